"""Q/K/V and output projections through the C-ABI. The GEMMs are checked against the oracle's
Linear within a tolerance stated here (bf16 operands, fp32 accumulation: |gpu - ref| <= 1e-3 *
max|ref|); everything after the GEMM is bit-exact against the oracle applied to the GPU's own GEMM
output: Q is its truncation to bf16 and the cache bytes (and int8 statistics) are pa_kv_append of
its K and V columns with fp32 input."""
import numpy as np
import pytest

import paged_attention as pa
import pa_oracle as orc
from helpers import empty_gpu, to_gpu, to_np
from test_oracle_blocks import caches

pytestmark = pytest.mark.gpu

GEMM_RTOL = 1e-3  # relative to the largest |y|


def gemm_close(got, ref, what):
    err = np.abs(np.asarray(got, np.float64) - ref).max()
    assert err <= GEMM_RTOL * np.abs(ref).max(), f"{what}: max error {err} vs max |y| {np.abs(ref).max()}"


@pytest.mark.parametrize("kv_dtype,hkv,hq,d,hidden,n_tok", [(1, 8, 32, 128, 512, 40), (2, 2, 8, 64, 256, 33),
                                                           (0, 4, 8, 128, 384, 17), (1, 8, 32, 128, 4096, 64)])
def test_qkv_project_append(kv_dtype, hkv, hq, d, hidden, n_tok):
    import torch

    rng = np.random.default_rng(20 + kv_dtype)
    cfg, k, v, stats = caches(kv_dtype, nb=64, hkv=hkv, d=d, seed=21)
    cfg.num_q_heads, cfg.q_dtype = hq, 1
    cols = (hq + 2 * hkv) * d
    x = orc.bf16_from_f32(rng.standard_normal((n_tok, hidden), dtype=np.float32))
    w = orc.bf16_from_f32((rng.standard_normal((cols, hidden), dtype=np.float32) / np.sqrt(hidden)).astype(np.float32))
    # one token per block (int8 appends need a block's tokens consecutive in the call)
    slots = (rng.permutation(64)[:n_tok] * 16 + rng.integers(0, 16, n_tok)).astype(np.int64)
    slots[3] = -1  # skipped
    gk, gv = to_gpu(k), to_gpu(v)
    gs = tuple(to_gpu(s) for s in stats) if stats else (None, None, None, None)
    q_out = empty_gpu((n_tok, hq, d), np.uint16)
    wsb = pa.qkv_workspace_size(cfg, n_tok)
    assert wsb == n_tok * cols * 4
    ws = empty_gpu((wsb,), np.uint8)
    print(f"qkv kv_dtype={kv_dtype} hq={hq} hkv={hkv} d={d} hidden={hidden} n_tok={n_tok}", flush=True)
    pa.qkv_project_append(None, cfg, to_gpu(x), to_gpu(w), hidden, n_tok, to_gpu(slots), q_out, gk, gv, *gs, ws, wsb)
    torch.cuda.synchronize()
    y = to_np(ws).view(np.float32).reshape(n_tok, cols)
    gemm_close(y, orc.linear(orc.f32_from_bf16(x), orc.f32_from_bf16(w)), "qkv gemm")
    np.testing.assert_array_equal(to_np(q_out, np.uint16).reshape(n_tok, -1), orc.bf16_from_f32(y[:, :hq * d]))
    cfg_app = pa.make_config(num_q_heads=hq, num_kv_heads=hkv, head_dim=d, kv_dtype=kv_dtype, q_dtype=0,
                             num_blocks=cfg.num_blocks)
    kn = np.ascontiguousarray(y[:, hq * d:(hq + hkv) * d])
    vn = np.ascontiguousarray(y[:, (hq + hkv) * d:])
    st = stats if stats else (None, None, None, None)
    orc.kv_append(cfg_app, kn, vn, slots, k, v, *st)
    dt = {0: np.float32, 1: np.uint16, 2: np.int8}[kv_dtype]
    np.testing.assert_array_equal(to_np(gk, dt), k)
    np.testing.assert_array_equal(to_np(gv, dt), v)
    if stats:
        for a, b in zip(gs, stats):
            np.testing.assert_array_equal(to_np(a), b)


@pytest.mark.parametrize("hq,d,hidden,n_tok", [(32, 128, 4096, 64), (8, 64, 256, 5)])
def test_o_project(hq, d, hidden, n_tok):
    import torch

    rng = np.random.default_rng(30)
    cfg = pa.make_config(num_q_heads=hq, num_kv_heads=hq // 4, head_dim=d, kv_dtype=1, q_dtype=1, num_blocks=4)
    attn = rng.standard_normal((n_tok, hq, d), dtype=np.float32)
    w = orc.bf16_from_f32((rng.standard_normal((hidden, hq * d), dtype=np.float32) / np.sqrt(hq * d)).astype(np.float32))
    y = empty_gpu((n_tok, hidden), np.float32)
    wsb = pa.o_workspace_size(cfg, n_tok)
    ws = empty_gpu((wsb,), np.uint8)
    pa.o_project(None, cfg, to_gpu(attn), to_gpu(w), hidden, n_tok, y, ws, wsb)
    torch.cuda.synchronize()
    a16 = to_np(ws).view(np.uint16).reshape(n_tok, hq * d)
    np.testing.assert_array_equal(a16, orc.bf16_from_f32(attn.reshape(n_tok, -1)))
    gemm_close(to_np(y), orc.linear(orc.f32_from_bf16(a16), orc.f32_from_bf16(w)), "o gemm")
