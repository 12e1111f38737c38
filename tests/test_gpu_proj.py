"""Q/K/V and output projections through the C-ABI. The GEMMs are checked against the oracle's
Linear within a tolerance stated here (bf16 operands, fp32 accumulation: |gpu - ref| <= 1e-3 *
max|ref|); everything after the GEMM is bit-exact against the oracle applied to the GPU's own GEMM
output: Q is its truncation to bf16 and the cache bytes (and int8 statistics) are pa_kv_append of
its K and V columns with fp32 input.

Batches of at most 64 tokens take the library's weight-streaming kernel (k split over workgroups,
partials added in a fixed order); larger ones rocBLAS. Cases cover both, a partial 64-column tile
(160 columns), a single token, a token count off the 16-token tiles, and determinism (two calls
agree bit for bit)."""
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


@pytest.mark.parametrize("kv_dtype,hkv,hq,d,hidden,n_tok", [
    (1, 8, 32, 128, 512, 40), (2, 2, 8, 64, 256, 33), (0, 4, 8, 128, 384, 17), (1, 8, 32, 128, 4096, 64),
    (1, 1, 3, 32, 1024, 1),     # 160 columns: a partial 64-column tile; one token
    (2, 8, 32, 128, 4096, 64),  # int8 cache at the Llama-3-8B shape
    (1, 2, 8, 64, 512, 100),    # past 64 tokens: rocBLAS
])
def test_qkv_project_append(kv_dtype, hkv, hq, d, hidden, n_tok):
    import torch

    rng = np.random.default_rng(20 + kv_dtype)
    nb = max(64, n_tok)
    cfg, k, v, stats = caches(kv_dtype, nb=nb, hkv=hkv, d=d, seed=21)
    cfg.num_q_heads, cfg.q_dtype = hq, 1
    cols = (hq + 2 * hkv) * d
    x = orc.bf16_from_f32(rng.standard_normal((n_tok, hidden), dtype=np.float32))
    w = orc.bf16_from_f32((rng.standard_normal((cols, hidden), dtype=np.float32) / np.sqrt(hidden)).astype(np.float32))
    # one token per block, at a random row of it
    slots = (rng.permutation(nb)[:n_tok] * 16 + rng.integers(0, 16, n_tok)).astype(np.int64)
    if n_tok > 3:
        slots[3] = -1  # skipped
    gk, gv = to_gpu(k), to_gpu(v)
    gs = tuple(to_gpu(s) for s in stats) if stats else (None, None, None, None)
    q_out = empty_gpu((n_tok, hq, d), np.uint16)
    wsb = pa.qkv_workspace_size(cfg, n_tok)
    assert wsb >= n_tok * cols * 4
    ws = empty_gpu((wsb,), np.uint8)
    print(f"qkv kv_dtype={kv_dtype} hq={hq} hkv={hkv} d={d} hidden={hidden} n_tok={n_tok}", flush=True)
    pa.qkv_project_append(None, cfg, to_gpu(x), to_gpu(w), hidden, n_tok, to_gpu(slots), q_out, gk, gv, *gs, ws, wsb)
    torch.cuda.synchronize()
    y = to_np(ws)[:n_tok * cols * 4].view(np.float32).reshape(n_tok, cols)
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


def test_qkv_project_is_deterministic():
    """Two calls on the same input give the same GEMM output and Q bit for bit (the split partials
    are added in a fixed order)."""
    import torch

    rng = np.random.default_rng(25)
    hq, hkv, d, hidden, n_tok = 32, 8, 128, 4096, 64
    cfg, k, v, _ = caches(1, nb=64, hkv=hkv, d=d, seed=26)
    cfg.num_q_heads, cfg.q_dtype = hq, 1
    cols = (hq + 2 * hkv) * d
    x = to_gpu(orc.bf16_from_f32(rng.standard_normal((n_tok, hidden), dtype=np.float32)))
    w = to_gpu(orc.bf16_from_f32((rng.standard_normal((cols, hidden), dtype=np.float32) / 64).astype(np.float32)))
    slots = to_gpu(np.full(n_tok, -1, np.int64))  # nothing appended
    wsb = pa.qkv_workspace_size(cfg, n_tok)
    outs = []
    for _ in range(2):
        q_out = empty_gpu((n_tok, hq, d), np.uint16)
        ws = empty_gpu((wsb,), np.uint8)
        pa.qkv_project_append(None, cfg, x, w, hidden, n_tok, slots, q_out, to_gpu(k), to_gpu(v), None, None, None,
                              None, ws, wsb)
        torch.cuda.synchronize()
        outs.append((to_np(ws)[:n_tok * cols * 4].copy(), to_np(q_out, np.uint16).copy()))
    np.testing.assert_array_equal(outs[0][0], outs[1][0])
    np.testing.assert_array_equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("hq,d,hidden,n_tok", [(32, 128, 4096, 64), (8, 64, 256, 5), (4, 64, 160, 21),
                                               (8, 64, 512, 100)])
def test_o_project(hq, d, hidden, n_tok):
    import torch

    rng = np.random.default_rng(30)
    cfg = pa.make_config(num_q_heads=hq, num_kv_heads=hq // 4, head_dim=d, kv_dtype=1, q_dtype=1, num_blocks=4)
    attn = rng.standard_normal((n_tok, hq, d), dtype=np.float32)
    w = orc.bf16_from_f32((rng.standard_normal((hidden, hq * d), dtype=np.float32) / np.sqrt(hq * d)).astype(np.float32))
    y = empty_gpu((n_tok, hidden), np.float32)
    wsb = pa.o_workspace_size(cfg, hidden, n_tok)
    ws = empty_gpu((wsb,), np.uint8)
    print(f"o hq={hq} d={d} hidden={hidden} n_tok={n_tok}", flush=True)
    pa.o_project(None, cfg, to_gpu(attn), to_gpu(w), hidden, n_tok, y, ws, wsb)
    torch.cuda.synchronize()
    a16 = orc.bf16_from_f32(attn.reshape(n_tok, -1))
    if n_tok > 64:  # the rocBLAS path multiplies a bf16 copy held in the workspace
        np.testing.assert_array_equal(to_np(ws)[:a16.nbytes].view(np.uint16).reshape(a16.shape), a16)
    gemm_close(to_np(y), orc.linear(orc.f32_from_bf16(a16), orc.f32_from_bf16(w)), "o gemm")


@pytest.mark.parametrize("n_tok", [64, 100])
def test_o_project_truncates_attention_output(n_tok):
    """The attention output is truncated to bf16, not rounded: every value sits just below the next
    bf16 (low 16 bits 0xff00) and all operands are positive, so rounding would raise y by about
    0.4% of its size, four times the tolerance."""
    import torch

    rng = np.random.default_rng(31)
    hq, d, hidden = 32, 128, 256
    cfg = pa.make_config(num_q_heads=hq, num_kv_heads=8, head_dim=d, kv_dtype=1, q_dtype=1, num_blocks=4)
    base = orc.bf16_from_f32(rng.uniform(0.5, 1.0, (n_tok, hq * d)).astype(np.float32))
    attn = ((base.astype(np.uint32) << 16) | 0xff00).view(np.float32).reshape(n_tok, hq, d)
    w = orc.bf16_from_f32(rng.uniform(0.0, 1.0 / (hq * d), (hidden, hq * d)).astype(np.float32))
    y = empty_gpu((n_tok, hidden), np.float32)
    wsb = pa.o_workspace_size(cfg, hidden, n_tok)
    ws = empty_gpu((wsb,), np.uint8)
    pa.o_project(None, cfg, to_gpu(attn), to_gpu(w), hidden, n_tok, y, ws, wsb)
    torch.cuda.synchronize()
    ref_t = orc.linear(orc.f32_from_bf16(base), orc.f32_from_bf16(w))
    ref_r = orc.linear(orc.f32_from_bf16(base + 1), orc.f32_from_bf16(w))  # what rounding to nearest gives
    assert np.abs(ref_r - ref_t).max() > 3 * GEMM_RTOL * np.abs(ref_t).max()  # the case separates the two
    gemm_close(to_np(y), ref_t, "o gemm (truncation)")
