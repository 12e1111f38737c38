"""GPU parity of pa_chunked_prefill against the CPU oracle (orc_chunked_prefill), through the C-ABI.

The oracle gathers each sequence's prefix + chunk through its block table and runs the reference's
StandardPagedAttentionKernel loops with the Decode-phase (bottom-right) mask
(Kernels/StandardPagedAttentionKernel.cs:57-66, :219-255). Bar: (1e-5, 1e-4) for fp32 KV,
(2e-3, 1e-2) for bf16 KV and (2e-2, 1e-2) for int8 KV, |gpu - oracle| <= atol + rtol*|oracle|.
"""
import os

import numpy as np
import pytest

import paged_attention as pa
import pa_oracle as orc
import workloads as wl
from helpers import build_int8_caches, check_close, config_for, empty_gpu, to_gpu, to_np, tol_for

pytestmark = pytest.mark.gpu
NTHREADS = min(16, os.cpu_count() or 1)


@pytest.fixture(scope="module")
def stream():
    import torch

    torch.cuda.init()
    s = pa.TorchStream.current(0)
    yield s.stream
    s.stream.destroy()
    s.device.close()


def run_prefill(stream, *, prefix, chunk, Hq, Hkv, D, kv_dtype, q_dtype, flags=0, seed=0, table_edit=None,
                input_edit=None):
    import torch

    prefix = np.asarray(prefix, np.int32)
    chunk = np.asarray(chunk, np.int32)
    totals = prefix + chunk
    w = wl.make_small(300 + seed, num_seqs=len(prefix), lens=totals, Hq=Hq, Hkv=Hkv, D=D, kv_dtype=kv_dtype,
                      q_dtype=q_dtype)
    if table_edit is not None:
        table_edit(w)
    inp = wl.numpy_inputs(w, 400 + seed)
    if input_edit is not None:
        input_edit(w, inp)
    cfg = config_for(w, flags=flags)
    if kv_dtype == 2:
        host, g = build_int8_caches(w, inp, stream)
        kc, vc, ks, vs = g["kc"], g["vc"], g["ks"], g["vs"]
    else:
        host = dict(k_cache=inp["k_cache"], v_cache=inp["v_cache"], k_scale=None, v_scale=None)
        kc, vc, ks, vs = to_gpu(inp["k_cache"]), to_gpu(inp["v_cache"]), None, None
    rng = np.random.default_rng(500 + seed)
    q_start = np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32)
    nq = int(q_start[-1])
    q = rng.standard_normal((nq, Hq, D)).astype(np.float32)
    if q_dtype == 1:
        q = orc.bf16_from_f32(q)
    ref = orc.chunked_prefill(cfg, q, q_start, prefix, host["k_cache"], host["v_cache"], host["k_scale"],
                              host["v_scale"], w.block_tables, n_threads=NTHREADS)
    out = empty_gpu((nq, Hq, D), np.float32)
    out.fill_(float("nan"))
    pa.chunked_prefill(stream, cfg, out, to_gpu(q), to_gpu(q_start), to_gpu(prefix), kc, vc, ks, vs,
                       to_gpu(w.block_tables), len(prefix), w.max_blocks, int(chunk.max()))
    torch.cuda.synchronize()
    return to_np(out), ref


PREFIX = [0, 1, 15, 16, 17, 37, 300, 1000]
CHUNK = [33, 1, 16, 17, 100, 64, 5, 130]


@pytest.mark.parametrize("flags", [0, pa.PA_FLAG_REFERENCE_LITERAL_MASK, pa.PA_FLAG_NO_MASK])
@pytest.mark.parametrize("kv_dtype,q_dtype,Hq,Hkv,D", [
    (1, 1, 32, 8, 128), (1, 0, 8, 8, 64), (2, 1, 16, 2, 128), (2, 0, 8, 1, 64), (1, 1, 8, 4, 256),
    (2, 1, 8, 2, 256),
])
def test_prefill_ragged(stream, flags, kv_dtype, q_dtype, Hq, Hkv, D):
    got, ref = run_prefill(stream, prefix=PREFIX, chunk=CHUNK, Hq=Hq, Hkv=Hkv, D=D, kv_dtype=kv_dtype,
                           q_dtype=q_dtype, flags=flags, seed=D + kv_dtype)
    check_close(got, ref, **tol_for(kv_dtype), what=f"prefill flags={flags} kv={kv_dtype} D={D} G={Hq // Hkv}")


@pytest.mark.parametrize("flags", [0, pa.PA_FLAG_REFERENCE_LITERAL_MASK, pa.PA_FLAG_NO_MASK])
@pytest.mark.parametrize("q_dtype,Hq,Hkv,D", [(0, 8, 8, 128), (1, 16, 4, 64), (0, 8, 2, 32), (0, 4, 1, 256)])
def test_prefill_fp32_cache(stream, flags, q_dtype, Hq, Hkv, D):
    """fp32 caches through the fp32 prefill kernel (fp32 operands and accumulation), held to the
    fp32 bar over ragged chunks, scattered block tables and every mask mode."""
    got, ref = run_prefill(stream, prefix=PREFIX, chunk=CHUNK, Hq=Hq, Hkv=Hkv, D=D, kv_dtype=0, q_dtype=q_dtype,
                           flags=flags, seed=D + Hq)
    check_close(got, ref, **tol_for(0), what=f"fp32 prefill flags={flags} D={D} G={Hq // Hkv}")


def test_prefill_fp32_long_prompt(stream):
    """A 512-query prompt after a 700-token prefix and a whole 512-token prompt, fp32 cache."""
    got, ref = run_prefill(stream, prefix=[700, 0], chunk=[512, 512], Hq=8, Hkv=8, D=128, kv_dtype=0, q_dtype=0,
                           seed=21)
    check_close(got, ref, **tol_for(0), what="fp32 512-query prefill")


def test_prefill_fp32_invalid_block_ids_read_as_zero(stream):
    def edit(w):
        w.block_tables[0, 1] = -1
        w.block_tables[1, 3] = w.num_blocks + 5

    got, ref = run_prefill(stream, prefix=[40, 20], chunk=[30, 50], Hq=8, Hkv=2, D=64, kv_dtype=0, q_dtype=0,
                           seed=22, table_edit=edit)
    check_close(got, ref, **tol_for(0), what="fp32 invalid ids")


def test_prefill_empty_chunks_and_single_query(stream):
    got, ref = run_prefill(stream, prefix=[5, 0, 40, 0], chunk=[0, 1, 0, 20], Hq=16, Hkv=4, D=128, kv_dtype=1,
                           q_dtype=1, seed=3)
    check_close(got, ref, **tol_for(1), what="empty chunks")


def test_prefill_invalid_block_ids_read_as_zero(stream):
    def edit(w):
        w.block_tables[0, 2] = -1
        w.block_tables[1, 1] = w.num_blocks + 3

    got, ref = run_prefill(stream, prefix=[40, 20], chunk=[30, 50], Hq=8, Hkv=2, D=64, kv_dtype=1, q_dtype=0,
                           seed=4, table_edit=edit)
    check_close(got, ref, **tol_for(1), what="invalid ids")


def test_prefill_c3_shape(stream):
    """C3's prefill geometry (Hq 32, Hkv 8, D 128, 512-token chunks) on two of its sequences."""
    got, ref = run_prefill(stream, prefix=[0, 700], chunk=[512, 512], Hq=32, Hkv=8, D=128, kv_dtype=1, q_dtype=1,
                           seed=5)
    check_close(got, ref, **tol_for(1), what="C3 prefill")


def test_prefill_rows_match_decode(stream):
    """The last query of a chunk attends to the whole context: its row equals a decode of that token."""
    import torch

    prefix, chunk = np.array([100, 0, 513], np.int32), np.array([20, 7, 64], np.int32)
    got, _ = run_prefill(stream, prefix=prefix, chunk=chunk, Hq=16, Hkv=4, D=128, kv_dtype=1, q_dtype=1, seed=6)
    # same inputs, rebuilt deterministically, decoded at the last position of every chunk
    totals = prefix + chunk
    w = wl.make_small(306, num_seqs=3, lens=totals, Hq=16, Hkv=4, D=128, kv_dtype=1, q_dtype=1)
    inp = wl.numpy_inputs(w, 406)
    rng = np.random.default_rng(506)
    q_start = np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32)
    q = orc.bf16_from_f32(rng.standard_normal((int(q_start[-1]), 16, 128)).astype(np.float32))
    q_last = np.ascontiguousarray(q[q_start[1:] - 1])
    cfg = config_for(w)
    out = empty_gpu((3, 16, 128), np.float32)
    wsb = pa.decode_workspace_size(cfg, 3, int(totals.max()))
    ws = empty_gpu((max(wsb, 1),), np.uint8)
    pa.paged_decode(stream, cfg, out, to_gpu(q_last), to_gpu(inp["k_cache"]), to_gpu(inp["v_cache"]), None, None,
                    to_gpu(w.block_tables), to_gpu(totals), 3, w.max_blocks, int(totals.max()), ws, wsb)
    torch.cuda.synchronize()
    check_close(got[q_start[1:] - 1], to_np(out), **tol_for(1), what="last prefill row vs decode")


def _bf16_outliers(w, inp):
    """About 0.3 % of the bf16 V cache set to +-[65536, 1e5): magnitudes fp16 cannot hold."""
    rng = np.random.default_rng(77)
    v = inp["v_cache"].view(np.uint16).reshape(-1)
    idx = rng.choice(v.size, size=max(8, v.size // 300), replace=False)
    mag = rng.uniform(65536.0, 1e5, size=idx.size).astype(np.float32)
    sign = np.where(rng.random(idx.size) < 0.5, -1.0, 1.0).astype(np.float32)
    v[idx] = orc.bf16_from_f32(mag * sign)


def _scale_v(factor):
    """The whole V cache multiplied by a power of two: every bf16 value and every int8 code stays
    the same up to the exact factor (int8: the scale absmax / 127 takes the factor exactly, the
    codes do not change), so the exact attention output is the unscaled one times the factor."""
    def edit(w, inp):
        if w.kv_dtype == 2:
            inp["v_src"] *= np.float32(factor)
        else:
            v = orc.f32_from_bf16(inp["v_cache"]) * np.float32(factor)
            inp["v_cache"] = orc.bf16_from_f32(v)
    edit.factor = factor
    return edit


@pytest.mark.parametrize("flags", [0, pa.PA_FLAG_REFERENCE_LITERAL_MASK, pa.PA_FLAG_NO_MASK])
@pytest.mark.parametrize("kv_dtype,q_dtype,Hq,Hkv,D,edit", [
    (1, 1, 32, 8, 128, _bf16_outliers), (1, 0, 8, 2, 64, _bf16_outliers),
    (1, 1, 32, 8, 128, _scale_v(2.0 ** 16)), (2, 1, 16, 4, 128, _scale_v(4096.0)), (2, 0, 8, 8, 64, _scale_v(4096.0)),
], ids=["bf16-outliers", "bf16-outliers-d64", "bf16-x65536", "int8-x4096", "int8-x4096-d64"])
def test_prefill_values_beyond_fp16_range(stream, flags, kv_dtype, q_dtype, Hq, Hkv, D, edit):
    """V magnitudes past fp16's 65504.
    bf16 outliers: 0.3 % of V entries at +-[65536, 1e5) among N(0,1) values, at the unchanged bar
    (an output dim mixes only that dim's V values, so the outliers' dims are held to 1e-2 of their
    size). Scaled V (bf16 x 2^16: |V| up to ~3e5; int8 x 4096: block V scales ~100, P times the scale
    far past fp16): attention is linear in V and the factor is exact, so outputs divided by the
    factor are held to the unit-scale bar -- the bar the errors of fp16 / bf16 probabilities scale
    with."""
    got, ref = run_prefill(stream, prefix=[0, 17, 300, 40], chunk=[40, 33, 64, 1], Hq=Hq, Hkv=Hkv, D=D,
                           kv_dtype=kv_dtype, q_dtype=q_dtype, flags=flags, seed=11 + D + kv_dtype,
                           input_edit=edit)
    f = getattr(edit, "factor", 1.0)
    assert np.abs(ref).max() > 1000.0, "the case must reach large outputs"
    check_close(got / f, ref / f, **tol_for(kv_dtype), what=f"large V kv={kv_dtype} D={D} flags={flags} x{f}")
