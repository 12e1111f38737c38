"""GPU parity at the benchmarked sizes: the exact calls bench.py times, on the full configurations,
against the CPU oracle.

  C2  pa_paged_decode_append on the whole batch (64 sequences, log-U[128, 4096], bf16 cache, the
      library-default split): the headline call.
  C4  the int8 step as bench.py times it: 128 sequences up to 8192 tokens, caches quantised from an
      fp32 source with 1 % outlier channels x 8, then the fused quantising 1-token append + decode.
  C3  the mixed step exactly as bench.py issues it: pa_paged_decode_append over the 48 decode
      sequences, pa_kv_append of the 8 prefill chunks (512 tokens each), pa_chunked_prefill over
      all 8 chunks.
  C1  (test_gpu_parity.py) and C5 (test_gpu_prefix.py) are covered next to their other cases.

Bar: cache bytes, int8 codes, scales and absmax bit-exact (orc_kv_append); attention outputs
within (2e-3, 1e-2) for bf16 and (2e-2, 1e-2) for int8 caches of the oracle's per-sequence
StandardPagedAttentionKernel restatement (DecodeOrchestrator.cs:85-109,
StandardPagedAttentionKernel.cs:21-84).
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


def _sync():
    import torch

    torch.cuda.synchronize()


def _new_tokens(w, rng, outliers=False):
    """The appended token of every sequence, [S][Hkv][D] in the activation dtype (fp32 source with
    the workload's outlier channels x 8 when asked)."""
    S, Hkv, D = w.num_seqs, w.num_kv_heads, w.head_dim
    k = (rng.standard_normal((S, Hkv, D), dtype=np.float32) * np.float32(w.value_scale)).astype(np.float32)
    v = (rng.standard_normal((S, Hkv, D), dtype=np.float32) * np.float32(w.value_scale)).astype(np.float32)
    if outliers and len(w.outlier_channels):
        for a in (k, v):
            a.reshape(S, Hkv * D)[:, w.outlier_channels] *= np.float32(8)
    if w.q_dtype == 1:
        k, v = orc.bf16_from_f32(k), orc.bf16_from_f32(v)
    return k, v


def _last_slots(w):
    pos = w.context_lens.astype(np.int64) - 1
    return w.block_tables[np.arange(w.num_seqs), pos // 16].astype(np.int64) * 16 + pos % 16


def _fused_step(stream, w, cfg, q, k_new, v_new, caches, scales):
    """One pa_paged_decode_append call over the whole batch with the library-default split."""
    S = w.num_seqs
    out = empty_gpu((S, w.num_q_heads, w.head_dim), np.float32)
    out.fill_(float("nan"))
    mcl = w.max_context_len
    wsb = pa.decode_workspace_size(cfg, S, mcl)
    ws = empty_gpu((max(wsb, 1),), np.uint8)
    ks, vs, ka, va = scales
    pa.paged_decode_append(stream, cfg, out, to_gpu(q), to_gpu(k_new), to_gpu(v_new), caches[0], caches[1], ks, vs,
                           ka, va, to_gpu(w.block_tables), to_gpu(w.context_lens), S, w.max_blocks, mcl, ws, wsb)
    _sync()
    return to_np(out).copy()


def test_c2_headline_call_full(stream):
    """C2 as benched: pa_paged_decode_append, 64 sequences, library-default partition."""
    w = wl.make_c2()
    assert w.num_seqs == 64 and w.kv_dtype == 1 and w.q_dtype == 1
    inp = wl.numpy_inputs(w, 202)
    cfg = config_for(w)
    k_new, v_new = _new_tokens(w, np.random.default_rng(203))
    hk, hv = inp["k_cache"].copy(), inp["v_cache"].copy()
    gk, gv = to_gpu(hk), to_gpu(hv)
    orc.kv_append(cfg, k_new, v_new, _last_slots(w), hk, hv)
    ref = orc.paged_decode(cfg, inp["q"], hk, hv, None, None, w.block_tables, w.context_lens, n_threads=NTHREADS)
    got = _fused_step(stream, w, cfg, inp["q"], k_new, v_new, (gk, gv), (None, None, None, None))
    np.testing.assert_array_equal(to_np(gk, np.uint16), hk, err_msg="C2: K cache after the fused append")
    np.testing.assert_array_equal(to_np(gv, np.uint16), hv, err_msg="C2: V cache after the fused append")
    check_close(got, ref, **tol_for(1), what="C2 pa_paged_decode_append")


def test_c4_step_full(stream):
    """C4 as benched: 128 sequences, int8 caches built by the quantising append from an fp32
    source with outlier channels, then the fused 1-token quantising append (outliers in the new
    token too, so scales grow and blocks are requantised) and the decode of the whole batch."""
    w = wl.make_c4()
    assert w.num_seqs == 128 and w.kv_dtype == 2
    inp = wl.numpy_inputs(w, 404)
    host, g = build_int8_caches(w, inp, stream)  # whole pool appended on the GPU and in the oracle
    q = inp["q"]
    del inp
    cfg = config_for(w)
    k_new, v_new = _new_tokens(w, np.random.default_rng(405), outliers=True)
    hk, hv = host["k_cache"], host["v_cache"]
    hks, hvs = host["k_scale"], host["v_scale"]
    hka, hva = to_np(g["ka"]).copy(), to_np(g["va"]).copy()
    orc.kv_append(cfg, k_new, v_new, _last_slots(w), hk, hv, hks, hvs, hka, hva)
    ref = orc.paged_decode(cfg, q, hk, hv, hks, hvs, w.block_tables, w.context_lens, n_threads=NTHREADS)
    got = _fused_step(stream, w, cfg, q, k_new, v_new, (g["kc"], g["vc"]), (g["ks"], g["vs"], g["ka"], g["va"]))
    for name, dev, ref_arr in (("K codes", g["kc"], hk), ("V codes", g["vc"], hv), ("k_scale", g["ks"], hks),
                               ("v_scale", g["vs"], hvs), ("k_absmax", g["ka"], hka), ("v_absmax", g["va"], hva)):
        np.testing.assert_array_equal(to_np(dev), ref_arr, err_msg=f"C4: {name} after the fused append")
    check_close(got, ref, **tol_for(2), what="C4 pa_paged_decode_append")


def test_c3_step_as_benched(stream):
    """C3 as bench.py issues it: fused decode-append of the 48 decode sequences, the append of the
    8 x 512 prefill tokens, then the chunked prefill of all 8 chunks over prefix + chunk."""
    w = wl.make_c3()
    assert w.num_seqs == 48 and len(w.prefill_prefix) == 8 and w.prefill_chunk == 512
    inp = wl.numpy_inputs(w, 303)
    cfg = config_for(w)
    rng = np.random.default_rng(304)
    S, Hq, Hkv, D = w.num_seqs, w.num_q_heads, w.num_kv_heads, w.head_dim
    # decode part
    k_new, v_new = _new_tokens(w, rng)
    hk, hv = inp["k_cache"].copy(), inp["v_cache"].copy()
    gk, gv = to_gpu(hk), to_gpu(hv)
    orc.kv_append(cfg, k_new, v_new, _last_slots(w), hk, hv)
    # prefill part: 8 chunks of 512 new tokens at positions prefix .. prefix + 511
    P, L = w.prefill_prefix.astype(np.int64), w.prefill_chunk
    n_pre, tot = len(P), len(P) * L
    tab = w.prefill_tables
    pos = P[:, None] + np.arange(L)[None, :]
    slots = (tab[np.arange(n_pre)[:, None], pos // 16].astype(np.int64) * 16 + pos % 16).reshape(-1)
    q_pre = orc.bf16_from_f32((rng.standard_normal((tot, Hq, D), dtype=np.float32) * 0.5).astype(np.float32))
    k_pre = orc.bf16_from_f32((rng.standard_normal((tot, Hkv, D), dtype=np.float32) * 0.5).astype(np.float32))
    v_pre = orc.bf16_from_f32((rng.standard_normal((tot, Hkv, D), dtype=np.float32) * 0.5).astype(np.float32))
    q_start = (np.arange(n_pre + 1) * L).astype(np.int32)
    # GPU: the three calls in bench.py's order
    got_dec = _fused_step(stream, w, cfg, inp["q"], k_new, v_new, (gk, gv), (None, None, None, None))
    pa.kv_append(stream, cfg, to_gpu(k_pre), to_gpu(v_pre), to_gpu(slots), tot, gk, gv)
    out_pre = empty_gpu((tot, Hq, D), np.float32)
    out_pre.fill_(float("nan"))
    pa.chunked_prefill(stream, cfg, out_pre, to_gpu(q_pre), to_gpu(q_start), to_gpu(P.astype(np.int32)), gk, gv,
                       None, None, to_gpu(tab), n_pre, tab.shape[1], L)
    _sync()
    # oracle: decode over the decode-appended cache, then the chunk append, then the prefill
    ref_dec = orc.paged_decode(cfg, inp["q"], hk, hv, None, None, w.block_tables, w.context_lens,
                               n_threads=NTHREADS)
    orc.kv_append(cfg, k_pre, v_pre, slots, hk, hv)
    ref_pre = orc.chunked_prefill(cfg, q_pre, q_start, P.astype(np.int32), hk, hv, None, None, tab,
                                  n_threads=NTHREADS)
    np.testing.assert_array_equal(to_np(gk, np.uint16), hk, err_msg="C3: K cache after both appends")
    np.testing.assert_array_equal(to_np(gv, np.uint16), hv, err_msg="C3: V cache after both appends")
    check_close(got_dec, ref_dec, **tol_for(1), what="C3 decode")
    check_close(to_np(out_pre), ref_pre, **tol_for(1), what="C3 prefill (8 chunks)")
