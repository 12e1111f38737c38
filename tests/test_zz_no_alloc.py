"""pa_paged_decode_noalloc: pa_paged_decode with its split-K workspace in the library's per-device
scratch array instead of a caller buffer. Each call is checked against pa_paged_decode with a
caller workspace on the same inputs (same kernels and split, so the outputs agree bit for bit, well
inside the parity bar), twice in a row with the second input smaller than the first (the scratch
keeps the first call's contents), and against the oracle; a shape whose workspace exceeds the
scratch is refused on the host."""
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
    dev = pa.Device(0)  # pa_device_open resolves the scratch address of device 0
    s = pa.Stream(dev)
    yield s
    s.destroy()
    dev.close()


def _case(seed, lens, Hq, Hkv, D, kv_dtype, q_dtype):
    w = wl.make_small(seed, num_seqs=len(lens), lens=lens, Hq=Hq, Hkv=Hkv, D=D, kv_dtype=kv_dtype, q_dtype=q_dtype)
    inp = wl.numpy_inputs(w, seed + 1)
    return w, inp


def _run_both(stream, w, inp):
    import torch

    cfg = config_for(w)
    S, mcl = w.num_seqs, w.max_context_len
    if w.kv_dtype == 2:  # int8: the pool quantised by the GPU append (checked against the oracle's)
        host, g = build_int8_caches(w, inp, stream)
        caches = (g["kc"], g["vc"], g["ks"], g["vs"])
    else:
        host = dict(k_cache=inp["k_cache"], v_cache=inp["v_cache"], k_scale=None, v_scale=None)
        caches = (to_gpu(inp["k_cache"]), to_gpu(inp["v_cache"]), None, None)
    args = (to_gpu(inp["q"]), *caches, to_gpu(w.block_tables), to_gpu(w.context_lens), S, w.max_blocks, mcl)
    wsb = pa.decode_workspace_size(cfg, S, mcl)
    ws = empty_gpu((max(wsb, 1),), np.uint8)
    ref_out = empty_gpu((S, w.num_q_heads, w.head_dim), np.float32)
    out = empty_gpu((S, w.num_q_heads, w.head_dim), np.float32)
    out.fill_(float("nan"))
    torch.cuda.synchronize()
    pa.paged_decode(stream, cfg, ref_out, *args, ws, wsb)
    pa.paged_decode_noalloc(stream, cfg, out, *args)
    stream.synchronize()
    got, want = to_np(out).copy(), to_np(ref_out).copy()
    ref = orc.paged_decode(cfg, inp["q"], host["k_cache"], host["v_cache"], host["k_scale"], host["v_scale"],
                           w.block_tables, w.context_lens, n_threads=NTHREADS)
    return got, want, ref, wsb


@pytest.mark.parametrize("kv_dtype,q_dtype,Hq,Hkv,D", [(1, 1, 32, 8, 128), (0, 0, 8, 2, 64), (2, 0, 32, 8, 128)])
def test_noalloc_decode_matches_workspace_decode_twice(stream, kv_dtype, q_dtype, Hq, Hkv, D):
    rng = np.random.default_rng(40 + kv_dtype)
    big = rng.integers(1, 3000, size=40).tolist() + [4096, 0, 1]
    small = rng.integers(1, 700, size=6).tolist() + [650]
    for i, lens in enumerate((big, small)):
        w, inp = _case(600 + 10 * i + kv_dtype, lens, Hq, Hkv, D, kv_dtype, q_dtype)
        got, want, ref, wsb = _run_both(stream, w, inp)
        assert wsb > 0, "the case must use a split-K workspace"
        np.testing.assert_array_equal(got, want, err_msg=f"call {i}: noalloc output differs from pa_paged_decode")
        check_close(got, ref, **tol_for(kv_dtype), what=f"call {i} vs oracle")


def test_noalloc_chunked_call_matches_workspace_decode_twice(stream):
    """More sequences than one persistent launch takes (2047): the call runs in chunks of
    sequences that reuse the same scratch one after another; twice in a row, the second smaller."""
    rng = np.random.default_rng(47)
    for i, n in enumerate((2300, 2100)):
        lens = rng.integers(1, 48, size=n).tolist()
        w, inp = _case(700 + i, lens, 8, 2, 64, 1, 1)
        got, want, ref, wsb = _run_both(stream, w, inp)
        assert 0 < wsb <= pa.PA_NOALLOC_SCRATCH_BYTES
        np.testing.assert_array_equal(got, want, err_msg=f"call {i}: noalloc output differs from pa_paged_decode")
        check_close(got, ref, **tol_for(1), what=f"chunked call {i} vs oracle")


def test_noalloc_refuses_a_shape_beyond_its_scratch(stream):
    # fp32 cache, 256-token partitions: 2000 sequences x 32 heads x 391 partials needs ~1.3 GB
    cfg = pa.make_config(num_q_heads=32, num_kv_heads=32, head_dim=128, kv_dtype=0, q_dtype=0, num_blocks=8)
    assert pa.decode_workspace_size(cfg, 2000, 100000) > (32 << 20)
    dummy = empty_gpu((1024,), np.uint8)
    with pytest.raises(pa.PagedAttentionError) as e:
        pa.paged_decode_noalloc(stream, cfg, dummy, dummy, dummy, dummy, None, None, dummy, dummy, 2000, 6250, 100000)
    assert e.value.status == pa.PA_ERROR_WORKSPACE_TOO_SMALL
