"""Shared helpers of the test-suite: device buffers, the C-ABI calls with torch-backed memory,
oracle-built int8 caches and the tolerance check."""
from __future__ import annotations

import numpy as np

import paged_attention as pa
import pa_oracle as orc

BLOCK = 16

# Tolerances of the parity bar: |gpu - oracle| <= atol + rtol * |oracle|, fp32 accumulation.
# bf16 and int8 caches: the bar north_star states. fp32 caches: the VALU kernel computes in fp32
# throughout (only the order of the sums and the exp differ from the oracle), so it is held to
# about 100 fp32 ulps of the outputs' scale.
TOL_BF16 = dict(atol=2e-3, rtol=1e-2)
TOL_FP32 = dict(atol=1e-5, rtol=1e-4)
TOL_INT8 = dict(atol=2e-2, rtol=1e-2)


def tol_for(kv_dtype):
    return {0: TOL_FP32, 1: TOL_BF16, 2: TOL_INT8}[kv_dtype]


def cuda():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    return torch.device("cuda:0")


_NP2TORCH = None


def to_gpu(a: np.ndarray):
    """Copies a numpy array to the GPU keeping its bytes (uint16 travels as int16)."""
    import torch

    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a.copy()).to(cuda())


def to_np(t, dtype=None) -> np.ndarray:
    a = t.detach().cpu().numpy()
    if dtype is not None:
        a = a.view(dtype)
    return a


def empty_gpu(shape, np_dtype):
    import torch

    tdt = {np.float32: torch.float32, np.int8: torch.int8, np.uint16: torch.int16,
           np.int16: torch.int16, np.int32: torch.int32, np.int64: torch.int64,
           np.uint8: torch.uint8}[np.dtype(np_dtype).type]
    return torch.zeros(shape, dtype=tdt, device=cuda())


def check_close(got: np.ndarray, ref: np.ndarray, atol: float, rtol: float, what: str = ""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} elements out of tolerance (atol={atol}, rtol={rtol}); "
                             f"worst at {i}: got {got[i]}, ref {ref[i]}, max-abs {err.max():.3e}")
    return float(err.max())


def full_pool_slots(num_blocks):
    """slot_mapping that appends every row of every block, block by block."""
    return np.arange(num_blocks * BLOCK, dtype=np.int64)


def pool_tokens(src: np.ndarray) -> np.ndarray:
    """[nb][Hkv][16][D] source rows -> [nb*16][Hkv][D] token-major append input."""
    nb, hkv, b, d = src.shape
    return np.ascontiguousarray(src.transpose(0, 2, 1, 3).reshape(nb * b, hkv, d))


def config_for(w, **kw):
    return pa.make_config(num_q_heads=w.num_q_heads, num_kv_heads=w.num_kv_heads, head_dim=w.head_dim,
                          kv_dtype=w.kv_dtype, q_dtype=w.q_dtype, num_blocks=w.num_blocks, **kw)


def build_int8_caches(w, inp, stream):
    """Quantises the fp32 source pool with the oracle and with the GPU append; they must agree."""
    import torch

    cfg = config_for(w)
    nb, hkv, d = w.num_blocks, w.num_kv_heads, w.head_dim
    slots = full_pool_slots(nb)
    k_tok, v_tok = pool_tokens(inp["k_src"]), pool_tokens(inp["v_src"])
    if w.q_dtype == 1:
        k_tok, v_tok = orc.bf16_from_f32(k_tok), orc.bf16_from_f32(v_tok)
    kc = np.zeros((nb, hkv, 16, d), np.int8)
    vc = np.zeros_like(kc)
    ks, vs, ka, va = (np.zeros((nb, hkv), np.float32) for _ in range(4))
    orc.kv_append(cfg, k_tok, v_tok, slots, kc, vc, ks, vs, ka, va)
    g = {n: empty_gpu(a.shape, a.dtype) for n, a in
         dict(kc=kc, vc=vc, ks=ks, vs=vs, ka=ka, va=va).items()}
    gk, gv, gsl = to_gpu(k_tok), to_gpu(v_tok), to_gpu(slots)
    pa.kv_append(stream, cfg, gk, gv, gsl, len(slots), g["kc"], g["vc"], g["ks"], g["vs"], g["ka"], g["va"])
    torch.cuda.synchronize()
    for n, a in dict(kc=kc, vc=vc, ks=ks, vs=vs, ka=ka, va=va).items():
        np.testing.assert_array_equal(to_np(g[n]), a, err_msg=f"int8 pool build: {n} differs")
    return dict(k_cache=kc, v_cache=vc, k_scale=ks, v_scale=vs), g
