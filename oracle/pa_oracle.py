"""ctypes wrapper of oracle/libpa_oracle.so -- TEST INFRASTRUCTURE ONLY.

Loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker / the
timed CPU baseline. The product path (ml-framework_amd/libpa_hip.so) never imports this module.
All arrays are numpy, C-contiguous, with the dtypes the C functions expect.
"""
from __future__ import annotations

import ctypes
import os
import sys

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libpa_oracle.so")

sys.path.insert(0, os.path.join(os.path.dirname(_HERE), "ml-framework_amd"))
from paged_attention import PaConfig  # noqa: E402  (the shared pa_config layout)

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_CFG = ctypes.POINTER(PaConfig)
_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        L.orc_bf16_from_f32.restype = ctypes.c_uint16
        L.orc_bf16_from_f32.argtypes = [ctypes.c_float]
        L.orc_f32_from_bf16.restype = ctypes.c_float
        L.orc_f32_from_bf16.argtypes = [ctypes.c_uint16]
        L.orc_round_half_away_from_zero.restype = ctypes.c_int32
        L.orc_round_half_away_from_zero.argtypes = [ctypes.c_float]
        L.orc_quantize_symmetric.restype = ctypes.c_int8
        L.orc_quantize_symmetric.argtypes = [ctypes.c_float, ctypes.c_float]
        L.orc_dequantize.restype = ctypes.c_float
        L.orc_dequantize.argtypes = [ctypes.c_int8, ctypes.c_float]
        L.orc_sdpa.restype = ctypes.c_int
        L.orc_sdpa.argtypes = [_P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32, ctypes.c_float, _I32]
        L.orc_bm_create.restype = _P
        L.orc_bm_create.argtypes = [_I32]
        L.orc_bm_destroy.restype = None
        L.orc_bm_destroy.argtypes = [_P]
        L.orc_bm_allocate_block.restype = _I32
        L.orc_bm_allocate_block.argtypes = [_P]
        L.orc_bm_allocate_blocks.restype = _I32
        L.orc_bm_allocate_blocks.argtypes = [_P, _I32, _P]
        L.orc_bm_free_block.restype = None
        L.orc_bm_free_block.argtypes = [_P, _I32]
        L.orc_bm_free_count.restype = _I32
        L.orc_bm_free_count.argtypes = [_P]
        L.orc_build_slot_mapping.restype = None
        L.orc_build_slot_mapping.argtypes = [_CFG, _P, _I32, _P, _P, _P, _I32, _P]
        L.orc_kv_append.restype = ctypes.c_int
        L.orc_kv_append.argtypes = [_CFG, _P, _P, _P, _I32, _P, _P, _P, _P, _P, _P]
        L.orc_paged_decode.restype = ctypes.c_int
        L.orc_paged_decode.argtypes = [_CFG, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32]
        L.orc_chunked_prefill.restype = ctypes.c_int
        L.orc_chunked_prefill.argtypes = [_CFG, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32]
        _lib = L
    return _lib


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def bf16_from_f32(x: np.ndarray) -> np.ndarray:
    """Vectorised BFloat16.cs:99-107 (identical to orc_bf16_from_f32, checked in tests)."""
    return (np.ascontiguousarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def f32_from_bf16(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def sdpa(q, k, v, phase, scale=-1.0, force_causal=False):
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    b, nq, H, D = q.shape
    nc = k.shape[1]
    out = np.zeros_like(q)
    rc = lib().orc_sdpa(_p(q), _p(k), _p(v), _p(out), b, nq, nc, H, D, phase, scale, int(force_causal))
    assert rc == 0
    return out


class BlockManager:
    def __init__(self, total):
        self.h = lib().orc_bm_create(total)

    def allocate_block(self):
        return lib().orc_bm_allocate_block(self.h)

    def allocate_blocks(self, n):
        out = np.zeros(max(n, 1), np.int32)
        got = lib().orc_bm_allocate_blocks(self.h, n, _p(out))
        return list(out[:got])

    def free_block(self, b):
        lib().orc_bm_free_block(self.h, b)

    def free_count(self):
        return lib().orc_bm_free_count(self.h)

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_bm_destroy(self.h)
            self.h = None


def build_slot_mapping(cfg, block_tables, start_pos, num_new, token_offset):
    block_tables = np.ascontiguousarray(block_tables, np.int32)
    start_pos = np.ascontiguousarray(start_pos, np.int32)
    num_new = np.ascontiguousarray(num_new, np.int32)
    token_offset = np.ascontiguousarray(token_offset, np.int32)
    n = int((token_offset + num_new).max()) if len(num_new) else 0
    out = np.full(max(n, 1), -2, np.int64)
    lib().orc_build_slot_mapping(ctypes.byref(cfg), _p(block_tables), block_tables.shape[1],
                                 _p(start_pos), _p(num_new), _p(token_offset), len(num_new), _p(out))
    return out[:n]


def kv_append(cfg, k_new, v_new, slot_mapping, k_cache, v_cache, k_scale=None, v_scale=None,
              k_absmax=None, v_absmax=None):
    """In-place on the cache arrays, like pa_kv_append."""
    slot_mapping = np.ascontiguousarray(slot_mapping, np.int64)
    rc = lib().orc_kv_append(ctypes.byref(cfg), _p(k_new), _p(v_new), _p(slot_mapping),
                             len(slot_mapping), _p(k_cache), _p(v_cache), _p(k_scale), _p(v_scale),
                             _p(k_absmax), _p(v_absmax))
    assert rc == 0


def paged_decode(cfg, q, k_cache, v_cache, k_scale, v_scale, block_tables, context_lens, n_threads=1):
    block_tables = np.ascontiguousarray(block_tables, np.int32)
    context_lens = np.ascontiguousarray(context_lens, np.int32)
    S = len(context_lens)
    out = np.zeros((S, cfg.num_q_heads, cfg.head_dim), np.float32)
    rc = lib().orc_paged_decode(ctypes.byref(cfg), _p(out), _p(q), _p(k_cache), _p(v_cache),
                                _p(k_scale), _p(v_scale), _p(block_tables), _p(context_lens), S,
                                block_tables.shape[1], n_threads)
    assert rc == 0
    return out


def chunked_prefill(cfg, q, q_start_loc, prefix_lens, k_cache, v_cache, k_scale, v_scale,
                    block_tables, n_threads=1):
    block_tables = np.ascontiguousarray(block_tables, np.int32)
    q_start_loc = np.ascontiguousarray(q_start_loc, np.int32)
    prefix_lens = np.ascontiguousarray(prefix_lens, np.int32)
    S = len(prefix_lens)
    out = np.zeros((int(q_start_loc[-1]), cfg.num_q_heads, cfg.head_dim), np.float32)
    rc = lib().orc_chunked_prefill(ctypes.byref(cfg), _p(out), _p(q), _p(q_start_loc),
                                   _p(prefix_lens), _p(k_cache), _p(v_cache), _p(k_scale),
                                   _p(v_scale), _p(block_tables), S, block_tables.shape[1], n_threads)
    assert rc == 0
    return out
