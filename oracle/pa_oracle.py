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


# ---- whole-block moves (numpy: pure data movement) ---------------------------------------------
# Copy-on-write and swap of paged blocks: the copy the reference leaves to a comment at beam
# divergence (Sharing/BeamSearchBlockSharing.cs:69-79) and the block data moves of
# IPagedAttentionCache.GetBlockData / StoreBlockData (ContinuousBatching/KVCache/
# IPagedAttentionCache.cs:40-47, CacheBlockData.cs:7-12). Caches are numpy arrays whose first axis
# is the block; the statistics (int8) are [num_blocks][Hkv] float32 arrays, in the order
# k_scale, v_scale, k_absmax, v_absmax.

def _rows(a, nb):
    return a.reshape(nb, -1)


def copy_blocks(cfg, k_cache, v_cache, stats, pairs):
    """In place: block dst := block src for each valid pair with src != dst (pa_copy_blocks)."""
    nb = cfg.num_blocks
    for src, dst in np.asarray(pairs, np.int64).reshape(-1, 2):
        if not (0 <= src < nb and 0 <= dst < nb) or src == dst:
            continue
        for a in (k_cache, v_cache) + tuple(s for s in (stats or ()) if s is not None):
            _rows(a, nb)[dst] = _rows(a, nb)[src]


def block_record_bytes(cfg):
    elt = {0: 4, 1: 2, 2: 1}[cfg.kv_dtype]
    part = cfg.num_kv_heads * 16 * cfg.head_dim * elt
    return 2 * part + (16 * cfg.num_kv_heads if cfg.kv_dtype == 2 else 0)


def gather_blocks(cfg, k_cache, v_cache, stats, block_ids, packed):
    """Record i of packed (uint8 [n][record]) := K bytes, V bytes, then k_scale, v_scale,
    k_absmax, v_absmax of block block_ids[i] (pa_gather_blocks); invalid ids leave the record."""
    nb = cfg.num_blocks
    for i, b in enumerate(np.asarray(block_ids, np.int64)):
        if not 0 <= b < nb:
            continue
        parts = [_rows(k_cache, nb)[b].view(np.uint8), _rows(v_cache, nb)[b].view(np.uint8)]
        if cfg.kv_dtype == 2:
            parts += [np.ascontiguousarray(s[b]).view(np.uint8) for s in stats]
        packed[i] = np.concatenate(parts)


def scatter_blocks(cfg, k_cache, v_cache, stats, block_ids, packed):
    """Block block_ids[i] := record i of packed (pa_scatter_blocks)."""
    nb = cfg.num_blocks
    part = _rows(k_cache, nb)[0].view(np.uint8).size
    for i, b in enumerate(np.asarray(block_ids, np.int64)):
        if not 0 <= b < nb:
            continue
        rec = packed[i]
        _rows(k_cache, nb)[b] = rec[:part].view(k_cache.dtype)
        _rows(v_cache, nb)[b] = rec[part:2 * part].view(v_cache.dtype)
        if cfg.kv_dtype == 2:
            hkv = cfg.num_kv_heads
            for j, s in enumerate(stats):
                s[b] = rec[2 * part + 4 * hkv * j:2 * part + 4 * hkv * (j + 1)].view(np.float32)


def read_block_f32(cfg, k_cache, v_cache, k_scale, v_scale, block, tokens):
    """Tokens [0, tokens) of a block as fp32 [tokens][Hkv][D] (pa_read_block_f32): K tile
    [16][D], V tile [D][16]; bf16 widened, int8 code * scale (Dequantize,
    Quantization/Operations/QuantizationOperations.cs:83-88)."""
    nb, hkv, d = cfg.num_blocks, cfg.num_kv_heads, cfg.head_dim
    kt = k_cache.reshape(nb, hkv, 16, d)[block, :, :tokens, :]        # [Hkv][t][D]
    vt = v_cache.reshape(nb, hkv, d, 16)[block, :, :, :tokens]        # [Hkv][D][t]
    if cfg.kv_dtype == 1:
        kt, vt = f32_from_bf16(kt), f32_from_bf16(vt)
    elif cfg.kv_dtype == 2:
        kt = kt.astype(np.float32) * k_scale[block][:, None, None]
        vt = vt.astype(np.float32) * v_scale[block][:, None, None]
    return (np.ascontiguousarray(np.transpose(kt, (1, 0, 2)).astype(np.float32)),
            np.ascontiguousarray(np.transpose(vt, (2, 0, 1)).astype(np.float32)))


# ---- projections either side of attention (numpy) ----------------------------------------------
def linear(x, w):
    """Linear.Forward without bias (src/MLFramework/Modules/Linear.cs:81-110): y = x W^T, here in
    float64 from the given (bf16-valued) operands; x [n][in], w [out][in]."""
    return np.asarray(x, np.float64) @ np.asarray(w, np.float64).T
