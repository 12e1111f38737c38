"""Seeded synthetic workloads for the five benchmark configurations (shapes, context lengths,
block tables) and their cache contents.

Shapes follow the configurations the backend is measured on:
  C1  fp32 KV, B=4, Hq=Hkv=8, D=64, ctx U{1..256}, 128-block pool (disjoint slices of one
      seeded permutation)                                   -- CPU-parity case
  C2  bf16 KV, B=64, Hq=32, Hkv=8, D=128, ctx log-U[128, 4096], pool = 1.1 x need, shuffled
  C3  48 decode (log-U[256, 4096]) + 8 prefill chunks of 512 on a prefix U{0..2048}
  C4  int8 KV (+ fp32 scale per block and KV head), B=128, ctx log-U[128, 8192], 1 % outlier
      channels x 8, one quantising append per sequence
  C5  bf16 KV, B=8, ctx U{16384..32768}, first 8192 tokens (512 blocks) shared by every table
Block size is 16 throughout. The block tables are what the reference's BlockTable /
KVCacheBlockManager would hand over once flattened (int32 [num_seqs][max_blocks], -1 padded).
numpy generates the index data and small caches; large caches are generated on the GPU with torch.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

BLOCK = 16


@dataclass
class Workload:
    name: str
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    kv_dtype: int  # PA_DTYPE_*
    q_dtype: int
    context_lens: np.ndarray  # int32 [S] -- tokens each decode query attends to (incl. the new one)
    block_tables: np.ndarray  # int32 [S][max_blocks]
    num_blocks: int
    value_scale: float = 1.0  # K/V/Q ~ N(0,1) * value_scale
    outlier_channels: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int64))
    shared_prefix_blocks: int = 0
    # prefill part (C3)
    prefill_prefix: np.ndarray | None = None
    prefill_chunk: int = 0
    prefill_tables: np.ndarray | None = None

    @property
    def num_seqs(self) -> int:
        return len(self.context_lens)

    @property
    def max_blocks(self) -> int:
        return self.block_tables.shape[1]

    @property
    def max_context_len(self) -> int:
        return int(self.context_lens.max()) if len(self.context_lens) else 0

    def kv_bytes_per_token(self) -> float:
        elt = {0: 4, 1: 2, 2: 1}[self.kv_dtype]
        b = 2 * self.num_kv_heads * self.head_dim * elt
        if self.kv_dtype == 2:
            b += 2 * self.num_kv_heads * 4 / BLOCK  # per-(block, head) scales, K and V
        return b

    def distinct_tokens(self) -> int:
        """Tokens whose KV bytes are distinct in HBM (a shared prefix counts once)."""
        total = int(self.context_lens.sum())
        if self.shared_prefix_blocks:
            shared = self.shared_prefix_blocks * BLOCK
            total -= (self.num_seqs - 1) * shared
        return total

    def decode_algorithmic_bytes(self) -> float:
        """Distinct KV bytes + Q read + O write (fp32) + block tables + context lengths."""
        q_elt = 2 if self.q_dtype == 1 else 4
        qo = self.num_seqs * self.num_q_heads * self.head_dim * (q_elt + 4)
        tables = self.block_tables.size * 4 + self.num_seqs * 4
        return self.distinct_tokens() * self.kv_bytes_per_token() + qo + tables


def _log_uniform_lengths(rng, n, lo, hi):
    # T = floor(exp(U(ln lo, ln(hi + 1)))), clipped to [lo, hi]
    t = np.floor(np.exp(rng.uniform(math.log(lo), math.log(hi + 1), size=n))).astype(np.int64)
    return np.clip(t, lo, hi).astype(np.int32)


def _tables_from_pool(rng, lens, pool_blocks, max_blocks=None, shared=None):
    need = [(int(t) + BLOCK - 1) // BLOCK for t in lens]
    perm = rng.permutation(pool_blocks).astype(np.int32)
    mb = max_blocks or max(need + [1])
    tables = np.full((len(lens), mb), -1, np.int32)
    pos = 0
    for s, n in enumerate(need):
        start = 0
        if shared is not None:
            k = min(len(shared), n)
            tables[s, :k] = shared[:k]
            start = k
        tables[s, start:n] = perm[pos:pos + n - start]
        pos += n - start
    return tables


def make_c1(seed=1, batch=4):
    rng = np.random.default_rng(seed)
    lens = rng.integers(1, 257, size=batch).astype(np.int32)
    pool = 128
    tables = _tables_from_pool(rng, lens, pool)
    return Workload("C1", 8, 8, 64, 0, 0, lens, tables, pool)


def make_c2(seed=2, batch=64, lo=128, hi=4096):
    rng = np.random.default_rng(seed)
    lens = _log_uniform_lengths(rng, batch, lo, hi)
    need = int(sum((int(t) + BLOCK - 1) // BLOCK for t in lens))
    pool = int(math.ceil(1.1 * need))
    tables = _tables_from_pool(rng, lens, pool)
    return Workload("C2", 32, 8, 128, 1, 1, lens, tables, pool, value_scale=0.5)


def make_c4(seed=4, batch=128, lo=128, hi=8192):
    rng = np.random.default_rng(seed)
    lens = _log_uniform_lengths(rng, batch, lo, hi)
    need = int(sum((int(t) + BLOCK - 1) // BLOCK for t in lens))
    pool = int(math.ceil(1.1 * need))
    tables = _tables_from_pool(rng, lens, pool)
    n_ch = 8 * 128
    outliers = np.sort(rng.choice(n_ch, size=max(1, round(0.01 * n_ch)), replace=False))
    return Workload("C4", 32, 8, 128, 2, 0, lens, tables, pool, outlier_channels=outliers)


def make_c5(seed=5, batch=8, lo=16384, hi=32768, prefix_tokens=8192):
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, size=batch).astype(np.int32)
    shared_n = prefix_tokens // BLOCK
    private = int(sum((int(t) + BLOCK - 1) // BLOCK - shared_n for t in lens))
    pool = shared_n + private
    perm = rng.permutation(pool).astype(np.int32)
    shared = perm[:shared_n]
    rest_rng = np.random.default_rng(seed + 1000)
    need = [(int(t) + BLOCK - 1) // BLOCK for t in lens]
    tables = np.full((batch, max(need)), -1, np.int32)
    pos = shared_n
    for s, n in enumerate(need):
        tables[s, :shared_n] = shared
        tables[s, shared_n:n] = perm[pos:pos + n - shared_n]
        pos += n - shared_n
    del rest_rng
    return Workload("C5", 32, 8, 128, 1, 1, lens, tables, pool, shared_prefix_blocks=shared_n)


def make_c3(seed=3, n_decode=48, n_prefill=8, chunk=512):
    rng = np.random.default_rng(seed)
    lens = _log_uniform_lengths(rng, n_decode, 256, 4096)
    prefix = rng.integers(0, 2049, size=n_prefill).astype(np.int32)
    pre_tot = prefix + chunk
    need_d = int(sum((int(t) + BLOCK - 1) // BLOCK for t in lens))
    need_p = int(sum((int(t) + BLOCK - 1) // BLOCK for t in pre_tot))
    pool = int(math.ceil(1.1 * (need_d + need_p)))
    all_lens = np.concatenate([lens, pre_tot]).astype(np.int32)
    tables_all = _tables_from_pool(rng, all_lens, pool)
    w = Workload("C3", 32, 8, 128, 1, 1, lens, np.ascontiguousarray(tables_all[:n_decode]), pool,
                 value_scale=0.5)
    w.prefill_prefix = prefix
    w.prefill_chunk = chunk
    w.prefill_tables = np.ascontiguousarray(tables_all[n_decode:])
    return w


def make_small(seed, *, num_seqs, lens, Hq, Hkv, D, kv_dtype, q_dtype, extra_blocks=7,
               value_scale=1.0):
    """Arbitrary small ragged case with a shuffled pool (used by parity tests)."""
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int32)
    assert len(lens) == num_seqs
    need = int(sum(max(0, (int(t) + BLOCK - 1) // BLOCK) for t in lens))
    pool = need + extra_blocks
    tables = _tables_from_pool(rng, lens, pool)
    return Workload("small", Hq, Hkv, D, kv_dtype, q_dtype, lens, tables, pool, value_scale=value_scale)


# ---- cache contents ------------------------------------------------------------------------------
def _bf16_bits(x: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def numpy_inputs(w: Workload, seed: int):
    """q and caches as numpy arrays (fp32 or bf16 bits / int8 codes + scales).

    fp32/bf16 caches: every pool row is N(0,1) * value_scale (bf16 by truncation).
    int8 caches: the fp32 source rows (with outlier channels x8) are quantised with absmax/127 per
    (block, KV head) over the block's 16 rows, which is what one append of a full block produces.
    Returns dict(q, k_cache, v_cache, k_scale, v_scale, k_absmax, v_absmax, k_src, v_src).
    """
    rng = np.random.default_rng(seed)
    S, Hq, Hkv, D, nb = w.num_seqs, w.num_q_heads, w.num_kv_heads, w.head_dim, w.num_blocks
    q = (rng.standard_normal((S, Hq, D), dtype=np.float32) * np.float32(w.value_scale)).astype(np.float32)
    shape = (nb, Hkv, BLOCK, D)
    k = (rng.standard_normal(shape, dtype=np.float32) * np.float32(w.value_scale)).astype(np.float32)
    v = (rng.standard_normal(shape, dtype=np.float32) * np.float32(w.value_scale)).astype(np.float32)
    out = {"k_scale": None, "v_scale": None, "k_absmax": None, "v_absmax": None}
    out["q"] = _bf16_bits(q) if w.q_dtype == 1 else q
    if w.kv_dtype == 0:
        out["k_cache"], out["v_cache"] = k, v
    elif w.kv_dtype == 1:
        out["k_cache"], out["v_cache"] = _bf16_bits(k), _bf16_bits(v)
    else:
        if len(w.outlier_channels):
            flat_k = k.transpose(0, 2, 1, 3).reshape(nb, BLOCK, Hkv * D)
            flat_v = v.transpose(0, 2, 1, 3).reshape(nb, BLOCK, Hkv * D)
            flat_k[:, :, w.outlier_channels] *= np.float32(8)
            flat_v[:, :, w.outlier_channels] *= np.float32(8)
            k = np.ascontiguousarray(flat_k.reshape(nb, BLOCK, Hkv, D).transpose(0, 2, 1, 3))
            v = np.ascontiguousarray(flat_v.reshape(nb, BLOCK, Hkv, D).transpose(0, 2, 1, 3))
        out["k_src"], out["v_src"] = k, v
    return out
