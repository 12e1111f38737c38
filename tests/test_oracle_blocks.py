"""The oracle's whole-block moves (copy-on-write copy, swap gather / scatter, fp32 block view).

These are data movement, so they are pinned by closed forms and invariants: copies and round
trips reproduce the source bytes and leave every other block alone, records have the documented
byte layout, the fp32 view reads K as [16][D] and V as [D][16] per tile (a transposed read of a
tile built as 1000 d + t fails), int8 values are the exact products code * scale, and the write
is pa_kv_append at slots block * 16 + t.
"""
import numpy as np
import pytest

import pa_oracle as orc
from paged_attention import make_config


def caches(kv_dtype, nb=9, hkv=2, d=64, seed=0):
    rng = np.random.default_rng(seed)
    cfg = make_config(num_q_heads=2 * hkv, num_kv_heads=hkv, head_dim=d, kv_dtype=kv_dtype, q_dtype=0,
                      num_blocks=nb)
    shape = (nb, hkv, 16, d)
    if kv_dtype == 0:
        k = rng.standard_normal(shape, dtype=np.float32)
        v = rng.standard_normal(shape, dtype=np.float32)
    elif kv_dtype == 1:
        k = rng.integers(0, 1 << 16, shape, dtype=np.uint16)
        v = rng.integers(0, 1 << 16, shape, dtype=np.uint16)
    else:
        k = rng.integers(-127, 128, shape, dtype=np.int8)
        v = rng.integers(-127, 128, shape, dtype=np.int8)
    stats = None
    if kv_dtype == 2:
        ks, vs = (rng.uniform(0.01, 0.1, (nb, hkv)).astype(np.float32) for _ in range(2))
        stats = (ks, vs, ks * 127, vs * 127)
    return cfg, k, v, stats


@pytest.mark.parametrize("kv_dtype", [0, 1, 2])
def test_copy_blocks_copies_pairs_and_nothing_else(kv_dtype):
    cfg, k, v, stats = caches(kv_dtype)
    k0, v0 = k.copy(), v.copy()
    s0 = tuple(s.copy() for s in stats) if stats else None
    pairs = [(1, 4), (7, 2), (3, 3), (-1, 5), (8, 99)]  # a self pair and two invalid ones
    orc.copy_blocks(cfg, k, v, stats, pairs)
    for b in range(cfg.num_blocks):
        src = {4: 1, 2: 7}.get(b, b)
        np.testing.assert_array_equal(k[b], k0[src])
        np.testing.assert_array_equal(v[b], v0[src])
        if stats:
            for s, o in zip(stats, s0):
                np.testing.assert_array_equal(s[b], o[src])


@pytest.mark.parametrize("kv_dtype", [0, 1, 2])
def test_gather_scatter_round_trip_and_record_layout(kv_dtype):
    cfg, k, v, stats = caches(kv_dtype, seed=1)
    rec = orc.block_record_bytes(cfg)
    part = k[0].nbytes
    assert rec == 2 * part + (16 * cfg.num_kv_heads if kv_dtype == 2 else 0) and rec % 16 == 0
    ids = np.array([5, -3, 0, 8], np.int32)
    packed = np.full((len(ids), rec), 0xAB, np.uint8)
    orc.gather_blocks(cfg, k, v, stats, ids, packed)
    assert (packed[1] == 0xAB).all()  # invalid id: record untouched
    np.testing.assert_array_equal(packed[0][:part], k[5].reshape(-1).view(np.uint8))
    np.testing.assert_array_equal(packed[0][part:2 * part], v[5].reshape(-1).view(np.uint8))
    if kv_dtype == 2:
        tail = packed[3][2 * part:].view(np.float32).reshape(4, cfg.num_kv_heads)
        for j, s in enumerate(stats):
            np.testing.assert_array_equal(tail[j], s[8])
    # swap back into other blocks: those blocks now equal the originals, the rest is unchanged
    cfg2, k2, v2, stats2 = caches(kv_dtype, seed=2)
    k2b, v2b = k2.copy(), v2.copy()
    dst = np.array([1, 6, 2, 3], np.int32)
    orc.scatter_blocks(cfg2, k2, v2, stats2, np.where(ids >= 0, dst, -1), packed)
    for i, (s_id, d_id) in enumerate(zip(ids, dst)):
        if s_id < 0:
            np.testing.assert_array_equal(k2[d_id], k2b[d_id])
            continue
        np.testing.assert_array_equal(k2[d_id], k[s_id])
        np.testing.assert_array_equal(v2[d_id], v[s_id])
        if kv_dtype == 2:
            for s_new, s_old in zip(stats2, stats):
                np.testing.assert_array_equal(s_new[d_id], s_old[s_id])
    for b in set(range(cfg2.num_blocks)) - set(dst.tolist()):
        np.testing.assert_array_equal(k2[b], k2b[b])
        np.testing.assert_array_equal(v2[b], v2b[b])


def test_read_block_layout_closed_form():
    cfg, k, v, _ = caches(0, nb=3, hkv=2, d=64)
    d_idx, t_idx = np.meshgrid(np.arange(64), np.arange(16), indexing="ij")
    v.reshape(3, 2, 64, 16)[1, 1] = 1000 * d_idx + t_idx          # V tile [D][16]
    k.reshape(3, 2, 16, 64)[1, 0] = 1000 * t_idx.T + d_idx.T      # K tile [16][D]: 1000 t + d
    ko, vo = orc.read_block_f32(cfg, k, v, None, None, 1, 5)
    assert ko.shape == (5, 2, 64) and vo.shape == (5, 2, 64)
    for t in range(5):
        np.testing.assert_array_equal(vo[t, 1], 1000 * np.arange(64) + t)
        np.testing.assert_array_equal(ko[t, 0], 1000 * t + np.arange(64))


def test_read_block_dequant_exact_products_and_bf16_widening():
    cfg, k, v, stats = caches(2, seed=3)
    ko, vo = orc.read_block_f32(cfg, k, v, stats[0], stats[1], 4, 16)
    kt = k.reshape(cfg.num_blocks, cfg.num_kv_heads, 16, 64)[4]
    for h in range(cfg.num_kv_heads):
        np.testing.assert_array_equal(ko[:, h, :], kt[h].astype(np.float32) * np.float32(stats[0][4, h]))
    cfg, k, v, _ = caches(1, seed=4)
    k.reshape(-1)[:4] = [0x3F80, 0xBF80, 0x4049, 0x0001]  # 1, -1, 3.140625, smallest subnormal
    ko, _ = orc.read_block_f32(cfg, k, v, None, None, 0, 1)
    np.testing.assert_array_equal(ko[0, 0, :4], np.array([1.0, -1.0, 3.140625, 2.0 ** -133], np.float32))


@pytest.mark.parametrize("kv_dtype", [0, 1, 2])
def test_write_block_is_append_at_block_slots(kv_dtype):
    cfg, k, v, stats = caches(kv_dtype, seed=5)
    rng = np.random.default_rng(6)
    tokens = 11
    x = rng.standard_normal((tokens, cfg.num_kv_heads, 64), dtype=np.float32)
    y = rng.standard_normal((tokens, cfg.num_kv_heads, 64), dtype=np.float32)
    st = tuple(s.copy() for s in stats) if stats else (None, None, None, None)
    orc.kv_append(cfg, x, y, 3 * 16 + np.arange(tokens), k, v, *st)
    ko, vo = orc.read_block_f32(cfg, k, v, st[0], st[1], 3, tokens)
    if kv_dtype == 0:
        np.testing.assert_array_equal(ko, x)
    elif kv_dtype == 1:
        np.testing.assert_array_equal(ko, orc.f32_from_bf16(orc.bf16_from_f32(x)))
    else:  # block starts afresh: scale = absmax / 127 per head, error <= scale / 2
        for h in range(cfg.num_kv_heads):
            sc = np.float32(np.abs(x[:, h]).max()) / np.float32(127)
            assert st[0][3, h] == sc
            assert np.abs(ko[:, h] - x[:, h]).max() <= sc / 2 * (1 + 1e-6)
