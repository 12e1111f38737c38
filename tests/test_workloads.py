"""Shapes of the seeded benchmark workloads (the five BASELINE.json configurations)."""
import numpy as np

import workloads as wl


def _check_tables(w, shared_blocks=0):
    seen = {}
    for s, T in enumerate(w.context_lens):
        n = (int(T) + 15) // 16
        row = w.block_tables[s]
        assert np.all(row[:n] >= 0) and np.all(row[:n] < w.num_blocks)
        assert np.all(row[n:] == -1)
        for i, b in enumerate(row[:n]):
            if i < shared_blocks:
                continue
            assert b not in seen, "private blocks must not be shared between sequences"
            seen[b] = s


def test_c1():
    w = wl.make_c1()
    assert (w.num_seqs, w.num_q_heads, w.num_kv_heads, w.head_dim, w.kv_dtype) == (4, 8, 8, 64, 0)
    assert w.num_blocks == 128 and w.context_lens.min() >= 1 and w.context_lens.max() <= 256
    _check_tables(w)


def test_c2():
    w = wl.make_c2()
    assert (w.num_seqs, w.num_q_heads, w.num_kv_heads, w.head_dim, w.kv_dtype) == (64, 32, 8, 128, 1)
    assert w.context_lens.min() >= 128 and w.context_lens.max() <= 4096
    need = sum((int(t) + 15) // 16 for t in w.context_lens)
    assert w.num_blocks == int(np.ceil(1.1 * need))
    _check_tables(w)
    assert w.kv_bytes_per_token() == 4096


def test_c3():
    w = wl.make_c3()
    assert w.num_seqs == 48 and len(w.prefill_prefix) == 8 and w.prefill_chunk == 512
    assert w.context_lens.min() >= 256 and w.context_lens.max() <= 4096
    assert w.prefill_prefix.min() >= 0 and w.prefill_prefix.max() <= 2048


def test_c4():
    w = wl.make_c4()
    assert (w.num_seqs, w.kv_dtype) == (128, 2) and w.context_lens.max() <= 8192
    assert len(w.outlier_channels) == 10  # 1 % of the 8 x 128 channels
    assert w.kv_bytes_per_token() == 2 * 8 * 128 + 2 * 8 * 4 / 16


def test_c5_shared_prefix():
    w = wl.make_c5()
    assert w.num_seqs == 8 and w.context_lens.min() >= 16384 and w.context_lens.max() <= 32768
    shared = w.block_tables[:, :512]
    assert np.all(shared == shared[0]), "the first 512 blocks appear in every table"
    _check_tables(w, shared_blocks=512)
    assert w.distinct_tokens() == int(w.context_lens.sum()) - 7 * 8192
