"""The shared-prefix plan's grouping (pa_prefix_plan_fill, host only: no GPU call).

Rule: shared_with_prev[s] links sequence s to s - 1; linked runs are cut into groups of at most
16 / G members (G = Hq / Hkv); a group of one is no group; a group shares the minimum link inside
it; every member records (group, shared), everyone else (-1, 0). Pinned by hand-worked cases and
by invariants over random links.
"""
import numpy as np
import pytest

import paged_attention as pa


def cfg(G):
    return pa.make_config(num_q_heads=8 * G, num_kv_heads=8, head_dim=128, kv_dtype=1, num_blocks=64)


def test_plan_hand_worked():
    # G = 4: groups of up to 4. Run 0..5 (links 7, 5, 9, 3, 3) -> {0..3 shares min(7,5,9)=5}, {4,5 shares 3};
    # 6 alone; run 7..8 (link 2) -> {7,8 shares 2}.
    links = [0, 7, 5, 9, 3, 3, 0, 0, 2]
    groups, seqinfo = pa.prefix_plan_fill(cfg(4), links)
    np.testing.assert_array_equal(groups, [[0, 4, 5], [4, 2, 3], [7, 2, 2]])
    np.testing.assert_array_equal(seqinfo, [[0, 5], [0, 5], [0, 5], [0, 5], [1, 3], [1, 3], [-1, 0], [2, 2], [2, 2]])


def test_plan_cap_by_head_ratio():
    links = [0] + [4] * 8  # one run of 9
    g1, _ = pa.prefix_plan_fill(cfg(1), links)   # cap 16: one group
    np.testing.assert_array_equal(g1, [[0, 9, 4]])
    g8, s8 = pa.prefix_plan_fill(cfg(8), links)  # cap 2: four pairs, sequence 8 alone
    np.testing.assert_array_equal(g8, [[0, 2, 4], [2, 2, 4], [4, 2, 4], [6, 2, 4]])
    assert tuple(s8[8]) == (-1, 0)
    g16, s16 = pa.prefix_plan_fill(cfg(16), links)  # cap 1: no group at all
    assert g16.shape == (0, 3) and np.all(s16[:, 0] == -1)


@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_plan_invariants_random(G):
    rng = np.random.default_rng(G)
    for _ in range(50):
        S = int(rng.integers(1, 60))
        links = np.where(rng.random(S) < 0.7, rng.integers(1, 40, S), 0).astype(np.int32)
        groups, seqinfo = pa.prefix_plan_fill(cfg(G), links)
        assert len(groups) <= S // 2
        covered = np.full(S, -1)
        for g, (first, nm, shared) in enumerate(groups):
            assert 2 <= nm <= 16 // G
            assert np.all(links[first + 1:first + nm] > 0)       # members are linked
            assert shared == links[first + 1:first + nm].min()   # and share the minimum link
            assert np.all(covered[first:first + nm] == -1)       # groups are disjoint
            covered[first:first + nm] = g
        np.testing.assert_array_equal(seqinfo[:, 0], covered)
        shared_of = np.array([groups[g][2] if g >= 0 else 0 for g in covered])
        np.testing.assert_array_equal(seqinfo[:, 1], shared_of)
        # a group is never cut short while its run continues and room is left
        for first, nm, _ in groups:
            end = first + nm
            if nm < 16 // G and end < S:
                assert links[end] == 0


def test_plan_rejects_bad_input():
    with pytest.raises(pa.PagedAttentionError):
        pa.prefix_plan_fill(cfg(4), [0, -1])
