"""Pins the CPU oracle (oracle/pa_oracle.c) before it is trusted as the GPU checker.

Each oracle function is checked against something other than a retyping of its own formula:
  - known-answer tests held by the reference's own test-suite
    (tests/MLFramework.Tests/Quantization/Operations/QuantizationOperationsTests.cs,
     .../Inference/PagedAttention/KVCacheBlockManagerTests.cs, BlockTableTests.cs,
     PagedAttentionFunctionalTests.cs);
  - closed forms and invariants (bf16 = upper 16 bits, slot = table[p/16]*16 + p%16, ties of the
    rounding rule, dequantisation error <= scale/2, T=1 => O=V, equal keys => O=mean(V));
  - an independent library routine: torch.nn.functional.scaled_dot_product_attention in float64
    on the CPU, with the reference's mask rules written as explicit boolean masks and the paged
    gather done by numpy fancy indexing;
  - brute force on small inputs (exact rational arithmetic with fractions.Fraction, a deque
    model of the FIFO free list).
"""
from collections import deque
from fractions import Fraction
import math

import numpy as np
import pytest
import torch

import pa_oracle as orc
import paged_attention as pa
import workloads as wl

L = orc.lib()
f32 = np.float32


# ---- bf16 (src/MLFramework/Amp/BFloat16.cs:99-117) -----------------------------------------------
def test_bf16_truncates_not_rounds():
    # bf16 keeps 7 mantissa bits (last one 2^-7). 1 + 2^-8 + 2^-9 drops 0.75 ulp: round-to-nearest
    # would give 1 + 2^-7 (0x3F81), truncation gives 1.0 (0x3F80).
    x = f32(1.0 + 2.0 ** -8 + 2.0 ** -9)
    b = L.orc_bf16_from_f32(x)
    assert b == 0x3F80
    assert L.orc_f32_from_bf16(b) == f32(1.0)
    assert L.orc_bf16_from_f32(f32(-(1.0 + 2.0 ** -7 + 2.0 ** -8))) == 0xBF81  # toward zero for negatives
    for v, bits in [(0.0, 0x0000), (-0.0, 0x8000), (1.0, 0x3F80), (-2.0, 0xC000), (float("inf"), 0x7F80),
                    (float("-inf"), 0xFF80)]:
        assert L.orc_bf16_from_f32(v) == bits
    assert (L.orc_bf16_from_f32(float("nan")) & 0x7F80) == 0x7F80


def test_bf16_vectorised_matches_scalar_and_closed_form():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(20000) * rng.choice([1e-30, 1e-3, 1.0, 1e3, 1e30], 20000)).astype(f32)
    v = orc.bf16_from_f32(x)
    assert np.array_equal(v, (x.view(np.uint32) >> 16).astype(np.uint16))
    for i in range(0, 20000, 997):
        assert L.orc_bf16_from_f32(float(x[i])) == v[i]
    back = orc.f32_from_bf16(v)
    assert np.array_equal(back.view(np.uint32), x.view(np.uint32) & 0xFFFF0000)


# ---- RoundHalfAwayFromZero / QuantizeSymmetric / Dequantize -------------------------------------
def test_quantize_reference_known_answers():
    # QuantizationOperationsTests.cs: QuantizeSymmetric_WithValidValue (1.0/0.5 -> 2),
    # Quantize_WithNegativeValue (-1.0/0.5 -> -2), Quantize_WithLargeValue (1000/0.5 -> 127),
    # Quantize_WithVeryNegativeValue (-1000/0.5 -> -128), QuantizeTensor ([-1,0,1,2]/0.5 ->
    # [-2,0,2,4]), QuantizeSymmetric_WithNaN_ReturnsZero.
    q = L.orc_quantize_symmetric
    assert q(1.0, 0.5) == 2
    assert q(-1.0, 0.5) == -2
    assert q(1000.0, 0.5) == 127
    assert q(-1000.0, 0.5) == -128
    assert [q(v, 0.5) for v in (-1.0, 0.0, 1.0, 2.0)] == [-2, 0, 2, 4]
    assert q(float("nan"), 0.5) == 0
    # Round half away from zero (the rule the reference's InlineData comments describe):
    # 1.25/0.5 = 2.5 -> 3, 1.75/0.5 = 3.5 -> 4, 0.25/0.5 = 0.5 -> 1, -0.25/0.5 = -0.5 -> -1.
    assert [q(v, 0.5) for v in (1.25, 1.75, 0.25, -0.25)] == [3, 4, 1, -1]


def test_round_half_away_ties_and_fp32_edge():
    r = L.orc_round_half_away_from_zero
    for k in range(-300, 301):
        assert r(k + 0.5) == (k + 1 if k >= 0 else k)  # ties go away from zero
        assert r(-(abs(k) + 0.5)) == -(abs(k) + 1)
        assert r(float(k)) == k
    # |v| + 0.5f is an fp32 add: 0.49999997f + 0.5f rounds to 1.0f, so the result is 1, not 0.
    assert r(float(f32(0.49999997))) == 1
    assert r(float(f32(-0.49999997))) == -1
    assert r(float("nan")) == 0
    assert r(float("inf")) == 2 ** 31 - 1 and r(float("-inf")) == -(2 ** 31)
    assert r(3e9) == 2 ** 31 - 1 and r(-3e9) == -(2 ** 31)  # saturating conversion


def _nearest_away(fr: Fraction) -> int:
    fl = math.floor(fr)
    d = fr - fl
    if d > Fraction(1, 2):
        return fl + 1
    if d < Fraction(1, 2):
        return fl
    return fl + 1 if fr > 0 else fl


def test_quantize_brute_force_exact_rationals():
    rng = np.random.default_rng(1)
    vals = (rng.standard_normal(6000) * 40).astype(f32)
    scales = rng.uniform(0.05, 2.0, 6000).astype(f32)
    for v, s in zip(vals, scales):
        quot = f32(v) / f32(s)  # the fp32 division the reference performs
        fr = Fraction(float(quot))
        frac_part = abs(fr - math.floor(fr))
        if abs(frac_part - Fraction(1, 2)) < Fraction(1, 2 ** 22):
            continue  # within an fp32 ulp of a tie: covered by the tie / edge tests above
        expect = max(-128, min(127, _nearest_away(fr)))
        assert L.orc_quantize_symmetric(float(v), float(s)) == expect, (v, s)


def test_dequantize_exact_product():
    rng = np.random.default_rng(2)
    for s in rng.uniform(1e-4, 3.0, 50).astype(f32):
        for qv in range(-128, 128):
            assert L.orc_dequantize(qv, float(s)) == f32(qv) * f32(s)


# ---- StandardPagedAttentionKernel (Kernels/StandardPagedAttentionKernel.cs:21-84) ---------------
def torch_sdpa(q, k, v, mask=None, scale=None):
    """float64 SDPA on [b, n, H, D] layouts; mask is [nq, nc] bool (True = attend)."""
    qt = torch.tensor(q, dtype=torch.float64).permute(0, 2, 1, 3)
    kt = torch.tensor(k, dtype=torch.float64).permute(0, 2, 1, 3)
    vt = torch.tensor(v, dtype=torch.float64).permute(0, 2, 1, 3)
    m = None if mask is None else torch.tensor(mask)
    o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=m, scale=scale)
    return o.permute(0, 2, 1, 3).numpy()


def bottom_right_mask(nq, nc):
    start = nc - nq
    return np.array([[c <= start + i for c in range(nc)] for i in range(nq)])


@pytest.mark.parametrize("phase", [pa.PA_PHASE_PREFILL, pa.PA_PHASE_DECODE])
@pytest.mark.parametrize("nq,nc", [(1, 1), (1, 9), (3, 7), (5, 5), (4, 11)])
def test_sdpa_matches_torch_with_reference_mask_rule(phase, nq, nc):
    rng = np.random.default_rng(10 * nq + nc + phase)
    b, H, D = 2, 3, 16
    q = rng.standard_normal((b, nq, H, D)).astype(f32)
    k = rng.standard_normal((b, nc, H, D)).astype(f32)
    v = rng.standard_normal((b, nc, H, D)).astype(f32)
    got = orc.sdpa(q, k, v, phase)
    # The reference masks only when phase == Decode and numCached > numQueries (:57).
    mask = bottom_right_mask(nq, nc) if (phase == pa.PA_PHASE_DECODE and nc > nq) else None
    np.testing.assert_allclose(got, torch_sdpa(q, k, v, mask), rtol=0, atol=2e-6)
    # force_causal applies the same bottom-right mask regardless of phase.
    got_c = orc.sdpa(q, k, v, phase, force_causal=True)
    np.testing.assert_allclose(got_c, torch_sdpa(q, k, v, bottom_right_mask(nq, nc)), rtol=0, atol=2e-6)


def test_sdpa_scale_rule():
    rng = np.random.default_rng(3)
    q, k, v = (rng.standard_normal((1, 2, 2, 32)).astype(f32) for _ in range(3))
    default = orc.sdpa(q, k, v, pa.PA_PHASE_PREFILL, scale=-1.0)
    np.testing.assert_allclose(default, torch_sdpa(q, k, v, scale=1 / math.sqrt(32)), atol=2e-6)
    custom = orc.sdpa(q, k, v, pa.PA_PHASE_PREFILL, scale=0.3)
    np.testing.assert_allclose(custom, torch_sdpa(q, k, v, scale=0.3), atol=2e-6)
    zero = orc.sdpa(q, k, v, pa.PA_PHASE_PREFILL, scale=0.0)  # scale <= 0 selects the default (:28)
    assert np.array_equal(zero, default)


def test_sdpa_closed_forms():
    rng = np.random.default_rng(4)
    # One cached token: the output is that token's value.
    q = rng.standard_normal((1, 1, 4, 8)).astype(f32)
    k = rng.standard_normal((1, 1, 4, 8)).astype(f32)
    v = rng.standard_normal((1, 1, 4, 8)).astype(f32)
    assert np.array_equal(orc.sdpa(q, k, v, pa.PA_PHASE_DECODE), v)
    # Identical keys: uniform weights, the output is the mean of the values.
    k = np.repeat(rng.standard_normal((1, 1, 4, 8)).astype(f32), 6, axis=1)
    v = rng.standard_normal((1, 6, 4, 8)).astype(f32)
    np.testing.assert_allclose(orc.sdpa(q, k, v, pa.PA_PHASE_DECODE)[0, 0], v[0].mean(axis=0), atol=1e-6)
    # One dominant score: the output is that token's value.
    k = rng.standard_normal((1, 6, 4, 8)).astype(f32) * 0.01
    k[0, 2] = q[0, 0] * 50
    np.testing.assert_allclose(orc.sdpa(q, k, v, pa.PA_PHASE_DECODE)[0, 0], v[0, 2], atol=1e-5)


def test_sdpa_single_query_decode_equals_prefill_and_stable_at_large_logits():
    # PagedAttentionFunctionalTests.cs:40-67 (one query: Decode == Prefill) and :255-277 (x100 inputs
    # produce finite outputs).
    rng = np.random.default_rng(5)
    q = (rng.uniform(-1, 1, (2, 1, 4, 32)) * 100).astype(f32)
    k = (rng.uniform(-1, 1, (2, 20, 4, 32)) * 100).astype(f32)
    v = rng.uniform(-1, 1, (2, 20, 4, 32)).astype(f32)
    d = orc.sdpa(q, k, v, pa.PA_PHASE_DECODE)
    p = orc.sdpa(q, k, v, pa.PA_PHASE_PREFILL)
    assert np.array_equal(d, p)
    assert np.all(np.isfinite(d))


# ---- KVCacheBlockManager (KVCacheBlockManager.cs:59-174) ------------------------------------------
def test_block_manager_reference_behaviour():
    bm = orc.BlockManager(100)
    assert bm.allocate_block() == 0  # KVCacheBlockManagerTests.cs:26-34: first id is 0 (FIFO from 0)
    assert bm.allocate_block() == 1
    assert bm.free_count() == 98
    # all-or-nothing AllocateBlocks (:71-83)
    assert bm.allocate_blocks(99) == []
    assert bm.free_count() == 98
    got = bm.allocate_blocks(98)
    assert got == list(range(2, 100)) and bm.free_count() == 0
    assert bm.allocate_block() == -1  # "No free blocks available" (:48-58)
    bm.free_block(7)
    bm.free_block(3)
    assert bm.allocate_blocks(2) == [7, 3]  # freed ids re-enqueued at the tail, in order


def test_block_manager_brute_force_against_deque():
    rng = np.random.default_rng(6)
    n = 37
    bm, model, live = orc.BlockManager(n), deque(range(n)), []
    for _ in range(3000):
        op = rng.integers(0, 3)
        if op == 0:
            got = bm.allocate_block()
            exp = model.popleft() if model else -1
            assert got == exp
            if got >= 0:
                live.append(got)
        elif op == 1 and live:
            b = live.pop(int(rng.integers(0, len(live))))
            bm.free_block(b)
            model.append(b)
        else:
            c = int(rng.integers(0, 6))
            got = bm.allocate_blocks(c)
            if len(model) >= c:
                exp = [model.popleft() for _ in range(c)]
                live.extend(exp)
            else:
                exp = []
            assert got == exp
        assert bm.free_count() == len(model)


# ---- slot mapping / BlockTable intent (BlockTableTests.cs:83-134) ----------------------------------
def test_slot_mapping_block_table_intent():
    cfg = pa.make_config(num_q_heads=1, num_kv_heads=1, head_dim=64, kv_dtype=0, num_blocks=10)
    tables = np.array([[5, 9, 2]], np.int32)
    slots = orc.build_slot_mapping(cfg, tables, [0], [48], [0])
    # block k of the sequence covers tokens [16k, 16k+15]
    for p in range(48):
        assert slots[p] == tables[0, p // 16] * 16 + p % 16
    assert slots[0] == 80 and slots[15] == 95 and slots[16] == 144 and slots[47] == 47


def test_slot_mapping_brute_force():
    rng = np.random.default_rng(7)
    S, mb = 9, 6
    tables = rng.integers(0, 200, (S, mb)).astype(np.int32)
    tables[rng.random((S, mb)) < 0.2] = -1
    start = rng.integers(0, mb * 16 + 5, S).astype(np.int32)
    num = rng.integers(0, 30, S).astype(np.int32)
    off = np.concatenate([[0], np.cumsum(num)[:-1]]).astype(np.int32)
    cfg = pa.make_config(num_q_heads=1, num_kv_heads=1, head_dim=64, kv_dtype=0, num_blocks=200)
    slots = orc.build_slot_mapping(cfg, tables, start, num, off)
    for s in range(S):
        for j in range(num[s]):
            p = start[s] + j
            lb = p // 16
            exp = -1
            if lb < mb and tables[s, lb] >= 0:
                exp = tables[s, lb] * 16 + p % 16
            assert slots[off[s] + j] == exp


# ---- KV append ------------------------------------------------------------------------------------
def _cache_index(is_v, blk, h, off, d, H, D):
    tile = (blk * H + h) * 16 * D
    return tile + (d * 16 + off if is_v else off * D + d)


@pytest.mark.parametrize("kv_dtype,q_dtype", [(0, 0), (1, 0), (1, 1), (0, 1)])
def test_append_plain_scatter(kv_dtype, q_dtype):
    rng = np.random.default_rng(8 + kv_dtype)
    nb, H, D, n = 12, 3, 64, 70
    cfg = pa.make_config(num_q_heads=H, num_kv_heads=H, head_dim=D, kv_dtype=kv_dtype, q_dtype=q_dtype,
                         num_blocks=nb)
    slots = rng.permutation(nb * 16)[:n].astype(np.int64)
    slots[::9] = -1
    slots[4] = nb * 16 + 2
    x = rng.standard_normal((n, H, D)).astype(f32)
    y = rng.standard_normal((n, H, D)).astype(f32)
    xin = orc.bf16_from_f32(x) if q_dtype == 1 else x
    yin = orc.bf16_from_f32(y) if q_dtype == 1 else y
    dt = np.uint16 if kv_dtype == 1 else f32
    kc = np.full((nb, H, 16, D), 7, dt)
    vc = np.full((nb, H, 16, D), 7, dt)
    orc.kv_append(cfg, xin, yin, slots, kc, vc)
    kf, vf = kc.reshape(-1), vc.reshape(-1)
    touched = np.zeros(kf.size, bool)
    for i in range(n):
        s = slots[i]
        if s < 0 or s >= nb * 16:
            continue
        for h in range(H):
            xv = orc.f32_from_bf16(xin[i, h]) if q_dtype == 1 else x[i, h]
            yv = orc.f32_from_bf16(yin[i, h]) if q_dtype == 1 else y[i, h]
            ek = orc.bf16_from_f32(xv) if kv_dtype == 1 else xv
            ev = orc.bf16_from_f32(yv) if kv_dtype == 1 else yv
            ki = np.array([_cache_index(False, s // 16, h, s % 16, d, H, D) for d in range(D)])
            vi = np.array([_cache_index(True, s // 16, h, s % 16, d, H, D) for d in range(D)])
            assert np.array_equal(kf[ki], ek) and np.array_equal(vf[vi], ev)
            touched[ki] = True
    assert np.all(kf[~touched] == 7)


def _int8_block(codes, scale, h, is_v, blk, D):
    """[16][D] dequantised view of one (block, head) tile."""
    tile = codes[blk, h].reshape(-1)
    rows = np.array([[tile[d * 16 + r] if is_v else tile[r * D + d] for d in range(D)] for r in range(16)])
    return rows.astype(f32) * f32(scale)


def test_append_int8_policy_invariants():
    rng = np.random.default_rng(9)
    nb, H, D = 4, 2, 64
    cfg = pa.make_config(num_q_heads=H, num_kv_heads=H, head_dim=D, kv_dtype=2, num_blocks=nb)
    kc = np.zeros((nb, H, 16, D), np.int8)
    vc = np.zeros_like(kc)
    ks, vs, ka, va = (np.zeros((nb, H), f32) for _ in range(4))
    # a full block from the fp32 source: scale = absmax / 127 (fp32 division), |codes| <= 127 and
    # the absmax element quantises to +-127; dequantisation error <= scale / 2.
    x = rng.standard_normal((16, H, D)).astype(f32)
    orc.kv_append(cfg, x, x, np.arange(16, dtype=np.int64) + 16, kc, vc, ks, vs, ka, va)
    for h in range(H):
        amax = np.abs(x[:, h]).max()
        assert ka[1, h] == amax and ks[1, h] == f32(amax) / f32(127)
        deq = _int8_block(kc, ks[1, h], h, False, 1, D)
        assert np.all(np.abs(deq - x[:, h]) <= ks[1, h] / 2 * (1 + 1e-6))
        assert np.abs(kc[1, h]).max() == 127
        assert np.array_equal(_int8_block(vc, vs[1, h], h, True, 1, D), deq)  # same data, V layout
    # a partial block, then a token within absmax (no growth: residents untouched), then an outlier
    # (growth: residents requantised, error bounded by the old + new half-steps).
    y = rng.standard_normal((5, H, D)).astype(f32)
    orc.kv_append(cfg, y, y, np.arange(5, dtype=np.int64) + 32, kc, vc, ks, vs, ka, va)
    before = kc[2].copy()
    small = (y[:1] * 0.5).astype(f32)
    orc.kv_append(cfg, small, small, np.array([32 + 5], np.int64), kc, vc, ks, vs, ka, va)
    assert np.array_equal(kc[2][:, :5], before[:, :5]) and ks[2, 0] == f32(np.abs(y[:, 0]).max()) / f32(127)
    old_scale = ks[2].copy()
    old_deq = [_int8_block(kc, old_scale[h], h, False, 2, D)[:6] for h in range(H)]
    big = (y[:1] * 9.0).astype(f32)
    orc.kv_append(cfg, big, big, np.array([32 + 6], np.int64), kc, vc, ks, vs, ka, va)
    for h in range(H):
        assert ks[2, h] == f32(np.abs(big[0, h]).max()) / f32(127) and ks[2, h] > old_scale[h]
        new_deq = _int8_block(kc, ks[2, h], h, False, 2, D)[:6]
        assert np.all(np.abs(new_deq - old_deq[h]) <= (ks[2, h] + old_scale[h]) / 2 * (1 + 1e-6))
    # writing row 0 starts the block afresh: statistics come from the new token only.
    z = (rng.standard_normal((1, H, D)) * 0.01).astype(f32)
    orc.kv_append(cfg, z, z, np.array([32], np.int64), kc, vc, ks, vs, ka, va)
    assert ka[2, 0] == np.abs(z[0, 0]).max()


def _requant_case(old_scale, new_amax, H=2, D=64, row=5):
    """One int8 block whose resident tile holds every code -128..127 (each 4 times per head) under
    old_scale, then an append at `row` whose max |x| is new_amax > the block's absmax: the
    state before and after, through the oracle's append."""
    nb = 2
    cfg = pa.make_config(num_q_heads=H, num_kv_heads=H, head_dim=D, kv_dtype=2, num_blocks=nb)
    codes = (np.arange(16 * D) % 256 - 128).astype(np.int8)
    kc = np.zeros((nb, H, 16, D), np.int8)
    for h in range(H):
        kc[1, h] = np.roll(codes, 37 * h).reshape(16, D)
    vc = kc.copy()
    ks = np.full((nb, H), f32(old_scale), f32)
    ka = np.full((nb, H), f32(old_scale) * f32(127), f32)
    vs, va = ks.copy(), ka.copy()
    x = np.zeros((1, H, D), f32)
    x[0, :, 0] = f32(new_amax)
    x[0, :, 1] = -f32(new_amax) / f32(3)
    before = kc.copy()
    orc.kv_append(cfg, x, x, np.array([16 + row], np.int64), kc, vc, ks, vs, ka, va)
    return before, kc, vc, ks, ka, x


@pytest.mark.parametrize("old_scale,new_amax,separates", [
    (0.5, 127.0, False),        # new scale exactly 2x: every odd code lands on a tie (k + 0.5)
    (0.25, 127.0, False),       # 4x: ties at odd multiples of 2
    (1.0, 190.5, False),        # 1.5x: mixed fractions
    (0.0078125, 3.0, False),    # tiny scales, large ratio: most codes collapse to 0 / +-1
    (0.3, 38.1 + 1e-3, False),  # ratio just above 1: codes almost unchanged, fp32 rounding decides
    (1.7, 1e4, False),          # huge growth: every resident code becomes 0 or +-1
    # a pair (found by search) where the fp32 rounding of the ratio moves code -125 to -43
    # instead of -44: the case that separates the shortcut q * (old / new)
    (0.2618793547153473, 95.5709228515625, True),
])
def test_append_int8_requantisation_exact(old_scale, new_amax, separates):
    """After a growth event every resident code equals QuantizeSymmetric(Dequantize(code, old),
    new) with the KAT-pinned primitives (QuantizationOperations.cs:83-88, 188-200): all 256 codes,
    ties included, and also the exact-rational rounding rule on the fp32 quotient. The ratio
    shortcut q * (old / new) is shown to differ on these inputs, so the test tells them apart."""
    H, D, row = 2, 64, 5
    old_scale = float(f32(old_scale))
    before, kc, vc, ks, ka, x = _requant_case(old_scale, new_amax, H, D, row)
    new_scale = f32(f32(new_amax) / f32(127))
    assert ks[1, 0] == new_scale and ka[1, 0] == f32(new_amax)
    shortcut_differs = False
    ratio = f32(f32(old_scale) / new_scale)
    for h in range(H):
        for r in range(16):
            for d in range(D):
                c = int(before[1, h, r, d])
                got = int(kc[1, h, r, d])
                if r == row:
                    assert got == L.orc_quantize_symmetric(float(x[0, h, d]), float(new_scale))
                    continue
                deq = L.orc_dequantize(c, float(old_scale))
                assert deq == f32(c) * f32(old_scale)
                expect = L.orc_quantize_symmetric(deq, float(new_scale))
                assert got == expect, (h, r, d, c, got, expect)
                # the rounding rule on the exact fp32 quotient, by rational arithmetic
                quot = Fraction(float(f32(f32(deq) / new_scale)))
                assert got == max(-128, min(127, _nearest_away(quot)))
                if L.orc_quantize_symmetric(float(f32(c) * ratio), 1.0) != expect:
                    shortcut_differs = True
    assert shortcut_differs == separates
    # V: the tile is dim-major; resident element (row r, dim d) sits at d * 16 + r
    for h in range(H):
        bt, vt = before[1, h].reshape(-1), vc[1, h].reshape(-1)
        for r in range(16):
            if r == row:
                continue
            for d in range(0, D, 7):
                c = int(bt[d * 16 + r])
                assert int(vt[d * 16 + r]) == L.orc_quantize_symmetric(L.orc_dequantize(c, float(old_scale)),
                                                                       float(new_scale))


def _segments(slots, nb):
    """Maximal runs of consecutive valid slots that lie in one block: (start, end) pairs."""
    segs, i, n = [], 0, len(slots)
    while i < n:
        if not 0 <= slots[i] < nb * 16:
            i += 1
            continue
        j = i + 1
        while j < n and 0 <= slots[j] < nb * 16 and slots[j] // 16 == slots[i] // 16:
            j += 1
        segs.append((i, j))
        i = j
    return segs


def test_append_int8_call_equals_its_segments_in_order():
    """The int8 append of a call whose blocks arrive out of order (runs split by -1 padding, a
    block revisited after other blocks, a slot written twice) equals its segments appended one by
    one as separate calls, in call order: the rule the GPU's per-block owner follows."""
    rng = np.random.default_rng(21)
    nb, H, D = 6, 2, 64
    cfg = pa.make_config(num_q_heads=H, num_kv_heads=H, head_dim=D, kv_dtype=2, num_blocks=nb)
    base = [np.zeros((nb, H, 16, D), np.int8) for _ in range(2)] + [np.zeros((nb, H), f32) for _ in range(4)]
    fill = rng.standard_normal((nb * 16, H, D)).astype(f32)
    orc.kv_append(cfg, fill, fill, np.arange(nb * 16, dtype=np.int64), *base)
    slots = np.array([16 + 3, 16 + 4, -1, 16 + 5, 48, 49, 16 + 6, 16 + 6, 80 + 7, -1, -1, 48 + 2, 16 + 9,
                      nb * 16 + 1, 16 + 10], np.int64)
    x = (rng.standard_normal((len(slots), H, D)) * rng.choice([0.5, 4.0], size=(len(slots), 1, 1))).astype(f32)
    whole = [a.copy() for a in base]
    orc.kv_append(cfg, x, x, slots, *whole)
    piecewise = [a.copy() for a in base]
    segs = _segments(slots, nb)
    assert len(segs) == 8 and sum(slots[a] // 16 == 1 for a, _ in segs) == 5  # block 1 comes back 5 times
    for s0, s1 in segs:
        xs = np.ascontiguousarray(x[s0:s1])
        orc.kv_append(cfg, xs, xs, np.ascontiguousarray(slots[s0:s1]), *piecewise)
    for a, b in zip(whole, piecewise):
        np.testing.assert_array_equal(a, b)
    # within one segment the later of two tokens with the same slot wins
    one = [a.copy() for a in base]
    xs = np.ascontiguousarray(x[6:8])
    orc.kv_append(cfg, xs, xs, np.ascontiguousarray(slots[6:8]), *one)
    q = np.array([L.orc_quantize_symmetric(float(v), float(one[2][1, 0])) for v in x[7, 0]], np.int8)
    np.testing.assert_array_equal(one[0][1, 0, 6], q)


# ---- paged decode / chunked prefill vs torch float64 on a numpy gather ---------------------------
def _gather(cache, scales, kv_dtype, table, T, Hq, G, is_v):
    nb, Hkv, B, D = cache.shape
    out = np.zeros((T, Hq, D))
    for t in range(T):
        blk = table[t // 16] if t // 16 < len(table) else -1
        if blk < 0 or blk >= nb:
            continue
        for h in range(Hq):
            tile = cache[blk, h // G].reshape(-1)
            idx = np.arange(D) * 16 + t % 16 if is_v else (t % 16) * D + np.arange(D)
            val = tile[idx]
            if kv_dtype == 1:
                val = orc.f32_from_bf16(val)
            elif kv_dtype == 2:
                val = val.astype(f32) * f32(scales[blk, h // G])
            out[t, h] = val
    return out


def _int8_cache(w, inp):
    cfg = pa.make_config(num_q_heads=w.num_q_heads, num_kv_heads=w.num_kv_heads, head_dim=w.head_dim,
                         kv_dtype=2, q_dtype=w.q_dtype, num_blocks=w.num_blocks)
    nb, H, D = w.num_blocks, w.num_kv_heads, w.head_dim
    kc, vc = np.zeros((nb, H, 16, D), np.int8), np.zeros((nb, H, 16, D), np.int8)
    sc = [np.zeros((nb, H), f32) for _ in range(4)]
    tok = lambda a: np.ascontiguousarray(a.transpose(0, 2, 1, 3).reshape(nb * 16, H, D))  # noqa: E731
    kin, vin = tok(inp["k_src"]), tok(inp["v_src"])
    if w.q_dtype == 1:
        kin, vin = orc.bf16_from_f32(kin), orc.bf16_from_f32(vin)
    orc.kv_append(cfg, kin, vin, np.arange(nb * 16, dtype=np.int64), kc, vc, *sc)
    return kc, vc, sc[0], sc[1]


@pytest.mark.parametrize("kv_dtype,q_dtype,Hq,Hkv,D", [(0, 0, 4, 4, 32), (1, 1, 8, 2, 64), (2, 0, 8, 4, 64)])
def test_paged_decode_against_torch(kv_dtype, q_dtype, Hq, Hkv, D):
    lens = [0, 1, 15, 16, 17, 40, 100]
    w = wl.make_small(11 + kv_dtype, num_seqs=len(lens), lens=lens, Hq=Hq, Hkv=Hkv, D=D, kv_dtype=kv_dtype,
                      q_dtype=q_dtype)
    w.block_tables[5, 1] = -1              # a hole: reads as zeros
    w.block_tables[6, 2] = w.num_blocks     # out of the pool: reads as zeros
    inp = wl.numpy_inputs(w, 12)
    if kv_dtype == 2:
        kc, vc, ks, vs = _int8_cache(w, inp)
    else:
        kc, vc, ks, vs = inp["k_cache"], inp["v_cache"], None, None
    cfg = pa.make_config(num_q_heads=Hq, num_kv_heads=Hkv, head_dim=D, kv_dtype=kv_dtype, q_dtype=q_dtype,
                         num_blocks=w.num_blocks)
    got = orc.paged_decode(cfg, inp["q"], kc, vc, ks, vs, w.block_tables, w.context_lens)
    G = Hq // Hkv
    qf = orc.f32_from_bf16(inp["q"]) if q_dtype == 1 else inp["q"]
    for s, T in enumerate(lens):
        if T <= 0:
            assert np.all(got[s] == 0)
            continue
        K = _gather(kc, ks, kv_dtype, w.block_tables[s], T, Hq, G, False)
        V = _gather(vc, vs, kv_dtype, w.block_tables[s], T, Hq, G, True)
        ref = torch_sdpa(qf[s][None, None].astype(np.float64), K[None], V[None])[0, 0]
        np.testing.assert_allclose(got[s], ref, rtol=0, atol=5e-6)


@pytest.mark.parametrize("flags", [0, pa.PA_FLAG_REFERENCE_LITERAL_MASK, pa.PA_FLAG_NO_MASK])
def test_chunked_prefill_against_torch(flags):
    rng = np.random.default_rng(13)
    Hq, Hkv, D = 8, 2, 32
    prefix = [0, 37, 5]
    chunk = [33, 20, 1]
    totals = [p + c for p, c in zip(prefix, chunk)]
    w = wl.make_small(14, num_seqs=3, lens=totals, Hq=Hq, Hkv=Hkv, D=D, kv_dtype=1, q_dtype=1)
    inp = wl.numpy_inputs(w, 15)
    q_start = np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32)
    q = orc.bf16_from_f32(rng.standard_normal((int(q_start[-1]), Hq, D)).astype(f32))
    cfg = pa.make_config(num_q_heads=Hq, num_kv_heads=Hkv, head_dim=D, kv_dtype=1, q_dtype=1,
                         num_blocks=w.num_blocks, flags=flags)
    got = orc.chunked_prefill(cfg, q, q_start, np.array(prefix, np.int32), inp["k_cache"], inp["v_cache"],
                              None, None, w.block_tables)
    qf = orc.f32_from_bf16(q)
    for s in range(3):
        T, Lc, P = totals[s], chunk[s], prefix[s]
        K = _gather(inp["k_cache"], None, 1, w.block_tables[s], T, Hq, Hq // Hkv, False)
        V = _gather(inp["v_cache"], None, 1, w.block_tables[s], T, Hq, Hq // Hkv, True)
        if flags == pa.PA_FLAG_NO_MASK or (flags == pa.PA_FLAG_REFERENCE_LITERAL_MASK and P == 0):
            mask = None
        else:
            mask = bottom_right_mask(Lc, T)
        ref = torch_sdpa(qf[q_start[s]:q_start[s + 1]][None].astype(np.float64), K[None], V[None], mask)[0]
        np.testing.assert_allclose(got[q_start[s]:q_start[s + 1]], ref, rtol=0, atol=5e-6)
