"""GPU parity of libpa_hip.so against the CPU oracle, called through the C-ABI.

Bar: slot mapping, fp32/bf16 stores and int8 codes/scales/absmax are bit-exact; attention
outputs satisfy |gpu - oracle| <= atol + rtol*|oracle| with (2e-3, 1e-2) for bf16 KV, (2e-2, 1e-2)
for int8 KV and (1e-5, 1e-4) for fp32 KV (tests/helpers.py), accumulation in fp32.
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


def run_decode(w, seed, stream, partition_size=0, n_threads=NTHREADS, num_splits=0):
    inp = wl.numpy_inputs(w, seed)
    cfg = config_for(w, partition_size=partition_size, num_splits=num_splits)
    if w.kv_dtype == 2:
        host, g = build_int8_caches(w, inp, stream)
        kc, vc, ks, vs = g["kc"], g["vc"], g["ks"], g["vs"]
    else:
        host = dict(k_cache=inp["k_cache"], v_cache=inp["v_cache"], k_scale=None, v_scale=None)
        kc, vc, ks, vs = to_gpu(inp["k_cache"]), to_gpu(inp["v_cache"]), None, None
    ref = orc.paged_decode(cfg, inp["q"], host["k_cache"], host["v_cache"], host["k_scale"],
                           host["v_scale"], w.block_tables, w.context_lens, n_threads=n_threads)
    S = w.num_seqs
    out = empty_gpu((S, w.num_q_heads, w.head_dim), np.float32)
    out.fill_(float("nan"))
    mcl = w.max_context_len
    wsb = pa.decode_workspace_size(cfg, S, mcl)
    ws = empty_gpu((max(wsb, 1),), np.uint8)
    args = (to_gpu(inp["q"]), kc, vc, ks, vs, to_gpu(w.block_tables), to_gpu(w.context_lens), S,
            w.max_blocks, mcl, ws, wsb)
    pa.paged_decode(stream, cfg, out, *args)
    _sync()
    first = to_np(out).copy()
    # A second call on the same (now dirty) workspace must reproduce the first bit for bit.
    out.fill_(float("nan"))
    pa.paged_decode(stream, cfg, out, *args)
    _sync()
    np.testing.assert_array_equal(to_np(out), first)
    return first, ref


# ---- slot mapping ----------------------------------------------------------------------------------
def test_slot_mapping_bit_exact(stream):
    rng = np.random.default_rng(11)
    S, mb = 37, 20
    tables = rng.integers(0, 500, size=(S, mb)).astype(np.int32)
    tables[rng.random((S, mb)) < 0.1] = -1
    start = rng.integers(0, mb * 16, size=S).astype(np.int32)
    num_new = rng.integers(0, 40, size=S).astype(np.int32)
    offs = np.concatenate([[0], np.cumsum(num_new)[:-1]]).astype(np.int32)
    cfg = pa.make_config(num_q_heads=8, num_kv_heads=8, head_dim=64, kv_dtype=1, num_blocks=500)
    ref = orc.build_slot_mapping(cfg, tables, start, num_new, offs)
    out = empty_gpu((int(num_new.sum()),), np.int64)
    pa.build_slot_mapping(stream, cfg, to_gpu(tables), mb, to_gpu(start), to_gpu(num_new), to_gpu(offs),
                          S, int(num_new.max()), out)
    _sync()
    np.testing.assert_array_equal(to_np(out), ref)
    assert (ref == -1).any() and (ref >= 0).any()


# ---- append -----------------------------------------------------------------------------------------
@pytest.mark.parametrize("kv_dtype,q_dtype,D", [(1, 0, 128), (0, 1, 64), (1, 1, 256), (0, 0, 128)])
def test_append_plain_bit_exact(stream, kv_dtype, q_dtype, D):
    rng = np.random.default_rng(20 + D + kv_dtype)
    nb, hkv, n = 40, 4, 300
    cfg = pa.make_config(num_q_heads=hkv, num_kv_heads=hkv, head_dim=D, kv_dtype=kv_dtype,
                         q_dtype=q_dtype, num_blocks=nb)
    slots = rng.permutation(nb * 16)[:n].astype(np.int64)
    slots[::17] = -1
    slots[5] = nb * 16 + 3  # beyond the pool: skipped
    src_k = rng.standard_normal((n, hkv, D), dtype=np.float32)
    src_v = rng.standard_normal((n, hkv, D), dtype=np.float32)
    if q_dtype == 1:
        src_k, src_v = orc.bf16_from_f32(src_k), orc.bf16_from_f32(src_v)
    cdt = np.uint16 if kv_dtype == 1 else np.float32
    init = rng.standard_normal((nb, hkv, 16, D), dtype=np.float32)
    kc = orc.bf16_from_f32(init) if kv_dtype == 1 else init.copy()
    vc = kc.copy()
    gk, gv = to_gpu(kc), to_gpu(vc)
    orc.kv_append(cfg, src_k, src_v, slots, kc, vc)
    pa.kv_append(stream, cfg, to_gpu(src_k), to_gpu(src_v), to_gpu(slots), n, gk, gv)
    _sync()
    np.testing.assert_array_equal(to_np(gk, cdt), kc)
    np.testing.assert_array_equal(to_np(gv, cdt), vc)


@pytest.mark.parametrize("kv_dtype,q_dtype,D", [(1, 1, 128), (0, 0, 64), (1, 0, 256), (0, 1, 128), (1, 1, 32),
                                                (0, 0, 32)])
def test_append_plain_whole_blocks_bit_exact(stream, kv_dtype, q_dtype, D):
    """Runs of 16 consecutive slots that fill a block take the kernel's whole-tile V path; the
    rest (partial runs, a run crossing a block boundary, one broken by an invalid slot or out of
    order) take the per-token path. Both must write exactly the oracle's bytes."""
    rng = np.random.default_rng(70 + D + kv_dtype)
    nb, hkv = 24, 3
    cfg = pa.make_config(num_q_heads=hkv, num_kv_heads=hkv, head_dim=D, kv_dtype=kv_dtype,
                         q_dtype=q_dtype, num_blocks=nb)
    runs = [np.arange(16) + 16 * 3,             # whole block 3
            np.arange(16) + 16 * 7,             # whole block 7
            np.arange(5, 16) + 16 * 9,          # tail of block 9
            np.arange(0, 7) + 16 * 11,          # head of block 11
            np.arange(16) + 16 * 12 + 5,        # crosses from block 12 into 13
            np.arange(16) + 16 * 15,            # block 15, one slot invalidated below
            (np.arange(16) + 16 * 17)[::-1],    # block 17, tokens in reverse order
            np.arange(16) + 16 * 20]            # whole block 20
    slots = np.concatenate(runs).astype(np.int64)
    slots[np.flatnonzero(slots == 16 * 15 + 9)] = -1
    n = len(slots)
    src_k = rng.standard_normal((n, hkv, D), dtype=np.float32)
    src_v = rng.standard_normal((n, hkv, D), dtype=np.float32)
    if q_dtype == 1:
        src_k, src_v = orc.bf16_from_f32(src_k), orc.bf16_from_f32(src_v)
    cdt = np.uint16 if kv_dtype == 1 else np.float32
    init = rng.standard_normal((nb, hkv, 16, D), dtype=np.float32)
    kc = orc.bf16_from_f32(init) if kv_dtype == 1 else init.copy()
    vc = kc.copy()
    gk, gv = to_gpu(kc), to_gpu(vc)
    orc.kv_append(cfg, src_k, src_v, slots, kc, vc)
    pa.kv_append(stream, cfg, to_gpu(src_k), to_gpu(src_v), to_gpu(slots), n, gk, gv)
    _sync()
    np.testing.assert_array_equal(to_np(gk, cdt), kc)
    np.testing.assert_array_equal(to_np(gv, cdt), vc)


@pytest.mark.parametrize("kv_dtype,q_dtype,D", [(1, 1, 128), (0, 1, 64), (1, 0, 256)])
def test_append_prefill_chunks_bit_exact(stream, kv_dtype, q_dtype, D):
    """Chunks of several sequences in one call, as a chunked-prefill step appends them: each chunk
    starts at an arbitrary position of its sequence (a partly filled first block), fills whole
    blocks whose 16 tokens straddle the call's 16-token groups, and may end mid-block."""
    rng = np.random.default_rng(90 + D + kv_dtype)
    hkv, nb = 2, 64
    cfg = pa.make_config(num_q_heads=hkv, num_kv_heads=hkv, head_dim=D, kv_dtype=kv_dtype,
                         q_dtype=q_dtype, num_blocks=nb)
    perm = rng.permutation(nb)
    prefix, chunk = [37, 0, 15, 100], [50, 33, 64, 45]
    slots, used = [], 0
    for p, c in zip(prefix, chunk):
        nblk = (p + c + 15) // 16
        tab = perm[used:used + nblk]
        used += nblk
        pos = p + np.arange(c)
        slots.append(tab[pos // 16].astype(np.int64) * 16 + pos % 16)
    slots = np.concatenate(slots)
    n = len(slots)
    src_k = rng.standard_normal((n, hkv, D), dtype=np.float32)
    src_v = rng.standard_normal((n, hkv, D), dtype=np.float32)
    if q_dtype == 1:
        src_k, src_v = orc.bf16_from_f32(src_k), orc.bf16_from_f32(src_v)
    cdt = np.uint16 if kv_dtype == 1 else np.float32
    init = rng.standard_normal((nb, hkv, 16, D), dtype=np.float32)
    kc = orc.bf16_from_f32(init) if kv_dtype == 1 else init.copy()
    vc = kc.copy()
    gk, gv = to_gpu(kc), to_gpu(vc)
    orc.kv_append(cfg, src_k, src_v, slots, kc, vc)
    pa.kv_append(stream, cfg, to_gpu(src_k), to_gpu(src_v), to_gpu(slots), n, gk, gv)
    _sync()
    np.testing.assert_array_equal(to_np(gk, cdt), kc)
    np.testing.assert_array_equal(to_np(gv, cdt), vc)


@pytest.mark.parametrize("kv_dtype,q_dtype", [(1, 1), (0, 0)])
def test_append_plain_unaligned_activations(stream, kv_dtype, q_dtype):
    """New K/V starting one element past a 16-byte boundary take the element-wise kernel; its
    bytes equal the oracle's too (whole blocks and partial ones)."""
    import torch

    rng = np.random.default_rng(95 + kv_dtype)
    nb, hkv, D = 8, 2, 64
    cfg = pa.make_config(num_q_heads=hkv, num_kv_heads=hkv, head_dim=D, kv_dtype=kv_dtype,
                         q_dtype=q_dtype, num_blocks=nb)
    slots = np.concatenate([np.arange(16) + 16 * 5, np.arange(3, 12) + 16 * 2]).astype(np.int64)
    n = len(slots)
    src_k = rng.standard_normal((n, hkv, D), dtype=np.float32)
    src_v = rng.standard_normal((n, hkv, D), dtype=np.float32)
    if q_dtype == 1:
        src_k, src_v = orc.bf16_from_f32(src_k), orc.bf16_from_f32(src_v)
    cdt = np.uint16 if kv_dtype == 1 else np.float32
    init = rng.standard_normal((nb, hkv, 16, D), dtype=np.float32)
    kc = orc.bf16_from_f32(init) if kv_dtype == 1 else init.copy()
    vc = kc.copy()
    gk, gv = to_gpu(kc), to_gpu(vc)

    def shifted(a):  # the same values one element into a fresh buffer
        buf = to_gpu(np.concatenate([np.zeros(1, a.dtype), a.reshape(-1)]))
        view = buf[1:].view(a.shape)
        assert view.data_ptr() % 16 != 0
        return buf, view

    (_, vk), (_, vv) = shifted(src_k), shifted(src_v)
    orc.kv_append(cfg, src_k, src_v, slots, kc, vc)
    pa.kv_append(stream, cfg, vk, vv, to_gpu(slots), n, gk, gv)
    _sync()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_np(gk, cdt), kc)
    np.testing.assert_array_equal(to_np(gv, cdt), vc)


@pytest.mark.parametrize("D,q_dtype", [(128, 0), (64, 1), (256, 0)])
def test_append_int8_bit_exact(stream, D, q_dtype):
    """Full-block build, then a decode-style 1-token append with outliers (scale growth and
    requantisation), then a ragged multi-token append that starts mid-block."""
    rng = np.random.default_rng(30 + D)
    nb, hkv = 24, 4
    cfg = pa.make_config(num_q_heads=hkv, num_kv_heads=hkv, head_dim=D, kv_dtype=2, q_dtype=q_dtype,
                         num_blocks=nb)
    host = dict(kc=np.zeros((nb, hkv, 16, D), np.int8), vc=np.zeros((nb, hkv, 16, D), np.int8),
                ks=np.zeros((nb, hkv), np.float32), vs=np.zeros((nb, hkv), np.float32),
                ka=np.zeros((nb, hkv), np.float32), va=np.zeros((nb, hkv), np.float32))
    dev = {n: to_gpu(a) for n, a in host.items()}

    def step(slots, k, v):
        if q_dtype == 1:
            k, v = orc.bf16_from_f32(k), orc.bf16_from_f32(v)
        orc.kv_append(cfg, k, v, slots, host["kc"], host["vc"], host["ks"], host["vs"], host["ka"], host["va"])
        pa.kv_append(stream, cfg, to_gpu(k), to_gpu(v), to_gpu(slots), len(slots), dev["kc"], dev["vc"],
                     dev["ks"], dev["vs"], dev["ka"], dev["va"])
        _sync()
        for n, a in host.items():
            np.testing.assert_array_equal(to_np(dev[n]), a, err_msg=n)

    # 1) 12 blocks filled to 1..16 rows
    fill = rng.integers(1, 17, size=12)
    slots = np.concatenate([b * 16 + np.arange(f) for b, f in enumerate(fill)]).astype(np.int64)
    k = rng.standard_normal((len(slots), hkv, D), dtype=np.float32)
    v = rng.standard_normal((len(slots), hkv, D), dtype=np.float32)
    step(slots, k, v)
    # 2) one new token per partially filled block, half of them with x8 outliers (growth)
    open_blocks = [b for b, f in enumerate(fill) if f < 16]
    slots = np.array([b * 16 + fill[b] for b in open_blocks], np.int64)
    k = rng.standard_normal((len(slots), hkv, D), dtype=np.float32)
    v = rng.standard_normal((len(slots), hkv, D), dtype=np.float32)
    k[::2, :, 3] *= 8
    v[1::2, :, 7] *= 8
    step(slots, k, v)
    # 3) a 37-token chunk starting at row 5 of block 14, then -1 padding, then a new block
    slots = np.concatenate([14 * 16 + 5 + np.arange(11), 15 * 16 + np.arange(16), 16 * 16 + np.arange(10),
                            [-1, -1], 20 * 16 + np.arange(3)]).astype(np.int64)
    k = rng.standard_normal((len(slots), hkv, D), dtype=np.float32) * 3
    v = rng.standard_normal((len(slots), hkv, D), dtype=np.float32) * 3
    step(slots, k, v)


@pytest.mark.parametrize("D,q_dtype", [(128, 0), (64, 1), (256, 0)])
def test_append_int8_out_of_order_bit_exact(stream, D, q_dtype):
    """A block's tokens split by -1 padding, revisited after other blocks' tokens, a slot written
    twice, out-of-range slots, and a random scatter with ~80 segments per block (more than one pass
    of the owner's segment list): the first token of the call in a block owns it and applies its
    segments in call order, so the GPU matches the oracle's sequential append bit for bit."""
    rng = np.random.default_rng(90 + D)
    nb, hkv = 12, 4
    cfg = pa.make_config(num_q_heads=hkv, num_kv_heads=hkv, head_dim=D, kv_dtype=2, q_dtype=q_dtype,
                         num_blocks=nb)
    host = dict(kc=np.zeros((nb, hkv, 16, D), np.int8), vc=np.zeros((nb, hkv, 16, D), np.int8),
                ks=np.zeros((nb, hkv), np.float32), vs=np.zeros((nb, hkv), np.float32),
                ka=np.zeros((nb, hkv), np.float32), va=np.zeros((nb, hkv), np.float32))
    dev = {n: to_gpu(a) for n, a in host.items()}

    def step(slots, scale_choices):
        slots = np.asarray(slots, np.int64)
        mult = rng.choice(scale_choices, size=(len(slots), 1, 1)).astype(np.float32)
        k = (rng.standard_normal((len(slots), hkv, D), dtype=np.float32) * mult).astype(np.float32)
        v = (rng.standard_normal((len(slots), hkv, D), dtype=np.float32) * mult[::-1]).astype(np.float32)
        if q_dtype == 1:
            k, v = orc.bf16_from_f32(k), orc.bf16_from_f32(v)
        orc.kv_append(cfg, k, v, slots, host["kc"], host["vc"], host["ks"], host["vs"], host["ka"], host["va"])
        pa.kv_append(stream, cfg, to_gpu(k), to_gpu(v), to_gpu(slots), len(slots), dev["kc"], dev["vc"],
                     dev["ks"], dev["vs"], dev["ka"], dev["va"])
        _sync()
        for n, a in host.items():
            np.testing.assert_array_equal(to_np(dev[n]), a, err_msg=n)

    step(np.arange(nb * 16), [1.0])  # every block filled in order
    # block 1 split by padding and revisited, block 3 and 5 in between, slot 22 twice, 97 / 500 invalid
    step([19, 20, -1, 21, 48, 49, 22, 22, 87, -1, -1, 50, 25, nb * 16 + 1, 26, 500, 16 + 15, 16 + 0], [0.5, 4.0])
    # a random scatter over 5 blocks: ~80 segments per block, many with scale growth
    slots = rng.choice(np.arange(16 * 5, 16 * 10), size=400).astype(np.int64)
    slots[rng.random(400) < 0.1] = -1
    step(slots, [0.25, 1.0, 8.0])


@pytest.mark.parametrize("old_scale,new_amax", [(0.5, 127.0), (0.0078125, 3.0), (0.2618793547153473, 95.5709228515625),
                                               (1.7, 1e4)])
def test_append_int8_requantisation_all_codes(stream, old_scale, new_amax):
    """A resident tile holding every code -128..127, then a growth event: the GPU's requantised
    codes, scales and absmax equal the oracle's bit for bit (the oracle's rule is pinned code by
    code against the quantiser primitives in test_oracle.py)."""
    nb, hkv, D, row = 2, 2, 64, 5
    cfg = pa.make_config(num_q_heads=hkv, num_kv_heads=hkv, head_dim=D, kv_dtype=2, q_dtype=0, num_blocks=nb)
    codes = (np.arange(16 * D) % 256 - 128).astype(np.int8)
    kc = np.zeros((nb, hkv, 16, D), np.int8)
    for h in range(hkv):
        kc[1, h] = np.roll(codes, 37 * h).reshape(16, D)
    os_ = np.float32(old_scale)
    host = dict(kc=kc, vc=kc.copy(), ks=np.full((nb, hkv), os_, np.float32), vs=np.full((nb, hkv), os_, np.float32),
                ka=np.full((nb, hkv), os_ * np.float32(127), np.float32),
                va=np.full((nb, hkv), os_ * np.float32(127), np.float32))
    dev = {n: to_gpu(a) for n, a in host.items()}
    x = np.zeros((1, hkv, D), np.float32)
    x[0, :, 0] = np.float32(new_amax)
    x[0, :, 1] = -np.float32(new_amax) / np.float32(3)
    slots = np.array([16 + row], np.int64)
    orc.kv_append(cfg, x, x, slots, host["kc"], host["vc"], host["ks"], host["vs"], host["ka"], host["va"])
    pa.kv_append(stream, cfg, to_gpu(x), to_gpu(x), to_gpu(slots), 1, dev["kc"], dev["vc"], dev["ks"], dev["vs"],
                 dev["ka"], dev["va"])
    _sync()
    for n, a in host.items():
        np.testing.assert_array_equal(to_np(dev[n]), a, err_msg=n)


def test_decode_append_int8_shared_last_block(stream):
    """Fused int8 append where several sequences' new tokens land in one block (their tables share
    the block at different rows, and one row twice): the workgroup of the first such token owns
    the block and applies the tokens in sequence order (the general path); the others take the
    one-token path. Bytes, scales and absmax against the oracle's pa_kv_append in call order."""
    lens = [20, 24, 40, 33, 1, 17, 300]
    w = wl.make_small(91, num_seqs=len(lens), lens=lens, Hq=16, Hkv=4, D=128, kv_dtype=2, q_dtype=1)
    w.block_tables[1, 1] = w.block_tables[0, 1]  # seq 1's last token (row 7) in seq 0's last block (row 3)
    w.block_tables[3, 2] = w.block_tables[0, 1]  # seq 3's last token at row 0 of that block: afresh
    inp = wl.numpy_inputs(w, 92)
    cfg = config_for(w)
    S, Hkv, D = w.num_seqs, w.num_kv_heads, w.head_dim
    rng = np.random.default_rng(93)
    k_new = rng.standard_normal((S, Hkv, D), dtype=np.float32)
    v_new = rng.standard_normal((S, Hkv, D), dtype=np.float32)
    k_new[1, :, 3] *= 8.0  # growth on the shared block
    k_new, v_new = orc.bf16_from_f32(k_new), orc.bf16_from_f32(v_new)
    pos = w.context_lens.astype(np.int64) - 1
    slots = w.block_tables[np.arange(S), pos // 16].astype(np.int64) * 16 + pos % 16
    host, g = build_int8_caches(w, inp, stream)
    hk, hv = host["k_cache"].copy(), host["v_cache"].copy()
    hks, hvs = host["k_scale"].copy(), host["v_scale"].copy()
    hka, hva = to_np(g["ka"]).copy(), to_np(g["va"]).copy()
    orc.kv_append(cfg, k_new, v_new, slots, hk, hv, hks, hvs, hka, hva)
    out = empty_gpu((S, w.num_q_heads, D), np.float32)
    wsb = pa.decode_workspace_size(cfg, S, w.max_context_len)
    ws = empty_gpu((max(wsb, 1),), np.uint8)
    pa.paged_decode_append(stream, cfg, out, to_gpu(inp["q"]), to_gpu(k_new), to_gpu(v_new), g["kc"], g["vc"], g["ks"],
                           g["vs"], g["ka"], g["va"], to_gpu(w.block_tables), to_gpu(w.context_lens), S, w.max_blocks,
                           w.max_context_len, ws, wsb)
    _sync()
    for n, want in dict(kc=hk, vc=hv, ks=hks, vs=hvs, ka=hka, va=hva).items():
        np.testing.assert_array_equal(to_np(g[n]), want, err_msg=n)
    ref = orc.paged_decode(cfg, inp["q"], hk, hv, hks, hvs, w.block_tables, w.context_lens, n_threads=NTHREADS)
    check_close(to_np(out), ref, **tol_for(2), what="int8 fused append, shared last block")


# ---- decode -----------------------------------------------------------------------------------------
def test_decode_c1_fp32(stream):
    """C1, the CPU-parity configuration (fp32 cache and query, VALU kernel), at the fp32 bar."""
    w = wl.make_c1()
    got, ref = run_decode(w, 101, stream)
    err = check_close(got, ref, **tol_for(0), what="C1")
    assert err < 1e-5


def test_decode_c2_bf16_full(stream):
    w = wl.make_c2()
    got, ref = run_decode(w, 102, stream)
    check_close(got, ref, **tol_for(1), what="C2")


def test_decode_c4_int8_subset(stream):
    w = wl.make_c4(batch=24)
    got, ref = run_decode(w, 104, stream)
    check_close(got, ref, **tol_for(2), what="C4 subset")


EDGE_LENS = [0, 1, 2, 15, 16, 17, 255, 256, 257, 511, 512, 513, 1000, 1023, 1024, 1025, 3000]


@pytest.mark.parametrize("part", [0, 256, 512])
@pytest.mark.parametrize("kv_dtype,q_dtype,Hq,Hkv,D", [
    (1, 1, 32, 8, 128), (1, 0, 16, 8, 64), (1, 1, 16, 2, 256), (0, 0, 8, 2, 128), (2, 0, 8, 8, 64),
    (2, 1, 32, 8, 128), (0, 1, 4, 4, 256),
])
def test_decode_edge_lengths(stream, part, kv_dtype, q_dtype, Hq, Hkv, D):
    w = wl.make_small(7 + D + kv_dtype, num_seqs=len(EDGE_LENS), lens=EDGE_LENS, Hq=Hq, Hkv=Hkv, D=D,
                      kv_dtype=kv_dtype, q_dtype=q_dtype)
    got, ref = run_decode(w, 55, stream, partition_size=part)
    check_close(got, ref, **tol_for(kv_dtype), what=f"edge lens kv={kv_dtype} D={D} G={Hq // Hkv}")
    assert np.all(got[0] == 0.0)  # context_len 0 -> zeros


@pytest.mark.parametrize("part", [64, 0])
@pytest.mark.parametrize("kv_dtype,q_dtype", [(1, 1), (2, 1), (2, 0)])
def test_decode_many_short_rows(stream, kv_dtype, q_dtype, part):
    """Hundreds of rows of 1 to 8 blocks: a worker's range crosses many row ends, so the pipeline
    is carried across many pieces (a piece of 1 or 2 blocks still hands the next piece its first two
    blocks). With a 4-block partition there are more units than workers, and with 3 KV heads a
    worker's next unit belongs to another KV head."""
    rng = np.random.default_rng(31 + kv_dtype)
    lens = rng.integers(1, 161, size=1000).astype(np.int32)
    lens[::37] = 16  # whole blocks
    w = wl.make_small(41 + kv_dtype, num_seqs=len(lens), lens=lens, Hq=12, Hkv=3, D=128,
                      kv_dtype=kv_dtype, q_dtype=q_dtype)
    got, ref = run_decode(w, 59, stream, partition_size=part)
    check_close(got, ref, **tol_for(kv_dtype), what=f"short rows kv={kv_dtype} part={part}")


@pytest.mark.parametrize("part", [0, 4096])
@pytest.mark.parametrize("kv_dtype", [1, 2])
def test_decode_long_segments(stream, kv_dtype, part):
    """Long rows: 256-block segments (64 blocks per wave), and more units than workgroups."""
    w = wl.make_small(12 + kv_dtype, num_seqs=len(LONG_LENS), lens=LONG_LENS, Hq=16, Hkv=4, D=128,
                      kv_dtype=kv_dtype, q_dtype=1)
    got, ref = run_decode(w, 57, stream, partition_size=part)
    check_close(got, ref, **tol_for(kv_dtype), what=f"long segments kv={kv_dtype} part={part}")


@pytest.mark.parametrize("nsp", [1, 3, 16, 200])
@pytest.mark.parametrize("kv_dtype,q_dtype,Hq,Hkv,D", [(1, 1, 32, 8, 128), (2, 0, 16, 4, 128), (1, 0, 8, 8, 64)])
def test_decode_num_splits(stream, nsp, kv_dtype, q_dtype, Hq, Hkv, D):
    """pa_config.num_splits = P: every sequence cut into P partitions of whole blocks (fewer when it
    has fewer blocks), one worker per (partition, KV head), merged per row; edge lengths and long
    rows, P above and below the block counts."""
    lens = EDGE_LENS + [5000, 40000, 16 * 200, 16 * 200 + 1]
    w = wl.make_small(300 + nsp + kv_dtype, num_seqs=len(lens), lens=lens, Hq=Hq, Hkv=Hkv, D=D, kv_dtype=kv_dtype,
                      q_dtype=q_dtype)
    got, ref = run_decode(w, 61, stream, num_splits=nsp)
    check_close(got, ref, **tol_for(kv_dtype), what=f"num_splits={nsp} kv={kv_dtype} D={D}")
    assert np.all(got[0] == 0.0)


@pytest.mark.parametrize("part", [0, 64])
@pytest.mark.parametrize("kv_dtype,q_dtype,Hq,Hkv,D", [(1, 1, 32, 8, 128), (1, 0, 8, 2, 64), (1, 1, 16, 4, 256),
                                                        (2, 0, 32, 8, 128), (2, 1, 8, 8, 64)])
def test_decode_every_tail_position(stream, part, kv_dtype, q_dtype, Hq, Hkv, D):
    """A row's last block holding 1 to 16 tokens, each in a row of its own (and rows of one to three
    blocks). The kernels hand a lane group four consecutive tokens of a block (the bf16 kernel
    with groups 1 and 2 exchanged, so its K rows and the tail mask follow the same numbering), so
    every count of tokens in the last block masks a different set of lanes."""
    lens = [16 * b + r for b in (0, 1, 2) for r in range(1, 17)]
    w = wl.make_small(500 + D + kv_dtype, num_seqs=len(lens), lens=lens, Hq=Hq, Hkv=Hkv, D=D,
                      kv_dtype=kv_dtype, q_dtype=q_dtype)
    got, ref = run_decode(w, 63, stream, partition_size=part)
    check_close(got, ref, **tol_for(kv_dtype), what=f"tail positions kv={kv_dtype} D={D} part={part}")


def test_decode_invalid_block_ids_read_as_zero(stream):
    w = wl.make_small(9, num_seqs=4, lens=[40, 300, 700, 33], Hq=16, Hkv=4, D=128, kv_dtype=1, q_dtype=1)
    w.block_tables[1, 3] = -1
    w.block_tables[2, 10] = w.num_blocks + 5
    got, ref = run_decode(w, 56, stream)
    check_close(got, ref, **tol_for(1), what="invalid ids")


# ---- fused append + decode ------------------------------------------------------------------------
# Positions T-1 with (T-1) % 16 == 0 start a block (fresh int8 statistics); the rest append mid-block.
APPEND_LENS = [1, 2, 16, 17, 33, 100, 256, 257, 300, 513, 1000, 1024, 1025, 2000]
TAIL_LENS = [16 * b + r for b in (0, 1, 2) for r in range(1, 17)]  # every position of the new token
# more sequences than one persistent launch takes (2047): the call runs in chunks of sequences
MANY_LENS = np.random.default_rng(83).integers(1, 60, size=2100).tolist()


# Long rows: segments of up to 256 blocks (64 per wave), the appended block at a late lane;
# 1025 and 2049 put the fused append's new token in the block after a piece of exactly 64 blocks.
LONG_LENS = [5000, 1, 4100, 3000, 17, 6000, 40000, 1025, 2049]


@pytest.mark.parametrize("kv_dtype,q_dtype,Hq,Hkv,D,part,lens", [
    (1, 1, 32, 8, 128, -16, APPEND_LENS), (2, 0, 32, 8, 128, -5, APPEND_LENS),
    (1, 1, 32, 8, 128, 0, APPEND_LENS), (1, 0, 16, 4, 64, 512, APPEND_LENS), (2, 0, 32, 8, 128, 0, APPEND_LENS),
    (2, 1, 8, 2, 256, 512, APPEND_LENS), (0, 0, 8, 8, 64, 256, APPEND_LENS), (0, 1, 16, 4, 128, 512, APPEND_LENS),
    (1, 1, 16, 4, 128, 256, APPEND_LENS), (1, 1, 8, 2, 128, 4096, LONG_LENS), (2, 1, 8, 2, 128, 0, LONG_LENS),
    (1, 1, 32, 8, 128, 0, TAIL_LENS), (2, 0, 32, 8, 128, 0, TAIL_LENS),
    # one range, no merge launch: the owning wave writes the token (V tile patched in LDS)
    (1, 1, 32, 8, 128, 0, [40]), (1, 0, 8, 2, 64, -1, [1000]), (1, 1, 8, 2, 128, -1, [33]), (1, 1, 16, 4, 256, 0, [64]),
    (1, 1, 8, 2, 64, 0, MANY_LENS), (2, 0, 8, 2, 64, 0, MANY_LENS),
], ids=["bf16-split16", "int8-split5", "bf16-auto", "bf16-d64", "int8-auto", "int8-d256", "fp32-d64", "fp32-d128", "bf16-256", "bf16-long",
        "int8-long", "bf16-tails", "int8-tails", "bf16-one-range", "bf16-one-split", "bf16-one-split-new-block",
        "bf16-one-range-d256", "bf16-many-seqs", "int8-many-seqs"])
def test_decode_append_matches_append_then_decode(stream, kv_dtype, q_dtype, Hq, Hkv, D, part, lens):
    w = wl.make_small(70 + D + kv_dtype, num_seqs=len(lens), lens=lens, Hq=Hq, Hkv=Hkv, D=D,
                      kv_dtype=kv_dtype, q_dtype=q_dtype)
    inp = wl.numpy_inputs(w, 77)
    # part < 0: num_splits = -part partitions per sequence instead of a partition length
    cfg = config_for(w, partition_size=max(part, 0), num_splits=max(-part, 0))
    S = w.num_seqs
    rng = np.random.default_rng(78)
    k_new = rng.standard_normal((S, Hkv, D), dtype=np.float32)
    v_new = rng.standard_normal((S, Hkv, D), dtype=np.float32)
    k_new[::2, :, 5] *= 8.0   # outliers: int8 scale growth for half of the sequences
    v_new[1::3, :, 9] *= 8.0
    if q_dtype == 1:
        k_new, v_new = orc.bf16_from_f32(k_new), orc.bf16_from_f32(v_new)
    pos = w.context_lens.astype(np.int64) - 1
    slots = w.block_tables[np.arange(S), pos // 16].astype(np.int64) * 16 + pos % 16

    if kv_dtype == 2:
        host, g = build_int8_caches(w, inp, stream)
        ka, va = g["ka"], g["va"]
        host_amax = (to_np(ka).copy(), to_np(va).copy())
        kc, vc, ks, vs = g["kc"], g["vc"], g["ks"], g["vs"]
        hk, hv = host["k_cache"].copy(), host["v_cache"].copy()
        hks, hvs = host["k_scale"].copy(), host["v_scale"].copy()
        orc.kv_append(cfg, k_new, v_new, slots, hk, hv, hks, hvs, host_amax[0], host_amax[1])
    else:
        kc, vc, ks, vs, ka, va = to_gpu(inp["k_cache"]), to_gpu(inp["v_cache"]), None, None, None, None
        hk, hv = inp["k_cache"].copy(), inp["v_cache"].copy()
        hks = hvs = None
        orc.kv_append(cfg, k_new, v_new, slots, hk, hv)
    ref = orc.paged_decode(cfg, inp["q"], hk, hv, hks, hvs, w.block_tables, w.context_lens, n_threads=NTHREADS)

    out = empty_gpu((S, Hq, D), np.float32)
    out.fill_(float("nan"))
    mcl = w.max_context_len
    wsb = pa.decode_workspace_size(cfg, S, mcl)
    ws = empty_gpu((max(wsb, 1),), np.uint8)
    pa.paged_decode_append(stream, cfg, out, to_gpu(inp["q"]), to_gpu(k_new), to_gpu(v_new), kc, vc, ks, vs, ka,
                           va, to_gpu(w.block_tables), to_gpu(w.context_lens), S, w.max_blocks, mcl, ws, wsb)
    _sync()
    cdt = {0: np.float32, 1: np.uint16, 2: np.int8}[kv_dtype]
    np.testing.assert_array_equal(to_np(kc, cdt), hk, err_msg="K cache after fused append")
    np.testing.assert_array_equal(to_np(vc, cdt), hv, err_msg="V cache after fused append")
    if kv_dtype == 2:
        np.testing.assert_array_equal(to_np(ks), hks, err_msg="k_scale")
        np.testing.assert_array_equal(to_np(vs), hvs, err_msg="v_scale")
        np.testing.assert_array_equal(to_np(ka), host_amax[0], err_msg="k_absmax")
        np.testing.assert_array_equal(to_np(va), host_amax[1], err_msg="v_absmax")
    check_close(to_np(out), ref, **tol_for(kv_dtype), what=f"fused append kv={kv_dtype} q={q_dtype} D={D}")
