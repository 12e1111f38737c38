"""Shared-prefix decode (pa_paged_decode_prefix) against the CPU oracle, through the C-ABI.

The result must be the attention of pa_paged_decode over each sequence's whole table (the oracle's
paged decode), within the same tolerances (tests/helpers.py): the prefix blocks are only read once
per group. Block tables are built so that group members really share their first blocks.
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


def shared_case(seed, lens, groups, *, Hq, Hkv, D, kv_dtype=1, q_dtype=1):
    """groups: list of (first sequence, members, shared blocks); members' tables start with the
    same shared blocks, every other block is private. Returns (workload, shared_with_prev)."""
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int32)
    S = len(lens)
    need = [(int(t) + 15) // 16 for t in lens]
    pool = sum(need) + 8
    perm = rng.permutation(pool).astype(np.int32)
    tables = np.full((S, max(max(need), 1) + 2), -1, np.int32)
    links = np.zeros(S, np.int32)
    pos = 0
    owner = {}
    for first, nm, shared in groups:
        ids = perm[pos:pos + shared]
        pos += shared
        for m in range(first, first + nm):
            tables[m, :shared] = ids
            owner[m] = shared
            if m > first:
                links[m] = shared
    for s in range(S):
        k = owner.get(s, 0)
        tables[s, k:need[s]] = perm[pos:pos + need[s] - k]
        pos += need[s] - k
    assert pos <= pool
    w = wl.Workload("prefix", Hq, Hkv, D, kv_dtype, q_dtype, lens, tables, pool)
    return w, links


def run_prefix(stream, w, links, seed=7):
    inp = wl.numpy_inputs(w, seed)
    cfg = config_for(w)
    if w.kv_dtype == 2:
        host, g = build_int8_caches(w, inp, stream)
        kc, vc, ks, vs = g["kc"], g["vc"], g["ks"], g["vs"]
    else:
        host = dict(k_cache=inp["k_cache"], v_cache=inp["v_cache"], k_scale=None, v_scale=None)
        kc, vc, ks, vs = to_gpu(inp["k_cache"]), to_gpu(inp["v_cache"]), None, None
    ref = orc.paged_decode(cfg, inp["q"], host["k_cache"], host["v_cache"], host["k_scale"],
                           host["v_scale"], w.block_tables, w.context_lens, n_threads=NTHREADS)
    S = w.num_seqs
    pb = pa.prefix_plan_bytes(S)
    plan = empty_gpu((max(pb, 4),), np.uint8)
    ng = pa.prefix_plan_build(stream, cfg, links, plan, pb)
    mcl = w.max_context_len
    wsb = pa.prefix_workspace_size(cfg, S, mcl)
    ws = empty_gpu((max(wsb, 1),), np.uint8)
    out = empty_gpu((S, w.num_q_heads, w.head_dim), np.float32)
    args = (to_gpu(inp["q"]), kc, vc, ks, vs, to_gpu(w.block_tables), to_gpu(w.context_lens), S,
            w.max_blocks, mcl, plan, ng, ws, wsb)
    out.fill_(float("nan"))
    pa.paged_decode_prefix(stream, cfg, out, *args)
    _sync()
    first = to_np(out).copy()
    out.fill_(float("nan"))  # a second call on the dirty workspace reproduces the first
    pa.paged_decode_prefix(stream, cfg, out, *args)
    _sync()
    np.testing.assert_array_equal(to_np(out), first)
    return first, ref, ng, to_np(plan, np.int32)


def expected_groups(links, G):
    """The grouping rule of pa_prefix_plan_build, restated: linked runs cut into chunks of
    16 / G, chunks of one dropped, a chunk's shared count the minimum of its inner links."""
    cap, S, out = 16 // G, len(links), []
    s = 0
    while s < S:
        e = s + 1
        while e < S and links[e] > 0:
            e += 1
        for c0 in range(s, e, cap):
            c1 = min(c0 + cap, e)
            if c1 - c0 >= 2:
                out.append((c0, c1 - c0, int(min(links[c0 + 1:c1]))))
        s = e
    return out


@pytest.mark.parametrize("kv_dtype,q_dtype,Hq,Hkv,D", [
    (1, 1, 32, 8, 128),   # C5 shape, G = 4: groups of up to 4
    (1, 0, 8, 8, 64),     # G = 1: groups of up to 16, fp32 q
    (1, 1, 16, 2, 256),   # G = 8: pairs
    (2, 1, 32, 8, 128),   # int8 cache
    (2, 0, 16, 4, 64),    # int8, fp32 q
])
def test_prefix_decode_matches_oracle(stream, kv_dtype, q_dtype, Hq, Hkv, D):
    rng = np.random.default_rng(100 + D + kv_dtype)
    S = 19
    lens = rng.integers(200, 700, size=S).astype(np.int32)
    groups = [(0, 8, 12), (8, 3, 5), (12, 5, 9), (17, 2, 1)]  # seq 11 alone
    lens[9] = 16 * 5            # suffix empty: the whole context is shared
    lens[14] = 16 * 9 + 1       # one private token
    w, links = shared_case(rng.integers(1 << 30), lens, groups, Hq=Hq, Hkv=Hkv, D=D, kv_dtype=kv_dtype,
                           q_dtype=q_dtype)
    got, ref, ng, plan = run_prefix(stream, w, links)
    G = Hq // Hkv
    exp = expected_groups(links, G)
    assert ng == len(exp)
    np.testing.assert_array_equal(plan[:3 * ng].reshape(-1, 3), np.array(exp, np.int32).reshape(-1, 3))
    check_close(got, ref, **tol_for(kv_dtype), what=f"prefix decode kv{kv_dtype} G{G} D{D}")


def test_prefix_decode_c5_subset(stream):
    """C5's structure at a reduced size: 8 sequences sharing 1024 tokens, contexts 2-4k."""
    w = wl.make_c5(seed=9, batch=8, lo=2048, hi=4096, prefix_tokens=1024)
    links = np.zeros(w.num_seqs, np.int32)
    links[1:] = w.shared_prefix_blocks
    got, ref, ng, _ = run_prefix(stream, w, links)
    assert ng == 2
    check_close(got, ref, **tol_for(w.kv_dtype), what="C5 subset")


def test_prefix_decode_without_groups_and_empty_rows(stream):
    """No links: every sequence is its own row (the plan holds no group); zero-length contexts
    give zeros; the result equals pa_paged_decode's."""
    lens = np.array([0, 37, 500, 16, 0, 1200], np.int32)
    w, links = shared_case(5, lens, [], Hq=8, Hkv=2, D=128)
    got, ref, ng, _ = run_prefix(stream, w, links)
    assert ng == 0
    check_close(got, ref, **tol_for(1), what="no groups")
    assert np.all(got[0] == 0) and np.all(got[4] == 0)


def test_prefix_plan_and_args_validated_on_the_host(stream):
    cfg = pa.make_config(num_q_heads=32, num_kv_heads=8, head_dim=128, kv_dtype=1, num_blocks=64)
    pb = pa.prefix_plan_bytes(4)
    plan = empty_gpu((pb,), np.uint8)
    with pytest.raises(pa.PagedAttentionError):
        pa.prefix_plan_build(stream, cfg, [0, -1, 0, 0], plan, pb)
    with pytest.raises(pa.PagedAttentionError):
        pa.prefix_plan_build(stream, cfg, [0, 1, 1, 1], plan, pb - 4)
    fcfg = pa.make_config(num_q_heads=32, num_kv_heads=8, head_dim=128, kv_dtype=0, num_blocks=64)
    dummy = empty_gpu((1 << 20,), np.uint8)
    with pytest.raises(pa.PagedAttentionError):  # fp32 caches are not served by this path
        pa.paged_decode_prefix(stream, fcfg, dummy, dummy, dummy, dummy, None, None, dummy, dummy, 4, 4, 64,
                               plan, 0, dummy, 1 << 20)
    with pytest.raises(pa.PagedAttentionError):  # more groups than pairs of sequences
        pa.paged_decode_prefix(stream, cfg, dummy, dummy, dummy, dummy, None, None, dummy, dummy, 4, 4, 64,
                               plan, 3, dummy, 1 << 20)


def test_prefix_decode_graph_replay_matches_eager():
    """The shared-prefix decode records kernels only: captured once, replayed with new queries,
    every replay equals the eager call bit for bit and the oracle within tolerance."""
    import torch

    torch.cuda.init()
    dev = pa.Device(0)
    gs = pa.Stream(dev)  # a library stream: the null stream cannot capture
    try:
        rng = np.random.default_rng(77)
        lens = rng.integers(300, 600, size=9).astype(np.int32)
        w, links = shared_case(78, lens, [(0, 4, 10), (4, 5, 6)], Hq=32, Hkv=8, D=128)
        inp = wl.numpy_inputs(w, 9)
        cfg = config_for(w)
        S = w.num_seqs
        pb = pa.prefix_plan_bytes(S)
        plan = empty_gpu((pb,), np.uint8)
        torch.cuda.synchronize()
        ng = pa.prefix_plan_build(gs, cfg, links, plan, pb)
        wsb = pa.prefix_workspace_size(cfg, S, w.max_context_len)
        ws = empty_gpu((wsb,), np.uint8)
        out = empty_gpu((S, w.num_q_heads, w.head_dim), np.float32)
        q = to_gpu(inp["q"])
        kc, vc = to_gpu(inp["k_cache"]), to_gpu(inp["v_cache"])
        args = (q, kc, vc, None, None, to_gpu(w.block_tables), to_gpu(w.context_lens), S, w.max_blocks,
                w.max_context_len, plan, ng, ws, wsb)
        torch.cuda.synchronize()
        g = pa.Graph().capture(gs)
        pa.paged_decode_prefix(gs, cfg, out, *args)
        g.end()
        try:
            for r in range(3):
                qv = orc.bf16_from_f32(rng.standard_normal(inp["q"].shape, dtype=np.float32))
                q.copy_(to_gpu(qv))
                torch.cuda.synchronize()
                g.launch(gs)
                gs.synchronize()
                replay = to_np(out).copy()
                pa.paged_decode_prefix(gs, cfg, out, *args)
                gs.synchronize()
                np.testing.assert_array_equal(replay, to_np(out))
                ref = orc.paged_decode(cfg, qv, inp["k_cache"], inp["v_cache"], None, None, w.block_tables,
                                       w.context_lens, n_threads=NTHREADS)
                check_close(replay, ref, **tol_for(1), what=f"graph replay {r}")
        finally:
            g.destroy()
    finally:
        gs.destroy()
        dev.close()


def test_c5_full_size_vs_oracle(stream):
    """Full C5 (8 sequences of 16-32k tokens, 512 shared blocks): pa_paged_decode with the default
    split and pa_paged_decode_prefix, the two calls bench.py times, each against the oracle's
    whole-context decode; the configuration's stated split (num_splits = 16 partitions per sequence
    with the log-sum-exp merge) against the oracle as well; a 64-token split (about 500 partials per
    row: the merge's multi-round path) against the default split."""
    import torch

    w = wl.make_c5()
    S, Hq, Hkv, D = w.num_seqs, w.num_q_heads, w.num_kv_heads, w.head_dim
    g = torch.Generator(device="cuda:0")
    g.manual_seed(55)

    def bf16(*shape):
        x = torch.randn(*shape, generator=g, device="cuda:0", dtype=torch.float32)
        return (x.view(torch.int32) >> 16).to(torch.int16)

    q = bf16(S, Hq, D)
    kc, vc = bf16(w.num_blocks, Hkv, 16, D), bf16(w.num_blocks, Hkv, 16, D)
    tables, lens = to_gpu(w.block_tables), to_gpu(w.context_lens)
    mcl = w.max_context_len
    outs = {}
    for name, part, nsp in (("default", 0, 0), ("p64", 64, 0), ("split16", 0, 16)):
        cfg = config_for(w, partition_size=part, num_splits=nsp)
        wsb = pa.decode_workspace_size(cfg, S, mcl)
        ws = empty_gpu((wsb,), np.uint8)
        out = empty_gpu((S, Hq, D), np.float32)
        pa.paged_decode(stream, cfg, out, q, kc, vc, None, None, tables, lens, S, w.max_blocks, mcl, ws, wsb)
        _sync()
        outs[name] = to_np(out).copy()
    cfg = config_for(w)
    links = np.zeros(S, np.int32)
    links[1:] = w.shared_prefix_blocks
    pb = pa.prefix_plan_bytes(S)
    plan = empty_gpu((pb,), np.uint8)
    ng = pa.prefix_plan_build(stream, cfg, links, plan, pb)
    assert ng == 2
    wsb = pa.prefix_workspace_size(cfg, S, mcl)
    ws = empty_gpu((wsb,), np.uint8)
    out = empty_gpu((S, Hq, D), np.float32)
    pa.paged_decode_prefix(stream, cfg, out, q, kc, vc, None, None, tables, lens, S, w.max_blocks, mcl, plan, ng,
                           ws, wsb)
    _sync()
    outs["prefix"] = to_np(out).copy()
    ref = orc.paged_decode(cfg, to_np(q, np.uint16), to_np(kc, np.uint16), to_np(vc, np.uint16), None, None,
                           w.block_tables, w.context_lens, n_threads=NTHREADS)
    check_close(outs["default"], ref, **tol_for(1), what="C5 pa_paged_decode vs oracle")
    check_close(outs["prefix"], ref, **tol_for(1), what="C5 pa_paged_decode_prefix vs oracle")
    check_close(outs["split16"], ref, **tol_for(1), what="C5 with 16 partitions per sequence vs oracle")
    check_close(outs["p64"], outs["default"], **tol_for(1), what="C5 64-token split vs default")
