#!/usr/bin/env python3
"""Paged-attention benchmark on one MI355X (the BASELINE.json metric, plus the other configurations).

Headline step = one decode layer-step of the C2 configuration (Llama-3-8B layer shape: Hq=32,
Hkv=8, D=128, bf16 KV, block 16, batch 64, contexts log-uniform in [128, 4096], shuffled physical
blocks): append the new token's K/V of every sequence into the paged cache and attend over each
sequence's whole context, as one pa_paged_decode_append call (the fused decode kernel plus the
split-K merge). Inputs are resident in HBM before timing starts; all launches go through the
C-ABI of libpa_hip.so on one pa_stream and are timed with pa_events recorded on that stream,
the timed calls queued behind a short spin kernel so that the start event marks the GPU starting
the first timed call, not the host starting to launch it (`Timer`; the headline is also reported
without that gate, `two_pool.ungated_us_per_layer_step`). The timed steps alternate between two
disjoint copies of the cache (about 2 x 300 MB), so no step finds K/V that the step before left
in the 256 MB last-level cache: the figure is the cold-HBM rate a serving loop sees when the other
layers' K/V pass through that cache between two steps of one layer. The same step repeated over
one pool is reported beside it as `one_pool`; it, the same step replayed from a captured graph
and the two-call form of the step are timed before the headline (unless `--only-step`), so that
the headline's warm-up and timed steps run on a GPU that has been working.

Output: one JSON line. `value` is the achieved algorithmic HBM bandwidth of the whole step
(distinct KV bytes read + Q + O + block tables + the appended K/V, divided by the step time);
tokens/s per layer and us per layer-step ride along. `roofline` covers the same call. `extra`
times the other configurations the same way: C4 (int8 KV, fused append + decode), C5 (long
contexts with a shared prefix, decode), C3 (mixed: fused decode of 48 sequences, the append of
8 prefill chunks and their chunked prefill, with the prefill's MFMA rate) and the whole-block
moves (copy-on-write copies and swap-out of 4096 blocks, HBM GB/s) and a whole C2 decode layer
with its Q/K/V and output projections (Llama-3-8B weights). `cpu_baseline` times
the CPU oracle (a C restatement of the reference's StandardPagedAttentionKernel with its
per-sequence decode loop) on a bounded sample of the C2 batch, on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "ml-framework_amd"))

import paged_attention as pa  # noqa: E402
import workloads as wl  # noqa: E402

METRIC = "paged decode HBM GB/s (% peak) + tokens/s per layer, Llama-3-8B shape, 1 GPU"
PEAK_HBM_GBPS = 8000.0
PEAK_BF16_TFLOPS = 2500.0  # dense MFMA
GATE_CLOCKS_PER_US = 2500  # the timer's spin: shader clocks per us, above MI355X's 2.4 GHz top clock
GATE_MAX_SPIN_US = 2000.0
# HBM traffic of the headline call measured with rocprofv3 counters (FETCH_SIZE, WRITE_SIZE per
# dispatch, scaled by the same counters' reading for a plain copy of known size); written by the
# profiling summary, absent until then.
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "c2_decode_append_traffic.json")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def bf16_trunc_torch(x):
    import torch

    return (x.contiguous().view(torch.int32) >> 16).to(torch.int16)


def tensor(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def make_inputs(w: wl.Workload, seed: int):
    """Caches, q, new-token K/V and index arrays on the GPU (torch tensors as device memory).

    bf16/fp32 caches hold N(0,1) * value_scale values; int8 caches hold random codes in
    [-127, 127] with per-(block, KV head) scales (absmax = 127 * scale), which is what the
    kernels read whatever the codes' origin."""
    import torch

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    S, Hq, Hkv, D, nb = w.num_seqs, w.num_q_heads, w.num_kv_heads, w.head_dim, w.num_blocks
    vs = w.value_scale

    def randn(*shape):
        return torch.randn(*shape, generator=g, device=dev, dtype=torch.float32) * vs

    def act(*shape):  # activations in the q dtype
        x = randn(*shape)
        return bf16_trunc_torch(x) if w.q_dtype == pa.PA_DTYPE_BF16 else x

    out = dict(q=act(S, Hq, D), k_new=act(S, Hkv, D), v_new=act(S, Hkv, D),
               tables=tensor(w.block_tables), lens=tensor(w.context_lens),
               k_scale=None, v_scale=None, k_absmax=None, v_absmax=None)
    if w.kv_dtype == pa.PA_DTYPE_INT8:
        for n in ("k", "v"):
            out[f"{n}_cache"] = torch.randint(-127, 128, (nb, Hkv, 16, D), generator=g, device=dev,
                                              dtype=torch.int8)
            sc = torch.rand(nb, Hkv, generator=g, device=dev, dtype=torch.float32) * 0.02 + 0.01
            out[f"{n}_scale"] = sc
            out[f"{n}_absmax"] = sc * 127.0
    elif w.kv_dtype == pa.PA_DTYPE_BF16:
        out["k_cache"] = bf16_trunc_torch(randn(nb, Hkv, 16, D))
        out["v_cache"] = bf16_trunc_torch(randn(nb, Hkv, 16, D))
    else:
        out["k_cache"] = randn(nb, Hkv, 16, D)
        out["v_cache"] = randn(nb, Hkv, 16, D)
    # The library runs on its own stream: torch's kernels (and the temporaries they free on enqueue,
    # whose memory torch hands out again at once) must be done before any of it is used there.
    torch.cuda.synchronize()
    return out


def config_of(w: wl.Workload, partition_size=0, num_splits=0):
    return pa.make_config(num_q_heads=w.num_q_heads, num_kv_heads=w.num_kv_heads, head_dim=w.head_dim,
                          kv_dtype=w.kv_dtype, q_dtype=w.q_dtype, num_blocks=w.num_blocks,
                          partition_size=partition_size, num_splits=num_splits)


class Timer:
    """Times a callable with pa_events recorded on the stream the library launches on.

    With `gate` (the default) the timed calls are queued behind a gate: after the synchronize,
    a spin kernel on torch's stream that the library's stream waits for, long enough for the host
    to enqueue all `steps` calls (twice the host's measured enqueue time per call, plus 200 us, at
    most 2 ms; the spin counts shader clocks, converted at 2.5 GHz, above the chip's top clock, so
    that it lasts at least that long at any clock). The MFMA-bound prefill legs are timed without
    the gate: after an idle spell the chip's clocks drop and that kernel runs slower for a while.
    The start event is then taken when the GPU begins the first timed call rather than when the
    host begins issuing it, so a short run measures the same per-step rate as a long one: without
    the gate, the first call of a run waits for its own launch from Python (about 10 us of host
    work per call) on an idle queue. `last_gate` records the spin and the host's enqueue time of
    the last timed run (`covered` is false if the host was still enqueueing when the spin ended)."""

    def __init__(self, dev, stream, gate=True):
        self.dev, self.stream, self.gate = dev, stream, gate
        self.last_gate = None
        self._torch_stream = None

    def __call__(self, fn, steps, warmup, gate=None):
        import torch

        # the gate's spin kernel is torch's own test helper; without it the run is timed ungated
        gate = (self.gate if gate is None else gate) and hasattr(torch.cuda, "_sleep")
        torch.cuda.synchronize()  # buffers allocated through torch are settled before the library's stream runs
        t0 = time.perf_counter()
        for _ in range(warmup):
            fn()
        host_per_call_us = (time.perf_counter() - t0) * 1e6 / warmup if warmup else 50.0
        self.stream.synchronize()
        e0, e1 = pa.Event(self.dev), pa.Event(self.dev)
        g0 = g1 = None
        torch.cuda.synchronize()
        if gate:
            if self._torch_stream is None:
                self._torch_stream = pa.TorchStream.current(0).stream
            g0, g1 = pa.Event(self.dev), pa.Event(self.dev)
            # at most 2 ms: a longer idle spin lets the clocks drop before the timed calls
            spin_us = min(200.0 + 2.0 * steps * host_per_call_us, GATE_MAX_SPIN_US)
            t_host = time.perf_counter()
            g0.record(self._torch_stream)
            torch.cuda._sleep(int(spin_us * GATE_CLOCKS_PER_US))
            g1.record(self._torch_stream)
            self.stream.wait_event(g1)
        e0.record(self.stream)
        for _ in range(steps):
            fn()
        e1.record(self.stream)
        if gate:
            host_us = (time.perf_counter() - t_host) * 1e6
        e1.synchronize()
        ms = e0.elapsed_ms(e1) / steps
        if gate:
            spun = g0.elapsed_ms(g1) * 1e3
            self.last_gate = {"spin_us": round(spun, 1), "host_enqueue_us": round(host_us, 1),
                              "covered": bool(host_us < spun)}
            g0.destroy()
            g1.destroy()
        e0.destroy()
        e1.destroy()
        return ms


def decode_step(w, inp, stream, cfg, fused, out, ws, wsb):
    S, mcl = w.num_seqs, w.max_context_len
    if fused:
        return lambda: pa.paged_decode_append(stream, cfg, out, inp["q"], inp["k_new"], inp["v_new"], inp["k_cache"],
                                              inp["v_cache"], inp["k_scale"], inp["v_scale"], inp["k_absmax"],
                                              inp["v_absmax"], inp["tables"], inp["lens"], S, w.max_blocks, mcl,
                                              ws, wsb)
    return lambda: pa.paged_decode(stream, cfg, out, inp["q"], inp["k_cache"], inp["v_cache"], inp["k_scale"],
                                   inp["v_scale"], inp["tables"], inp["lens"], S, w.max_blocks, mcl, ws, wsb)


def decode_buffers(w, cfg):
    import torch

    out = torch.empty((w.num_seqs, w.num_q_heads, w.head_dim), dtype=torch.float32, device="cuda:0")
    wsb = pa.decode_workspace_size(cfg, w.num_seqs, w.max_context_len)
    ws = torch.empty((max(wsb, 1),), dtype=torch.uint8, device="cuda:0")
    return out, ws, wsb


def append_bytes(w):
    """The appended token of every sequence: new K/V read in the activation dtype + cache write."""
    act = 2 if w.q_dtype == pa.PA_DTYPE_BF16 else 4
    cache = {0: 4, 1: 2, 2: 1}[w.kv_dtype]
    return 2 * w.num_seqs * w.num_kv_heads * w.head_dim * (act + cache)


def run_decode_config(w, timer, stream, steps, warmup, fused, seed, num_splits=0):
    inp = make_inputs(w, seed)
    cfg = config_of(w, num_splits=num_splits)
    out, ws, wsb = decode_buffers(w, cfg)
    ms = timer(decode_step(w, inp, stream, cfg, fused, out, ws, wsb), steps, warmup)
    nbytes = w.decode_algorithmic_bytes() + (append_bytes(w) if fused else 0)
    gbps = nbytes / (ms * 1e-3) / 1e9
    res = {"us_per_layer_step": round(ms * 1e3, 3), "algorithmic_bytes": int(nbytes), "gbps": round(gbps, 1),
           "frac_hbm": round(gbps / PEAK_HBM_GBPS, 4), "tokens_per_s_per_layer": round(w.num_seqs / (ms * 1e-3), 1),
           "context_tokens": int(w.context_lens.sum()), "num_seqs": w.num_seqs,
           "step": "pa_paged_decode_append" if fused else "pa_paged_decode",
           "split": f"{num_splits} partitions per sequence" if num_splits else "library default (equal ranges)"}
    del inp, out, ws
    return res


def run_two_pool(w, inp, timer, stream, cfg, steps, warmup):
    """The headline step alternating between two disjoint copies of the C2 cache (same tables, a
    second pool in its own memory): a pair of steps touches about twice the 256 MB last-level
    cache, so no step finds its K/V left in that cache by the step before. Returns (ms per step,
    summary)."""
    inp2 = make_inputs(w, seed=4321)
    out, ws, wsb = decode_buffers(w, cfg)
    s1 = decode_step(w, inp, stream, cfg, True, out, ws, wsb)
    s2 = decode_step(w, inp2, stream, cfg, True, out, ws, wsb)

    def pair():
        s1()
        s2()

    ms = timer(pair, max(1, steps // 2), warmup) / 2
    gate = timer.last_gate
    # the same run without the gate: the host's launch of the first call is then inside the timed
    # region (the difference shrinks as steps grow)
    ms_ungated = timer(pair, max(1, steps // 2), warmup, gate=False) / 2
    nbytes = w.decode_algorithmic_bytes() + append_bytes(w)
    gbps = nbytes / (ms * 1e-3) / 1e9
    res = {"us_per_layer_step": round(ms * 1e3, 3), "gbps": round(gbps, 1), "frac_hbm": round(gbps / PEAK_HBM_GBPS, 4),
           "kv_bytes_per_pool": int(2 * inp["k_cache"].numel() * inp["k_cache"].element_size()),
           "step": "pa_paged_decode_append, pools alternating",
           "gate": gate, "ungated_us_per_layer_step": round(ms_ungated * 1e3, 3)}
    del inp2, out, ws
    return ms, res


def run_prefix_decode(w, timer, stream, steps, warmup, seed):
    """C5 through pa_paged_decode_prefix: the sequences' shared blocks are read once per group of
    16 / G sequences; same inputs, output and algorithmic (distinct) bytes as the plain decode."""
    import torch

    inp = make_inputs(w, seed)
    cfg = config_of(w)
    S = w.num_seqs
    links = np.zeros(S, np.int32)
    links[1:] = w.shared_prefix_blocks
    pb = pa.prefix_plan_bytes(S)
    plan = torch.empty((max(pb, 4),), dtype=torch.uint8, device="cuda:0")
    out = torch.empty((S, w.num_q_heads, w.head_dim), dtype=torch.float32, device="cuda:0")
    wsb = pa.prefix_workspace_size(cfg, S, w.max_context_len)
    ws = torch.empty((max(wsb, 1),), dtype=torch.uint8, device="cuda:0")
    torch.cuda.synchronize()
    ng = pa.prefix_plan_build(stream, cfg, links, plan, pb)

    def step():
        pa.paged_decode_prefix(stream, cfg, out, inp["q"], inp["k_cache"], inp["v_cache"], inp["k_scale"],
                               inp["v_scale"], inp["tables"], inp["lens"], S, w.max_blocks, w.max_context_len,
                               plan, ng, ws, wsb)

    ms = timer(step, steps, warmup)
    nbytes = w.decode_algorithmic_bytes()
    gbps = nbytes / (ms * 1e-3) / 1e9
    res = {"us_per_layer_step": round(ms * 1e3, 3), "algorithmic_bytes": int(nbytes), "gbps": round(gbps, 1),
           "frac_hbm": round(gbps / PEAK_HBM_GBPS, 4), "groups": ng, "step": "pa_paged_decode_prefix"}
    del inp, out, ws, plan
    return res


def c3_setup(stream, seed):
    """C3 inputs and the three calls of its layer-step: (workload, decode, chunk append, prefill, prefix lengths)."""
    import torch

    w = wl.make_c3()
    inp = make_inputs(w, seed)
    cfg = config_of(w)
    out, ws, wsb = decode_buffers(w, cfg)
    dec = decode_step(w, inp, stream, cfg, True, out, ws, wsb)

    P = w.prefill_prefix.astype(np.int64)
    L = w.prefill_chunk
    n_pre = len(P)
    g = torch.Generator(device="cuda:0")
    g.manual_seed(seed + 1)
    tot = n_pre * L
    q_pre = bf16_trunc_torch(torch.randn(tot, w.num_q_heads, w.head_dim, generator=g, device="cuda:0") * 0.5)
    k_pre = bf16_trunc_torch(torch.randn(tot, w.num_kv_heads, w.head_dim, generator=g, device="cuda:0") * 0.5)
    v_pre = bf16_trunc_torch(torch.randn(tot, w.num_kv_heads, w.head_dim, generator=g, device="cuda:0") * 0.5)
    pos = (P[:, None] + np.arange(L)[None, :])
    tab = w.prefill_tables
    slots = (tab[np.arange(n_pre)[:, None], pos // 16].astype(np.int64) * 16 + pos % 16).reshape(-1)
    slots_g = tensor(slots)
    q_start = tensor(np.arange(n_pre + 1, dtype=np.int32) * L)
    prefix_g = tensor(P.astype(np.int32))
    tab_g = tensor(tab)
    out_pre = torch.empty((tot, w.num_q_heads, w.head_dim), dtype=torch.float32, device="cuda:0")

    def app():
        pa.kv_append(stream, cfg, k_pre, v_pre, slots_g, tot, inp["k_cache"], inp["v_cache"])

    def pre():
        pa.chunked_prefill(stream, cfg, out_pre, q_pre, q_start, prefix_g, inp["k_cache"], inp["v_cache"], None,
                           None, tab_g, n_pre, tab.shape[1], L)

    return w, dec, app, pre, P, L, tot


# Untimed prefill calls before the C3 prefill and step are timed: the MFMA-bound prefill runs
# at lower clocks until the chip has been busy for some 50 ms (measured: 144.9 / 132.8 / 127.8 us
# per call after 10 / 100 / 400 warm-up calls), and a serving loop runs at the steady clocks.
PREFILL_WARMUP_CALLS = 400
DECODE_WARMUP_CALLS = 200


def run_c3(timer, stream, steps, warmup, seed):
    """C3: fused decode of 48 sequences + append of 8 prefill chunks (512 tokens each) + their prefill."""
    w, dec, app, pre, P, L, tot = c3_setup(stream, seed)
    n_pre = len(P)

    def step():
        dec()
        app()
        pre()

    ms_dec = timer(dec, steps, warmup)
    ms_app = timer(app, steps, warmup)
    # the MFMA-bound prefill runs at lower clocks after an idle spell, so its legs are timed ungated
    ms_pre = timer(pre, steps, max(warmup, PREFILL_WARMUP_CALLS), gate=False)
    ms_step = timer(step, steps, max(warmup, PREFILL_WARMUP_CALLS), gate=False)
    flops = float(4 * w.num_q_heads * w.head_dim * np.sum(L * P + L * (L + 1) / 2))
    pre_kv_bytes = float(np.sum(P + L)) * w.kv_bytes_per_token()
    dec_bytes = w.decode_algorithmic_bytes() + append_bytes(w)
    app_bytes = tot * w.num_kv_heads * w.head_dim * 2 * (2 + 2)
    tflops = flops / (ms_pre * 1e-3) / 1e12
    return {
        "us_per_layer_step": round(ms_step * 1e3, 3),
        "decode": {"us": round(ms_dec * 1e3, 3), "num_seqs": w.num_seqs, "algorithmic_bytes": int(dec_bytes),
                   "gbps": round(dec_bytes / (ms_dec * 1e-3) / 1e9, 1),
                   "frac_hbm": round(dec_bytes / (ms_dec * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)},
        "chunk_append": {"us": round(ms_app * 1e3, 3), "tokens": tot, "algorithmic_bytes": int(app_bytes),
                         "gbps": round(app_bytes / (ms_app * 1e-3) / 1e9, 1)},
        "prefill": {"us": round(ms_pre * 1e3, 3), "chunks": n_pre, "chunk_len": L,
                    "prefix_lens": [int(x) for x in P], "flops": flops, "tflops": round(tflops, 1),
                    "frac_mfma_bf16_dense": round(tflops / PEAK_BF16_TFLOPS, 4), "kv_bytes": int(pre_kv_bytes)},
    }


def cpu_baseline(w: wl.Workload, inp, budget_s: float):
    """Times the CPU oracle (1 thread) on the first n sequences of the batch, n grown until the
    sample costs about `budget_s` seconds, and scales to the whole batch by context tokens."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pa_oracle as orc  # test infrastructure: the timed CPU baseline only

    cfg = config_of(w)
    kc = inp["k_cache"].cpu().numpy().view(np.uint16)
    vc = inp["v_cache"].cpu().numpy().view(np.uint16)
    q = inp["q"].cpu().numpy().view(np.uint16)
    n, spent, toks = 0, 0.0, 0
    t_start = time.perf_counter()
    while n < w.num_seqs and spent < budget_s:
        t0 = time.perf_counter()
        orc.paged_decode(cfg, np.ascontiguousarray(q[n:n + 1]), kc, vc, None, None,
                         w.block_tables[n:n + 1], w.context_lens[n:n + 1], n_threads=1)
        spent += time.perf_counter() - t0
        toks += int(w.context_lens[n])
        n += 1
    wall = time.perf_counter() - t_start
    full_time = spent * (int(w.context_lens.sum()) / max(toks, 1))
    # Anchor at the reference's one published shape (batch 1, 16 cached tokens, 32 heads x 128, fp32,
    # MHA): 420.0 us on a Ryzen 7 3800X under .NET 9 (different CPU: a sanity check only).
    acfg = pa.make_config(num_q_heads=32, num_kv_heads=32, head_dim=128, kv_dtype=0, q_dtype=0, num_blocks=1)
    rng = np.random.default_rng(42)
    aq = rng.random((1, 32, 128), dtype=np.float32)
    akc = rng.random((1, 32, 16, 128), dtype=np.float32)
    avc = rng.random((1, 32, 16, 128), dtype=np.float32)
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < 1.0:
        orc.paged_decode(acfg, aq, akc, avc, None, None, np.zeros((1, 1), np.int32),
                         np.array([16], np.int32), n_threads=1)
        reps += 1
    anchor_us = (time.perf_counter() - t0) / reps * 1e6
    # All host cores (OpenMP over sequences, capped at the 16-core share of a one-GPU box): the
    # whole batch in one call, best of three.
    threads = max(1, min(16, os.cpu_count() or 1))
    best = float("inf")
    for _ in range(3):
        t0 = time.perf_counter()
        orc.paged_decode(cfg, q, kc, vc, None, None, w.block_tables, w.context_lens, n_threads=threads)
        best = min(best, time.perf_counter() - t0)
    return {
        "value": w.num_seqs / full_time,
        "unit": "tokens/s per layer",
        "cores": 1,
        "kind": "port",
        "sample": (f"{n} of {w.num_seqs} sequences ({toks} context tokens) of the same C2 batch, "
                   f"oracle paged decode (C restatement of StandardPagedAttentionKernel, per-sequence "
                   f"calls), 1 thread, {spent:.1f} s measured ({wall:.1f} s wall), scaled to all "
                   f"{int(w.context_lens.sum())} context tokens"),
        "us_per_layer_step": full_time * 1e6,
        "gbps_equivalent": w.decode_algorithmic_bytes() / full_time / 1e9,
        "anchor_published_shape_us": anchor_us,
        "anchor_published_reference_us": 420.0,
        "host_cpu": _cpu_model(),
        "host_nproc": os.cpu_count(),
        "all_cores": {"threads": threads, "value": w.num_seqs / best, "unit": "tokens/s per layer",
                      "us_per_layer_step": best * 1e6,
                      "sample": f"the whole C2 batch in one oracle call, {threads} OpenMP threads, best of 3"},
    }


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def load_traffic():
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return float(t["hbm_bytes_per_call"]), t
    except (OSError, KeyError, ValueError):
        return None, None


def run_block_moves(timer, stream, steps, warmup, seed):
    """Copy-on-write (pa_copy_blocks) and swap-out (pa_gather_blocks into a device buffer) of 4096
    blocks of a C2-shaped bf16 cache (Hkv 8, D 128: 64 KiB of K and V per block); bytes are read +
    written, 512 MB per call, twice the 256 MB last-level cache, so the rate is HBM's."""
    import torch

    nb, pairs_n = 16384, 4096
    cfg = pa.make_config(num_q_heads=32, num_kv_heads=8, head_dim=128, kv_dtype=1, q_dtype=1, num_blocks=nb)
    kc = torch.zeros((nb, 8, 16, 128), dtype=torch.int16, device="cuda:0")
    vc = torch.zeros_like(kc)
    perm = np.random.default_rng(seed).permutation(nb).astype(np.int32)
    pairs = torch.tensor(np.stack([perm[:pairs_n], perm[pairs_n:2 * pairs_n]], 1), device="cuda:0")
    ids = torch.tensor(perm[:pairs_n], device="cuda:0")
    rec = pa.block_bytes(cfg)
    packed = torch.empty((pairs_n, rec), dtype=torch.uint8, device="cuda:0")
    ms_copy = timer(lambda: pa.copy_blocks(stream, cfg, kc, vc, None, None, None, None, pairs, pairs_n), steps, warmup)
    ms_gather = timer(lambda: pa.gather_blocks(stream, cfg, kc, vc, None, None, None, None, ids, pairs_n, packed),
                      steps, warmup)
    moved = 2 * pairs_n * rec  # bytes read + written
    return {"blocks": pairs_n, "bytes_per_block": rec,
            "copy_blocks_us": round(ms_copy * 1e3, 2), "copy_blocks_gbps": round(moved / (ms_copy * 1e-3) / 1e9, 1),
            "gather_blocks_us": round(ms_gather * 1e3, 2),
            "gather_blocks_gbps": round(moved / (ms_gather * 1e-3) / 1e9, 1)}


WEIGHT_ROTATION_BYTES = 320 << 20  # more than the 256 MB last-level cache


def run_layer(timer, stream, w, inp, steps, warmup, seed):
    """One whole decode layer of the C2 batch with Llama-3-8B projection weights (hidden 4096,
    bf16): pa_qkv_project_append (x . W_qkv^T, Q out, K/V appended), pa_paged_decode over the
    cache, pa_o_project. Times each call and the three in sequence; the GEMMs are weight-bound, so
    their rate is weight bytes per second. Successive calls cycle through copies of each weight that
    together exceed the last-level cache, as the layers of a model do (each has its own weights),
    so the weights come from HBM."""
    import itertools

    import torch

    hidden, S = 4096, w.num_seqs
    cfg = config_of(w, 0)
    hq, hkv, d = w.num_q_heads, w.num_kv_heads, w.head_dim
    g = torch.Generator(device="cuda:0")
    g.manual_seed(seed)
    bf = lambda *shape: (torch.randn(*shape, generator=g, device="cuda:0") * 0.02).to(torch.bfloat16)
    x = bf(S, hidden)
    w_qkv = bf((hq + 2 * hkv) * d, hidden)
    w_o = bf(hidden, hq * d)
    copies = lambda t: itertools.cycle([t] + [t.clone() for _ in range(-(-WEIGHT_ROTATION_BYTES // (t.numel() * 2)) - 1)])
    wq_cycle, wo_cycle = copies(w_qkv), copies(w_o)
    q = torch.empty((S, hq, d), dtype=torch.bfloat16, device="cuda:0")
    attn = torch.empty((S, hq, d), dtype=torch.float32, device="cuda:0")
    y = torch.empty((S, hidden), dtype=torch.float32, device="cuda:0")
    qws_b, ows_b = pa.qkv_workspace_size(cfg, S), pa.o_workspace_size(cfg, hidden, S)
    qws = torch.empty(qws_b, dtype=torch.uint8, device="cuda:0")
    ows = torch.empty(ows_b, dtype=torch.uint8, device="cuda:0")
    dws_b = pa.decode_workspace_size(cfg, S, w.max_context_len)
    dws = torch.empty(max(dws_b, 1), dtype=torch.uint8, device="cuda:0")
    pos = w.context_lens.astype(np.int64) - 1
    slots = tensor(w.block_tables[np.arange(S), pos // 16].astype(np.int64) * 16 + pos % 16)

    def qkv():
        pa.qkv_project_append(stream, cfg, x, next(wq_cycle), hidden, S, slots, q, inp["k_cache"], inp["v_cache"],
                              None, None, None, None, qws, qws_b)

    def dec():
        pa.paged_decode(stream, cfg, attn, q, inp["k_cache"], inp["v_cache"], None, None, inp["tables"], inp["lens"],
                        S, w.max_blocks, w.max_context_len, dws, dws_b)

    def oproj():
        pa.o_project(stream, cfg, attn, next(wo_cycle), hidden, S, y, ows, ows_b)

    def layer():
        qkv(); dec(); oproj()

    qkv()  # creates the device's rocBLAS handle outside the timed region
    stream.synchronize()
    t = {k: timer(f, steps, warmup) * 1e3 for k, f in (("qkv", qkv), ("decode", dec), ("o", oproj), ("layer", layer))}
    wq_bytes, wo_bytes = w_qkv.numel() * 2, w_o.numel() * 2
    return {"hidden": hidden, "weights": "cycled through copies over 320 MB (HBM, not the last-level cache)",
            "qkv_project_append_us": round(t["qkv"], 2),
            "qkv_weight_gbps": round(wq_bytes / (t["qkv"] * 1e-6) / 1e9, 1),
            "decode_us": round(t["decode"], 2), "o_project_us": round(t["o"], 2),
            "o_weight_gbps": round(wo_bytes / (t["o"] * 1e-6) / 1e9, 1), "layer_us": round(t["layer"], 2)}


def copy_calibration(args, stream):
    """10 plain device-to-device copies of --copy-calibration-mb MiB (pa_memcpy): the reference
    dispatches for scaling hardware byte counters (FETCH_SIZE, WRITE_SIZE) in the same process."""
    import torch

    if args.copy_calibration_mb <= 0:
        return
    nbytes = args.copy_calibration_mb << 20
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty(nbytes, dtype=torch.uint8, device="cuda:0")
    torch.cuda.synchronize()
    for _ in range(10):
        pa.call("pa_memcpy", dst.data_ptr(), src.data_ptr(), nbytes, pa.PA_MEMCPY_DEVICE_TO_DEVICE, stream.handle)
    stream.synchronize()
    log(f"[bench] copy calibration: 10 x {nbytes} bytes device-to-device")


GRAPH_CALLS = 32  # layer-steps per captured graph: one decode step of a 32-layer (Llama-3-8B) model


def time_graph_replay(step, timer, stream, steps):
    """Captures GRAPH_CALLS fused layer-steps into one graph (pa_graph_*) and returns the time per
    layer-step of its replays on `stream` (the calls reuse one layer's buffers)."""
    stream.synchronize()
    g = pa.Graph().capture(stream)
    for _ in range(GRAPH_CALLS):
        step()
    g.end()
    try:
        return timer(lambda: g.launch(stream), max(1, steps // GRAPH_CALLS), 2) / GRAPH_CALLS
    finally:
        stream.synchronize()
        g.destroy()


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--seed", type=int, default=2)
    ap.add_argument("--partition-size", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="budget of the CPU-baseline sample (0 disables it)")
    ap.add_argument("--only-step", action="store_true",
                    help="time the headline step only (two pools alternating; no one-pool or two-call comparison, "
                         "no other configurations, no CPU baseline): for profiling")
    ap.add_argument("--no-extra", action="store_true", help="skip the C3/C4/C5 measurements")
    ap.add_argument("--only-prefill", action="store_true",
                    help="time the C3 chunked prefill call only and print its own JSON line: for profiling")
    ap.add_argument("--only-c3", action="store_true",
                    help="time the C3 calls (decode, chunk append, prefill) alone and as one step, print their JSON line")
    ap.add_argument("--only-c5", action="store_true",
                    help="time C5 through pa_paged_decode and pa_paged_decode_prefix and print their JSON line")
    ap.add_argument("--only-layer", action="store_true",
                    help="time only the C2 decode layer with its projections (and print that)")
    ap.add_argument("--only-c4", action="store_true",
                    help="time the C4 step (int8 fused append + decode) only and print its JSON line: for profiling")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="also run 10 plain device-to-device copies of this many MiB through pa_memcpy, the "
                         "reference kernel for scaling hardware byte counters")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this benchmark runs on exactly one GPU: the paged-decode path has "
                                   "no cross-GPU exchange (one-GPU build); run with --gpus 1"}))
        sys.exit(2)

    import torch

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    pa.load_library()
    w = wl.make_c2(seed=args.seed)
    log(f"[bench] C2: {w.num_seqs} seqs, {int(w.context_lens.sum())} context tokens, "
        f"{w.num_blocks} blocks, max ctx {w.max_context_len}")
    inp = make_inputs(w, seed=1234)
    torch.cuda.synchronize()

    dev = pa.Device(0)
    props = dev.props()
    stream = pa.Stream(dev)
    timer = Timer(dev, stream)
    if args.only_prefill:
        w3, _, _, pre, P, L, _ = c3_setup(stream, 3)
        ms = timer(pre, args.steps, max(args.warmup, PREFILL_WARMUP_CALLS), gate=False)
        flops = float(4 * w3.num_q_heads * w3.head_dim * np.sum(P * L + L * (L + 1) / 2))
        print(json.dumps({"mode": "only-prefill", "workload": "C3 chunked prefill", "us": round(ms * 1e3, 3),
                          "tflops": round(flops / (ms * 1e-3) / 1e12, 1), "steps": args.steps}), flush=True)
        copy_calibration(args, stream)
        return
    if args.only_c4:
        c4 = run_decode_config(wl.make_c4(), timer, stream, args.steps, args.warmup, True, 4)
        print(json.dumps({"mode": "only-c4", "workload": "C4 int8 fused append + decode", **c4,
                          "steps": args.steps}), flush=True)
        copy_calibration(args, stream)
        return
    if args.only_c3:
        c3 = run_c3(timer, stream, args.steps, args.warmup, 3)
        print(json.dumps({"mode": "only-c3", "workload": "C3 mixed step", **c3, "steps": args.steps}), flush=True)
        return
    if args.only_c5:
        w5 = wl.make_c5()
        plain = run_decode_config(w5, timer, stream, args.steps, args.warmup, False, 5)
        split16 = run_decode_config(w5, timer, stream, args.steps, args.warmup, False, 5, num_splits=16)
        shared = run_prefix_decode(w5, timer, stream, args.steps, args.warmup, 5)
        print(json.dumps({"mode": "only-c5", "workload": "C5 decode", "pa_paged_decode": plain,
                          "pa_paged_decode_split16": split16, "pa_paged_decode_prefix": shared,
                          "steps": args.steps}), flush=True)
        copy_calibration(args, stream)
        return
    if args.only_layer:
        lay = run_layer(timer, stream, w, inp, args.steps, args.warmup, 5)
        print(json.dumps({"mode": "only-layer", "workload": "C2 decode layer with projections", **lay,
                          "steps": args.steps}), flush=True)
        return
    cfg = config_of(w, args.partition_size)
    S = w.num_seqs
    out, ws, wsb = decode_buffers(w, cfg)
    step = decode_step(w, inp, stream, cfg, True, out, ws, wsb)

    def two_call_step():
        pa.kv_append(stream, cfg, inp["k_new"], inp["v_new"], inp["slots"], S, inp["k_cache"], inp["v_cache"])
        pa.paged_decode(stream, cfg, out, inp["q"], inp["k_cache"], inp["v_cache"], None, None,
                        inp["tables"], inp["lens"], S, w.max_blocks, w.max_context_len, ws, wsb)

    two_call_ms = float("nan")
    graph_ms = float("nan")
    one_pool = None
    extra = None
    # The variants of the C2 step run before the headline, so that the headline is timed on a GPU
    # that has been working, at the clocks a serving loop runs at: the first measurement of a fresh
    # process reads about 1 us per step more than the ones after it (56.0 against 54.8-55.4 us for
    # the same 20-step measurement repeated in one process).
    if not args.only_step:
        graph_ms = time_graph_replay(step, timer, stream, args.steps)
        log(f"[bench] C2 fused step replayed from a captured graph of {GRAPH_CALLS} steps (one pool) "
            f"{graph_ms * 1e3:.2f} us per step")
        one_ms = timer(step, args.steps, args.warmup)
        one_gbps = (w.decode_algorithmic_bytes() + append_bytes(w)) / (one_ms * 1e-3) / 1e9
        one_pool = {"us_per_layer_step": round(one_ms * 1e3, 3), "gbps": round(one_gbps, 1),
                    "frac_hbm": round(one_gbps / PEAK_HBM_GBPS, 4),
                    "step": "pa_paged_decode_append repeated over one pool (part of K/V still in the 256 MB "
                            "last-level cache from the step before)"}
        pos = w.context_lens.astype(np.int64) - 1
        inp["slots"] = tensor(w.block_tables[np.arange(S), pos // 16].astype(np.int64) * 16 + pos % 16)
        two_call_ms = timer(two_call_step, args.steps, args.warmup)
        log(f"[bench] C2 fused step over one pool {one_ms * 1e3:.2f} us, two-call step (one pool) "
            f"{two_call_ms * 1e3:.2f} us")
    step_ms, two_pool = run_two_pool(w, inp, timer, stream, cfg, args.steps, args.warmup)
    log(f"[bench] C2 fused step alternating two cache pools {step_ms * 1e3:.2f} us (without the launch gate "
        f"{two_pool['ungated_us_per_layer_step']:.2f} us; gate {two_pool['gate']})")
    if not args.only_step:
        if not args.no_extra:
            extra = {}
            n = max(20, args.steps // 2)
            # The long decode steps (C4, C5) run their timed calls after DECODE_WARMUP_CALLS untimed
            # ones: over the first hundred calls of a process the C4 decode kernel's time swings
            # between 113 and 131 us (kernel trace), and a serving loop runs at the steady rate.
            nw = max(args.warmup, DECODE_WARMUP_CALLS)
            extra["C4"] = run_decode_config(wl.make_c4(), timer, stream, n, nw, True, 4)
            log(f"[bench] C4 {extra['C4']['us_per_layer_step']} us")
            w5 = wl.make_c5()
            c5 = run_decode_config(w5, timer, stream, n, nw, False, 5)
            logical = float(w5.context_lens.sum()) * w5.kv_bytes_per_token()
            c5["logical_kv_bytes"] = int(logical)
            c5["logical_gbps"] = round(logical / (c5["us_per_layer_step"] * 1e-6) / 1e9, 1)
            extra["C5"] = c5
            log(f"[bench] C5 {c5['us_per_layer_step']} us")
            # the configuration's stated split: 16 partitions per sequence, merged with log-sum-exp
            extra["C5_split16"] = run_decode_config(w5, timer, stream, n, nw, False, 5, num_splits=16)
            log(f"[bench] C5 with 16 partitions per sequence {extra['C5_split16']['us_per_layer_step']} us")
            extra["C5_prefix"] = run_prefix_decode(w5, timer, stream, n, nw, 5)
            log(f"[bench] C5 shared-prefix decode {extra['C5_prefix']['us_per_layer_step']} us")
            extra["C3"] = run_c3(timer, stream, n, args.warmup, 3)
            log(f"[bench] C3 {extra['C3']['us_per_layer_step']} us")
            extra["block_moves"] = run_block_moves(timer, stream, n, args.warmup, 4)
            log(f"[bench] block moves {extra['block_moves']}")
            extra["C2_layer"] = run_layer(timer, stream, w, inp, n, args.warmup, 5)
            log(f"[bench] C2 layer with projections {extra['C2_layer']}")
            torch.cuda.empty_cache()
    torch.cuda.synchronize()
    copy_calibration(args, stream)

    dec_bytes = w.decode_algorithmic_bytes()
    step_bytes = dec_bytes + append_bytes(w)
    value = step_bytes / (step_ms * 1e-3) / 1e9
    traffic, traffic_src = load_traffic()

    cpu = None
    if args.cpu_seconds > 0 and not args.only_step:
        log("[bench] CPU baseline ...")
        cpu = cpu_baseline(w, inp, args.cpu_seconds)

    res = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "C2: Llama-3-8B-shaped single-layer paged decode (append + attention), bf16 KV, "
                        "fp32 accumulate; steps alternate two cache pools (cold HBM)",
            "num_seqs": S, "num_q_heads": w.num_q_heads, "num_kv_heads": w.num_kv_heads,
            "head_dim": w.head_dim, "block_size": 16, "context_lens": "log-uniform [128, 4096]",
            "context_tokens": int(w.context_lens.sum()), "num_blocks": w.num_blocks,
            "partition_size": args.partition_size or "library default", "parallelism": "single GPU",
        },
        "pct_peak_hbm": round(100.0 * value / PEAK_HBM_GBPS, 2),
        "tokens_per_s_per_layer": round(S / (step_ms * 1e-3), 1),
        "us_per_layer_step": round(step_ms * 1e3, 3),
        "roofline": {
            "kernel": "pa_paged_decode_append call: paged_decode_mfma_persistent_kernel<128, bf16, bf16 q, "
                      "append> + paged_decode_merge_split_kernel<128>",
            "bound": "hbm",
            "achieved": round(value, 2),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(value / PEAK_HBM_GBPS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "algorithmic_bytes_per_launch": int(step_bytes),
            "us_per_launch": round(step_ms * 1e3, 3),
        },
        "two_call_us_per_layer_step": None if two_call_ms != two_call_ms else round(two_call_ms * 1e3, 3),
        "graph_replay_us_per_layer_step": None if graph_ms != graph_ms else round(graph_ms * 1e3, 3),
        "graph_layer_steps_per_replay": GRAPH_CALLS,
        "two_pool": two_pool,
        "one_pool": one_pool,
        "extra": extra,
        "cpu_baseline": cpu,
        "device": {"name": props.name.decode(), "arch": props.arch.decode(), "cus": props.compute_units},
    }
    stream.destroy()
    dev.close()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
