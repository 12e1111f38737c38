#!/usr/bin/env python3
"""Paged-decode benchmark on one MI355X (the BASELINE.json metric).

Step = one decode layer-step of the C2 configuration (Llama-3-8B layer shape: Hq=32, Hkv=8,
D=128, bf16 KV, block 16, batch 64, contexts log-uniform in [128, 4096], shuffled physical
blocks): append the new token's K/V of every sequence into the paged cache and attend over each
sequence's whole context, as one pa_paged_decode_append call (the fused kernel plus the split-K
merge). Inputs are resident in HBM before timing starts; all launches go through the C-ABI of
libpa_hip.so on one pa_stream and are timed with pa_events on that stream.

Output: one JSON line. `value` is the achieved algorithmic HBM bandwidth of the whole step
(distinct KV bytes read + Q + O + block tables + the appended K/V, divided by the step time);
tokens/s per layer and us per layer-step ride along. `roofline` covers the same call; the
two-call path (pa_kv_append + pa_paged_decode) is timed beside it for reference.
`cpu_baseline` times the CPU oracle (a C restatement of the reference's StandardPagedAttentionKernel
with its per-sequence decode loop) on a bounded sample of the same batch, on this host.
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


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def bf16_trunc_torch(x):
    import torch

    return (x.contiguous().view(torch.int32) >> 16).to(torch.int16)


def make_inputs(w: wl.Workload, seed: int):
    """Caches, q, new-token K/V and index arrays on the GPU (torch tensors as device memory)."""
    import torch

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    S, Hq, Hkv, D, nb = w.num_seqs, w.num_q_heads, w.num_kv_heads, w.head_dim, w.num_blocks
    vs = w.value_scale

    def randn(*shape):
        return torch.randn(*shape, generator=g, device=dev, dtype=torch.float32) * vs

    assert w.kv_dtype == pa.PA_DTYPE_BF16 and w.q_dtype == pa.PA_DTYPE_BF16
    k_cache = bf16_trunc_torch(randn(nb, Hkv, 16, D))
    v_cache = bf16_trunc_torch(randn(nb, Hkv, 16, D))
    q = bf16_trunc_torch(randn(S, Hq, D))
    k_new = bf16_trunc_torch(randn(S, Hkv, D))
    v_new = bf16_trunc_torch(randn(S, Hkv, D))
    # The new token of sequence s sits at position context_len - 1.
    pos = w.context_lens.astype(np.int64) - 1
    slots = w.block_tables[np.arange(S), pos // 16].astype(np.int64) * 16 + pos % 16
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    return dict(k_cache=k_cache, v_cache=v_cache, q=q, k_new=k_new, v_new=v_new,
                slots=t(slots), tables=t(w.block_tables), lens=t(w.context_lens))


def cpu_baseline(w: wl.Workload, inp, budget_s: float):
    """Times the CPU oracle (1 thread) on the first n sequences of the batch, n grown until the
    sample costs about `budget_s` seconds, and scales to the whole batch by context tokens."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pa_oracle as orc  # test infrastructure: the timed CPU baseline only

    cfg = pa.make_config(num_q_heads=w.num_q_heads, num_kv_heads=w.num_kv_heads, head_dim=w.head_dim,
                         kv_dtype=w.kv_dtype, q_dtype=w.q_dtype, num_blocks=w.num_blocks)
    kc = inp["k_cache"].cpu().numpy().view(np.uint16)
    vc = inp["v_cache"].cpu().numpy().view(np.uint16)
    q = inp["q"].cpu().numpy().view(np.uint16)
    order = np.arange(w.num_seqs)
    n, spent, toks = 0, 0.0, 0
    t_start = time.perf_counter()
    while n < w.num_seqs and spent < budget_s:
        s = order[n]
        t0 = time.perf_counter()
        orc.paged_decode(cfg, np.ascontiguousarray(q[s:s + 1]), kc, vc, None, None,
                         w.block_tables[s:s + 1], w.context_lens[s:s + 1], n_threads=1)
        spent += time.perf_counter() - t0
        toks += int(w.context_lens[s])
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
                    help="time the fused step only (no two-call comparison, no CPU baseline): for profiling")
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
    cfg = pa.make_config(num_q_heads=w.num_q_heads, num_kv_heads=w.num_kv_heads, head_dim=w.head_dim,
                         kv_dtype=w.kv_dtype, q_dtype=w.q_dtype, num_blocks=w.num_blocks,
                         partition_size=args.partition_size)
    S, mcl = w.num_seqs, w.max_context_len
    out = torch.empty((S, w.num_q_heads, w.head_dim), dtype=torch.float32, device="cuda:0")
    wsb = pa.decode_workspace_size(cfg, S, mcl)
    ws = torch.zeros((max(wsb, 1),), dtype=torch.uint8, device="cuda:0")  # zero-filled once
    torch.cuda.synchronize()

    def step():
        pa.paged_decode_append(stream, cfg, out, inp["q"], inp["k_new"], inp["v_new"], inp["k_cache"],
                               inp["v_cache"], None, None, None, None, inp["tables"], inp["lens"], S,
                               w.max_blocks, mcl, ws, wsb)

    def two_call_step():
        pa.kv_append(stream, cfg, inp["k_new"], inp["v_new"], inp["slots"], S, inp["k_cache"], inp["v_cache"])
        pa.paged_decode(stream, cfg, out, inp["q"], inp["k_cache"], inp["v_cache"], None, None,
                        inp["tables"], inp["lens"], S, w.max_blocks, mcl, ws, wsb)

    def timed(fn, n):
        e0, e1 = pa.Event(dev), pa.Event(dev)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        e1.synchronize()
        ms = e0.elapsed_ms(e1) / n
        e0.destroy()
        e1.destroy()
        return ms

    for _ in range(args.warmup):
        step()
    stream.synchronize()
    step_ms = timed(step, args.steps)
    two_call_ms = float("nan")
    if not args.only_step:
        for _ in range(args.warmup):
            two_call_step()
        two_call_ms = timed(two_call_step, args.steps)
    torch.cuda.synchronize()
    if args.copy_calibration_mb > 0:
        nbytes = args.copy_calibration_mb << 20
        src = torch.empty(nbytes, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty(nbytes, dtype=torch.uint8, device="cuda:0")
        for _ in range(10):
            pa.call("pa_memcpy", dst.data_ptr(), src.data_ptr(), nbytes, pa.PA_MEMCPY_DEVICE_TO_DEVICE, stream.handle)
        stream.synchronize()
        log(f"[bench] copy calibration: 10 x {nbytes} bytes device-to-device")
    log(f"[bench] fused step {step_ms * 1e3:.2f} us, two-call step {two_call_ms * 1e3:.2f} us")

    dec_bytes = w.decode_algorithmic_bytes()
    # the appended token: new K/V read (bf16) + written into the cache
    app_bytes = 2 * S * w.num_kv_heads * w.head_dim * 2 * 2
    step_bytes = dec_bytes + app_bytes
    value = step_bytes / (step_ms * 1e-3) / 1e9
    achieved = value

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
                        "fp32 accumulate",
            "num_seqs": S, "num_q_heads": w.num_q_heads, "num_kv_heads": w.num_kv_heads,
            "head_dim": w.head_dim, "block_size": 16, "context_lens": "log-uniform [128, 4096]",
            "context_tokens": int(w.context_lens.sum()), "num_blocks": w.num_blocks,
            "partition_size": args.partition_size or "library default", "parallelism": "single GPU",
        },
        "pct_peak_hbm": round(100.0 * value / PEAK_HBM_GBPS, 2),
        "tokens_per_s_per_layer": round(S / (step_ms * 1e-3), 1),
        "us_per_layer_step": round(step_ms * 1e3, 3),
        "roofline": {
            "kernel": "pa_paged_decode_append (fused append + paged decode kernel, then split-K merge)",
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBPS, 4),
            "traffic": None,
            "algorithmic_bytes_per_launch": int(step_bytes),
            "us_per_launch": round(step_ms * 1e3, 3),
        },
        "two_call_us_per_layer_step": None if two_call_ms != two_call_ms else round(two_call_ms * 1e3, 3),
        "cpu_baseline": cpu,
        "device": {"name": props.name.decode(), "arch": props.arch.decode(), "cus": props.compute_units},
    }
    stream.destroy()
    dev.close()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
