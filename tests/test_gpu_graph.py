"""Graph capture and replay of the decode layer-step through the C-ABI (pa_graph_*).

Mirrors the reference CUDA HAL's capture / replay (HAL/CUDA/Graphs/CUDAGraphCapture.cs:24-61,
CUDAGraph.cs:33-119): one fused append + decode call is captured on a stream, then replayed
several times with new inputs written between the replays (eager work and synchronisations in
between). Every replay must equal an eager call on the same inputs bit for bit (outputs and the
appended cache bytes) and the oracle within the tolerance of the cache type.
"""
import numpy as np
import pytest

import paged_attention as pa
import pa_oracle as orc
import workloads as wl
from helpers import build_int8_caches, check_close, config_for, empty_gpu, to_gpu, to_np, tol_for

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kv_dtype,q_dtype", [(1, 1), (2, 0)])
def test_graph_replays_decode_append(kv_dtype, q_dtype):
    import torch

    torch.cuda.init()
    dev = pa.Device(0)
    gs = pa.Stream(dev)  # a library stream: the null stream cannot capture
    try:
        lens = [100, 1, 17, 300, 1025, 64]
        w = wl.make_small(31 + kv_dtype, num_seqs=len(lens), lens=lens, Hq=32, Hkv=8, D=128,
                          kv_dtype=kv_dtype, q_dtype=q_dtype)
        inp = wl.numpy_inputs(w, 5)
        cfg = config_for(w)
        S, Hq, Hkv, D = w.num_seqs, w.num_q_heads, w.num_kv_heads, w.head_dim
        mcl = w.max_context_len
        rng = np.random.default_rng(3)

        def act(*shape):
            x = rng.standard_normal(shape, dtype=np.float32) * 0.5
            return orc.bf16_from_f32(x) if q_dtype == 1 else x

        if kv_dtype == 2:
            # the int8 pool is quantised by one full-pool append (checked against the oracle)
            host, g8 = build_int8_caches(w, inp, gs)
            caches = dict(kc=host["k_cache"], vc=host["v_cache"], ks=host["k_scale"], vs=host["v_scale"],
                          ka=to_np(g8["ka"]).copy(), va=to_np(g8["va"]).copy())
        else:
            caches = dict(kc=inp["k_cache"], vc=inp["v_cache"])
        dev_c = {n: to_gpu(a) for n, a in caches.items()}
        q, k_new, v_new = to_gpu(act(S, Hq, D)), to_gpu(act(S, Hkv, D)), to_gpu(act(S, Hkv, D))
        out = empty_gpu((S, Hq, D), np.float32)
        wsb = pa.decode_workspace_size(cfg, S, mcl)
        ws = empty_gpu((max(wsb, 1),), np.uint8)
        tables, ctx = to_gpu(w.block_tables), to_gpu(w.context_lens)
        args = (q, k_new, v_new, dev_c["kc"], dev_c["vc"], dev_c.get("ks"), dev_c.get("vs"), dev_c.get("ka"),
                dev_c.get("va"), tables, ctx, S, w.max_blocks, mcl, ws, wsb)

        def restore():
            for n, a in caches.items():
                dev_c[n].copy_(to_gpu(a))
            out.fill_(float("nan"))
            torch.cuda.synchronize()

        def snapshot():
            cdt = {1: np.uint16, 2: np.int8}[kv_dtype]
            return (to_np(out).copy(), to_np(dev_c["kc"], cdt).copy(), to_np(dev_c["vc"], cdt).copy())

        torch.cuda.synchronize()
        g = pa.Graph().capture(gs)
        with pytest.raises(pa.PagedAttentionError, match="capturing"):
            pa.call("pa_memset", ws.data_ptr(), 0, 64, gs.handle)  # refused before anything is recorded
        pa.paged_decode_append(gs, cfg, out, *args)
        g.end()
        try:
            assert g.node_count() >= 1
            for r in range(3):
                qv, kv_, vv = act(S, Hq, D), act(S, Hkv, D), act(S, Hkv, D)
                q.copy_(to_gpu(qv))
                k_new.copy_(to_gpu(kv_))
                v_new.copy_(to_gpu(vv))
                restore()
                g.launch(gs)
                gs.synchronize()
                replay = snapshot()
                restore()
                pa.paged_decode_append(gs, cfg, out, *args)
                gs.synchronize()
                eager = snapshot()
                for a, b in zip(replay, eager):
                    np.testing.assert_array_equal(a, b)
                # and the right values: append on the host, then the oracle's decode
                hk, hv = caches["kc"].copy(), caches["vc"].copy()
                pos = w.context_lens.astype(np.int64) - 1
                slots = w.block_tables[np.arange(S), pos // 16].astype(np.int64) * 16 + pos % 16
                if kv_dtype == 2:
                    hks, hvs = caches["ks"].copy(), caches["vs"].copy()
                    hka, hva = caches["ka"].copy(), caches["va"].copy()
                    orc.kv_append(cfg, kv_, vv, slots, hk, hv, hks, hvs, hka, hva)
                    ref = orc.paged_decode(cfg, qv, hk, hv, hks, hvs, w.block_tables, w.context_lens)
                else:
                    orc.kv_append(cfg, kv_, vv, slots, hk, hv)
                    ref = orc.paged_decode(cfg, qv, hk, hv, None, None, w.block_tables, w.context_lens)
                check_close(replay[0], ref, **tol_for(kv_dtype), what=f"graph replay {r}")
        finally:
            g.destroy()
    finally:
        gs.destroy()
        dev.close()


def test_graph_capture_needs_a_stream():
    with pytest.raises(pa.PagedAttentionError):
        pa.call("pa_graph_capture_begin", None)
