"""GPU results against the committed golden fixtures (same seeded inputs as the oracle used)."""
import os
import sys

import numpy as np
import pytest

import paged_attention as pa
from helpers import check_close, empty_gpu, to_gpu, to_np, tol_for

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import cases  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def stream():
    import torch

    torch.cuda.init()
    s = pa.TorchStream.current(0)
    yield s.stream
    s.stream.destroy()
    s.device.close()


@pytest.mark.parametrize("name", ["decode_c1", "decode_c2_seq", "decode_c5_mini"])
def test_decode_matches_fixture(stream, name):
    import torch

    stored = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    w, inp, extra = cases.decode_inputs(name)
    cfg = cases.cfg_for(w, **extra)
    S, mcl = w.num_seqs, w.max_context_len
    out = empty_gpu((S, w.num_q_heads, w.head_dim), np.float32)
    wsb = pa.decode_workspace_size(cfg, S, mcl)
    ws = empty_gpu((max(wsb, 1),), np.uint8)
    pa.paged_decode(stream, cfg, out, to_gpu(inp["q"]), to_gpu(inp["k_cache"]), to_gpu(inp["v_cache"]), None,
                    None, to_gpu(w.block_tables), to_gpu(w.context_lens), S, w.max_blocks, mcl, ws, wsb)
    torch.cuda.synchronize()
    check_close(to_np(out), stored["out"], **tol_for(w.kv_dtype), what=name)


def test_int8_append_trace_matches_fixture(stream):
    import torch

    stored = np.load(os.path.join(GOLDEN, "int8_append_trace.npz"))
    nb, H, D, steps = cases.int8_append_inputs()
    cfg = pa.make_config(num_q_heads=H, num_kv_heads=H, head_dim=D, kv_dtype=2, num_blocks=nb)
    kc, vc = empty_gpu((nb, H, 16, D), np.int8), empty_gpu((nb, H, 16, D), np.int8)
    ks, vs, ka, va = (empty_gpu((nb, H), np.float32) for _ in range(4))
    for slots, x in steps:
        y = (-x[:, :, ::-1]).copy()
        pa.kv_append(stream, cfg, to_gpu(x), to_gpu(y), to_gpu(slots), len(slots), kc, vc, ks, vs, ka, va)
    torch.cuda.synchronize()
    for name, t in (("k_codes", kc), ("v_codes", vc), ("k_scale", ks), ("v_scale", vs), ("k_absmax", ka),
                    ("v_absmax", va)):
        np.testing.assert_array_equal(to_np(t), stored[name], err_msg=name)


def test_prefill_matches_fixture(stream):
    import torch

    stored = np.load(os.path.join(GOLDEN, "prefill_chunk.npz"))
    w, inp, q, q_start, prefix = cases.prefill_inputs()
    cfg = cases.cfg_for(w)
    out = empty_gpu(stored["out"].shape, np.float32)
    pa.chunked_prefill(stream, cfg, out, to_gpu(q), to_gpu(q_start), to_gpu(prefix), to_gpu(inp["k_cache"]),
                       to_gpu(inp["v_cache"]), None, None, to_gpu(w.block_tables), len(prefix), w.max_blocks,
                       int(np.diff(q_start).max()))
    torch.cuda.synchronize()
    check_close(to_np(out), stored["out"], **tol_for(w.kv_dtype), what="prefill_chunk")
