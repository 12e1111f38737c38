"""Golden cases: seeded inputs and the oracle outputs stored for them.

Each case builds its inputs deterministically (numpy PCG64) and runs the CPU oracle; the stored
fixture holds the outputs and a digest of the inputs. GPU tests rebuild the same inputs and compare
the library's results to the stored outputs.
"""
import hashlib

import numpy as np

import pa_oracle as orc
import paged_attention as pa
import workloads as wl

CASES = ("quantizer_kat", "decode_c1", "decode_c2_seq", "int8_append_trace", "prefill_chunk", "decode_c5_mini")


def digest(inputs: dict) -> str:
    h = hashlib.sha256()
    for k in sorted(inputs):
        a = np.ascontiguousarray(inputs[k])
        h.update(k.encode())
        h.update(str(a.dtype).encode())
        h.update(str(a.shape).encode())
        h.update(a.tobytes())
    return h.hexdigest()


def cfg_for(w, **kw):
    return pa.make_config(num_q_heads=w.num_q_heads, num_kv_heads=w.num_kv_heads, head_dim=w.head_dim,
                          kv_dtype=w.kv_dtype, q_dtype=w.q_dtype, num_blocks=w.num_blocks, **kw)


def quantizer_kat():
    rng = np.random.default_rng(2024)
    ties = np.array([k + 0.5 for k in range(-130, 130)], np.float32)
    vals = np.concatenate([ties, (rng.standard_normal(2000) * 60).astype(np.float32),
                           np.array([0.49999997, -0.49999997, 1000, -1000, 0, -0.0], np.float32)])
    scales = np.concatenate([np.ones(len(ties), np.float32), rng.uniform(0.05, 2, 2000).astype(np.float32),
                             np.array([1, 1, 0.5, 0.5, 0.5, 0.5], np.float32)])
    codes = np.array([orc.lib().orc_quantize_symmetric(float(v), float(s)) for v, s in zip(vals, scales)], np.int8)
    return {"values": vals, "scales": scales}, {"codes": codes}


def decode_inputs(name):
    if name == "decode_c1":
        w = wl.make_c1()
        return w, wl.numpy_inputs(w, 101), {}
    if name == "decode_c2_seq":
        w = wl.make_small(300, num_seqs=1, lens=[300], Hq=32, Hkv=8, D=128, kv_dtype=1, q_dtype=1,
                          value_scale=0.5)
        return w, wl.numpy_inputs(w, 301), {}
    if name == "decode_c5_mini":
        # two sequences sharing a 64-token prefix (4 blocks in both tables), split into 16 partitions
        w = wl.make_small(500, num_seqs=2, lens=[1000, 1024], Hq=32, Hkv=8, D=128, kv_dtype=1, q_dtype=1,
                          value_scale=0.5)
        w.block_tables[1, :4] = w.block_tables[0, :4]
        return w, wl.numpy_inputs(w, 501), {"partition_size": 64}
    raise KeyError(name)


def decode_case(name):
    w, inp, extra = decode_inputs(name)
    cfg = cfg_for(w)
    out = orc.paged_decode(cfg, inp["q"], inp["k_cache"], inp["v_cache"], None, None, w.block_tables,
                           w.context_lens)
    inputs = {"q": inp["q"], "k": inp["k_cache"], "v": inp["v_cache"], "tables": w.block_tables,
              "lens": w.context_lens}
    return inputs, {"out": out}


def int8_append_inputs():
    rng = np.random.default_rng(77)
    nb, H, D = 6, 2, 64
    steps = []
    fill = [16, 7, 1, 12]
    slots = np.concatenate([b * 16 + np.arange(f) for b, f in enumerate(fill)]).astype(np.int64)
    steps.append((slots, rng.standard_normal((len(slots), H, D)).astype(np.float32)))
    slots = np.array([1 * 16 + 7, 2 * 16 + 1, 3 * 16 + 12, 4 * 16], np.int64)
    x = rng.standard_normal((4, H, D)).astype(np.float32)
    x[0, :, 3] *= 10  # growth in block 1
    steps.append((slots, x))
    slots = np.concatenate([3 * 16 + 13 + np.arange(3), 5 * 16 + np.arange(5)]).astype(np.int64)
    steps.append((slots, (rng.standard_normal((8, H, D)) * 2).astype(np.float32)))
    return nb, H, D, steps


def int8_append_trace():
    nb, H, D, steps = int8_append_inputs()
    cfg = pa.make_config(num_q_heads=H, num_kv_heads=H, head_dim=D, kv_dtype=2, num_blocks=nb)
    kc = np.zeros((nb, H, 16, D), np.int8)
    vc = np.zeros_like(kc)
    ks, vs, ka, va = (np.zeros((nb, H), np.float32) for _ in range(4))
    inputs = {}
    for i, (slots, x) in enumerate(steps):
        y = (-x[:, :, ::-1]).copy()
        orc.kv_append(cfg, x, y, slots, kc, vc, ks, vs, ka, va)
        inputs[f"slots{i}"], inputs[f"x{i}"] = slots, x
    return inputs, {"k_codes": kc, "v_codes": vc, "k_scale": ks, "v_scale": vs, "k_absmax": ka, "v_absmax": va}


def prefill_inputs():
    rng = np.random.default_rng(91)
    prefix, chunk = [0, 37], [33, 33]
    totals = [p + c for p, c in zip(prefix, chunk)]
    w = wl.make_small(92, num_seqs=2, lens=totals, Hq=8, Hkv=2, D=64, kv_dtype=1, q_dtype=1)
    inp = wl.numpy_inputs(w, 93)
    q_start = np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32)
    q = orc.bf16_from_f32(rng.standard_normal((int(q_start[-1]), 8, 64)).astype(np.float32))
    return w, inp, q, q_start, np.array(prefix, np.int32)


def prefill_chunk():
    w, inp, q, q_start, prefix = prefill_inputs()
    cfg = cfg_for(w)
    out = orc.chunked_prefill(cfg, q, q_start, prefix, inp["k_cache"], inp["v_cache"], None, None, w.block_tables)
    inputs = {"q": q, "k": inp["k_cache"], "v": inp["v_cache"], "tables": w.block_tables, "q_start": q_start,
              "prefix": prefix}
    return inputs, {"out": out}


def build(name):
    if name == "quantizer_kat":
        return quantizer_kat()
    if name.startswith("decode_"):
        return decode_case(name)
    if name == "int8_append_trace":
        return int8_append_trace()
    if name == "prefill_chunk":
        return prefill_chunk()
    raise KeyError(name)
