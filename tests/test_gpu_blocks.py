"""Whole-block moves on the GPU through the C-ABI: copy-on-write copies, swap gather / scatter and
the fp32 block view, each bit-exact against the oracle (tests/test_oracle_blocks.py pins it)."""
import numpy as np
import pytest

import paged_attention as pa
import pa_oracle as orc
from helpers import empty_gpu, to_gpu, to_np
from test_oracle_blocks import caches

pytestmark = pytest.mark.gpu

SHAPES = [(0, 2, 64), (1, 8, 128), (2, 8, 128), (2, 2, 64), (1, 4, 256)]


def dev_caches(kv_dtype, hkv, d, seed, nb=40):
    cfg, k, v, stats = caches(kv_dtype, nb=nb, hkv=hkv, d=d, seed=seed)
    g = dict(k=to_gpu(k), v=to_gpu(v))
    gs = tuple(to_gpu(s) for s in stats) if stats else (None, None, None, None)
    return cfg, k, v, stats, g, gs


def np_dtype(kv_dtype):
    return {0: np.float32, 1: np.uint16, 2: np.int8}[kv_dtype]


def check_caches(kv_dtype, g, gs, k, v, stats, what):
    dt = np_dtype(kv_dtype)
    np.testing.assert_array_equal(to_np(g["k"], dt), k, err_msg=f"{what}: K")
    np.testing.assert_array_equal(to_np(g["v"], dt), v, err_msg=f"{what}: V")
    if stats:
        for name, a, b in zip(("k_scale", "v_scale", "k_absmax", "v_absmax"), gs, stats):
            np.testing.assert_array_equal(to_np(a), b, err_msg=f"{what}: {name}")


@pytest.mark.parametrize("kv_dtype,hkv,d", SHAPES)
def test_copy_blocks_bit_exact(kv_dtype, hkv, d):
    import torch

    cfg, k, v, stats, g, gs = dev_caches(kv_dtype, hkv, d, seed=10)
    rng = np.random.default_rng(11)
    perm = rng.permutation(cfg.num_blocks)
    pairs = np.stack([perm[:12], perm[12:24]], 1).astype(np.int32)  # disjoint sources and targets
    pairs[3] = (pairs[3][0], pairs[3][0])                            # self pair: no-op
    pairs[5] = (-1, pairs[5][1])                                     # invalid source: skipped
    pairs[7] = (pairs[7][0], cfg.num_blocks)                         # invalid target: skipped
    print(f"copy_blocks kv_dtype={kv_dtype} hkv={hkv} d={d} pairs={len(pairs)}", flush=True)
    pa.copy_blocks(None, cfg, g["k"], g["v"], *gs, to_gpu(pairs), len(pairs))
    torch.cuda.synchronize()
    orc.copy_blocks(cfg, k, v, stats, pairs)
    check_caches(kv_dtype, g, gs, k, v, stats, "copy_blocks")


@pytest.mark.parametrize("kv_dtype,hkv,d", SHAPES)
def test_swap_out_and_in_bit_exact(kv_dtype, hkv, d):
    import torch

    cfg, k, v, stats, g, gs = dev_caches(kv_dtype, hkv, d, seed=12)
    rec = pa.block_bytes(cfg)
    assert rec == orc.block_record_bytes(cfg)
    ids = np.array([3, 17, -1, 39, 0, 22], np.int32)
    print(f"gather/scatter kv_dtype={kv_dtype} hkv={hkv} d={d} record={rec}", flush=True)
    packed = empty_gpu((len(ids), rec), np.uint8)
    packed.fill_(0xAB)
    pa.gather_blocks(None, cfg, g["k"], g["v"], *gs, to_gpu(ids), len(ids), packed)
    torch.cuda.synchronize()
    ref = np.full((len(ids), rec), 0xAB, np.uint8)
    orc.gather_blocks(cfg, k, v, stats, ids, ref)
    np.testing.assert_array_equal(to_np(packed), ref)
    # swap the records back in elsewhere (a host round trip through pa_memcpy on the way)
    host = np.empty_like(ref)
    pa.call("pa_memcpy", host.ctypes.data, packed.data_ptr(), host.nbytes, pa.PA_MEMCPY_DEVICE_TO_HOST, None)
    np.testing.assert_array_equal(host, ref)
    back = to_gpu(host)
    cfg2, k2, v2, stats2, g2, gs2 = dev_caches(kv_dtype, hkv, d, seed=13)
    dst = np.array([30, 1, 5, 11, 12, 38], np.int32)
    dst[2] = -1
    pa.scatter_blocks(None, cfg2, g2["k"], g2["v"], *gs2, to_gpu(dst), len(dst), back)
    torch.cuda.synchronize()
    orc.scatter_blocks(cfg2, k2, v2, stats2, dst, host)
    check_caches(kv_dtype, g2, gs2, k2, v2, stats2, "scatter_blocks")


@pytest.mark.parametrize("kv_dtype,hkv,d", SHAPES)
@pytest.mark.parametrize("tokens", [1, 9, 16])
def test_read_block_f32_exact(kv_dtype, hkv, d, tokens):
    import torch

    cfg, k, v, stats, g, gs = dev_caches(kv_dtype, hkv, d, seed=14)
    ko = empty_gpu((tokens, hkv, d), np.float32)
    vo = empty_gpu((tokens, hkv, d), np.float32)
    pa.read_block_f32(None, cfg, g["k"], g["v"], gs[0], gs[1], 21, tokens, ko, vo)
    torch.cuda.synchronize()
    rk, rv = orc.read_block_f32(cfg, k, v, stats[0] if stats else None, stats[1] if stats else None, 21, tokens)
    np.testing.assert_array_equal(to_np(ko), rk)
    np.testing.assert_array_equal(to_np(vo), rv)


@pytest.mark.parametrize("kv_dtype,hkv,d", SHAPES)
@pytest.mark.parametrize("tokens", [1, 7, 16])
def test_write_block_f32_is_append(kv_dtype, hkv, d, tokens):
    import torch

    cfg, k, v, stats, g, gs = dev_caches(kv_dtype, hkv, d, seed=15)
    rng = np.random.default_rng(16)
    x = (rng.standard_normal((tokens, hkv, d), dtype=np.float32) * 3).astype(np.float32)
    y = (rng.standard_normal((tokens, hkv, d), dtype=np.float32) * 3).astype(np.float32)
    pa.write_block_f32(None, cfg, g["k"], g["v"], *gs, 6, tokens, to_gpu(x), to_gpu(y))
    torch.cuda.synchronize()
    st = stats if stats else (None, None, None, None)
    orc.kv_append(cfg, x, y, 6 * 16 + np.arange(tokens), k, v, *st)
    check_caches(kv_dtype, g, gs, k, v, stats, "write_block_f32")
