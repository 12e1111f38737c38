"""The C-ABI of libpa_hip.so on a machine without a GPU: the library loads, exports every function
include/paged_attn.h declares, and its host-side validation returns the documented status codes
before anything is launched (no call here reaches a kernel launch)."""
import ctypes
import os
import re

import pytest

import paged_attention as pa

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "paged_attn.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:pa_status|const char\*)\s+(pa_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_function():
    lib = pa.load_library()
    names = declared_functions()
    assert len(names) >= 30
    for n in names:
        assert hasattr(lib, n), f"{n} declared in paged_attn.h but not exported"
    assert sorted(pa.EXPORTS) == names, "binding's export list differs from the header"


def test_version_and_status_strings():
    lib = pa.load_library()
    major, minor = ctypes.c_int32(), ctypes.c_int32()
    assert lib.pa_get_version(ctypes.byref(major), ctypes.byref(minor)) == 0
    assert (major.value, minor.value) == (1, 1)
    for code, name in [(0, b"PA_SUCCESS"), (1, b"PA_ERROR_INVALID_ARGUMENT"), (2, b"PA_ERROR_INVALID_CONFIG"),
                       (3, b"PA_ERROR_OUT_OF_MEMORY"), (4, b"PA_ERROR_HIP"), (5, b"PA_ERROR_UNSUPPORTED"),
                       (6, b"PA_ERROR_WORKSPACE_TOO_SMALL"), (7, b"PA_ERROR_NO_DEVICE")]:
        assert lib.pa_status_string(code) == name
    assert lib.pa_status_string(99) == b"PA_ERROR_UNKNOWN"


def cfg(**kw):
    base = dict(num_q_heads=32, num_kv_heads=8, head_dim=128, kv_dtype=pa.PA_DTYPE_BF16,
                q_dtype=pa.PA_DTYPE_BF16, num_blocks=100)
    base.update(kw)
    return pa.make_config(**base)


FAKE = 0x1000  # never dereferenced: every call below fails validation first


@pytest.mark.parametrize("c,status,msg", [
    (cfg(block_size=32), pa.PA_ERROR_UNSUPPORTED, "block_size"),
    (cfg(num_q_heads=12), pa.PA_ERROR_INVALID_CONFIG, "multiple"),
    (cfg(head_dim=96), pa.PA_ERROR_UNSUPPORTED, "head_dim"),
    (cfg(kv_dtype=7), pa.PA_ERROR_UNSUPPORTED, "kv_dtype"),
    (cfg(q_dtype=pa.PA_DTYPE_INT8), pa.PA_ERROR_UNSUPPORTED, "q_dtype"),
    (cfg(num_blocks=-1), pa.PA_ERROR_INVALID_CONFIG, "num_blocks"),
    (cfg(scale=float("nan")), pa.PA_ERROR_INVALID_CONFIG, "scale"),
])
def test_config_validation(c, status, msg):
    with pytest.raises(pa.PagedAttentionError) as e:
        pa.paged_decode(None, c, FAKE, FAKE, FAKE, FAKE, None, None, FAKE, FAKE, 4, 10, 100)
    assert e.value.status == status and msg in str(e.value)


def test_argument_validation():
    c = cfg()
    with pytest.raises(pa.PagedAttentionError) as e:
        pa.call("pa_paged_decode", None, None, FAKE, FAKE, FAKE, FAKE, None, None, FAKE, FAKE, 1, 1, 1, None, 0)
    assert e.value.status == pa.PA_ERROR_INVALID_ARGUMENT
    with pytest.raises(pa.PagedAttentionError) as e:
        pa.paged_decode(None, c, None, FAKE, FAKE, FAKE, None, None, FAKE, FAKE, 4, 10, 100)
    assert e.value.status == pa.PA_ERROR_INVALID_ARGUMENT
    with pytest.raises(pa.PagedAttentionError) as e:
        pa.paged_decode(None, c, FAKE, FAKE, FAKE, FAKE, None, None, FAKE, FAKE, -1, 10, 100)
    assert e.value.status == pa.PA_ERROR_INVALID_ARGUMENT
    with pytest.raises(pa.PagedAttentionError) as e:  # int8 without scales
        pa.paged_decode(None, cfg(kv_dtype=2), FAKE, FAKE, FAKE, FAKE, None, None, FAKE, FAKE, 4, 10, 100)
    assert e.value.status == pa.PA_ERROR_INVALID_ARGUMENT
    with pytest.raises(pa.PagedAttentionError) as e:  # Hq / Hkv = 3
        pa.paged_decode(None, cfg(num_q_heads=24), FAKE, FAKE, FAKE, FAKE, None, None, FAKE, FAKE, 4, 10, 100)
    assert e.value.status == pa.PA_ERROR_UNSUPPORTED
    with pytest.raises(pa.PagedAttentionError) as e:  # long contexts need a workspace
        pa.paged_decode(None, c, FAKE, FAKE, FAKE, FAKE, None, None, FAKE, FAKE, 4, 300, 4096, None, 0)
    assert e.value.status == pa.PA_ERROR_WORKSPACE_TOO_SMALL
    with pytest.raises(pa.PagedAttentionError) as e:
        pa.paged_decode_append(None, c, FAKE, FAKE, None, FAKE, FAKE, FAKE, None, None, None, None, FAKE, FAKE,
                               4, 10, 100)
    assert e.value.status == pa.PA_ERROR_INVALID_ARGUMENT
    with pytest.raises(pa.PagedAttentionError) as e:  # int8 append without running absmax
        pa.paged_decode_append(None, cfg(kv_dtype=2), FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, None,
                               FAKE, FAKE, 4, 10, 100)
    assert e.value.status == pa.PA_ERROR_INVALID_ARGUMENT
    with pytest.raises(pa.PagedAttentionError) as e:
        pa.kv_append(None, c, FAKE, FAKE, FAKE, -3, FAKE, FAKE)
    assert e.value.status == pa.PA_ERROR_INVALID_ARGUMENT
    with pytest.raises(pa.PagedAttentionError) as e:
        pa.kv_append(None, cfg(kv_dtype=2), FAKE, FAKE, FAKE, 5, FAKE, FAKE)
    assert e.value.status == pa.PA_ERROR_INVALID_ARGUMENT
    with pytest.raises(pa.PagedAttentionError) as e:
        pa.build_slot_mapping(None, cfg(block_size=8), FAKE, 4, FAKE, FAKE, FAKE, 2, 3, FAKE)
    assert e.value.status == pa.PA_ERROR_UNSUPPORTED
    # empty batches are no-ops that succeed without touching any pointer
    pa.paged_decode(None, c, None, None, None, None, None, None, None, None, 0, 0, 0)
    pa.kv_append(None, c, None, None, None, 0, None, None)


@pytest.mark.parametrize("c,args,status,msg", [
    (cfg(), (-1, 4, 16), pa.PA_ERROR_INVALID_ARGUMENT, "negative"),
    (cfg(), (70000, 4, 16), pa.PA_ERROR_UNSUPPORTED, "65535"),
    (cfg(), (2, 0, 16), pa.PA_ERROR_INVALID_ARGUMENT, "block"),
    (cfg(flags=pa.PA_FLAG_REFERENCE_LITERAL_MASK | pa.PA_FLAG_NO_MASK), (2, 4, 16), pa.PA_ERROR_INVALID_CONFIG,
     "mask"),
    (cfg(head_dim=32), (2, 4, 16), pa.PA_ERROR_UNSUPPORTED, "head_dim"),
    (cfg(kv_dtype=pa.PA_DTYPE_INT8), (2, 4, 16), pa.PA_ERROR_INVALID_ARGUMENT, "k_scale"),
])
def test_prefill_argument_validation(c, args, status, msg):
    with pytest.raises(pa.PagedAttentionError) as e:
        pa.chunked_prefill(None, c, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, None, FAKE, *args)
    assert e.value.status == status and msg in str(e.value)
    with pytest.raises(pa.PagedAttentionError) as e:  # null block table
        pa.chunked_prefill(None, cfg(), FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, None, None, 2, 4, 16)
    assert e.value.status == pa.PA_ERROR_INVALID_ARGUMENT
    # no sequences or no queries: a no-op that touches no pointer
    pa.chunked_prefill(None, cfg(), None, None, None, None, None, None, None, None, None, 0, 4, 16)
    pa.chunked_prefill(None, cfg(), None, None, None, None, None, None, None, None, None, 2, 4, 0)


def test_workspace_size():
    c = cfg()  # Hq 32, Hkv 8, D 128, bf16
    # bf16/int8, default split: 2 partial slots per unit (range, KV head) of (D + 2) floats per query
    # head of the group (G = 4); ranges <= min(4096 workers / Hkv, ceil(blocks / 4)) where blocks
    # counts one KV head; plus num_seqs + 1 ints of sequence offsets.
    # 64 x 4096 tokens = 16384 blocks -> min(512, 4096) = 512 ranges x 8 KV heads
    assert pa.decode_workspace_size(c, 64, 4096) == 2 * 4096 * 4 * 130 * 4 + 65 * 4
    # 1 sequence of 16 tokens: 1 block -> 1 range x 8 KV heads
    assert pa.decode_workspace_size(c, 1, 16) == 2 * 8 * 4 * 130 * 4 + 2 * 4
    # fixed 512-token ranges (32 blocks): 16384 / 32 = 512 ranges x 8 KV heads
    assert pa.decode_workspace_size(cfg(partition_size=512), 64, 4096) == 2 * 4096 * 4 * 130 * 4 + 65 * 4
    # beyond one launch's 2047 sequences the launches reuse the workspace: sized for 2047
    assert pa.decode_workspace_size(c, 5000, 64) == 2 * 4096 * 4 * 130 * 4 + 2048 * 4
    assert pa.decode_workspace_size(c, 0, 4096) == 0
    # fp32: per-partition partials only when some sequence needs more than one partition
    assert pa.decode_workspace_size(cfg(kv_dtype=0), 4, 256) == 0
    assert pa.decode_workspace_size(cfg(kv_dtype=0), 4, 1000) == 4 * 32 * 4 * 130 * 4
    with pytest.raises(pa.PagedAttentionError) as e:
        pa.decode_workspace_size(cfg(partition_size=100), 4, 256)
    assert e.value.status == pa.PA_ERROR_UNSUPPORTED
    with pytest.raises(pa.PagedAttentionError):
        pa.decode_workspace_size(cfg(kv_dtype=0, partition_size=1024), 4, 256)
    # per-sequence split P: P units per (sequence, KV head), 2 slots each
    assert pa.decode_workspace_size(cfg(num_splits=16), 8, 32768) == 2 * 8 * 16 * 8 * 4 * 130 * 4 + 9 * 4
    assert pa.decode_workspace_size(cfg(num_splits=1), 3, 100) == 2 * 3 * 8 * 4 * 130 * 4 + 4 * 4
    for bad in (dict(num_splits=-1), dict(num_splits=257), dict(num_splits=4, partition_size=512),
                dict(num_splits=4, kv_dtype=0)):
        with pytest.raises(pa.PagedAttentionError) as e:
            pa.decode_workspace_size(cfg(**bad), 4, 256)
        assert e.value.status == pa.PA_ERROR_UNSUPPORTED, bad


def test_last_error_is_per_call():
    with pytest.raises(pa.PagedAttentionError):
        pa.paged_decode(None, cfg(head_dim=48), FAKE, FAKE, FAKE, FAKE, None, None, FAKE, FAKE, 4, 10, 100)
    assert "head_dim" in pa.last_error()
    assert pa.decode_workspace_size(cfg(), 1, 16) > 0
    assert pa.last_error() == ""


def test_device_open_without_gpu_reports_no_device():
    n = ctypes.c_int32(-1)
    assert pa.load_library().pa_device_count(ctypes.byref(n)) == 0
    if n.value == 0:
        with pytest.raises(pa.PagedAttentionError) as e:
            pa.Device(0)
        assert e.value.status == pa.PA_ERROR_NO_DEVICE


def test_block_moves_validate_on_the_host():
    c = cfg()  # bf16, Hkv 8, D 128
    assert pa.block_bytes(c) == 2 * 8 * 16 * 128 * 2
    assert pa.block_bytes(cfg(kv_dtype=2)) == 2 * 8 * 16 * 128 + 4 * 8 * 4
    bad = [
        lambda: pa.read_block_f32(None, c, 4096, 4096, None, None, c.num_blocks, 4, 4096, 4096),  # block
        lambda: pa.read_block_f32(None, c, 4096, 4096, None, None, 0, 17, 4096, 4096),            # tokens
        lambda: pa.write_block_f32(None, c, 4096, 4096, None, None, None, None, -1, 4, 4096, 4096),
        lambda: pa.copy_blocks(None, c, 4100, 4096, None, None, None, None, 4096, 1),              # alignment
        lambda: pa.copy_blocks(None, c, 4096, 4096, None, None, None, None, None, 1),              # pairs
        lambda: pa.gather_blocks(None, c, 4096, 4096, None, None, None, None, 4096, 1, 4104),       # packed
        lambda: pa.scatter_blocks(None, cfg(kv_dtype=2), 4096, 4096, None, None, None, None, 4096, 1, 4096),
    ]
    for f in bad:
        with pytest.raises(pa.PagedAttentionError) as e:
            f()
        assert e.value.status == pa.PA_ERROR_INVALID_ARGUMENT
    # empty calls are no-ops that succeed without touching memory
    pa.copy_blocks(None, c, 4096, 4096, None, None, None, None, None, 0)
    pa.gather_blocks(None, c, 4096, 4096, None, None, None, None, None, 0, None)
    pa.read_block_f32(None, c, 4096, 4096, None, None, 0, 0, None, None)
