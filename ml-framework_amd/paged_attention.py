"""ctypes binding of libpa_hip.so, the C-ABI declared in include/paged_attn.h.

This is what the reference's P/Invoke layer would bind (CallingConvention.Cdecl entry points, plain
pointers, integer status codes mapped to exceptions -- src/MLFramework/HAL/CUDA/CudaApi.cs:18,
CudaError.cs). Tests and bench.py call the library through it; tensors are torch tensors on the
GPU used only as device memory. There is no fallback: if the shared library is missing or does not
load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libpa_hip.so")

PA_SUCCESS = 0
PA_ERROR_INVALID_ARGUMENT = 1
PA_ERROR_INVALID_CONFIG = 2
PA_ERROR_OUT_OF_MEMORY = 3
PA_ERROR_HIP = 4
PA_ERROR_UNSUPPORTED = 5
PA_ERROR_WORKSPACE_TOO_SMALL = 6
PA_ERROR_NO_DEVICE = 7

PA_DTYPE_FP32 = 0
PA_DTYPE_BF16 = 1
PA_DTYPE_INT8 = 2

PA_PHASE_PREFILL = 0
PA_PHASE_DECODE = 1

PA_FLAG_NONE = 0
PA_FLAG_REFERENCE_LITERAL_MASK = 1
PA_FLAG_NO_MASK = 2

# bytes of the per-device scratch array of pa_paged_decode_noalloc (PA_NOALLOC_SCRATCH_BYTES)
PA_NOALLOC_SCRATCH_BYTES = 32 << 20

PA_MEMCPY_HOST_TO_DEVICE = 1
PA_MEMCPY_DEVICE_TO_HOST = 2
PA_MEMCPY_DEVICE_TO_DEVICE = 3

# Every function the header declares, in declaration order.
EXPORTS = (
    "pa_get_version", "pa_status_string", "pa_get_last_error",
    "pa_device_count", "pa_device_open", "pa_device_close", "pa_device_get_props",
    "pa_device_synchronize",
    "pa_alloc", "pa_free", "pa_memcpy", "pa_memset",
    "pa_stream_create", "pa_stream_wrap", "pa_stream_native", "pa_stream_destroy",
    "pa_stream_synchronize", "pa_stream_wait_event",
    "pa_event_create", "pa_event_destroy", "pa_event_record", "pa_event_query",
    "pa_event_synchronize", "pa_event_elapsed_ms",
    "pa_graph_capture_begin", "pa_graph_capture_end", "pa_graph_launch", "pa_graph_node_count",
    "pa_graph_destroy",
    "pa_build_slot_mapping", "pa_kv_append", "pa_decode_workspace_size", "pa_paged_decode",
    "pa_paged_decode_append", "pa_paged_decode_noalloc", "pa_chunked_prefill",
    "pa_block_bytes", "pa_copy_blocks", "pa_gather_blocks", "pa_scatter_blocks", "pa_read_block_f32",
    "pa_write_block_f32",
    "pa_qkv_workspace_size", "pa_qkv_project_append", "pa_o_workspace_size", "pa_o_project",
    "pa_prefix_plan_bytes", "pa_prefix_plan_build", "pa_prefix_plan_fill", "pa_prefix_workspace_size",
    "pa_paged_decode_prefix",
)


class PaConfig(ctypes.Structure):
    """struct pa_config (include/paged_attn.h)."""

    _fields_ = [
        ("block_size", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("kv_dtype", ctypes.c_int32),
        ("q_dtype", ctypes.c_int32),
        ("num_blocks", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("partition_size", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
        ("num_splits", ctypes.c_int32),
    ]


class PaDeviceProps(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 256),
        ("arch", ctypes.c_char * 64),
        ("total_memory", ctypes.c_size_t),
        ("compute_units", ctypes.c_int32),
        ("ordinal", ctypes.c_int32),
    ]


def make_config(*, num_q_heads, num_kv_heads, head_dim, kv_dtype, q_dtype=PA_DTYPE_FP32,
                num_blocks, block_size=16, scale=-1.0, partition_size=0, flags=0, num_splits=0) -> PaConfig:
    return PaConfig(block_size, num_q_heads, num_kv_heads, head_dim, kv_dtype, q_dtype,
                    num_blocks, scale, partition_size, flags, num_splits)


class PagedAttentionError(RuntimeError):
    """Raised for a non-zero pa_status; carries the status code and the library's message."""

    def __init__(self, status: int, fn: str, message: str):
        self.status = status
        super().__init__(f"{fn} failed with status {status}: {message}")


_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_SZ = ctypes.c_size_t
_CFG = ctypes.POINTER(PaConfig)

_SIGNATURES = {
    "pa_get_version": [ctypes.POINTER(_I32), ctypes.POINTER(_I32)],
    "pa_get_last_error": [ctypes.c_char_p, _SZ],
    "pa_device_count": [ctypes.POINTER(_I32)],
    "pa_device_open": [_I32, ctypes.POINTER(_P)],
    "pa_device_close": [_P],
    "pa_device_get_props": [_P, ctypes.POINTER(PaDeviceProps)],
    "pa_device_synchronize": [_P],
    "pa_alloc": [_P, _SZ, ctypes.POINTER(_P)],
    "pa_free": [_P, _P],
    "pa_memcpy": [_P, _P, _SZ, _I32, _P],
    "pa_memset": [_P, _I32, _SZ, _P],
    "pa_stream_create": [_P, ctypes.POINTER(_P)],
    "pa_stream_wrap": [_P, _P, ctypes.POINTER(_P)],
    "pa_stream_native": [_P, ctypes.POINTER(_P)],
    "pa_stream_destroy": [_P],
    "pa_stream_synchronize": [_P],
    "pa_stream_wait_event": [_P, _P],
    "pa_event_create": [_P, ctypes.POINTER(_P)],
    "pa_event_destroy": [_P],
    "pa_event_record": [_P, _P],
    "pa_event_query": [_P, ctypes.POINTER(_I32)],
    "pa_event_synchronize": [_P],
    "pa_event_elapsed_ms": [_P, _P, ctypes.POINTER(ctypes.c_float)],
    "pa_graph_capture_begin": [_P],
    "pa_graph_capture_end": [_P, ctypes.POINTER(_P)],
    "pa_graph_launch": [_P, _P],
    "pa_graph_node_count": [_P, ctypes.POINTER(_SZ)],
    "pa_graph_destroy": [_P],
    "pa_build_slot_mapping": [_P, _CFG, _P, _I32, _P, _P, _P, _I32, _I32, _P],
    "pa_kv_append": [_P, _CFG, _P, _P, _P, _I32, _P, _P, _P, _P, _P, _P],
    "pa_decode_workspace_size": [_CFG, _I32, _I32, ctypes.POINTER(_SZ)],
    "pa_paged_decode": [_P, _CFG, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _P, _SZ],
    "pa_paged_decode_append": [_P, _CFG, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32,
                               _P, _SZ],
    "pa_paged_decode_noalloc": [_P, _CFG, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32],
    "pa_chunked_prefill": [_P, _CFG, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32],
    "pa_prefix_plan_bytes": [_I32, ctypes.POINTER(_SZ)],
    "pa_prefix_plan_build": [_P, _CFG, _I32, _P, _P, _SZ, ctypes.POINTER(_I32)],
    "pa_prefix_plan_fill": [_CFG, _I32, _P, _P, _SZ, ctypes.POINTER(_I32)],
    "pa_prefix_workspace_size": [_CFG, _I32, _I32, ctypes.POINTER(_SZ)],
    "pa_paged_decode_prefix": [_P, _CFG, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _P, _I32, _P, _SZ],
    "pa_block_bytes": [_CFG, ctypes.POINTER(_SZ)],
    "pa_copy_blocks": [_P, _CFG, _P, _P, _P, _P, _P, _P, _P, _I32],
    "pa_gather_blocks": [_P, _CFG, _P, _P, _P, _P, _P, _P, _P, _I32, _P],
    "pa_scatter_blocks": [_P, _CFG, _P, _P, _P, _P, _P, _P, _P, _I32, _P],
    "pa_read_block_f32": [_P, _CFG, _P, _P, _P, _P, _I32, _I32, _P, _P],
    "pa_write_block_f32": [_P, _CFG, _P, _P, _P, _P, _P, _P, _I32, _I32, _P, _P],
    "pa_qkv_workspace_size": [_CFG, _I32, ctypes.POINTER(_SZ)],
    "pa_qkv_project_append": [_P, _CFG, _P, _P, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ],
    "pa_o_workspace_size": [_CFG, _I32, _I32, ctypes.POINTER(_SZ)],
    "pa_o_project": [_P, _CFG, _P, _P, _I32, _I32, _P, _P, _SZ],
}

_lib = None


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Loads libpa_hip.so once. Raises FileNotFoundError / OSError when it is absent or broken."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(
            f"{path} is missing: build it with `make -C ml-framework_amd` (or __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    for name in EXPORTS:
        fn = getattr(lib, name)
        if name == "pa_status_string":
            fn.restype = ctypes.c_char_p
            fn.argtypes = [ctypes.c_int]
            continue
        fn.restype = ctypes.c_int
        fn.argtypes = _SIGNATURES[name]
    _lib = lib
    return lib


def last_error() -> str:
    buf = ctypes.create_string_buffer(1024)
    load_library().pa_get_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(status: int, fn: str) -> None:
    if status != PA_SUCCESS:
        raise PagedAttentionError(status, fn, last_error())


def call(name: str, *args) -> None:
    lib = load_library()
    check(getattr(lib, name)(*args), name)


def _ptr(t) -> int | None:
    """Device (or host) address of a torch tensor / numpy array / int / None."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    if hasattr(t, "data_ptr"):
        return t.data_ptr()
    if hasattr(t, "ctypes"):
        return t.ctypes.data
    raise TypeError(f"cannot take the address of {type(t)}")


# ---- device / stream / event helpers ------------------------------------------------------------
class Device:
    def __init__(self, ordinal: int = 0):
        self.handle = ctypes.c_void_p()
        call("pa_device_open", ordinal, ctypes.byref(self.handle))

    def props(self) -> PaDeviceProps:
        p = PaDeviceProps()
        call("pa_device_get_props", self.handle, ctypes.byref(p))
        return p

    def close(self):
        if self.handle:
            call("pa_device_close", self.handle)
            self.handle = ctypes.c_void_p()


class Stream:
    """A pa_stream; `wrap` adopts an existing hipStream_t (e.g. torch's current stream)."""

    def __init__(self, device: Device, native: int | None = None):
        self.handle = ctypes.c_void_p()
        if native is None:
            call("pa_stream_create", device.handle, ctypes.byref(self.handle))
        else:
            call("pa_stream_wrap", device.handle, ctypes.c_void_p(native), ctypes.byref(self.handle))

    def native(self) -> int:
        out = ctypes.c_void_p()
        call("pa_stream_native", self.handle, ctypes.byref(out))
        return out.value or 0

    def synchronize(self):
        call("pa_stream_synchronize", self.handle)

    def wait_event(self, event: "Event"):
        """Work enqueued on this stream from now on starts after `event`'s recorded work."""
        call("pa_stream_wait_event", self.handle, event.handle)

    def destroy(self):
        if self.handle:
            call("pa_stream_destroy", self.handle)
            self.handle = ctypes.c_void_p()


class Event:
    def __init__(self, device: Device):
        self.handle = ctypes.c_void_p()
        call("pa_event_create", device.handle, ctypes.byref(self.handle))

    def record(self, stream: Stream):
        call("pa_event_record", self.handle, stream.handle)

    def synchronize(self):
        call("pa_event_synchronize", self.handle)

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        call("pa_event_elapsed_ms", self.handle, end.handle, ctypes.byref(ms))
        return ms.value

    def destroy(self):
        if self.handle:
            call("pa_event_destroy", self.handle)
            self.handle = ctypes.c_void_p()


class Graph:
    """A pa_graph: the work enqueued on `stream` between `capture(stream)` and `end()`, replayed
    with `launch` (mirrors CUDAGraphCapture / CUDAGraph of the reference's CUDA HAL)."""

    def __init__(self):
        self.handle = ctypes.c_void_p()
        self._stream = None

    def capture(self, stream: Stream) -> "Graph":
        call("pa_graph_capture_begin", stream.handle)
        self._stream = stream
        return self

    def end(self) -> "Graph":
        call("pa_graph_capture_end", self._stream.handle, ctypes.byref(self.handle))
        self._stream = None
        return self

    def launch(self, stream: Stream):
        call("pa_graph_launch", self.handle, stream.handle)

    def node_count(self) -> int:
        n = ctypes.c_size_t()
        call("pa_graph_node_count", self.handle, ctypes.byref(n))
        return n.value

    def destroy(self):
        if self.handle:
            call("pa_graph_destroy", self.handle)
            self.handle = ctypes.c_void_p()


# ---- operators -----------------------------------------------------------------------------------
def build_slot_mapping(stream, cfg: PaConfig, block_tables, max_blocks_per_seq, start_pos, num_new,
                       token_offset, num_seqs, max_new_per_seq, slot_mapping):
    call("pa_build_slot_mapping", stream.handle if stream else None, ctypes.byref(cfg),
         _ptr(block_tables), max_blocks_per_seq, _ptr(start_pos), _ptr(num_new), _ptr(token_offset),
         num_seqs, max_new_per_seq, _ptr(slot_mapping))


def kv_append(stream, cfg: PaConfig, k_new, v_new, slot_mapping, n_tok, k_cache, v_cache,
              k_scale=None, v_scale=None, k_absmax=None, v_absmax=None):
    call("pa_kv_append", stream.handle if stream else None, ctypes.byref(cfg), _ptr(k_new),
         _ptr(v_new), _ptr(slot_mapping), n_tok, _ptr(k_cache), _ptr(v_cache), _ptr(k_scale),
         _ptr(v_scale), _ptr(k_absmax), _ptr(v_absmax))


def decode_workspace_size(cfg: PaConfig, num_seqs: int, max_context_len: int) -> int:
    out = ctypes.c_size_t()
    call("pa_decode_workspace_size", ctypes.byref(cfg), num_seqs, max_context_len, ctypes.byref(out))
    return out.value


def paged_decode(stream, cfg: PaConfig, out, q, k_cache, v_cache, k_scale, v_scale, block_tables,
                 context_lens, num_seqs, max_blocks_per_seq, max_context_len, workspace=None,
                 workspace_bytes=0):
    call("pa_paged_decode", stream.handle if stream else None, ctypes.byref(cfg), _ptr(out), _ptr(q),
         _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale), _ptr(block_tables),
         _ptr(context_lens), num_seqs, max_blocks_per_seq, max_context_len, _ptr(workspace),
         workspace_bytes)


def paged_decode_append(stream, cfg: PaConfig, out, q, k_new, v_new, k_cache, v_cache, k_scale, v_scale,
                        k_absmax, v_absmax, block_tables, context_lens, num_seqs, max_blocks_per_seq,
                        max_context_len, workspace=None, workspace_bytes=0):
    call("pa_paged_decode_append", stream.handle if stream else None, ctypes.byref(cfg), _ptr(out), _ptr(q),
         _ptr(k_new), _ptr(v_new), _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale),
         _ptr(k_absmax), _ptr(v_absmax), _ptr(block_tables), _ptr(context_lens), num_seqs,
         max_blocks_per_seq, max_context_len, _ptr(workspace), workspace_bytes)


def paged_decode_noalloc(stream, cfg: PaConfig, out, q, k_cache, v_cache, k_scale, v_scale, block_tables,
                         context_lens, num_seqs, max_blocks_per_seq, max_context_len):
    call("pa_paged_decode_noalloc", stream.handle if stream else None, ctypes.byref(cfg), _ptr(out), _ptr(q),
         _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale), _ptr(block_tables), _ptr(context_lens),
         num_seqs, max_blocks_per_seq, max_context_len)


def prefix_plan_bytes(num_seqs: int) -> int:
    out = ctypes.c_size_t()
    call("pa_prefix_plan_bytes", num_seqs, ctypes.byref(out))
    return out.value


def prefix_plan_build(stream, cfg: PaConfig, shared_with_prev, plan, plan_bytes) -> int:
    """shared_with_prev: host int32 sequence (leading table entries sequence s shares with s - 1).
    Writes the device plan and returns the group count for paged_decode_prefix."""
    import numpy as np
    links = np.ascontiguousarray(np.asarray(shared_with_prev, dtype=np.int32))
    ng = ctypes.c_int32()
    call("pa_prefix_plan_build", stream.handle if stream else None, ctypes.byref(cfg), int(links.size),
         links.ctypes.data_as(ctypes.c_void_p), _ptr(plan), plan_bytes, ctypes.byref(ng))
    return ng.value


def prefix_plan_fill(cfg: PaConfig, shared_with_prev):
    """Host-side plan (no GPU): returns (groups int32 [G][3], seqinfo int32 [S][2])."""
    import numpy as np
    links = np.ascontiguousarray(np.asarray(shared_with_prev, dtype=np.int32))
    S = int(links.size)
    nbytes = prefix_plan_bytes(S)
    buf = np.zeros(max(nbytes // 4, 1), np.int32)
    ng = ctypes.c_int32()
    call("pa_prefix_plan_fill", ctypes.byref(cfg), S, links.ctypes.data_as(ctypes.c_void_p),
         buf.ctypes.data_as(ctypes.c_void_p), nbytes, ctypes.byref(ng))
    g = ng.value
    return buf[:3 * g].reshape(g, 3).copy(), buf[3 * g:3 * g + 2 * S].reshape(S, 2).copy()


def prefix_workspace_size(cfg: PaConfig, num_seqs: int, max_context_len: int) -> int:
    out = ctypes.c_size_t()
    call("pa_prefix_workspace_size", ctypes.byref(cfg), num_seqs, max_context_len, ctypes.byref(out))
    return out.value


def paged_decode_prefix(stream, cfg: PaConfig, out, q, k_cache, v_cache, k_scale, v_scale, block_tables,
                        context_lens, num_seqs, max_blocks_per_seq, max_context_len, plan, num_groups,
                        workspace, workspace_bytes):
    call("pa_paged_decode_prefix", stream.handle if stream else None, ctypes.byref(cfg), _ptr(out), _ptr(q),
         _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale), _ptr(block_tables),
         _ptr(context_lens), num_seqs, max_blocks_per_seq, max_context_len, _ptr(plan), num_groups,
         _ptr(workspace), workspace_bytes)


def chunked_prefill(stream, cfg: PaConfig, out, q, q_start_loc, prefix_lens, k_cache, v_cache,
                    k_scale, v_scale, block_tables, num_seqs, max_blocks_per_seq, max_chunk_len):
    call("pa_chunked_prefill", stream.handle if stream else None, ctypes.byref(cfg), _ptr(out),
         _ptr(q), _ptr(q_start_loc), _ptr(prefix_lens), _ptr(k_cache), _ptr(v_cache), _ptr(k_scale),
         _ptr(v_scale), _ptr(block_tables), num_seqs, max_blocks_per_seq, max_chunk_len)


# ---- whole-block moves (copy-on-write, swap) ---------------------------------------------------
def block_bytes(cfg: PaConfig) -> int:
    n = ctypes.c_size_t()
    call("pa_block_bytes", ctypes.byref(cfg), ctypes.byref(n))
    return n.value


def copy_blocks(stream, cfg: PaConfig, k_cache, v_cache, k_scale, v_scale, k_absmax, v_absmax, block_pairs,
                num_pairs):
    call("pa_copy_blocks", stream.handle if stream else None, ctypes.byref(cfg), _ptr(k_cache), _ptr(v_cache),
         _ptr(k_scale), _ptr(v_scale), _ptr(k_absmax), _ptr(v_absmax), _ptr(block_pairs), num_pairs)


def gather_blocks(stream, cfg: PaConfig, k_cache, v_cache, k_scale, v_scale, k_absmax, v_absmax, block_ids, n,
                  packed):
    call("pa_gather_blocks", stream.handle if stream else None, ctypes.byref(cfg), _ptr(k_cache), _ptr(v_cache),
         _ptr(k_scale), _ptr(v_scale), _ptr(k_absmax), _ptr(v_absmax), _ptr(block_ids), n, _ptr(packed))


def scatter_blocks(stream, cfg: PaConfig, k_cache, v_cache, k_scale, v_scale, k_absmax, v_absmax, block_ids, n,
                   packed):
    call("pa_scatter_blocks", stream.handle if stream else None, ctypes.byref(cfg), _ptr(k_cache), _ptr(v_cache),
         _ptr(k_scale), _ptr(v_scale), _ptr(k_absmax), _ptr(v_absmax), _ptr(block_ids), n, _ptr(packed))


def read_block_f32(stream, cfg: PaConfig, k_cache, v_cache, k_scale, v_scale, block, tokens, k_out, v_out):
    call("pa_read_block_f32", stream.handle if stream else None, ctypes.byref(cfg), _ptr(k_cache), _ptr(v_cache),
         _ptr(k_scale), _ptr(v_scale), block, tokens, _ptr(k_out), _ptr(v_out))


def write_block_f32(stream, cfg: PaConfig, k_cache, v_cache, k_scale, v_scale, k_absmax, v_absmax, block, tokens,
                    k_in, v_in):
    call("pa_write_block_f32", stream.handle if stream else None, ctypes.byref(cfg), _ptr(k_cache), _ptr(v_cache),
         _ptr(k_scale), _ptr(v_scale), _ptr(k_absmax), _ptr(v_absmax), block, tokens, _ptr(k_in), _ptr(v_in))


# ---- projections either side of attention ----------------------------------------------------
def qkv_workspace_size(cfg: PaConfig, n_tok: int) -> int:
    n = ctypes.c_size_t()
    call("pa_qkv_workspace_size", ctypes.byref(cfg), n_tok, ctypes.byref(n))
    return n.value


def qkv_project_append(stream, cfg: PaConfig, x, w_qkv, hidden, n_tok, slot_mapping, q_out, k_cache, v_cache,
                       k_scale, v_scale, k_absmax, v_absmax, workspace, workspace_bytes):
    call("pa_qkv_project_append", stream.handle if stream else None, ctypes.byref(cfg), _ptr(x), _ptr(w_qkv), hidden,
         n_tok, _ptr(slot_mapping), _ptr(q_out), _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale),
         _ptr(k_absmax), _ptr(v_absmax), _ptr(workspace), workspace_bytes)


def o_workspace_size(cfg: PaConfig, hidden: int, n_tok: int) -> int:
    n = ctypes.c_size_t()
    call("pa_o_workspace_size", ctypes.byref(cfg), hidden, n_tok, ctypes.byref(n))
    return n.value


def o_project(stream, cfg: PaConfig, attn, w_o, hidden, n_tok, y, workspace, workspace_bytes):
    call("pa_o_project", stream.handle if stream else None, ctypes.byref(cfg), _ptr(attn), _ptr(w_o), hidden, n_tok,
         _ptr(y), _ptr(workspace), workspace_bytes)


@dataclass
class TorchStream:
    """pa_stream wrapping torch's current HIP stream, so library launches order with torch work."""

    device: Device
    stream: Stream

    @classmethod
    def current(cls, ordinal: int = 0) -> "TorchStream":
        import torch

        dev = Device(ordinal)
        native = torch.cuda.current_stream(ordinal).cuda_stream
        return cls(dev, Stream(dev, native))
