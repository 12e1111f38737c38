// pa_internal.h -- shared host/device definitions of libpa_hip.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "paged_attn.h"

// ---- opaque handle types behind the C-ABI ------------------------------------------------------
struct pa_device {
    int32_t ordinal;
};

struct pa_stream {
    int32_t ordinal;
    hipStream_t stream;
    bool owned;  // false for pa_stream_wrap
};

struct pa_event {
    int32_t ordinal;
    hipEvent_t event;
};

struct pa_graph {
    int32_t ordinal;
    hipGraph_t graph;
    hipGraphExec_t exec;
    size_t nodes;
};

// ---- host-side error plumbing (pa_runtime.hip) -------------------------------------------------
namespace pa {

pa_status set_error(pa_status st, const std::string& msg);
pa_status set_hip_error(hipError_t err, const char* what);
pa_status clear_error();

// Stream handed to a launch (null pa_stream -> legacy default stream).
inline hipStream_t native(const pa_stream* s) { return s ? s->stream : nullptr; }

// Fixed block size of every compiled kernel.
constexpr int kBlockSize = 16;

// Validates the fields every operator needs; on failure sets the last error.
pa_status check_config(const pa_config* cfg, const char* fn);
// The append of pa_kv_append on stream s, for new K/V whose token t starts at t * tok_stride
// elements (pa_kv_append: num_kv_heads * head_dim); in_bf16 selects the activation dtype.
pa_status launch_kv_append(const char* f, hipStream_t s, const pa_config* cfg, const void* k_new, const void* v_new,
                           bool in_bf16, int64_t tok_stride, const int64_t* slot_mapping, int32_t n_tok,
                           void* k_cache, void* v_cache, float* k_scale, float* v_scale, float* k_absmax,
                           float* v_absmax);

// pa_chunked_prefill over an fp32 cache (chunked_prefill_fp32.hip); the caller has validated the
// arguments. mask_mode: 0 causal, 1 causal only when the prefix is non-empty, 2 no mask.
pa_status launch_chunked_prefill_fp32(hipStream_t s, const pa_config* cfg, float* out, const void* q,
                                      const int32_t* q_start_loc, const int32_t* prefix_lens, const float* k_cache,
                                      const float* v_cache, const int32_t* block_tables, int32_t num_seqs,
                                      int32_t max_blocks_per_seq, int32_t max_chunk_len, int32_t mask_mode);
// Resolves the device address of pa_paged_decode_noalloc's scratch array on device `ordinal`
// (paged_decode.hip); pa_device_open calls it once per device.
pa_status init_decode_scratch(int ordinal);

inline float resolve_scale(const pa_config* cfg) {
    // StandardPagedAttentionKernel.cs:18,28 -- scale > 0 overrides 1/sqrt(headDim).
    return cfg->scale > 0.0f ? cfg->scale : 1.0f / sqrtf(static_cast<float>(cfg->head_dim));
}

}  // namespace pa

#define PA_HIP_CHECK(expr)                                            \
    do {                                                              \
        hipError_t _e = (expr);                                       \
        if (_e != hipSuccess) return pa::set_hip_error(_e, #expr);    \
    } while (0)

// ---- device helpers ------------------------------------------------------------------------
namespace pa {

// bf16 <-> fp32 with the reference's rules: fp32 -> bf16 keeps the upper 16 bits (truncation,
// src/MLFramework/Amp/BFloat16.cs:99-107); bf16 -> fp32 shifts back (:109-117).
__device__ __forceinline__ uint16_t bf16_trunc(float x) {
    return static_cast<uint16_t>(__float_as_uint(x) >> 16);
}
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Sign-extended byte k of a 32-bit word, as fp32.
__device__ __forceinline__ float i8_at(uint32_t w, int k) {
    return static_cast<float>(static_cast<int32_t>(w << (24 - 8 * k)) >> 24);
}

// Sum over aligned groups of W lanes (W a power of two <= 64), result in every lane of the group.
// Groups of up to 16 lanes use DPP within a row: quad_perm xor1 (0xB1), quad_perm xor2 (0x4E),
// row_half_mirror (0x141: lane i <-> 7-i), row_mirror (0x140: lane i <-> 15-i). Once every lane of
// a sub-group holds that sub-group's sum, a mirror adds the partner sub-group's sum.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(W >= 1 && W <= 64 && (W & (W - 1)) == 0, "W must be a power of two <= 64");
    if constexpr (W >= 2)
        v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
    if constexpr (W >= 4)
        v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));
    if constexpr (W >= 8)
        v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false));
    if constexpr (W >= 16)
        v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false));
    if constexpr (W >= 32) v += __shfl_xor(v, 16, 64);
    if constexpr (W >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// QuantizationUtils.RoundHalfAwayFromZero (Quantization/Operations/QuantizationUtils.cs:146-159)
// followed by Clamp to [-128, 127] (:110-115), as QuantizeSymmetric applies them
// (QuantizationOperations.cs:188-200). fabsf(v) + 0.5f is an fp32 add; floor of that fp32 value
// is exact in fp32; the saturating int conversion and the clamp meet at the int8 bounds.
__device__ __forceinline__ int8_t quantize_symmetric(float v, float scale) {
#pragma clang fp contract(off)
    float scaled = v / scale;  // IEEE division (hipcc default: correctly rounded fp32 divide)
    if (scaled != scaled) return 0;  // NaN (value NaN, 0/0) -> 0
    float a = floorf(fabsf(scaled) + 0.5f);
    float r = copysignf(a, scaled);
    if (r >= 127.0f) return 127;
    if (r <= -128.0f) return -128;
    return static_cast<int8_t>(static_cast<int>(r));
}

}  // namespace pa
