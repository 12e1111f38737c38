// append_int8.h -- the quantising append of one segment into an int8 paged cache, shared by
// pa_kv_append and the last-token append of pa_paged_decode_append.
//
// Policy (the reference's QuantizeSymmetric / Dequantize, Quantization/Operations/
// QuantizationOperations.cs:188-200, applied per (block, KV head) with a running absmax): a
// segment is a run of consecutive tokens of the call that land in the same block; its first
// token's wave owns that (block, head) for the call. Writing row 0 starts the block afresh
// (scale = segment absmax / 127); otherwise a segment whose absmax exceeds the block's grows the
// scale and requantises every row it does not overwrite; the new rows are quantised with the
// block's (possibly grown) scale.
#pragma once

#include "pa_internal.h"

namespace pa {

__device__ __forceinline__ float load_act(const void* p, bool bf16, int64_t i) {
    return bf16 ? bf16_to_f32(static_cast<const uint16_t*>(p)[i]) : static_cast<const float*>(p)[i];
}

// Wave (64 lanes) for token i of the call, KV head h, K (is_v false) or V. slot_at(t) is the slot
// of token t (out of [0, capacity): skipped); src holds the tokens' values in the activation dtype,
// token t's (head h, dim d) at t * tok_stride + h * D + d. The tile of (block, h) is K [16][D] or
// V [D][16] in `cache`.
template <int D, typename SlotAt>
__device__ __forceinline__ void append_int8_segment(const void* src, bool in_bf16, int64_t tok_stride, SlotAt slot_at,
                                                    int32_t i,
                                                    int32_t n_tok, int8_t* cache, float* scale, float* absmax,
                                                    int h, int32_t num_kv_heads, int64_t capacity, bool is_v) {
#pragma clang fp contract(off)
    constexpr int kPer = D / 64;  // elements per lane
    const int lane = threadIdx.x & 63;
    const int64_t slot = slot_at(i);
    if (slot < 0 || slot >= capacity) return;
    const int64_t blk = slot / kBlockSize;
    if (i > 0) {
        const int64_t prev = slot_at(i - 1);
        if (prev >= 0 && prev < capacity && prev / kBlockSize == blk) return;  // not a segment head
    }
    // Extent of the segment, the slots it writes and the absmax of its values for head h.
    int end = i;
    uint32_t written = 0;
    bool fresh = false;
    float seg_amax = 0.0f;
    while (end < n_tok) {
        const int64_t s = slot_at(end);
        if (s < 0 || s >= capacity || s / kBlockSize != blk) break;
        const int off = static_cast<int>(s % kBlockSize);
        written |= 1u << off;
        fresh |= off == 0;
        const int64_t base = static_cast<int64_t>(end) * tok_stride + static_cast<int64_t>(h) * D;
#pragma unroll
        for (int k = 0; k < kPer; k++) {
            const float a = fabsf(load_act(src, in_bf16, base + lane + 64 * k));
            seg_amax = a > seg_amax ? a : seg_amax;  // NaN never wins, as `if (a > m) m = a`
        }
        end++;
    }
    seg_amax = wave_max(seg_amax);

    const int64_t sidx = blk * num_kv_heads + h;
    int8_t* block_codes = cache + ((blk * num_kv_heads + h) * kBlockSize) * D;
    // Element (row off, dim d) of the tile: K is [16][D], V is [D][16].
    auto at = [&](int off, int d) -> int8_t* {
        return is_v ? block_codes + d * kBlockSize + off : block_codes + off * D + d;
    };
    float cur_scale;
    if (fresh) {
        // Writing row 0 starts the block: earlier contents and statistics are discarded.
        cur_scale = seg_amax / 127.0f;
        if (lane == 0) {
            absmax[sidx] = seg_amax;
            scale[sidx] = cur_scale;
        }
    } else {
        const float old_amax = absmax[sidx];
        const float old_scale = scale[sidx];
        cur_scale = old_scale;
        if (seg_amax > old_amax) {
            cur_scale = seg_amax / 127.0f;
            // Requantise every row this segment does not overwrite:
            // QuantizeSymmetric(Dequantize(q, old_scale), new_scale).
            for (int off = 0; off < kBlockSize; off++) {
                if (written & (1u << off)) continue;
#pragma unroll
                for (int k = 0; k < kPer; k++) {
                    int8_t* c = at(off, lane + 64 * k);
                    const float deq = static_cast<float>(static_cast<int32_t>(*c)) * old_scale;
                    *c = quantize_symmetric(deq, cur_scale);
                }
            }
            if (lane == 0) {
                absmax[sidx] = seg_amax;
                scale[sidx] = cur_scale;
            }
        }
    }
    for (int t = i; t < end; t++) {
        const int off = static_cast<int>(slot_at(t) % kBlockSize);
        const int64_t base = static_cast<int64_t>(t) * tok_stride + static_cast<int64_t>(h) * D;
#pragma unroll
        for (int k = 0; k < kPer; k++) {
            const float x = load_act(src, in_bf16, base + lane + 64 * k);
            *at(off, lane + 64 * k) = quantize_symmetric(x, cur_scale);
        }
    }
}

}  // namespace pa
