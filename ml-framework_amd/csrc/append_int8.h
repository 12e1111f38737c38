// append_int8.h -- the quantising append into an int8 paged cache, shared by pa_kv_append, the
// last-token append of pa_paged_decode_append and pa_write_block_f32.
//
// Policy (the reference's QuantizeSymmetric / Dequantize, Quantization/Operations/
// QuantizationOperations.cs:188-200, applied per (block, KV head) with a running absmax): a
// segment is a maximal run of consecutive tokens of the call whose slots are valid and lie in one
// block. Segments are applied in call order. Writing row 0 starts the block afresh (scale =
// segment absmax / 127); otherwise a segment whose absmax exceeds the block's grows the scale and
// requantises every row it does not overwrite; the segment's rows are then quantised with the
// block's (possibly grown) scale.
//
// Ownership: one workgroup per token of the call; the workgroup of the first token of the call
// that lands in a block owns that block and applies every segment of it, in call order, one wave
// per (KV head, K|V). A block's tokens may therefore arrive in any order, split by invalid slots
// or by other blocks' tokens, without two workgroups touching one block.
#pragma once

#include "pa_internal.h"

namespace pa {

__device__ __forceinline__ float load_act(const void* p, bool bf16, int64_t i) {
    return bf16 ? bf16_to_f32(static_cast<const uint16_t*>(p)[i]) : static_cast<const float*>(p)[i];
}

// One segment [s, e) of block blk for KV head h, K (is_v false) or V, applied by one wave (64
// lanes; lane l owns dims l, l + 64, ..). slot_at(t) is token t's slot; src holds the tokens'
// values in the activation dtype, token t's (head h, dim d) at t * tok_stride + h * D + d. The
// tile of (blk, h) is K [16][D] or V [D][16] in `cache`. (amax, cur_scale) carry the block's
// statistics from one segment of this (block, head) to the next: have_stats false loads them.
template <int D, typename SlotAt>
__device__ __forceinline__ void append_int8_apply(const void* src, bool in_bf16, int64_t tok_stride, SlotAt slot_at,
                                                  int32_t s, int32_t e, int64_t blk, int8_t* cache, float* scale,
                                                  float* absmax, int h, int32_t num_kv_heads, bool is_v, float& amax,
                                                  float& cur_scale, bool& have_stats) {
#pragma clang fp contract(off)
    static_assert(D % 64 == 0, "int8 caches take head_dim 64, 128 or 256");
    constexpr int kPer = D / 64;  // elements per lane
    const int lane = threadIdx.x & 63;
    // Rows the segment writes (lane j looks at tokens s + j, s + j + 64, ..) and its absmax.
    uint32_t written = 0;
    for (int t = s + lane; t < e; t += 64) written |= 1u << static_cast<int>(slot_at(t) % kBlockSize);
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) written |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(written), o, 64));
    const bool fresh = (written & 1u) != 0;
    const int64_t sidx = blk * num_kv_heads + h;
    int8_t* block_codes = cache + ((blk * num_kv_heads + h) * kBlockSize) * D;
    // Element (row off, dim d) of the tile: K is [16][D], V is [D][16].
    auto at = [&](int off, int d) -> int8_t* {
        return is_v ? block_codes + d * kBlockSize + off : block_codes + off * D + d;
    };
    // One round trip for everything the segment reads: the block's statistics, its codes (needed
    // only if the scale grows, so fetched unless the segment starts the block) as 16-byte chunks
    // of the tile (chunk c of lane: c = lane + 64 i, K row c / (D/16) or V dim c), and, for a
    // one-token segment, the token's values (kept for its quantisation).
    const float amax_mem = have_stats ? 0.0f : absmax[sidx];
    const float scale_mem = have_stats ? 0.0f : scale[sidx];
    constexpr int kChunks = kBlockSize * D / 16 / 64;  // 16-byte chunks of the tile per lane
    uint4 old_chunk[kChunks];
    if (!fresh) {
#pragma unroll
        for (int i = 0; i < kChunks; i++) old_chunk[i] = reinterpret_cast<const uint4*>(block_codes)[lane + 64 * i];
    }
    const bool one = e - s == 1;
    float x1[kPer];
    float seg_amax = 0.0f;
    for (int t = s; t < e; t++) {
        const int64_t base = static_cast<int64_t>(t) * tok_stride + static_cast<int64_t>(h) * D;
#pragma unroll
        for (int k = 0; k < kPer; k++) {
            const float x = load_act(src, in_bf16, base + lane + 64 * k);
            if (t == s) x1[k] = x;
            const float a = fabsf(x);
            seg_amax = a > seg_amax ? a : seg_amax;  // NaN never wins, as `if (a > m) m = a`
        }
    }
    seg_amax = wave_max(seg_amax);

    if (fresh) {
        // Writing row 0 starts the block: earlier contents and statistics are discarded.
        amax = seg_amax;
        cur_scale = seg_amax / 127.0f;
        if (lane == 0) {
            absmax[sidx] = amax;
            scale[sidx] = cur_scale;
        }
    } else {
        if (!have_stats) {
            amax = amax_mem;
            cur_scale = scale_mem;
        }
        if (seg_amax > amax) {
            const float old_scale = cur_scale;
            cur_scale = seg_amax / 127.0f;
            amax = seg_amax;
            // Requantise every row this segment does not overwrite:
            // QuantizeSymmetric(Dequantize(q, old_scale), new_scale). The rows it writes keep
            // their old codes here; its own stores below replace them, after these have landed.
#pragma unroll
            for (int i = 0; i < kChunks; i++) {
                const int c = lane + 64 * i;
                uint32_t w[4] = {old_chunk[i].x, old_chunk[i].y, old_chunk[i].z, old_chunk[i].w};
#pragma unroll
                for (int b = 0; b < 16; b++) {
                    const int row = is_v ? b : c / (D / 16);
                    if (written & (1u << row)) continue;
                    const uint32_t sh = 8 * (b & 3);
                    const int32_t q = static_cast<int32_t>(w[b >> 2] << (24 - sh)) >> 24;
                    const float deq = static_cast<float>(q) * old_scale;
                    const uint32_t nq = static_cast<uint32_t>(static_cast<uint8_t>(quantize_symmetric(deq, cur_scale)));
                    w[b >> 2] = (w[b >> 2] & ~(0xffu << sh)) | (nq << sh);
                }
                reinterpret_cast<uint4*>(block_codes)[c] = make_uint4(w[0], w[1], w[2], w[3]);
            }
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the tile's stores precede the new rows'

            if (lane == 0) {
                absmax[sidx] = amax;
                scale[sidx] = cur_scale;
            }
        }
    }
    have_stats = true;
    for (int t = s; t < e; t++) {
        const int off = static_cast<int>(slot_at(t) % kBlockSize);
        const int64_t base = static_cast<int64_t>(t) * tok_stride + static_cast<int64_t>(h) * D;
#pragma unroll
        for (int k = 0; k < kPer; k++) {
            const float x = one ? x1[k] : load_act(src, in_bf16, base + lane + 64 * k);
            *at(off, lane + 64 * k) = quantize_symmetric(x, cur_scale);
        }
    }
}

// One token appended alone into its block (the block receives no other token of the call), by one
// wave for (KV head h, K or V): the same bytes and statistics as append_int8_apply with a one-token
// segment, in fewer memory round trips. x holds the token's values (lane l: dims l, l + 64, ..),
// loaded by the caller before the slot was known. The block's statistics and its codes come in one
// round trip; the token's codes are merged into the tile's 16-byte chunks (V: byte off of the chunk
// of each dim, the lane's own dims; K: row off's chunks, staged through `stage`, D bytes of LDS), so
// the tile goes back in one set of whole-chunk stores with no store-then-wait ordering between the
// requantised rows and the token's row.
template <int D>
__device__ __forceinline__ void append_int8_one_token(const float (&x)[D / 64], int64_t slot, int8_t* cache,
                                                      float* scale, float* absmax, int h, int32_t num_kv_heads,
                                                      bool is_v, int8_t* stage) {
#pragma clang fp contract(off)
    constexpr int kPer = D / 64;
    constexpr int kChunks = kBlockSize * D / 16 / 64;  // 16-byte chunks of the tile per lane (= kPer)
    const int lane = threadIdx.x & 63;
    const int64_t blk = slot / kBlockSize;
    const int off = static_cast<int>(slot % kBlockSize);
    const int64_t sidx = blk * num_kv_heads + h;
    int8_t* block_codes = cache + ((blk * num_kv_heads + h) * kBlockSize) * D;
    uint4* chunks = reinterpret_cast<uint4*>(block_codes);
    const float amax_mem = absmax[sidx];
    const float scale_mem = scale[sidx];
    uint4 ch[kChunks];
#pragma unroll
    for (int i = 0; i < kChunks; i++) ch[i] = chunks[lane + 64 * i];
    float seg_amax = 0.0f;
#pragma unroll
    for (int k = 0; k < kPer; k++) {
        const float a = fabsf(x[k]);
        seg_amax = a > seg_amax ? a : seg_amax;  // NaN never wins, as `if (a > m) m = a`
    }
    seg_amax = wave_max(seg_amax);
    const bool fresh = off == 0;  // writing row 0 starts the block afresh
    float cur_scale;
    bool grow = false, new_stats = false;
    float old_scale = 0.0f, amax = 0.0f;
    if (fresh) {
        amax = seg_amax;
        cur_scale = seg_amax / 127.0f;
        new_stats = true;
    } else {
        amax = amax_mem;
        cur_scale = scale_mem;
        if (seg_amax > amax) {
            old_scale = cur_scale;
            cur_scale = seg_amax / 127.0f;
            amax = seg_amax;
            grow = true;
            new_stats = true;
        }
    }
    // the token's codes: lane l, dims l + 64 k
    uint32_t code[kPer];
#pragma unroll
    for (int k = 0; k < kPer; k++) code[k] = static_cast<uint32_t>(static_cast<uint8_t>(quantize_symmetric(x[k], cur_scale)));
    if (!is_v) {  // K row off: D consecutive bytes, chunks off * D / 16 .. (+ D / 16), via LDS
#pragma unroll
        for (int k = 0; k < kPer; k++) stage[lane + 64 * k] = static_cast<int8_t>(code[k]);
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
        __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int i = 0; i < kChunks; i++) {
        const int c = lane + 64 * i;  // K: row c / (D / 16), dims 16 (c % (D / 16)) ..; V: dim c, tokens 0 .. 15
        uint32_t w[4] = {ch[i].x, ch[i].y, ch[i].z, ch[i].w};
        if (grow) {
            // QuantizeSymmetric(Dequantize(q, old_scale), new_scale) on every row but `off`
#pragma unroll
            for (int b = 0; b < 16; b++) {
                const int row = is_v ? b : c / (D / 16);
                if (row == off) continue;
                const uint32_t sh = 8 * (b & 3);
                const int32_t q = static_cast<int32_t>(w[b >> 2] << (24 - sh)) >> 24;
                const float deq = static_cast<float>(q) * old_scale;
                const uint32_t nq = static_cast<uint32_t>(static_cast<uint8_t>(quantize_symmetric(deq, cur_scale)));
                w[b >> 2] = (w[b >> 2] & ~(0xffu << sh)) | (nq << sh);
            }
        }
        if (is_v) {  // byte off of dim c's chunk: this lane's own code of dim c = lane + 64 i
            const uint32_t sh = 8 * (off & 3);
            w[off >> 2] = (w[off >> 2] & ~(0xffu << sh)) | (code[i] << sh);
        } else if (c / (D / 16) == off) {  // a chunk of row off: 16 codes from the stage
            const uint4 n = *reinterpret_cast<const uint4*>(stage + 16 * (c % (D / 16)));
            w[0] = n.x;
            w[1] = n.y;
            w[2] = n.z;
            w[3] = n.w;
        }
        chunks[c] = make_uint4(w[0], w[1], w[2], w[3]);
    }
    if (new_stats && lane == 0) {
        absmax[sidx] = amax;
        scale[sidx] = cur_scale;
    }
}

// Segments collected per pass of the owner's scan (a block has at most 16 rows, so more than one
// pass only happens when slots repeat).
constexpr int kAppendSegList = 64;
// Threads of an int8 append workgroup: one wave per (KV head, K|V) up to 16 waves.
constexpr int kAppendMaxThreads = 1024;
inline int append_int8_threads(int32_t num_kv_heads) {
    const int64_t waves = 2 * static_cast<int64_t>(num_kv_heads);
    return static_cast<int>(64 * (waves < kAppendMaxThreads / 64 ? waves : kAppendMaxThreads / 64));
}

// Tokens per thread of the owner's coarse scan (a chunk of kAppendCoarse * blockDim.x tokens is
// skipped when none of them lands in the block).
constexpr int kAppendCoarse = 8;

// The workgroup of token i (blockDim.x a multiple of 64, at most kAppendMaxThreads): if token i
// is the first token of the call that lands in its block, applies every segment of that block, in
// call order; otherwise returns. The owner reads the call's slot list once, kAppendCoarse slots per
// thread at a time, and looks closer only at chunks that hold tokens of its block: a call of n
// tokens costs each touched block one pass over n slots (a few memory round trips for calls of up
// to ~16k tokens; split much larger calls).
template <int D, typename SlotAt>
__device__ __forceinline__ void append_int8_block(const void* k_src, const void* v_src, bool in_bf16,
                                                  int64_t tok_stride, SlotAt slot_at, int32_t i, int32_t n_tok,
                                                  int8_t* k_cache, int8_t* v_cache, float* k_scale, float* v_scale,
                                                  float* k_absmax, float* v_absmax, int32_t num_kv_heads,
                                                  int64_t capacity) {
    __shared__ int s_start[kAppendSegList], s_end[kAppendSegList];
    __shared__ int s_wcnt[2][kAppendMaxThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nthreads = blockDim.x, nwaves = nthreads >> 6;
    auto valid = [&](int64_t sl) { return sl >= 0 && sl < capacity; };
    // Token i's slot and its predecessor's, loaded together.
    const int64_t slot_i = slot_at(i);
    const int64_t slot_p = i > 0 ? slot_at(i - 1) : -1;
    if (!valid(slot_i)) return;
    const int64_t blk = slot_i / kBlockSize;
    if (valid(slot_p) && slot_p / kBlockSize == blk) return;  // not the first token of its segment
    auto in_blk = [&](int t) {
        if (t < 0 || t >= n_tok) return false;
        const int64_t sl = slot_at(t);
        return valid(sl) && sl / kBlockSize == blk;
    };
    // Does any token of [lo, hi) land in the block? (coarse: kAppendCoarse tokens per thread)
    auto any_in = [&](int lo, int hi) {
        bool f = false;
#pragma unroll
        for (int k = 0; k < kAppendCoarse; k++) {
            const int t = lo + k * nthreads + tid;
            f |= t < hi && in_blk(t);
        }
        return __syncthreads_or(f) != 0;
    };
    const int coarse = kAppendCoarse * nthreads;
    // An earlier token of the call in the block: its workgroup owns the block.
    for (int c0 = 0; c0 < i; c0 += coarse)
        if (any_in(c0, i)) return;

    // Passes: from seg_from on, segment starts and ends are compacted, in order, into s_start /
    // s_end until kAppendSegList segments are complete or the call ends; then they are applied.
    int seg_from = i;
    while (seg_from < n_tok) {
        int nseg = 0, nstart = 0;
        int resume = n_tok;  // where the next pass starts if this one fills the list
        for (int c0 = seg_from; c0 < n_tok && resume == n_tok; c0 += coarse) {
            if (!any_in(c0, n_tok)) continue;
            const int c1 = min(n_tok, c0 + coarse);
            for (int f0 = c0; f0 < c1; f0 += nthreads) {
                const int t = f0 + tid;
                const bool cur = t < c1 && in_blk(t);
                const bool st = cur && !in_blk(t - 1);
                const bool en = cur && !in_blk(t + 1);
                const uint64_t ms = __ballot(st), me = __ballot(en);
                const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
                if (lane == 0) {
                    s_wcnt[0][wave] = __popcll(ms);
                    s_wcnt[1][wave] = __popcll(me);
                }
                __syncthreads();
                int bs = nstart, be = nseg, ts = 0, te = 0;
                for (int w = 0; w < nwaves; w++) {
                    if (w < wave) {
                        bs += s_wcnt[0][w];
                        be += s_wcnt[1][w];
                    }
                    ts += s_wcnt[0][w];
                    te += s_wcnt[1][w];
                }
                const int rs = bs + __popcll(ms & below), re = be + __popcll(me & below);
                if (st && rs < kAppendSegList) s_start[rs] = t;
                if (en && re < kAppendSegList) s_end[re] = t + 1;
                __syncthreads();
                nstart += ts;
                nseg += te;
                if (nseg >= kAppendSegList) {
                    nseg = kAppendSegList;
                    resume = s_end[kAppendSegList - 1];
                    break;
                }
            }
        }
        // Apply the complete segments, in order, one wave per (KV head, K|V).
        for (int p = wave; p < 2 * num_kv_heads; p += nwaves) {
            const int h = p >> 1;
            const bool is_v = (p & 1) != 0;
            float amax = 0.0f, cur_scale = 0.0f;
            bool have = false;  // statistics of an earlier pass are re-read (written before the barrier)
            for (int k = 0; k < nseg; k++)
                append_int8_apply<D>(is_v ? v_src : k_src, in_bf16, tok_stride, slot_at, s_start[k], s_end[k], blk,
                                     is_v ? v_cache : k_cache, is_v ? v_scale : k_scale, is_v ? v_absmax : k_absmax,
                                     h, num_kv_heads, is_v, amax, cur_scale, have);
        }
        if (resume >= n_tok) break;
        __syncthreads();  // this pass's statistics and codes are visible to the next pass's waves
        seg_from = resume;
    }
}

}  // namespace pa
