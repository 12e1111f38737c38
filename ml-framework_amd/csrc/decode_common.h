// decode_common.h -- shared definitions of the paged-decode kernels (argument block, helpers,
// partition merge, fused-append register patches). Included by the decode translation units.
#pragma once

#include <string>

#include "pa_internal.h"

namespace pa {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));

struct DecodeArgs {
    float* out;
    const void* q;
    const void* k_cache;
    const void* v_cache;
    const float* k_scale;
    const float* v_scale;
    const int32_t* block_tables;
    const int32_t* context_lens;
    // split-K partials. fp32 kernel: row = (seq * Hq + head) * max_parts + part. MFMA kernel:
    // row = slot * G + head-in-group, slot = 2 * unit + (0: first row portion of the unit, 1: last).
    float* ws_o;  // [rows][D], unnormalised
    float* ws_m;  // [rows]
    float* ws_l;  // [rows]
    int32_t* ws_pref;  // MFMA kernel: [num_seqs + 1] blocks per KV-head row before each sequence
    // fused append (pa_paged_decode_append): the token at position context_len - 1
    const void* k_new;  // [num_seqs][Hkv][D] of the activation dtype
    const void* v_new;
    float* k_absmax;    // int8 caches: running absmax / scale per (block, KV head), updated
    float* v_absmax;
    int32_t num_kv_heads;
    int32_t group;  // G = Hq / Hkv
    int32_t max_blocks_per_seq;
    int32_t num_blocks;
    int32_t max_context_len;
    int32_t max_parts;
    int32_t part;  // fp32 kernel: partition length in tokens
    // MFMA kernel: the flattened (sequence, KV head, block) list is cut into ranges of
    // split_blocks blocks (0: one range per split_grid / Hkv workers, at least 4 blocks)
    int32_t split_blocks;
    int32_t split_grid;  // workers (waves) of the launch
    int32_t q_bf16;
    float scale;
    // shared-prefix decode (pa_paged_decode_prefix): the plan (prefix groups, then per sequence
    // its group and shared block count) and its group count; unused by the other entry points.
    const int32_t* plan;
    int32_t num_groups;
    // Slot of row r, KV head h when the row lies whole inside one range: row_slot_base + r * Hkv +
    // h (a range has slots for its first and last row portions only, and grouped rows never write
    // the output directly).
    int32_t row_slot_base;
    // MFMA kernel: units (range, KV head) the workspace has slots for (2 per unit), computed on the
    // host from the call's shape; the merges follow no slot index at or past 2 * max_units.
    int64_t max_units;
    // MFMA kernel: > 0 cuts every row (sequence, KV head) into this many partitions of whole
    // blocks instead of the batch-wide equal ranges (pa_config.num_splits)
    int32_t num_splits;
    // Fused append (bf16 caches) when the merge kernel runs: the decode folds the new token into
    // attention from k_new / v_new and the merge kernel writes it into the cache.
    int32_t append_in_merge;
};


// Shared-prefix plan, in device memory: num_groups records {first sequence, members, shared
// blocks}, then per sequence {group or -1, shared blocks or 0}. The members of a group are
// consecutive sequences whose block tables agree on the shared blocks; with G query heads per KV
// head a group has at most 16 / G members (one MFMA column tile of query heads).
constexpr int kPlanGroupInts = 3;
constexpr int kPlanSeqInts = 2;
// Workspace slot width of the shared-prefix decode: a slot holds the 16 MFMA columns (the query
// heads of up to 16 / G sequences) of one KV head.
constexpr int kPrefixSlotRows = 16;

// Context length clamped to what the table holds and to max_context_len (raw: context_lens[seq]).
__device__ __forceinline__ int clamp_len(const DecodeArgs& a, int raw) {
    return min(min(raw, a.max_blocks_per_seq * pa::kBlockSize), a.max_context_len);
}

// Element i of an activation array (the fused append's new K/V): fp32, or bf16 widened exactly.
__device__ __forceinline__ float act_at(const void* p, bool f32, int64_t i) {
    return f32 ? static_cast<const float*>(p)[i] : pa::bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}

// The new token (position T - 1 of sequence seq, KV head kvh; T = its clamped context length >= 2)
// written into a bf16 cache as pa_kv_append stores it: K row (T - 1) % 16 and V column (T - 1) % 16
// of the block the table gives for it, bf16 by truncation. One wave, lane l takes dims l, l + 64, ..
// Written by the merge kernel's fifth wave (beside the four merging ones, so its round trip is not
// added to theirs), after the decode's streaming, with non-temporal stores: the V column
// touches one line per two dims of the transposed tile, and written among the decode's reads, or
// left dirty in the caches for the next step's reads to evict, those lines cost the C2 step 3-4 us
// (measured: in the decode, in the merge kernel with plain stores, as whole tiles read and
// rewritten; non-temporal 2-byte stores here cost the least).
template <int D, bool F32>
__device__ __forceinline__ void append_token_bf16_as(const DecodeArgs& a, int seq, int kvh) {
    // Every load goes out before any is used: the length, the token's values and, for tables of up
    // to kRowIds * 64 blocks, the sequence's table row, from which the token's block is picked; the
    // stores then wait for one round trip instead of three (length, then table entry, then values).
    constexpr int NPL = (D + 63) / 64;
    constexpr int kRowIds = 4;
    const int lane = threadIdx.x & 63;
    const int64_t src = (static_cast<int64_t>(seq) * a.num_kv_heads + kvh) * D;
    uint32_t kraw[NPL], vraw[NPL];
#pragma unroll
    for (int e = 0; e < NPL; e++) {
        const int d = lane + 64 * e;
        kraw[e] = 0;
        vraw[e] = 0;
        if (d < D) {
            if constexpr (F32) {
                kraw[e] = static_cast<const uint32_t*>(a.k_new)[src + d];
                vraw[e] = static_cast<const uint32_t*>(a.v_new)[src + d];
            } else {
                kraw[e] = static_cast<uint32_t>(static_cast<const uint16_t*>(a.k_new)[src + d]) << 16;
                vraw[e] = static_cast<uint32_t>(static_cast<const uint16_t*>(a.v_new)[src + d]) << 16;
            }
        }
    }
    const int32_t* row = a.block_tables + static_cast<int64_t>(seq) * a.max_blocks_per_seq;
    const bool whole_row = a.max_blocks_per_seq <= kRowIds * 64;
    int ids[kRowIds];
#pragma unroll
    for (int k = 0; k < kRowIds; k++) {
        const int b = lane + 64 * k;
        ids[k] = whole_row && b < a.max_blocks_per_seq ? row[b] : -1;
    }
    const int T = clamp_len(a, a.context_lens[seq]);
    if (T < 2) return;  // T == 1: the decode writes it (no streamed block); T <= 0: nothing
    const int bi = (T - 1) / 16;
    int bid;
    if (whole_row) {
        int w = ids[0];
#pragma unroll
        for (int k = 1; k < kRowIds; k++) w = (bi >> 6) == k ? ids[k] : w;
        bid = __builtin_amdgcn_readlane(w, bi & 63);
    } else {
        bid = row[bi];
    }
    if (bid < 0 || bid >= a.num_blocks) return;
    const int r = (T - 1) & 15;
    const int64_t tile = (static_cast<int64_t>(bid) * a.num_kv_heads + kvh) * 16 * D;
    uint16_t* kc = static_cast<uint16_t*>(const_cast<void*>(a.k_cache)) + tile;
    uint16_t* vc = static_cast<uint16_t*>(const_cast<void*>(a.v_cache)) + tile;
#pragma unroll
    for (int e = 0; e < NPL; e++) {
        const int d = lane + 64 * e;
        if (d < D) {
            __builtin_nontemporal_store(pa::bf16_trunc(__uint_as_float(kraw[e])), kc + r * D + d);
            __builtin_nontemporal_store(pa::bf16_trunc(__uint_as_float(vraw[e])), vc + d * 16 + r);
        }
    }
}
template <int D>
__device__ __forceinline__ void append_token_bf16(const DecodeArgs& a, int seq, int kvh) {
    if (a.q_bf16) append_token_bf16_as<D, false>(a, seq, kvh);
    else append_token_bf16_as<D, true>(a, seq, kvh);
}

// Final write of one (sequence, query head, dim): normalised output, or the partition's partial.
__device__ __forceinline__ void emit(const DecodeArgs& a, int seq, int h, int part, int nparts, int D,
                                     int d, float o, float m, float l) {
    const int64_t row = static_cast<int64_t>(seq) * a.num_kv_heads * a.group + h;
    if (nparts == 1) {
        a.out[row * D + d] = o / l;
    } else {
        const int64_t pidx = row * a.max_parts + part;
        a.ws_o[pidx * D + d] = o;
        if (d == 0) {
            a.ws_m[pidx] = m;
            a.ws_l[pidx] = l;
        }
    }
}

// ================================================================================================
// bf16 / int8 caches: MFMA kernel.
// ================================================================================================
template <int KV> struct MfmaRaw;
template <> struct MfmaRaw<PA_DTYPE_BF16> {
    using K = uint4;  // 8 bf16 of one token row (A operand of the 16x16x32 MFMA)
    using V = uint2;  // 4 bf16: 4 consecutive tokens of one dim (B operand of the 16x16x16 MFMA)
    static constexpr int kElt = 2;
};
template <> struct MfmaRaw<PA_DTYPE_INT8> {
    using K = uint2;     // 8 int8 codes
    using V = uint32_t;  // 4 int8 codes
    static constexpr int kElt = 1;
};

// fp32 -> bf16 bits by truncation (the reference's conversion, BFloat16.cs:99-107).
// One v_perm_b32: bytes 3, 2 of hi over bytes 3, 2 of lo, i.e. (hi & 0xffff0000) | (lo >> 16).
__device__ __forceinline__ uint32_t pack_bf16_trunc(float lo, float hi) {
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// fp32 -> bf16 bits rounded to nearest even, two at a time (gfx950's v_cvt_pk_bf16_f32).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16_rne(float lo, float hi) {
    const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint32_t pack_i8pair(uint32_t w, int k) {
    // Codes k and k+1 of w as two bf16 (exact: |code| <= 128 needs 8 significant bits).
    return pack_bf16_trunc(pa::i8_at(w, k), pa::i8_at(w, k + 1));
}

// Reductions across the 4 rows of 16 lanes with gfx950's v_permlane16/32_swap (VALU, no LDS):
// each swap returns the pair {x[l], x[l ^ 16]} (resp. x[l ^ 32]) in some order.
__device__ __forceinline__ float rows_max(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows_sum(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Log-sum-exp merge of split partials. Partials [pbeg, pend) of head g merged into (M, L, o) (this lane's dims lane, lane + 64, ..):
// lane j loads partial j's (max, sum), 64 partials per round, the wave reduces them to the round's
// max and weighted sum, and the outputs are loaded UNROLL partials at a time, each weighted by the
// value its lane computed. An empty range leaves M = -inf, L = 0, o = 0.
template <int D, typename PidxOf>
__device__ __forceinline__ void merge_range(const DecodeArgs& a, int g, int pbeg, int pend, PidxOf pidx_of, float& M,
                                            float& L, float (&o)[(D + 63) / 64]) {
    constexpr int DPL = (D + 63) / 64;  // dims per lane (lanes past D hold none when D = 32)
    constexpr int UNROLL = 16;   // partials whose output loads are issued together
    const int lane = threadIdx.x & 63;
    M = -INFINITY;
    L = 0.0f;
#pragma unroll
    for (int k = 0; k < DPL; k++) o[k] = 0.0f;
    for (int p0 = pbeg; p0 < pend; p0 += 64) {
        const int cnt = min(64, pend - p0);
        const bool ok = lane < cnt;
        const int64_t pi = pidx_of(p0 + (ok ? lane : 0), g);
        const float pm = ok ? a.ws_m[pi] : -INFINITY;
        const float pl = ok ? a.ws_l[pi] : 0.0f;
        // Every load of a batch is issued before any is used; past cnt (uniform) nothing is
        // loaded and the weight read is lane 63's or beyond-cnt zero, times zero.
        float x[UNROLL][DPL];
        auto load_batch = [&](int u) {
#pragma unroll
            for (int j = 0; j < UNROLL; j++) {
                if (u + j < cnt) {
                    const int64_t pj = pidx_of(p0 + u + j, g);
#pragma unroll
                    for (int k = 0; k < DPL; k++) x[j][k] = lane + 64 * k < D ? a.ws_o[pj * D + lane + 64 * k] : 0.0f;
                } else {
#pragma unroll
                    for (int k = 0; k < DPL; k++) x[j][k] = 0.0f;
                }
            }
        };
        load_batch(0);  // needs the slot indices only: in flight with the (max, sum) loads
        const float cm = fmaxf(M, wave_max(pm));  // finite: every partial saw a token
        const float r = __expf(M - cm);           // rescale of earlier rounds (0 on the first)
        const float w = ok ? __expf(pm - cm) : 0.0f;
        L = L * r + wave_sum(pl * w);
#pragma unroll
        for (int k = 0; k < DPL; k++) o[k] *= r;
        for (int u = 0; u < cnt; u += UNROLL) {
            if (u > 0) load_batch(u);
#pragma unroll
            for (int j = 0; j < UNROLL; j++) {
                const float wj = readlane_f(w, min(u + j, 63));
#pragma unroll
                for (int k = 0; k < DPL; k++) o[k] += x[j][k] * wj;
            }
        }
        M = cm;
    }
}

// Merge of the nparts partials of (sequence, KV head): wave w takes heads w, w + 4, ... of the
// group. pidx_of(u, g) is the workspace row of partial u of head g of the group.
template <int D, typename PidxOf>
__device__ __forceinline__ void merge_partitions(const DecodeArgs& a, int seq, int kvh, int nparts, PidxOf pidx_of) {
    constexpr int DPL = (D + 63) / 64;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int G = a.group;
    for (int g = wave; g < G; g += 4) {
        const int64_t row = static_cast<int64_t>(seq) * a.num_kv_heads * G + kvh * G + g;
        float M, L, o[DPL];
        merge_range<D>(a, g, 0, nparts, pidx_of, M, L, o);
        const float inv = 1.0f / L;
#pragma unroll
        for (int k = 0; k < DPL; k++)
            if (lane + 64 * k < D) a.out[row * D + lane + 64 * k] = o[k] * inv;
    }
}

// Merge of the nparts partials of one head g of (sequence, KV head) by the 4 waves of the
// workgroup: wave w merges a quarter of the partials, and wave 0 combines the four states.
template <int D, typename PidxOf>
__device__ __forceinline__ void merge_head_wide(const DecodeArgs& a, int seq, int kvh, int g, int nparts,
                                                PidxOf pidx_of) {
    constexpr int DPL = (D + 63) / 64;
    __shared__ float s_m[4], s_l[4], s_o[4][DPL * 64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = (nparts + 3) / 4;
    float M, L, o[DPL];
    merge_range<D>(a, g, min(wave * q, nparts), min((wave + 1) * q, nparts), pidx_of, M, L, o);
    if (lane == 0) {
        s_m[wave] = M;
        s_l[wave] = L;
    }
#pragma unroll
    for (int k = 0; k < DPL; k++) s_o[wave][lane + 64 * k] = o[k];
    __syncthreads();
    if (wave != 0) return;
    float cm = s_m[0];  // finite: wave 0's quarter is never empty
    for (int w = 1; w < 4; w++) cm = fmaxf(cm, s_m[w]);
    float lt = 0.0f, ot[DPL];
#pragma unroll
    for (int k = 0; k < DPL; k++) ot[k] = 0.0f;
    for (int w = 0; w < 4; w++) {
        const float f = __expf(s_m[w] - cm);  // 0 for an empty quarter (-inf)
        lt += s_l[w] * f;
#pragma unroll
        for (int k = 0; k < DPL; k++) ot[k] += s_o[w][lane + 64 * k] * f;
    }
    const int64_t row = static_cast<int64_t>(seq) * a.num_kv_heads * a.group + kvh * a.group + g;
    const float inv = 1.0f / lt;
#pragma unroll
    for (int k = 0; k < DPL; k++)
        if (lane + 64 * k < D) a.out[row * D + lane + 64 * k] = ot[k] * inv;
}

// Merge pass: one workgroup per (KV head, sequence).
template <int D>
__global__ __launch_bounds__(256) void paged_decode_merge_kernel(const DecodeArgs a) {
    const int kvh = blockIdx.x, seq = blockIdx.y;
    const int T = clamp_len(a, a.context_lens[seq]);
    if (T <= 0) return;
    const int nparts = (T + a.part - 1) / a.part;
    if (nparts <= 1) return;
    merge_partitions<D>(a, seq, kvh, nparts, [&](int u, int g) {
        return (static_cast<int64_t>(seq) * a.num_kv_heads * a.group + kvh * a.group + g) * a.max_parts + u;
    });
}

// Range length (blocks) of the MFMA kernel's split of the `total` blocks of all sequences (one KV
// head's worth); the decode and the merge kernel derive the same value from the same arguments.
// By default the split_grid workers (waves) form split_grid / Hkv ranges of equal length, each
// range done by Hkv workers, one per KV head; a range holds at least 4 blocks.
__device__ __forceinline__ int64_t split_range_blocks(const DecodeArgs& a, int64_t total) {
    if (a.split_blocks > 0) return a.split_blocks;
    const int64_t nr = a.split_grid >= a.num_kv_heads ? a.split_grid / a.num_kv_heads : 1;
    const int64_t c = (total + nr - 1) / nr;
    return c < 4 ? 4 : c;
}

// Merge pass of the MFMA kernel: one workgroup per (KV head, sequence). Sequence seq occupies
// blocks [R0, R0 + nbr) of the sequence-major block list; its rows were split iff R0 and
// R0 + nbr - 1 fall in different ranges, and then ranges w1 .. w2 each left one partial per KV
// head, in unit u = w * Hkv + kvh: slot 2u, except range w1 when the sequence starts inside it (the
// row is then that unit's last row portion, slot 2u + 1).
// Launched with kMergeThreads threads, or kMergeThreads + 64 when it also writes the fused
// append's token (a.append_in_merge): that fifth wave only writes the token.
constexpr int kMergeThreads = 256;
template <int D>
__global__ __launch_bounds__(kMergeThreads + 64) void paged_decode_merge_split_kernel(const DecodeArgs a,
                                                                                      int32_t num_seqs) {
    const int kvh = blockIdx.x, seq = blockIdx.y;
    if (threadIdx.x >= kMergeThreads) {
        if (a.append_in_merge) append_token_bf16<D>(a, seq, kvh);
        return;
    }
    const int64_t R0 = a.ws_pref[seq];
    const int nbr = a.ws_pref[seq + 1] - a.ws_pref[seq];
    const int64_t total = a.ws_pref[num_seqs];
    if (nbr <= 0) return;
    // The prefix table comes from the decode launch through the workspace: one that does not fit
    // (the workspace overwritten in between) is not followed outside the slots.
    if (R0 < 0 || R0 + nbr > total) return;
    const int Hkv = a.num_kv_heads;
    const int G = a.group;
    if (a.num_splits > 0) {
        // Per-sequence split: partitions k < ceil(nbr / c) of c = ceil(nbr / P) blocks, the partial
        // of partition k in slot 2 ((seq P + k) Hkv + kvh).
        const int P = a.num_splits;
        const int c = (nbr + P - 1) / P;
        const int np = (nbr + c - 1) / c;
        if (np <= 1) return;  // written whole by the decode kernel
        if ((static_cast<int64_t>(seq) * P + np) * Hkv > a.max_units) return;
        merge_partitions<D>(a, seq, kvh, np, [&](int u, int g) {
            return (2 * ((static_cast<int64_t>(seq) * P + u) * Hkv + kvh)) * G + g;
        });
        return;
    }
    const int64_t C = split_range_blocks(a, total);
    const int64_t w1 = R0 / C, w2 = (R0 + nbr - 1) / C;
    if (w1 == w2) return;  // written whole by the decode kernel
    if ((w2 + 1) * Hkv > a.max_units) return;  // slots the workspace does not have
    const bool starts_inside = R0 != w1 * C;
    merge_partitions<D>(a, seq, kvh, static_cast<int>(w2 - w1 + 1), [&](int u, int g) {
        const int64_t unit = (w1 + u) * Hkv + kvh;
        return (2 * unit + (u == 0 && starts_inside ? 1 : 0)) * G + g;
    });
}

// Shared-prefix decode merge: one workgroup per (KV head, sequence, query head of the group), its
// 4 waves sharing the head's partials (a sequence's partials are many here). Rows of the decode's list
// are the num_groups prefix rows, then one suffix row per sequence (its blocks after the shared
// ones); every row's partials sit in 16-wide slots (slot 2u + {0, 1} of unit u, as above, or the
// row's own slot row_slot_base + r * Hkv + kvh when the row lies inside one range). A
// sequence in a group combines its suffix row's partials with those of its group's prefix row
// (columns mi * G .. mi * G + G - 1, mi its place in the group); an ungrouped sequence whose row
// was written whole by the decode is skipped.
template <int D>
__global__ __launch_bounds__(256) void paged_decode_merge_prefix_kernel(const DecodeArgs a, int32_t num_seqs) {
    const int kvh = blockIdx.x, seq = blockIdx.y;
    const int NG = a.num_groups;
    const int Hkv = a.num_kv_heads, G = a.group;
    const int32_t* groups = a.plan;
    const int32_t* seqinfo = a.plan + static_cast<int64_t>(NG) * kPlanGroupInts;
    const int row = NG + seq;
    // Independent loads first (a test between them would serialise their round trips).
    const int raw_len = a.context_lens[seq];
    int grp = seqinfo[static_cast<int64_t>(seq) * kPlanSeqInts];
    const int64_t total = a.ws_pref[NG + num_seqs];
    const int64_t R0 = a.ws_pref[row];
    const int64_t R1 = a.ws_pref[row + 1];
    if (clamp_len(a, raw_len) <= 0) return;  // zero output, written by the decode
    if (grp >= NG) grp = -1;
    const int64_t C = split_range_blocks(a, total);
    const int nbr = static_cast<int>(R1 - R0);
    if (R0 < 0 || nbr < 0 || R1 > total) return;  // a prefix table that does not fit the slots
    int ns = 0;
    int64_t w1 = 0;
    bool s_inside = false;
    if (nbr > 0) {
        w1 = R0 / C;
        ns = static_cast<int>((R0 + nbr - 1) / C - w1 + 1);
        s_inside = R0 != w1 * C;
    }
    int np = 0, mi = 0;
    int64_t pw1 = 0;
    bool p_inside = false;
    if (grp >= 0) {
        const int64_t P0 = a.ws_pref[grp];
        const int pn = a.ws_pref[grp + 1] - a.ws_pref[grp];
        if (P0 < 0 || pn < 0 || P0 + pn > total) return;
        mi = seq - groups[static_cast<int64_t>(grp) * kPlanGroupInts];
        if (mi < 0 || (mi + 1) * G > kPrefixSlotRows) return;  // not a member: a plan that does not fit
        if (pn > 0) {
            pw1 = P0 / C;
            np = static_cast<int>((P0 + pn - 1) / C - pw1 + 1);
            p_inside = P0 != pw1 * C;
        }
    }
    if (grp < 0 && ns <= 1) return;  // written whole by the decode kernel
    if (ns + np == 0) return;
    // Unit slots the workspace does not have (a prefix table that does not fit the call). Row slots
    // are bounded by the host-checked group count.
    if (ns > 1 && (w1 + ns) * Hkv > a.max_units) return;
    if (np > 1 && (pw1 + np) * Hkv > a.max_units) return;
    // A row inside one range left its partial in its row slot, a split row one per range.
    merge_head_wide<D>(a, seq, kvh, static_cast<int>(blockIdx.z), ns + np, [&](int u, int g) -> int64_t {
        if (u < ns) {
            if (ns == 1) return (a.row_slot_base + static_cast<int64_t>(row) * Hkv + kvh) * kPrefixSlotRows + g;
            const int64_t unit = (w1 + u) * Hkv + kvh;
            return (2 * unit + (u == 0 && s_inside ? 1 : 0)) * kPrefixSlotRows + g;
        }
        u -= ns;
        if (np == 1)
            return (a.row_slot_base + static_cast<int64_t>(grp) * Hkv + kvh) * kPrefixSlotRows + mi * G + g;
        const int64_t unit = (pw1 + u) * Hkv + kvh;
        return (2 * unit + (u == 0 && p_inside ? 1 : 0)) * kPrefixSlotRows + mi * G + g;
    });
}

__device__ __forceinline__ bf16x8_t k_operand(const uint4& r) { return __builtin_bit_cast(bf16x8_t, r); }
__device__ __forceinline__ bf16x8_t k_operand(const uint2& r) {
    const uint4 p = make_uint4(pack_i8pair(r.x, 0), pack_i8pair(r.x, 2), pack_i8pair(r.y, 0), pack_i8pair(r.y, 2));
    return __builtin_bit_cast(bf16x8_t, p);
}
__device__ __forceinline__ s16x4_t v_operand(const uint2& r) { return __builtin_bit_cast(s16x4_t, r); }
__device__ __forceinline__ s16x4_t v_operand(const uint32_t& r) {
    const uint2 p = make_uint2(pack_i8pair(r, 0), pack_i8pair(r, 2));
    return __builtin_bit_cast(s16x4_t, p);
}

// First of the 8 consecutive dims of K slab sl (32 dims of one QK MFMA) that lane group q4 feeds
// in the decode kernel. The dot product does not depend on which dims go to which MFMA k slot as
// long as K and Q agree, so the choice is made for the loads:
//  - bf16: slab sl, lane group q4 -> dims 32 sl + 8 q4 (bytes 64 sl + 16 q4 of the row): one K
//    load instruction reads 64 contiguous bytes of each of 16 rows (timed equal to a contiguous
//    quarter of the dims per lane group, whose pieces land on both lines of each row);
//  - int8: a contiguous quarter of the dims per lane group, so a lane's piece of a K row is two
//    16-byte loads instead of four 8-byte ones (each instruction still covers 16 lines).
template <int D, int KV>
__device__ __forceinline__ int k_dim0(int sl, int q4) {
    return KV == PA_DTYPE_INT8 ? (D / 4) * q4 + 8 * sl : 32 * sl + 8 * q4;
}


// Word 3 of a raw buffer descriptor on gfx9 (32-bit data format, no swizzle).
constexpr int kBufferFlags = 0x00020000;

// CP: the load's cache-policy operand; kLoadNonTemporal marks data that is not read again soon.
// Measured on the decode's K/V stream (us per step): int8 caches, K and V non-temporal, C4 136.0
// -> 125.8; bf16 caches, V only: C2 over two pools 67.3 -> 58.6, C5 128.2 -> 123.9, C5 through
// the shared-prefix decode 113.2 -> 99.5 (K and V: 61.9, 131.6, 108.8; K only: 63.2, 124.9).
constexpr int kLoadDefault = 0;
constexpr int kLoadNonTemporal = 2;
template <typename T, int CP = kLoadDefault> __device__ __forceinline__ T buffer_load(__amdgpu_buffer_rsrc_t r, int off) {
    if constexpr (sizeof(T) == 16) {
        return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CP));
    } else if constexpr (sizeof(T) == 8) {
        return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, CP));
    } else {
        static_assert(sizeof(T) == 4, "16-, 8- or 4-byte loads");
        return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, CP));
    }
}

// 16 bytes per lane from a buffer into LDS: lane l's bytes land at LDS address lds + 16 l
// (buffer_load_dwordx4 with the LDS bit; M0 holds the LDS address, and one wait state must
// separate the M0 write from the load; M0 is restored afterwards). A zero-sized descriptor
// writes zeros. Written as inline asm so that the compiler, which does not see these LDS
// writes, adds no wait on them before its own LDS reads: the kernel orders them itself (vmcnt
// wait + barrier per step). The LDS address is an operand and the asm clobbers memory, so the
// compiler treats the array as written by it.
using u32x4_t = uint32_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void lds_load16(u32x4_t rsrc, uint32_t voffset, uint32_t lds) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
        "buffer_load_dwordx4 %2, %1, 0 offen lds\n\ts_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(rsrc), "v"(voffset), "s"(lds)
        : "memory");
}
__device__ __forceinline__ u32x4_t buffer_rsrc_words(const void* base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    return u32x4_t{static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32) & 0xffffu, bytes,
                   static_cast<uint32_t>(kBufferFlags)};
}
__device__ __forceinline__ uint32_t lds_address(const void* p) {
    using lds_char = const __attribute__((address_space(3))) char;
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_char*)p));  // generic -> LDS offset
}

// ---- launchers (one translation unit per kernel family) ----------------------------------------
constexpr int kMaxPersistentSeqs = 2048;  // per-sequence tables of the persistent kernel (LDS)
constexpr int kMaxDecodeWorkers = 4096;   // workers (waves) of one MFMA decode launch, at most
// Workers (waves) per MFMA decode workgroup. Waves sharing a SIMD do not progress evenly (the older
// one runs ahead and finishes first) but the chip's bandwidth stays in use either way; one 8-wave
// workgroup per CU instead of two 4-wave ones measured slower.
__host__ __device__ constexpr int decode_waves(int) { return 4; }
int device_cus();
// bf16 / int8 caches; num_seqs < kMaxPersistentSeqs. Launches the resident workgroups, each of
// decode_waves(D) independent workers, with no more than kMaxDecodeWorkers and max_units workers
// in all; records the worker count in a.split_grid (the merge kernel needs it).
// shared: the shared-prefix decode (a.plan, a.num_groups; no append), whose row list is the
// num_groups prefix rows and then one suffix row per sequence.
template <int D>
void launch_decode_mfma(DecodeArgs& a, int kv_dtype, bool q_f32, bool append, bool shared, int num_seqs,
                        int64_t max_grid, hipStream_t s);
extern template void launch_decode_mfma<32>(DecodeArgs&, int, bool, bool, bool, int, int64_t, hipStream_t);
extern template void launch_decode_mfma<64>(DecodeArgs&, int, bool, bool, bool, int, int64_t, hipStream_t);
extern template void launch_decode_mfma<128>(DecodeArgs&, int, bool, bool, bool, int, int64_t, hipStream_t);
extern template void launch_decode_mfma<256>(DecodeArgs&, int, bool, bool, bool, int, int64_t, hipStream_t);
// fp32 caches: grid (max_parts, Hkv, num_seqs); returns false for an uncompiled shape.
bool launch_decode_fp32(const DecodeArgs& a, int head_dim, dim3 grid, hipStream_t s);

}  // namespace pa
