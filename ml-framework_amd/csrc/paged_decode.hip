// paged_decode.hip -- ragged paged decode for gfx950 (wave64).
//
// Replaces the reference's per-sequence decode loop (DecodeOrchestrator.BatchDecode /
// ComputeDecodeAttention, src/MLFramework/Inference/PagedAttention/Phases/DecodeOrchestrator.cs:64-109,
// which gathers each sequence's K/V and calls StandardPagedAttentionKernel once per sequence,
// Kernels/StandardPagedAttentionKernel.cs:21-84) with one launch over the whole ragged batch.
//
// Work decomposition: one workgroup (4 waves) per (partition, KV head, sequence). A partition is a
// run of `part` tokens (whole 16-token blocks) of one sequence. A sequence that fits in one
// partition is finished in place; longer ones write per-partition (max, sum, unnormalised output)
// to the workspace and paged_decode_merge_kernel combines them with a log-sum-exp reduction.
// The G = Hq / Hkv query heads of a KV head share every K/V byte loaded (GQA).
//
// bf16 / int8 caches (paged_decode_mfma_kernel): each wave streams its blocks (every 4th block of
// the partition) with a one-block prefetch. Per block, S^T[16 tokens][16 heads] = K . Q^T runs on
// v_mfma_f32_16x16x32_bf16 (query heads padded to 16 rows) and O[16 heads][D] += P . V on
// v_mfma_f32_16x16x16_bf16 with P split into bf16 high and low parts, so the probabilities keep
// ~16 bits. The score layout the first MFMA leaves in registers (lane = (token group, head)) is
// exactly the A-operand layout of the second, so P never leaves registers. Softmax is online per
// wave in fp32; the four waves are combined through LDS at the end.
// fp32 caches (paged_decode_fp32_kernel): VALU dot products reduced across lanes with DPP, a
// partition-wide softmax in LDS, and VALU P.V.
#include <string>
#include <type_traits>

#include "pa_internal.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

struct DecodeArgs {
    float* out;
    const void* q;
    const void* k_cache;
    const void* v_cache;
    const float* k_scale;
    const float* v_scale;
    const int32_t* block_tables;
    const int32_t* context_lens;
    float* ws_o;  // [num_seqs][Hq][max_parts][D]
    float* ws_m;  // [num_seqs][Hq][max_parts]
    float* ws_l;  // [num_seqs][Hq][max_parts]
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
    int32_t part;  // partition length in tokens (multiple of 64)
    int32_t q_bf16;
    float scale;
};

__device__ __forceinline__ int clamp_len(const DecodeArgs& a, int seq) {
    int T = a.context_lens[seq];
    T = min(T, a.max_blocks_per_seq * pa::kBlockSize);
    T = min(T, a.max_context_len);
    return T;
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
__device__ __forceinline__ uint32_t pack_bf16_trunc(float lo, float hi) {
    return (__float_as_uint(hi) & 0xffff0000u) | (__float_as_uint(lo) >> 16);
}

__device__ __forceinline__ uint32_t pack_i8pair(uint32_t w, int k) {
    // Codes k and k+1 of w as two bf16 (exact: |code| <= 128 needs 8 significant bits).
    return pack_bf16_trunc(pa::i8_at(w, k), pa::i8_at(w, k + 1));
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Log-sum-exp merge of the partitions of one (sequence, KV head): wave w takes query heads
// w, w + 4, ... Partition statistics are read 64 at a time (one per lane); the weighted sum over
// partitions issues its loads in groups of 8 so their latencies overlap.
template <int D>
__device__ __forceinline__ void merge_partitions(const DecodeArgs& a, int seq, int kvh, int nparts) {
    constexpr int DPL = D / 64;  // dims per lane
    constexpr int CHUNK = 16;    // partitions whose loads are issued together
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int G = a.group;
    for (int g = wave; g < G; g += 4) {
        const int64_t row = static_cast<int64_t>(seq) * a.num_kv_heads * G + kvh * G + g;
        const int64_t base = row * a.max_parts;
        float M = -INFINITY, L = 0.0f;
        float o[DPL];
#pragma unroll
        for (int k = 0; k < DPL; k++) o[k] = 0.0f;
        // Running log-sum-exp over chunks of partitions; within a chunk every load (m, l and the
        // partial outputs) is issued before any is used.
        for (int p0 = 0; p0 < nparts; p0 += CHUNK) {
            const int cnt = min(CHUNK, nparts - p0);
            float pm[CHUNK], pl[CHUNK], po[CHUNK][DPL];
#pragma unroll
            for (int u = 0; u < CHUNK; u++) {
                const bool ok = u < cnt;
                const int64_t pi = base + p0 + (ok ? u : 0);
                pm[u] = ok ? a.ws_m[pi] : -INFINITY;
                pl[u] = ok ? a.ws_l[pi] : 0.0f;
#pragma unroll
                for (int k = 0; k < DPL; k++) po[u][k] = ok ? a.ws_o[pi * D + lane + 64 * k] : 0.0f;
            }
            float cm = M;
#pragma unroll
            for (int u = 0; u < CHUNK; u++) cm = fmaxf(cm, pm[u]);
            const float r = __expf(M - cm);  // rescale of what was accumulated (0 on the first chunk)
            L *= r;
#pragma unroll
            for (int k = 0; k < DPL; k++) o[k] *= r;
#pragma unroll
            for (int u = 0; u < CHUNK; u++) {
                const float w = __expf(pm[u] - cm);
                L += pl[u] * w;
#pragma unroll
                for (int k = 0; k < DPL; k++) o[k] += po[u][k] * w;
            }
            M = cm;
        }
        const float inv = 1.0f / L;
#pragma unroll
        for (int k = 0; k < DPL; k++) a.out[row * D + lane + 64 * k] = o[k] * inv;
    }
}

// Separate merge pass (fp32 caches): one workgroup per (KV head, sequence).
template <int D>
__global__ __launch_bounds__(256) void paged_decode_merge_kernel(const DecodeArgs a) {
    const int kvh = blockIdx.x, seq = blockIdx.y;
    const int T = clamp_len(a, seq);
    if (T <= 0) return;
    const int nparts = (T + a.part - 1) / a.part;
    if (nparts <= 1) return;
    merge_partitions<D>(a, seq, kvh, nparts);
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

// ---- fused append: the new token (row r of the sequence's last block) enters the owning wave's
// registers and the cache. Values and cache bytes are those of pa_kv_append for that one token.
__device__ __forceinline__ float act_at(const void* p, bool f32, int64_t i) {
    return f32 ? static_cast<const float*>(p)[i] : pa::bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}

template <int D, bool QF32>
__device__ __forceinline__ void append_bf16_regs(const DecodeArgs& a, int64_t tile, int64_t src, int r, int q4,
                                                 int n, uint4 (&kr)[D / 32], uint2 (&vr)[D / 16]) {
    constexpr int NSLAB = D / 32, NT = D / 16;
    uint16_t* kc = static_cast<uint16_t*>(const_cast<void*>(a.k_cache));
    uint16_t* vc = static_cast<uint16_t*>(const_cast<void*>(a.v_cache));
    if (n == r) {  // K row r: dims 32s + 8q4 .. +8 of this lane
#pragma unroll
        for (int sl = 0; sl < NSLAB; sl++) {
            const int d0 = 32 * sl + 8 * q4;
            uint4 v;
            if constexpr (QF32) {
                const float* x = static_cast<const float*>(a.k_new) + src + d0;
                v = make_uint4(pack_bf16_trunc(x[0], x[1]), pack_bf16_trunc(x[2], x[3]),
                               pack_bf16_trunc(x[4], x[5]), pack_bf16_trunc(x[6], x[7]));
            } else {
                v = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.k_new) + src + d0);
            }
            kr[sl] = v;
            *reinterpret_cast<uint4*>(kc + tile + r * D + d0) = v;
        }
    }
    if (q4 == (r >> 2)) {  // V column r: element r & 3 of this lane's 4-token run, dims 16t + n
        const int e = r & 3;
        const uint32_t sh = (e & 1) * 16;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int d = 16 * t + n;
            uint32_t b;
            if constexpr (QF32) b = __float_as_uint(static_cast<const float*>(a.v_new)[src + d]) >> 16;
            else b = static_cast<const uint16_t*>(a.v_new)[src + d];
            const uint32_t mask = ~(0xffffu << sh);
            if (e < 2) vr[t].x = (vr[t].x & mask) | (b << sh);
            else vr[t].y = (vr[t].y & mask) | (b << sh);
            vc[tile + d * 16 + r] = static_cast<uint16_t>(b);
        }
    }
}

__device__ __forceinline__ int code_at(uint32_t w, int k) { return static_cast<int32_t>(w << (24 - 8 * k)) >> 24; }
__device__ __forceinline__ uint32_t with_code(uint32_t w, int k, int8_t c) {
    return (w & ~(0xffu << (8 * k))) | (static_cast<uint32_t>(static_cast<uint8_t>(c)) << (8 * k));
}

// int8: the owning wave holds the whole (block, head) tile in registers (K: 8 codes per lane per
// 32-dim slab, V: 4 codes per lane per 16-dim tile), so the scale growth and requantisation of
// pa_kv_append run in place. Returns the tile's K and V scales after the append.
template <int D, bool QF32>
__device__ __forceinline__ void append_int8_regs(const DecodeArgs& a, int64_t tile, int64_t src, int64_t sidx,
                                                 int r, int q4, int n, uint2 (&kr)[D / 32], uint32_t (&vr)[D / 16],
                                                 float& k_scale_out, float& v_scale_out) {
#pragma clang fp contract(off)
    constexpr int NSLAB = D / 32, NT = D / 16;
    int8_t* kc = static_cast<int8_t*>(const_cast<void*>(a.k_cache));
    int8_t* vc = static_cast<int8_t*>(const_cast<void*>(a.v_cache));
    float* kscale = const_cast<float*>(a.k_scale);
    float* vscale = const_cast<float*>(a.v_scale);
    const bool fresh = r == 0;  // writing row 0 starts the block afresh
    const int lane = threadIdx.x & 63;
    // ---------------- K ----------------
    {
        float x[NSLAB][8];
        float amax = 0.0f;
#pragma unroll
        for (int sl = 0; sl < NSLAB; sl++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                x[sl][e] = n == r ? act_at(a.k_new, QF32, src + 32 * sl + 8 * q4 + e) : 0.0f;
                const float ax = fabsf(x[sl][e]);
                amax = ax > amax ? ax : amax;
            }
        amax = pa::wave_max(amax);
        const float old_amax = fresh ? 0.0f : a.k_absmax[sidx];
        const float old_scale = fresh ? 0.0f : kscale[sidx];
        const bool grow = !fresh && amax > old_amax;
        const float sc = (fresh || grow) ? amax / 127.0f : old_scale;
#pragma unroll
        for (int sl = 0; sl < NSLAB; sl++) {
            uint32_t w[2] = {kr[sl].x, kr[sl].y};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                int8_t c;
                if (n == r) c = pa::quantize_symmetric(x[sl][e], sc);
                else if (grow) c = pa::quantize_symmetric(static_cast<float>(code_at(w[e >> 2], e & 3)) * old_scale, sc);
                else c = static_cast<int8_t>(code_at(w[e >> 2], e & 3));
                w[e >> 2] = with_code(w[e >> 2], e & 3, c);
            }
            kr[sl] = make_uint2(w[0], w[1]);
            if (grow || n == r) *reinterpret_cast<uint2*>(kc + tile + n * D + 32 * sl + 8 * q4) = kr[sl];
        }
        if (lane == 0 && (fresh || grow)) {
            a.k_absmax[sidx] = amax;
            kscale[sidx] = sc;
        }
        k_scale_out = sc;
    }
    // ---------------- V (tile is [D][16]: lane holds tokens 4q4..4q4+3 of dim 16t+n) ----------------
    {
        const bool mine = q4 == (r >> 2);
        const int er = r & 3;
        float x[NT];
        float amax = 0.0f;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            x[t] = mine ? act_at(a.v_new, QF32, src + 16 * t + n) : 0.0f;
            const float ax = fabsf(x[t]);
            amax = ax > amax ? ax : amax;
        }
        amax = pa::wave_max(amax);
        const float old_amax = fresh ? 0.0f : a.v_absmax[sidx];
        const float old_scale = fresh ? 0.0f : vscale[sidx];
        const bool grow = !fresh && amax > old_amax;
        const float sc = (fresh || grow) ? amax / 127.0f : old_scale;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            uint32_t w = vr[t];
            int8_t newc = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const bool is_new = mine && e == er;
                int8_t c;
                if (is_new) c = newc = pa::quantize_symmetric(x[t], sc);
                else if (grow) c = pa::quantize_symmetric(static_cast<float>(code_at(w, e)) * old_scale, sc);
                else c = static_cast<int8_t>(code_at(w, e));
                w = with_code(w, e, c);
            }
            vr[t] = w;
            int8_t* dst = vc + tile + (16 * t + n) * 16;
            if (grow) *reinterpret_cast<uint32_t*>(dst + 4 * q4) = w;
            else if (mine) dst[r] = newc;
        }
        if (lane == 0 && (fresh || grow)) {
            a.v_absmax[sidx] = amax;
            vscale[sidx] = sc;
        }
        v_scale_out = sc;
    }
}

// Online-softmax rescaling is deferred until a block's max exceeds the running max by more than
// this (natural-log units): probabilities then stay below e^8 and fp32 sums stay exact enough,
// while the O accumulators are rescaled on few blocks instead of on most of them.
constexpr float kRescaleThreshold = 8.0f;
constexpr int kMaxPersistentSeqs = 4096;  // sequence-prefix table held in LDS

struct MfmaShared {
    float m[4][16];
    float l[4][16];
    int pref[kMaxPersistentSeqs + 1];  // items before sequence s (persistent mode)
};

// One work item: (sequence, KV head, partition). Called by all 256 threads of a workgroup.
template <int D, int KV, bool QF32, bool APPEND>
__device__ __forceinline__ void mfma_item(const DecodeArgs& a, int seq, int kvh, int part, MfmaShared& sh,
                                          float (*s_x)[D][16]) {
    using Raw = MfmaRaw<KV>;
    constexpr int ELT = Raw::kElt;
    constexpr int NSLAB = D / 32;  // QK MFMAs (k = 32 dims each)
    constexpr int NT = D / 16;     // PV n-tiles of 16 dims
    constexpr int TILE = 16 * D;   // elements per (block, KV head) tile

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q4 = lane >> 4;  // token group (QK C rows) / k group of the MFMA operands
    const int n = lane & 15;   // head column of S^T / row of P / dim within a PV tile
    const int G = a.group, Hkv = a.num_kv_heads;

    const int T = clamp_len(a, seq);
    const int tok0 = part * a.part;
    if (T <= 0) {
        if (part == 0)
            for (int idx = tid; idx < G * D; idx += 256)
                a.out[(static_cast<int64_t>(seq) * Hkv * G + kvh * G) * D + idx] = 0.0f;
        return;
    }
    if (tok0 >= T) return;
    const int tok_end = min(T, tok0 + a.part);
    const int nparts = (T + a.part - 1) / a.part;

    // This wave's blocks: lb0 + wave + 4j, j < nb. Lane j holds block j's id (and int8 scales).
    const int lb0 = tok0 / 16;
    // Fused append: the last block of the sequence belongs to wave (rel & 3), iteration rel >> 2.
    int j_app = -1;
    if constexpr (APPEND) {
        const int rel = (T - 1) / 16 - lb0;
        if (part == nparts - 1 && (rel & 3) == wave) j_app = rel >> 2;
    }
    const int nblk = (tok_end - tok0 + 15) / 16;
    const int nb = nblk > wave ? (nblk - wave + 3) / 4 : 0;
    const int32_t* table = a.block_tables + static_cast<int64_t>(seq) * a.max_blocks_per_seq;
    int my_bid = -1;
    float my_ks = 0.0f, my_vs = 0.0f;
    if (lane < nb) {
        my_bid = table[lb0 + wave + 4 * lane];
        if (my_bid >= a.num_blocks) my_bid = -1;
        if constexpr (KV == PA_DTYPE_INT8) {
            if (my_bid >= 0) {
                my_ks = a.k_scale[static_cast<int64_t>(my_bid) * Hkv + kvh];
                my_vs = a.v_scale[static_cast<int64_t>(my_bid) * Hkv + kvh];
            }
        }
    }

    // Q^T operand: lane (q4, n) holds head n, dims 32s + 8q4 .. +8 (zero rows for n >= G).
    bf16x8_t qhi[NSLAB], qlo[QF32 ? NSLAB : 1];
    {
        const bool hv = n < G;
        const int64_t qrow = (static_cast<int64_t>(seq) * Hkv * G + kvh * G + (hv ? n : 0)) * D;
#pragma unroll
        for (int s = 0; s < NSLAB; s++) {
            const int d0 = 32 * s + 8 * q4;
            if constexpr (QF32) {
                const float* qp = static_cast<const float*>(a.q) + qrow + d0;
                float x[8];
#pragma unroll
                for (int e = 0; e < 8; e++) x[e] = hv ? qp[e] : 0.0f;
                uint32_t h[4], l[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    h[e] = pack_bf16_trunc(x[2 * e], x[2 * e + 1]);
                    const float r0 = x[2 * e] - __uint_as_float(__float_as_uint(x[2 * e]) & 0xffff0000u);
                    const float r1 = x[2 * e + 1] - __uint_as_float(__float_as_uint(x[2 * e + 1]) & 0xffff0000u);
                    l[e] = pack_bf16_trunc(r0, r1);
                }
                qhi[s] = __builtin_bit_cast(bf16x8_t, make_uint4(h[0], h[1], h[2], h[3]));
                qlo[s] = __builtin_bit_cast(bf16x8_t, make_uint4(l[0], l[1], l[2], l[3]));
            } else {
                const uint4 raw = hv ? *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.q) + qrow + d0)
                                     : make_uint4(0, 0, 0, 0);
                qhi[s] = __builtin_bit_cast(bf16x8_t, raw);
            }
        }
    }

    const char* kc = static_cast<const char*>(a.k_cache);
    const char* vc = static_cast<const char*>(a.v_cache);
    using KR = typename Raw::K;
    using VR = typename Raw::V;
    auto load = [&](KR (&kr)[NSLAB], VR (&vr)[NT], int j) {
        const int bid = __builtin_amdgcn_readlane(my_bid, j);
        if (bid >= 0) {
            const int64_t tile = (static_cast<int64_t>(bid) * Hkv + kvh) * TILE;
            const char* kt = kc + (tile + n * D + 8 * q4) * ELT;
            const char* vt = vc + (tile + n * 16 + 4 * q4) * ELT;
#pragma unroll
            for (int s = 0; s < NSLAB; s++) kr[s] = *reinterpret_cast<const KR*>(kt + 32 * s * ELT);
#pragma unroll
            for (int t = 0; t < NT; t++) vr[t] = *reinterpret_cast<const VR*>(vt + 256 * t * ELT);
        } else {
#pragma unroll
            for (int s = 0; s < NSLAB; s++) kr[s] = KR{};
#pragma unroll
            for (int t = 0; t < NT; t++) vr[t] = VR{};
        }
    };

    float m_run = -INFINITY;  // reference max of head n (exceeded by at most kRescaleThreshold)
    float l_run = 0.0f;       // this lane's share of the running sum of head n
    f32x4_t acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    auto compute = [&](KR (&kr)[NSLAB], VR (&vr)[NT], int j) {
        float ks = 1.0f, vfac = 1.0f;
        if constexpr (KV == PA_DTYPE_INT8) {
            ks = readlane_f(my_ks, j);
            vfac = readlane_f(my_vs, j);
        }
        if constexpr (APPEND) {
            const int bid = __builtin_amdgcn_readlane(my_bid, j);
            if (j == j_app && bid >= 0) {
                const int64_t tile = (static_cast<int64_t>(bid) * Hkv + kvh) * TILE;
                const int64_t src = (static_cast<int64_t>(seq) * Hkv + kvh) * D;
                const int r = (T - 1) & 15;
                if constexpr (KV == PA_DTYPE_INT8)
                    append_int8_regs<D, QF32>(a, tile, src, static_cast<int64_t>(bid) * Hkv + kvh, r, q4, n, kr, vr,
                                              ks, vfac);
                else
                    append_bf16_regs<D, QF32>(a, tile, src, r, q4, n, kr, vr);
            }
        }
        // S^T[token 4q4+i][head n]
        f32x4_t s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int sl = 0; sl < NSLAB; sl++) {
            const bf16x8_t kop = k_operand(kr[sl]);
            s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qhi[sl], s, 0, 0, 0);
            if constexpr (QF32) s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qlo[sl], s, 0, 0, 0);
        }
        const int tbase = (lb0 + wave + 4 * j) * 16 + 4 * q4;
        float sc[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float v = s[i];
            if constexpr (KV == PA_DTYPE_INT8) v = v * ks;  // (q . code) * k_scale, then * scale
            v = v * a.scale;
            sc[i] = tbase + i < T ? v : -INFINITY;
        }
        float bm = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
        bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
        bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
        const bool grow = bm > m_run + kRescaleThreshold;
        if (__any(grow)) {
            const float m_new = grow ? bm : m_run;
            const float alpha = __expf(m_run - m_new);  // 1 where the max did not move, 0 from -inf
            l_run *= alpha;
            m_run = m_new;
            float ar[4];
#pragma unroll
            for (int i = 0; i < 4; i++) ar[i] = __shfl(alpha, 4 * q4 + i, 64);
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[t][i] *= ar[i];
        }
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            p[i] = __expf(sc[i] - m_run);
            l_run += p[i];
            if constexpr (KV == PA_DTYPE_INT8) p[i] *= vfac;
        }
        uint32_t hi[2], lo[2];
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const float a0 = p[2 * e], a1 = p[2 * e + 1];
            const float h0 = __uint_as_float(__float_as_uint(a0) & 0xffff0000u);
            const float h1 = __uint_as_float(__float_as_uint(a1) & 0xffff0000u);
            hi[e] = pack_bf16_trunc(a0, a1);
            lo[e] = pack_bf16_trunc(a0 - h0, a1 - h1);
        }
        const s16x4_t phi = __builtin_bit_cast(s16x4_t, make_uint2(hi[0], hi[1]));
        const s16x4_t plo = __builtin_bit_cast(s16x4_t, make_uint2(lo[0], lo[1]));
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const s16x4_t vop = v_operand(vr[t]);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(phi, vop, acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(plo, vop, acc[t], 0, 0, 0);
        }
    };

    {
        // Three rotating register buffers: two blocks in flight while a third is consumed.
        KR ka[NSLAB], kb[NSLAB], kx[NSLAB];
        VR va[NT], vb[NT], vx[NT];
        int j = 0;
        if (nb > 0) load(ka, va, 0);
        if (nb > 1) load(kb, vb, 1);
        while (j < nb) {
            if (j + 2 < nb) load(kx, vx, j + 2);
            compute(ka, va, j);
            if (++j >= nb) break;
            if (j + 2 < nb) load(ka, va, j + 2);
            compute(kb, vb, j);
            if (++j >= nb) break;
            if (j + 2 < nb) load(kb, vb, j + 2);
            compute(kx, vx, j);
            ++j;
        }
    }

    // ---- combine the 4 waves: weights exp(m_w - M) per head, then a 2-level tree in LDS ----
    float l_tot = l_run + __shfl_xor(l_run, 16, 64);
    l_tot += __shfl_xor(l_tot, 32, 64);
    if (q4 == 0) {
        sh.m[wave][n] = m_run;
        sh.l[wave][n] = l_tot;
    }
    __syncthreads();
    float M[4], f_own[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int h = 4 * q4 + i;
        M[i] = fmaxf(fmaxf(sh.m[0][h], sh.m[1][h]), fmaxf(sh.m[2][h], sh.m[3][h]));
        f_own[i] = __expf(sh.m[wave][h] - M[i]);  // 0 for a wave that saw no block
    }
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[t][i] *= f_own[i];
    // acc[t] holds rows 4q4..4q4+3 of dim 16t+n: one 16-byte LDS store in the [dim][row] layout.
    if (wave >= 2) {
#pragma unroll
        for (int t = 0; t < NT; t++) *reinterpret_cast<f32x4_t*>(&s_x[wave - 2][16 * t + n][4 * q4]) = acc[t];
    }
    __syncthreads();
    if (wave < 2) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            f32x4_t* slot = reinterpret_cast<f32x4_t*>(&s_x[wave][16 * t + n][4 * q4]);
            acc[t] += *slot;
            if (wave == 1) *slot = acc[t];
        }
    }
    __syncthreads();
    if (wave == 0) {
        float L[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int h = 4 * q4 + i;
            L[i] = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; w++) L[i] += sh.l[w][h] * __expf(sh.m[w][h] - M[i]);
        }
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const f32x4_t other = *reinterpret_cast<const f32x4_t*>(&s_x[1][16 * t + n][4 * q4]);
            acc[t] += other;
        }
        if (4 * q4 < G) {
            const int64_t row0 = static_cast<int64_t>(seq) * Hkv * G + kvh * G;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int h = 4 * q4 + i;
                if (h >= G) break;
                const int64_t row = row0 + h;
                if (nparts == 1) {
                    const float inv = 1.0f / L[i];
#pragma unroll
                    for (int t = 0; t < NT; t++) a.out[row * D + 16 * t + n] = acc[t][i] * inv;
                } else {
                    const int64_t pidx = row * a.max_parts + part;
#pragma unroll
                    for (int t = 0; t < NT; t++) a.ws_o[pidx * D + 16 * t + n] = acc[t][i];
                    if (n == 0) {
                        a.ws_m[pidx] = M[i];
                        a.ws_l[pidx] = L[i];
                    }
                }
            }
        }
    }
    __syncthreads();  // LDS reuse by the next item
}

// Grid mode: one workgroup per (partition, KV head, sequence).
template <int D, int KV, bool QF32, bool APPEND>
__global__ __launch_bounds__(256, 2) void paged_decode_mfma_kernel(const DecodeArgs a) {
    __shared__ MfmaShared sh;
    __shared__ float s_x[2][D][16];
    mfma_item<D, KV, QF32, APPEND>(a, blockIdx.z, blockIdx.y, blockIdx.x, sh, s_x);
}

// Persistent mode: gridDim.x workgroups walk the compacted list of non-empty items
// (sequence s owns items pref[s]*Hkv .. pref[s+1]*Hkv - 1, KV head fastest), item w, w + grid, ...
// Every workgroup leaves its loop after a bounded number of items.
template <int D, int KV, bool QF32, bool APPEND>
__global__ __launch_bounds__(256, 2) void paged_decode_mfma_persistent_kernel(const DecodeArgs a, int32_t num_seqs) {
    __shared__ MfmaShared sh;
    __shared__ float s_x[2][D][16];
    const int tid = threadIdx.x;
    // Items per sequence: its partition count (a zero-length sequence still gets one item, which
    // writes its zero output). Exclusive prefix over sequences, built by the whole workgroup.
    constexpr int PER = (kMaxPersistentSeqs + 255) / 256;
    int cnt[PER];
    int local = 0;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int s = tid * PER + k;
        int c = 0;
        if (s < num_seqs) {
            const int T = clamp_len(a, s);
            c = T <= 0 ? 1 : (T + a.part - 1) / a.part;
        }
        cnt[k] = c;
        local += c;
    }
    // block-wide exclusive scan of `local`
    const int lane = tid & 63, wave = tid >> 6;
    int incl = local;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(incl, o, 64);
        if (lane >= o) incl += v;
    }
    if (lane == 63) sh.pref[wave] = incl;  // wave totals (scratch, overwritten below)
    __syncthreads();
    int wave_off = 0;
    for (int w = 0; w < wave; w++) wave_off += sh.pref[w];
    const int total_parts = sh.pref[0] + sh.pref[1] + sh.pref[2] + sh.pref[3];
    __syncthreads();
    int run = wave_off + incl - local;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int s = tid * PER + k;
        if (s <= num_seqs) sh.pref[s] = run;
        run += cnt[k];
    }
    __syncthreads();

    const int Hkv = a.num_kv_heads;
    const int64_t total = static_cast<int64_t>(total_parts) * Hkv;
    int seq = 0;
    for (int64_t item = blockIdx.x; item < total; item += gridDim.x) {
        const int pi = static_cast<int>(item / Hkv);
        const int kvh = static_cast<int>(item - static_cast<int64_t>(pi) * Hkv);
        // Items only increase, so the owning sequence is found by scanning forward.
        while (seq + 1 < num_seqs && sh.pref[seq + 1] <= pi) seq++;
        mfma_item<D, KV, QF32, APPEND>(a, seq, kvh, pi - sh.pref[seq], sh, s_x);
    }
}

// ================================================================================================
// fp32 caches: VALU kernel.
// ================================================================================================
template <int D, int G, int PART>
__global__ __launch_bounds__(256) void paged_decode_fp32_kernel(const DecodeArgs a) {
    constexpr int CH = D / 4;      // 16-byte chunks per K row
    constexpr int TPI = 64 / CH;   // K rows per wave load instruction
    constexpr int LPB = 16 / TPI;  // K load instructions per block per lane
    constexpr int RPL = D / 16;    // V dim rows per lane per block (lane = (dim row, 4-token chunk))
    constexpr int NBW = PART / 64; // blocks per wave
    constexpr int TPT = PART / 256;
    constexpr int TILE = 16 * D;
    static_assert(CH >= 16 && CH <= 64, "fp32 kernel covers head_dim 64..256");

    __shared__ float s_logits[G][PART];
    __shared__ float s_red[4][G];
    __shared__ float s_o[4][G][D];

    const int part = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int Hkv = a.num_kv_heads, Hq = Hkv * G;

    const int T = clamp_len(a, seq);
    const int tok0 = part * PART;
    if (T <= 0) {
        if (part == 0)
            for (int idx = tid; idx < G * D; idx += 256)
                a.out[(static_cast<int64_t>(seq) * Hq + kvh * G) * D + idx] = 0.0f;
        return;
    }
    if (tok0 >= T) return;
    const int ntok = min(PART, T - tok0);
    const int nparts = (T + PART - 1) / PART;
    const int ti = lane / CH, ch = lane % CH;

    float qf[G][4];
    {
        const int64_t qb = (static_cast<int64_t>(seq) * Hq + kvh * G) * D + ch * 4;
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                qf[g][e] = a.q_bf16 ? pa::bf16_to_f32(static_cast<const uint16_t*>(a.q)[qb + g * D + e])
                                    : static_cast<const float*>(a.q)[qb + g * D + e];
    }

    const int32_t* table = a.block_tables + static_cast<int64_t>(seq) * a.max_blocks_per_seq;
    const int lb0 = tok0 / 16;
    int bid[NBW];
#pragma unroll
    for (int i = 0; i < NBW; i++) {
        const int lb = lb0 + i * 4 + wave;
        int id = -1;
        if ((lb - lb0) * 16 < ntok) {
            id = table[lb];
            if (id >= a.num_blocks) id = -1;
        }
        bid[i] = __builtin_amdgcn_readfirstlane(id);
    }
    const float* kc = static_cast<const float*>(a.k_cache);
    const float* vc = static_cast<const float*>(a.v_cache);
    auto kload = [&](int b, int j) -> uint4 {
        if (b < 0) return make_uint4(0, 0, 0, 0);
        return *reinterpret_cast<const uint4*>(kc + (static_cast<int64_t>(b) * Hkv + kvh) * TILE +
                                               (j * TPI + ti) * D + ch * 4);
    };

    // ---- scores ----
#pragma unroll
    for (int i = 0; i < NBW; i++) {
        uint4 kr[LPB];
#pragma unroll
        for (int j = 0; j < LPB; j++) kr[j] = kload(bid[i], j);
#pragma unroll
        for (int j = 0; j < LPB; j++) {
            const float kf[4] = {__uint_as_float(kr[j].x), __uint_as_float(kr[j].y), __uint_as_float(kr[j].z),
                                 __uint_as_float(kr[j].w)};
            float dot[G];
#pragma unroll
            for (int g = 0; g < G; g++) {
                float acc = 0.0f;
#pragma unroll
                for (int e = 0; e < 4; e++) acc += qf[g][e] * kf[e];
                dot[g] = pa::group_sum<CH>(acc);
            }
            const int lt = (i * 4 + wave) * 16 + j * TPI + ti;
            if (ch == 0)
#pragma unroll
                for (int g = 0; g < G; g++) s_logits[g][lt] = lt < ntok ? dot[g] * a.scale : -INFINITY;
        }
    }
    __syncthreads();

    // ---- partition softmax ----
    float m[G], l[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        float mx = -INFINITY;
#pragma unroll
        for (int k = 0; k < TPT; k++) mx = fmaxf(mx, s_logits[g][tid + 256 * k]);
        mx = pa::wave_max(mx);
        if (lane == 0) s_red[wave][g] = mx;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; g++) m[g] = fmaxf(fmaxf(s_red[0][g], s_red[1][g]), fmaxf(s_red[2][g], s_red[3][g]));
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; g++) {
        float sum = 0.0f;
#pragma unroll
        for (int k = 0; k < TPT; k++) {
            const float p = __expf(s_logits[g][tid + 256 * k] - m[g]);
            s_logits[g][tid + 256 * k] = p;
            sum += p;
        }
        sum = pa::wave_sum(sum);
        if (lane == 0) s_red[wave][g] = sum;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; g++) l[g] = (s_red[0][g] + s_red[1][g]) + (s_red[2][g] + s_red[3][g]);

    // ---- o = sum_t p_t v_t; V tile is [D][16]: lane = (dim row vd + 16 r, tokens 4vc..4vc+3) ----
    const int vc4 = lane & 3, vd = lane >> 2;
    float acc[G][RPL];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int r = 0; r < RPL; r++) acc[g][r] = 0.0f;
#pragma unroll
    for (int i = 0; i < NBW; i++) {
        if (bid[i] < 0) continue;  // zero values contribute nothing
        const float* vt = vc + (static_cast<int64_t>(bid[i]) * Hkv + kvh) * TILE + vd * 16 + 4 * vc4;
        uint4 vr[RPL];
#pragma unroll
        for (int r = 0; r < RPL; r++) vr[r] = *reinterpret_cast<const uint4*>(vt + r * 256);
        const int lt = (i * 4 + wave) * 16 + 4 * vc4;
        float4 p[G];
#pragma unroll
        for (int g = 0; g < G; g++) p[g] = *reinterpret_cast<const float4*>(&s_logits[g][lt]);
#pragma unroll
        for (int r = 0; r < RPL; r++) {
            const float v0 = __uint_as_float(vr[r].x), v1 = __uint_as_float(vr[r].y);
            const float v2 = __uint_as_float(vr[r].z), v3 = __uint_as_float(vr[r].w);
#pragma unroll
            for (int g = 0; g < G; g++) acc[g][r] += p[g].x * v0 + p[g].y * v1 + p[g].z * v2 + p[g].w * v3;
        }
    }
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int r = 0; r < RPL; r++) acc[g][r] = pa::group_sum<4>(acc[g][r]);
    if (vc4 == 0)
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int r = 0; r < RPL; r++) s_o[wave][g][vd + 16 * r] = acc[g][r];
    __syncthreads();

    for (int idx = tid; idx < G * D; idx += 256) {
        const int g = idx / D, d = idx - g * D;
        const float o = (s_o[0][g][d] + s_o[1][g][d]) + (s_o[2][g][d] + s_o[3][g][d]);
        emit(a, seq, kvh * G + g, part, nparts, D, d, o, m[g], l[g]);
    }
}

// ================================================================================================
// ---- host side ---------------------------------------------------------------------------------
constexpr int kMaxPart = 4096;  // a wave's block ids must fit one VGPR (64 lanes x 4 waves x 16)

// Partition length for this call. fp32 caches use 256 or 512 (VALU kernel templates); bf16/int8
// take any multiple of 64 up to 4096, defaulting to about 1/16 of the longest context (at least
// 256), which keeps the partial count per sequence at or under 16.
int resolve_part(const pa_config* cfg, int32_t max_len, std::string* err) {
    const int req = cfg->partition_size;
    if (cfg->kv_dtype == PA_DTYPE_FP32) {
        if (req == 0) return 256;
        if (req == 256 || req == 512) return req;
        *err = "partition_size must be 0, 256 or 512 for an fp32 cache";
        return -1;
    }
    if (req == 0) {
        int p = (max_len + 15) / 16;
        p = (p + 255) / 256 * 256;
        return p < 256 ? 256 : (p > kMaxPart ? kMaxPart : p);
    }
    if (req < 64 || req > kMaxPart || req % 64 != 0) {
        *err = "partition_size must be a multiple of 64 in [64, 4096]";
        return -1;
    }
    return req;
}

// Workspace: [o fp32 rows*D][m fp32 rows][l fp32 rows] with rows = num_seqs * Hq * max_parts.
size_t workspace_bytes_for(const pa_config* cfg, int32_t num_seqs, int32_t max_len, int part) {
    const int64_t max_parts = (static_cast<int64_t>(max_len) + part - 1) / part;
    if (max_parts <= 1 || num_seqs <= 0) return 0;
    const int64_t rows = static_cast<int64_t>(num_seqs) * cfg->num_q_heads * max_parts;
    return static_cast<size_t>(rows) * (cfg->head_dim + 2) * sizeof(float);
}

int32_t effective_max_len(int32_t max_context_len, int32_t max_blocks_per_seq) {
    // Tokens beyond the table are never read, so the grid only needs to cover what the table holds.
    const int64_t table_tokens = static_cast<int64_t>(max_blocks_per_seq) * pa::kBlockSize;
    return max_context_len > table_tokens ? static_cast<int32_t>(table_tokens) : max_context_len;
}

// Resident workgroups per CU of a kernel, and CUs of the current device (queried once each;
// read-only afterwards).
template <typename K>
int resident_wgs(K kernel) {
    static int cached = [&] {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, 256, 0) != hipSuccess || n < 1) n = 1;
        return n;
    }();
    return cached;
}

int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

template <int D, int KV, bool QF32, bool APPEND>
void launch_mfma(const DecodeArgs& a, dim3 grid, int num_seqs, hipStream_t s) {
    if (num_seqs < kMaxPersistentSeqs) {
        auto kern = paged_decode_mfma_persistent_kernel<D, KV, QF32, APPEND>;
        const int64_t upper = static_cast<int64_t>(grid.x) * grid.y * grid.z;
        int64_t nwg = static_cast<int64_t>(device_cus()) * resident_wgs(kern);
        if (nwg > upper) nwg = upper;
        if (nwg < 1) nwg = 1;
        kern<<<static_cast<unsigned>(nwg), 256, 0, s>>>(a, num_seqs);
    } else {
        paged_decode_mfma_kernel<D, KV, QF32, APPEND><<<grid, 256, 0, s>>>(a);
    }
}

// fp32 caches, fused entry point: append the token at position context_len - 1 of every
// sequence (one workgroup per sequence, K row and V column of every KV head), before the decode.
__global__ __launch_bounds__(256) void append_last_token_fp32_kernel(const DecodeArgs a, int32_t head_dim) {
    const int seq = blockIdx.x;
    const int T = clamp_len(a, seq);
    if (T <= 0) return;
    const int bid = a.block_tables[static_cast<int64_t>(seq) * a.max_blocks_per_seq + (T - 1) / 16];
    if (bid < 0 || bid >= a.num_blocks) return;
    const int r = (T - 1) & 15;
    const int Hkv = a.num_kv_heads, n = Hkv * head_dim;
    float* kc = static_cast<float*>(const_cast<void*>(a.k_cache));
    float* vc = static_cast<float*>(const_cast<void*>(a.v_cache));
    const bool f32 = !a.q_bf16;
    for (int idx = threadIdx.x; idx < n; idx += blockDim.x) {
        const int h = idx / head_dim, d = idx - h * head_dim;
        const int64_t src = static_cast<int64_t>(seq) * n + idx;
        const int64_t tile = (static_cast<int64_t>(bid) * Hkv + h) * 16 * head_dim;
        kc[tile + r * head_dim + d] = act_at(a.k_new, f32, src);
        vc[tile + d * 16 + r] = act_at(a.v_new, f32, src);
    }
}

template <int D, int G>
void launch_fp32(const DecodeArgs& a, dim3 grid, hipStream_t s) {
    if (a.part == 512) paged_decode_fp32_kernel<D, G, 512><<<grid, 256, 0, s>>>(a);
    else paged_decode_fp32_kernel<D, G, 256><<<grid, 256, 0, s>>>(a);
}

template <int D, bool APPEND>
bool launch_decode(const pa_config* cfg, const DecodeArgs& a, dim3 grid, hipStream_t s) {
    if (cfg->kv_dtype == PA_DTYPE_FP32) {
        if (APPEND) append_last_token_fp32_kernel<<<grid.z, 256, 0, s>>>(a, D);
        switch (a.group) {
            case 1: launch_fp32<D, 1>(a, grid, s); return true;
            case 2: launch_fp32<D, 2>(a, grid, s); return true;
            case 4: launch_fp32<D, 4>(a, grid, s); return true;
            case 8: launch_fp32<D, 8>(a, grid, s); return true;
            default: return false;
        }
    }
    const bool qf32 = cfg->q_dtype == PA_DTYPE_FP32;
    const int num_seqs = static_cast<int>(grid.z);
    if (cfg->kv_dtype == PA_DTYPE_BF16) {
        if (qf32) launch_mfma<D, PA_DTYPE_BF16, true, APPEND>(a, grid, num_seqs, s);
        else launch_mfma<D, PA_DTYPE_BF16, false, APPEND>(a, grid, num_seqs, s);
    } else {
        if (qf32) launch_mfma<D, PA_DTYPE_INT8, true, APPEND>(a, grid, num_seqs, s);
        else launch_mfma<D, PA_DTYPE_INT8, false, APPEND>(a, grid, num_seqs, s);
    }
    return true;
}

}  // namespace

extern "C" {

pa_status pa_decode_workspace_size(const pa_config* cfg, int32_t num_seqs, int32_t max_context_len,
                                   size_t* bytes) {
    pa_status st = pa::check_config(cfg, "pa_decode_workspace_size");
    if (st != PA_SUCCESS) return st;
    if (!bytes) return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_decode_workspace_size: bytes is null");
    if (num_seqs < 0 || max_context_len < 0)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_decode_workspace_size: negative size");
    std::string err;
    const int part = resolve_part(cfg, max_context_len, &err);
    if (part < 0) return pa::set_error(PA_ERROR_UNSUPPORTED, "pa_decode_workspace_size: " + err);
    *bytes = workspace_bytes_for(cfg, num_seqs, max_context_len, part);
    return pa::clear_error();
}

}  // extern "C"

namespace {

pa_status decode_impl(const char* fn, bool append, pa_stream* stream, const pa_config* cfg, float* out,
                      const void* q, const void* k_new, const void* v_new, const void* k_cache,
                      const void* v_cache, const float* k_scale, const float* v_scale, float* k_absmax,
                      float* v_absmax, const int32_t* block_tables, const int32_t* context_lens,
                      int32_t num_seqs, int32_t max_blocks_per_seq, int32_t max_context_len, void* workspace,
                      size_t workspace_bytes) {
    const std::string f(fn);
    pa_status st = pa::check_config(cfg, fn);
    if (st != PA_SUCCESS) return st;
    if (num_seqs < 0 || max_blocks_per_seq < 0 || max_context_len < 0)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, f + ": negative size");
    if (num_seqs == 0) return pa::clear_error();
    if (num_seqs > 65535) return pa::set_error(PA_ERROR_UNSUPPORTED, f + ": num_seqs > 65535");
    if (!out || !q || !k_cache || !v_cache || !block_tables || !context_lens)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, f + ": null pointer");
    if (append && (!k_new || !v_new)) return pa::set_error(PA_ERROR_INVALID_ARGUMENT, f + ": null k_new/v_new");
    if (cfg->kv_dtype == PA_DTYPE_INT8 && (!k_scale || !v_scale))
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, f + ": int8 cache needs k_scale and v_scale");
    if (append && cfg->kv_dtype == PA_DTYPE_INT8 && (!k_absmax || !v_absmax))
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, f + ": int8 append needs k_absmax and v_absmax");
    const int G = cfg->num_q_heads / cfg->num_kv_heads;
    const bool g_ok = cfg->kv_dtype == PA_DTYPE_FP32 ? (G == 1 || G == 2 || G == 4 || G == 8)
                                                     : (G == 1 || G == 2 || G == 4 || G == 8 || G == 16);
    if (!g_ok) return pa::set_error(PA_ERROR_UNSUPPORTED, f + ": unsupported Hq / Hkv ratio");
    if (cfg->num_kv_heads > 65535) return pa::set_error(PA_ERROR_UNSUPPORTED, f + ": too many KV heads");

    const int32_t max_len = effective_max_len(max_context_len, max_blocks_per_seq);
    std::string err;
    // The partition length is resolved from the caller's max_context_len, exactly as
    // pa_decode_workspace_size does, so both agree on the workspace layout.
    const int part = resolve_part(cfg, max_context_len, &err);
    if (part < 0) return pa::set_error(PA_ERROR_UNSUPPORTED, f + ": " + err);
    const int32_t max_parts = max_len > 0 ? (max_len + part - 1) / part : 1;
    const size_t need = workspace_bytes_for(cfg, num_seqs, max_len, part);
    if (need > 0 && (!workspace || workspace_bytes < need))
        return pa::set_error(PA_ERROR_WORKSPACE_TOO_SMALL,
                             f + ": workspace of " + std::to_string(need) + " bytes required");

    DecodeArgs a{};
    a.out = out;
    a.q = q;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.k_scale = k_scale;
    a.v_scale = v_scale;
    a.block_tables = block_tables;
    a.context_lens = context_lens;
    a.k_new = k_new;
    a.v_new = v_new;
    a.k_absmax = k_absmax;
    a.v_absmax = v_absmax;
    a.num_kv_heads = cfg->num_kv_heads;
    a.group = G;
    a.max_blocks_per_seq = max_blocks_per_seq;
    a.num_blocks = cfg->num_blocks;
    a.max_context_len = max_len;
    a.max_parts = max_parts;
    a.part = part;
    a.q_bf16 = cfg->q_dtype == PA_DTYPE_BF16;
    a.scale = pa::resolve_scale(cfg);
    if (need > 0) {
        const int64_t rows = static_cast<int64_t>(num_seqs) * cfg->num_q_heads * max_parts;
        a.ws_o = static_cast<float*>(workspace);
        a.ws_m = a.ws_o + rows * cfg->head_dim;
        a.ws_l = a.ws_m + rows;
    }

    hipStream_t s = pa::native(stream);
    dim3 grid(max_parts, cfg->num_kv_heads, num_seqs);
    bool ok = false;
    switch (cfg->head_dim) {
        case 64: ok = append ? launch_decode<64, true>(cfg, a, grid, s) : launch_decode<64, false>(cfg, a, grid, s); break;
        case 128: ok = append ? launch_decode<128, true>(cfg, a, grid, s) : launch_decode<128, false>(cfg, a, grid, s); break;
        case 256: ok = append ? launch_decode<256, true>(cfg, a, grid, s) : launch_decode<256, false>(cfg, a, grid, s); break;
    }
    if (!ok) return pa::set_error(PA_ERROR_UNSUPPORTED, f + ": configuration not compiled");
    PA_HIP_CHECK(hipGetLastError());
    if (max_parts > 1) {
        dim3 mgrid(cfg->num_kv_heads, num_seqs);
        switch (cfg->head_dim) {
            case 64: paged_decode_merge_kernel<64><<<mgrid, 256, 0, s>>>(a); break;
            case 128: paged_decode_merge_kernel<128><<<mgrid, 256, 0, s>>>(a); break;
            default: paged_decode_merge_kernel<256><<<mgrid, 256, 0, s>>>(a); break;
        }
        PA_HIP_CHECK(hipGetLastError());
    }
    return pa::clear_error();
}

}  // namespace

extern "C" {

pa_status pa_paged_decode(pa_stream* stream, const pa_config* cfg, float* out, const void* q,
                          const void* k_cache, const void* v_cache, const float* k_scale,
                          const float* v_scale, const int32_t* block_tables, const int32_t* context_lens,
                          int32_t num_seqs, int32_t max_blocks_per_seq, int32_t max_context_len,
                          void* workspace, size_t workspace_bytes) {
    return decode_impl("pa_paged_decode", false, stream, cfg, out, q, nullptr, nullptr, k_cache, v_cache, k_scale,
                       v_scale, nullptr, nullptr, block_tables, context_lens, num_seqs, max_blocks_per_seq,
                       max_context_len, workspace, workspace_bytes);
}

pa_status pa_paged_decode_append(pa_stream* stream, const pa_config* cfg, float* out, const void* q,
                                 const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                                 float* k_scale, float* v_scale, float* k_absmax, float* v_absmax,
                                 const int32_t* block_tables, const int32_t* context_lens, int32_t num_seqs,
                                 int32_t max_blocks_per_seq, int32_t max_context_len, void* workspace,
                                 size_t workspace_bytes) {
    return decode_impl("pa_paged_decode_append", true, stream, cfg, out, q, k_new, v_new, k_cache, v_cache,
                       k_scale, v_scale, k_absmax, v_absmax, block_tables, context_lens, num_seqs,
                       max_blocks_per_seq, max_context_len, workspace, workspace_bytes);
}

}  // extern "C"
