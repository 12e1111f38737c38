// chunked_prefill_fp32.hip -- chunked prefill over an fp32 paged cache, fp32 throughout.
//
// The same operation as the bf16 / int8 chunked prefill (queries at positions prefix_lens[s] + i
// over keys [0, prefix_lens[s] + chunk_len) of the block table, the reference's
// StandardPagedAttentionKernel, Kernels/StandardPagedAttentionKernel.cs:21-84, with the mask of
// :57-66 / :219-255), for caches that hold fp32: K tile [16][D], V tile [D][16] per
// (block, KV head). It serves callers that hand over fp32 activations and expect fp32 results,
// such as the dense ComputePagedAttention(query, cachedKeys, cachedValues, phase) of the
// reference's IPagedAttentionKernel (Kernels/IPagedAttentionKernel.cs:13-28) with more than one
// query: one launch in which a key block is read once per 64 queries instead of once per query.
//
// Work decomposition: a unit is one 16-query tile of one query head; a workgroup of 4 waves takes
// 4 consecutive units of one (sequence, KV head) -- for G > 1 the heads of the group first, so
// waves that read the same key blocks share a CU -- and the workgroups of one (sequence, KV head)
// run on one XCD, the ones with the most keys first. Each wave streams its key blocks from
// memory into registers (16-byte loads, the next block's issued before the current block's
// MFMAs) and computes, per block, on v_mfma_f32_16x16x4_f32 (fp32 operands, fp32 accumulation):
//   S^T[16 keys][16 queries] = K . Q^T, with head dim d = (lane / 16) * D / 4 + c on MFMA c, so a
//     lane's K and Q operands are D / 4 consecutive floats of one row;
//   online softmax per query in fp32 (log2 domain: the scale times log2(e) folded into Q);
//   O^T[D][16 queries] += V^T . P^T, where MFMA s of an output tile takes keys 4 (lane / 16) + s:
//     the lane's own four S^T values are its P operands, its V operand is one 16-byte read of
//     the [D][16] V tile, and all of the lane's accumulators belong to its own query, so the
//     rescale by the running maximum needs no exchange between lanes.
#include <string>

#include "pa_internal.h"

namespace pa {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kF32Waves = 4;
constexpr int kF32Threads = 64 * kF32Waves;

struct PrefillF32Args {
    float* out;
    const void* q;
    const float* k_cache;
    const float* v_cache;
    const int32_t* q_start_loc;
    const int32_t* prefix_lens;
    const int32_t* block_tables;
    int32_t num_kv_heads;
    int32_t group;
    int32_t max_blocks_per_seq;
    int32_t num_blocks;
    int32_t mask_mode;  // 0 causal, 1 causal only when the prefix is non-empty, 2 no mask
    float scale;
    int32_t wg_per_group;  // workgroups per (sequence, KV head)
    int32_t num_groups;    // num_seqs * num_kv_heads
    int32_t q_bf16;
};

// One key block's operands for this lane: its quarter of K row (lane % 16) and, per 16-dim
// output tile t, V^T rows 16 t + lane % 16 at keys 4 (lane / 16) .. +3. An invalid block id reads
// as zeros (the oracle's gather does the same).
template <int D>
struct BlockOps {
    f32x4 k[D / 16];
    f32x4 v[D / 16];
};

template <int D>
__device__ __forceinline__ void load_block(BlockOps<D>& o, const PrefillF32Args& a, const int32_t* table, int b,
                                           int kvh, int lane) {
    const int bid = table[b];
    if (bid < 0 || bid >= a.num_blocks) {
#pragma unroll
        for (int t = 0; t < D / 16; t++) {
            o.k[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            o.v[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        return;
    }
    const int64_t tile = (static_cast<int64_t>(bid) * a.num_kv_heads + kvh) * (16 * D);
    const f32x4* kp = reinterpret_cast<const f32x4*>(a.k_cache + tile + (lane & 15) * D + (lane >> 4) * (D / 4));
    const f32x4* vp = reinterpret_cast<const f32x4*>(a.v_cache + tile + (lane & 15) * 16 + (lane >> 4) * 4);
#pragma unroll
    for (int t = 0; t < D / 16; t++) {
        o.k[t] = kp[t];
        o.v[t] = vp[t * 64];  // 16 dims of 16 floats further
    }
}

template <int D>
__global__ __launch_bounds__(kF32Threads) void chunked_prefill_fp32_kernel(const PrefillF32Args a) {
    constexpr int NC = D / 4;   // MFMAs of the QK product (4 dims each)
    constexpr int NT = D / 16;  // 16-dim output tiles
    const int lid = blockIdx.x;
    const int wk = lid >> 3;
    const int m = wk / a.wg_per_group;
    const int qg = a.wg_per_group - 1 - (wk - m * a.wg_per_group);
    const int gi = (lid & 7) + 8 * m;
    if (gi >= a.num_groups) return;
    const int seq = gi / a.num_kv_heads, kvh = gi - seq * a.num_kv_heads;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int G = a.group, Hq = a.num_kv_heads * G;
    const int u = qg * kF32Waves + wave;
    const int qt = u / G, hq = kvh * G + (u - qt * G);

    const int q0 = a.q_start_loc[seq];
    const int Lc = a.q_start_loc[seq + 1] - q0;
    const int i0 = qt * 16;
    if (i0 >= Lc) return;
    const int P = max(a.prefix_lens[seq], 0);
    const int T = min(P + Lc, a.max_blocks_per_seq * 16);
    const bool causal = a.mask_mode == 0 || (a.mask_mode == 1 && P > 0);
    const int n = lane & 15, q4 = lane >> 4;
    const int qi = i0 + n;  // this lane's query (tile rows past the chunk are computed, not stored)
    const int kend = causal ? min(T, P + min(i0 + 16, Lc)) : T;
    const int qlim = causal ? min(T, P + qi + 1) : T;
    const int nkb = (kend + 15) / 16;

    // Q operand: dims (lane / 16) * D / 4 .. + D / 4 of query qi, times scale * log2(e).
    const float c2 = a.scale * 1.4426950408889634f;
    float qv[NC];
    {
        const int64_t row = (static_cast<int64_t>(q0) + min(qi, Lc - 1)) * Hq + hq;
        const int64_t base = row * D + q4 * NC;
        if (a.q_bf16) {
            const uint16_t* qp = static_cast<const uint16_t*>(a.q) + base;
#pragma unroll
            for (int c = 0; c < NC; c++) qv[c] = bf16_to_f32(qp[c]) * c2;
        } else {
            const f32x4* qp = reinterpret_cast<const f32x4*>(static_cast<const float*>(a.q) + base);
#pragma unroll
            for (int c4 = 0; c4 < NC / 4; c4++) {
                const f32x4 x = qp[c4];
#pragma unroll
                for (int e = 0; e < 4; e++) qv[4 * c4 + e] = x[e] * c2;
            }
        }
    }

    const int32_t* table = a.block_tables + static_cast<int64_t>(seq) * a.max_blocks_per_seq;
    f32x4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -INFINITY, l_run = 0.0f;

    BlockOps<D> cur;
    load_block<D>(cur, a, table, 0, kvh, lane);
    for (int b = 0; b < nkb; b++) {
        BlockOps<D> nxt;
        if (b + 1 < nkb) load_block<D>(nxt, a, table, b + 1, kvh, lane);
        // S^T = K . Q^T
        f32x4 s = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < NC; c++)
            s = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.k[c >> 2][c & 3], qv[c], s, 0, 0, 0);
        // lane holds keys 16 b + 4 q4 + i of query qi
        const int key0 = 16 * b + 4 * q4;
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (key0 + i >= qlim) s[i] = -INFINITY;
        float mb = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        mb = fmaxf(mb, __shfl_xor(mb, 16, 64));
        mb = fmaxf(mb, __shfl_xor(mb, 32, 64));
        const float m_new = fmaxf(m_run, mb);
        // key 0 is visible to every query, so m_new is finite from the first block on
        const float alpha = exp2f(m_run - m_new);
        m_run = m_new;
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; i++) p[i] = exp2f(s[i] - m_new);
        l_run = l_run * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
#pragma unroll
        for (int t = 0; t < NT; t++) acc[t] *= alpha;
        // O^T += V^T . P^T: MFMA (t, i) takes keys 4 q4 + i of the block
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.v[t][i], p[i], acc[t], 0, 0, 0);
        if (b + 1 < nkb) cur = nxt;
    }
    // lanes n, n + 16, n + 32, n + 48 hold partial sums of query n over their keys
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    if (qi >= Lc) return;
    const float inv = 1.0f / l_run;
    float* op = a.out + ((static_cast<int64_t>(q0) + qi) * Hq + hq) * D + 4 * q4;
#pragma unroll
    for (int t = 0; t < NT; t++) *reinterpret_cast<f32x4*>(op + 16 * t) = acc[t] * inv;
}

}  // namespace

pa_status launch_chunked_prefill_fp32(hipStream_t s, const pa_config* cfg, float* out, const void* q,
                                      const int32_t* q_start_loc, const int32_t* prefix_lens, const float* k_cache,
                                      const float* v_cache, const int32_t* block_tables, int32_t num_seqs,
                                      int32_t max_blocks_per_seq, int32_t max_chunk_len, int32_t mask_mode) {
    PrefillF32Args a{};
    a.out = out;
    a.q = q;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.q_start_loc = q_start_loc;
    a.prefix_lens = prefix_lens;
    a.block_tables = block_tables;
    a.num_kv_heads = cfg->num_kv_heads;
    a.group = cfg->num_q_heads / cfg->num_kv_heads;
    a.max_blocks_per_seq = max_blocks_per_seq;
    a.num_blocks = cfg->num_blocks;
    a.mask_mode = mask_mode;
    a.scale = resolve_scale(cfg);
    a.q_bf16 = cfg->q_dtype == PA_DTYPE_BF16;
    const int64_t units = static_cast<int64_t>(a.group) * ((max_chunk_len + 15) / 16);
    const int64_t wpg = (units + kF32Waves - 1) / kF32Waves;
    const int64_t ng = static_cast<int64_t>(num_seqs) * cfg->num_kv_heads;
    const int64_t nwg = wpg * ((ng + 7) / 8) * 8;
    if (nwg > 0x7fffffff) return set_error(PA_ERROR_UNSUPPORTED, "pa_chunked_prefill: grid too large");
    a.wg_per_group = static_cast<int32_t>(wpg);
    a.num_groups = static_cast<int32_t>(ng);
    const dim3 grid(static_cast<uint32_t>(nwg));
    switch (cfg->head_dim) {
        case 32: chunked_prefill_fp32_kernel<32><<<grid, kF32Threads, 0, s>>>(a); break;
        case 64: chunked_prefill_fp32_kernel<64><<<grid, kF32Threads, 0, s>>>(a); break;
        case 128: chunked_prefill_fp32_kernel<128><<<grid, kF32Threads, 0, s>>>(a); break;
        default: chunked_prefill_fp32_kernel<256><<<grid, kF32Threads, 0, s>>>(a); break;
    }
    PA_HIP_CHECK(hipGetLastError());
    return clear_error();
}

}  // namespace pa
