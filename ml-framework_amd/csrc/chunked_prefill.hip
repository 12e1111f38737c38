// chunked_prefill.hip -- chunked prefill over the paged cache on gfx950 MFMA.
//
// Computes, for each prefill sequence s, attention of its chunk's queries (positions
// prefix_lens[s] + i) over keys [0, prefix_lens[s] + chunk_len) read through the block table --
// the reference's StandardPagedAttentionKernel (Kernels/StandardPagedAttentionKernel.cs:21-84)
// called with phase Decode on the gathered prefix + chunk, whose mask is bottom-right aligned
// (:57-66, :219-255). The reference splits long prompts into 512-token chunks on the host
// (ContinuousBatching/Prefill/PrefillHandler.cs:85-89, PrefillConfiguration.cs:21); each chunk is
// one call here.
//
// Work decomposition: one workgroup per (16-query tile, KV head, sequence); wave w computes query
// head w (w + 4, ...) of the KV head's group. The workgroup streams the key blocks through LDS:
// each thread loads its 16-byte pieces of a block's K and V tiles into registers R blocks ahead,
// writes them into one of two LDS slots, and after one barrier every wave reads its MFMA operands
// from that slot. A K/V tile thus crosses from memory once per workgroup and R blocks are in
// flight per workgroup. The LDS tiles are stored with an XOR swizzle of 16-byte chunks so the
// operand reads are free of bank conflicts. Per 16-key block and head:
// S^T[16 keys][16 queries] = K . Q^T on v_mfma_f32_16x16x32_bf16, online softmax per query in fp32
// with the causal limit per query, O[16 queries][D] += P . V on v_mfma_f32_16x16x16_bf16 with P
// split into bf16 high and low parts. These are the decode kernel's operand layouts with the 16
// MFMA rows holding 16 queries instead of (padded) heads.
#include <string>

#include "decode_common.h"

namespace pa {
namespace {

struct PrefillArgs {
    float* out;
    const void* q;
    const void* k_cache;
    const void* v_cache;
    const float* k_scale;
    const float* v_scale;
    const int32_t* q_start_loc;
    const int32_t* prefix_lens;
    const int32_t* block_tables;
    int32_t num_kv_heads;
    int32_t group;
    int32_t max_blocks_per_seq;
    int32_t num_blocks;
    int32_t mask_mode;  // 0 causal, 1 causal only when the prefix is non-empty, 2 no mask
    float scale;
};

constexpr float kPrefillRescaleThreshold = 8.0f;

// LDS geometry of one staged block (K tile then V tile) for head_dim D and element size ELT.
template <int D, int ELT> struct PrefillTile {
    static constexpr int RC = D * ELT / 16;             // 16-byte chunks per K row
    static constexpr int K_CHUNKS = 16 * RC;             // K tile [16][D]
    static constexpr int VRC = ELT;                      // 16-byte chunks per V row (16 tokens)
    static constexpr int CHUNKS = 2 * K_CHUNKS;          // K + V tiles, same size
    static constexpr int BYTES = CHUNKS * 16;
    static constexpr int KP = (K_CHUNKS + 255) / 256;  // per-thread chunks of each tile
    static constexpr int PER_THREAD = 2 * KP;          // K chunks first, then V chunks
    // XOR applied to the chunk index of K row r: the 16 rows read by one 16-lane group land in
    // distinct bank groups
    __device__ static constexpr int kx(int r) { return RC >= 16 ? (r & 15) : ((r * RC / 16) & (RC - 1)); }
    // LDS chunk of V row d, half h (bf16 rows are 2 chunks: rows 8..15 of a 16-row group swap halves)
    __device__ static constexpr int vpos(int d, int h) { return K_CHUNKS + d * VRC + (VRC == 2 ? (h ^ ((d >> 3) & 1)) : h); }
};

template <int D, int KV, bool QF32>
__global__ __launch_bounds__(256, D > 128 ? 1 : 2) void chunked_prefill_kernel(const PrefillArgs a) {
    using Raw = MfmaRaw<KV>;
    constexpr int ELT = Raw::kElt;
    constexpr int NSLAB = D / 32;
    constexpr int NT = D / 16;
    constexpr int TILE = 16 * D;
    using KR = typename Raw::K;
    using VR = typename Raw::V;
    using TL = PrefillTile<D, ELT>;
    constexpr int PT = TL::PER_THREAD;
    constexpr int R = 4;  // blocks in flight (register staging)
    __shared__ __align__(16) uint4 s_tile[2][TL::CHUNKS];

    const int qt = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q4 = lane >> 4, n = lane & 15;
    const int G = a.group, Hkv = a.num_kv_heads, Hq = Hkv * G;

    const int q0 = a.q_start_loc[seq];
    const int Lc = a.q_start_loc[seq + 1] - q0;
    const int P = max(a.prefix_lens[seq], 0);
    const int i0 = qt * 16;
    if (i0 >= Lc) return;
    const int nq = min(16, Lc - i0);
    const int T = min(P + Lc, a.max_blocks_per_seq * 16);
    const bool causal = a.mask_mode == 0 || (a.mask_mode == 1 && P > 0);
    const int kmax = causal ? min(T, P + i0 + nq) : T;  // keys any query of the tile may see
    const int nkb = (kmax + 15) / 16;
    const bool qvalid = n < nq;
    const int klim = causal ? min(T, P + i0 + n + 1) : T;  // this lane's query sees keys [0, klim)

    const int32_t* table = a.block_tables + static_cast<int64_t>(seq) * a.max_blocks_per_seq;
    const char* kc = static_cast<const char*>(a.k_cache);
    const char* vc = static_cast<const char*>(a.v_cache);

    // This thread's chunks of a block: entry k < KP is a K chunk, the others V chunks (so each
    // load uses one descriptor for the whole wave); byte offset within the tile (past the end for a
    // thread without a chunk: such loads return zeros) and LDS chunk.
    int g_off[PT], l_pos[PT];
    bool live[PT];
#pragma unroll
    for (int k = 0; k < PT; k++) {
        const int c = tid + 256 * (k % TL::KP);
        live[k] = c < TL::K_CHUNKS;
        g_off[k] = live[k] ? c * 16 : TILE * ELT;
        if (k < TL::KP) {
            const int r = c / TL::RC, cc = c % TL::RC;
            l_pos[k] = r * TL::RC + (cc ^ TL::kx(r));
        } else {
            l_pos[k] = TL::vpos(c / TL::VRC, c % TL::VRC);
        }
    }
    // Block ids (and int8 scales) of up to KCH key blocks at a time, in LDS: reading them there
    // costs no wait on the streaming loads (a table load inside the stream would).
    constexpr int KCH = 1024;
    __shared__ int s_ids[KCH];
    __shared__ float s_ksc[KV == PA_DTYPE_INT8 ? KCH : 1], s_vsc[KV == PA_DTYPE_INT8 ? KCH : 1];
    // Loads of a block into staging registers through per-block buffer descriptors: an invalid
    // block or one past the end gets zero-sized descriptors and reads as zeros. The loads are the
    // same on every step (no branches), so each wait is for exactly the block it needs.
    auto stage = [&](uint4 (&st)[PT], int jl, int nkc) {
        const int bid = jl < nkc ? s_ids[jl] : -1;
        const int64_t tile = bid >= 0 ? (static_cast<int64_t>(bid) * Hkv + kvh) * TILE * ELT : 0;
        const int bytes = bid >= 0 ? TILE * ELT : 0;
        const __amdgpu_buffer_rsrc_t rk =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(kc + tile), 0, bytes, kBufferFlags);
        const __amdgpu_buffer_rsrc_t rv =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(vc + tile), 0, bytes, kBufferFlags);
#pragma unroll
        for (int k = 0; k < PT; k++) st[k] = buffer_load<uint4>(k < TL::KP ? rk : rv, g_off[k]);
    };
    auto publish = [&](const uint4 (&st)[PT], int slot) {
#pragma unroll
        for (int k = 0; k < PT; k++)
            if (live[k]) s_tile[slot][l_pos[k]] = st[k];
    };

    for (int g0 = 0; g0 < G; g0 += 4) {
        const int g = g0 + wave;
        const bool active = g < G;  // waves without a head still stage blocks
        const int head = kvh * G + (active ? g : 0);
        // Q^T operand: lane (q4, n) holds query i0 + n of this head, dims 32s + 8q4 .. +8.
        bf16x8_t qhi[NSLAB], qlo[QF32 ? NSLAB : 1];
        {
            const int64_t qrow = (static_cast<int64_t>(q0 + i0 + (qvalid ? n : 0)) * Hq + head) * D;
#pragma unroll
            for (int sl = 0; sl < NSLAB; sl++) {
                const int d0 = 32 * sl + 8 * q4;
                if constexpr (QF32) {
                    const float* qp = static_cast<const float*>(a.q) + qrow + d0;
                    float x[8];
#pragma unroll
                    for (int e = 0; e < 8; e++) x[e] = qvalid ? qp[e] : 0.0f;
                    uint32_t hh[4], ll[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        hh[e] = pack_bf16_trunc(x[2 * e], x[2 * e + 1]);
                        const float r0 = x[2 * e] - __uint_as_float(__float_as_uint(x[2 * e]) & 0xffff0000u);
                        const float r1 = x[2 * e + 1] - __uint_as_float(__float_as_uint(x[2 * e + 1]) & 0xffff0000u);
                        ll[e] = pack_bf16_trunc(r0, r1);
                    }
                    qhi[sl] = __builtin_bit_cast(bf16x8_t, make_uint4(hh[0], hh[1], hh[2], hh[3]));
                    qlo[sl] = __builtin_bit_cast(bf16x8_t, make_uint4(ll[0], ll[1], ll[2], ll[3]));
                } else {
                    const uint4 raw = qvalid
                        ? *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.q) + qrow + d0)
                        : make_uint4(0, 0, 0, 0);
                    qhi[sl] = __builtin_bit_cast(bf16x8_t, raw);
                }
            }
        }

        float m_run = -INFINITY, l_run = 0.0f;
        f32x4_t acc[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) acc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

        auto compute = [&](int slot, int lb, int jl) {
            const uint4* tl = s_tile[slot];
            const char* tb = reinterpret_cast<const char*>(tl);
            KR kr[NSLAB];
            VR vr[NT];
#pragma unroll
            for (int sl = 0; sl < NSLAB; sl++) {
                if constexpr (ELT == 2) {  // 8 bf16 = one 16-byte chunk
                    const int cc = 4 * sl + q4;
                    kr[sl] = tl[n * TL::RC + (cc ^ TL::kx(n))];
                } else {  // 8 int8 codes = half a chunk
                    const int cc = 2 * sl + (q4 >> 1);
                    kr[sl] = *reinterpret_cast<const KR*>(tb + (n * TL::RC + (cc ^ TL::kx(n))) * 16 + (q4 & 1) * 8);
                }
            }
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const int d = 16 * t + n;
                if constexpr (ELT == 2)
                    vr[t] = *reinterpret_cast<const VR*>(tb + TL::vpos(d, q4 >> 1) * 16 + (q4 & 1) * 8);
                else
                    vr[t] = *reinterpret_cast<const VR*>(tb + TL::vpos(d, 0) * 16 + q4 * 4);
            }
            float ks = 1.0f, vfac = 1.0f;
            if constexpr (KV == PA_DTYPE_INT8) {  // 0 for an invalid block (its tile reads as zeros)
                ks = s_ksc[jl];
                vfac = s_vsc[jl];
            }
            f32x4_t s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int sl = 0; sl < NSLAB; sl++) {
                const bf16x8_t kop = k_operand(kr[sl]);
                s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qhi[sl], s, 0, 0, 0);
                if constexpr (QF32) s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qlo[sl], s, 0, 0, 0);
            }
            const int kbase = lb * 16 + 4 * q4;
            float sc[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float v = s[i];
                if constexpr (KV == PA_DTYPE_INT8) v = v * ks;
                v = v * a.scale;
                // queries past the tile keep finite scores (their rows are never stored)
                sc[i] = !qvalid ? 0.0f : (kbase + i < klim ? v : -INFINITY);
            }
            const float bm = rows_max(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
            const bool grow = bm > m_run + kPrefillRescaleThreshold;
            if (__any(grow)) {
                const float m_new = grow ? bm : m_run;
                const float alpha = m_new == -INFINITY ? 1.0f : __expf(m_run - m_new);
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
                p[i] = sc[i] == -INFINITY ? 0.0f : __expf(sc[i] - m_run);
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

        // Stream: block j is published into slot j % 2 at step j (its staging registers were
        // loaded R steps earlier), the registers are refilled with block j + R, one barrier, then
        // every wave computes block j. Slot j % 2 was last read by compute(j - 2), which every
        // wave finished before the barrier of step j - 1. Whole rounds of R steps keep the
        // staging registers' indices static.
        for (int c0 = 0; c0 < nkb; c0 += KCH) {
            const int nkc = min(KCH, nkb - c0);
            __syncthreads();  // the previous chunk's ids and the slots are no longer read
            for (int i = tid; i < nkc; i += 256) {
                int id = table[c0 + i];
                id = id < a.num_blocks ? id : -1;
                s_ids[i] = id;
                if constexpr (KV == PA_DTYPE_INT8) {
                    s_ksc[i] = id >= 0 ? a.k_scale[static_cast<int64_t>(id) * Hkv + kvh] : 0.0f;
                    s_vsc[i] = id >= 0 ? a.v_scale[static_cast<int64_t>(id) * Hkv + kvh] : 0.0f;
                }
            }
            __syncthreads();
            uint4 stg[R][PT];
#pragma unroll
            for (int r = 0; r < R; r++) stage(stg[r], r, nkc);
            for (int j0 = 0; j0 < nkc; j0 += R) {
#pragma unroll
                for (int r = 0; r < R; r++) {
                    // the last round's steps past the end publish and stage zeros: harmless, and
                    // the loads stay the same on every step
                    const int jl = j0 + r;
                    publish(stg[r], jl & 1);
                    stage(stg[r], jl + R, nkc);
                    __syncthreads();
                    if (active && jl < nkc) compute(jl & 1, c0 + jl, jl);
                }
            }
        }
        __syncthreads();  // the slots are reused by the next head group

        // rows of acc are queries 4q4 + i; their sums live in lanes (any q4, n = 4q4 + i)
        const float l_tot = rows_sum(l_run);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int qi = 4 * q4 + i;
            const float li = __shfl(l_tot, qi, 64);
            if (active && qi < nq) {
                const float inv = 1.0f / li;
                float* o = a.out + (static_cast<int64_t>(q0 + i0 + qi) * Hq + head) * D;
#pragma unroll
                for (int t = 0; t < NT; t++) o[16 * t + n] = acc[t][i] * inv;
            }
        }
    }
}

template <int D, int KV>
void launch(const PrefillArgs& a, bool qf32, dim3 grid, hipStream_t s) {
    if (qf32) chunked_prefill_kernel<D, KV, true><<<grid, 256, 0, s>>>(a);
    else chunked_prefill_kernel<D, KV, false><<<grid, 256, 0, s>>>(a);
}

template <int D>
void launch_kv(const PrefillArgs& a, int kv, bool qf32, dim3 grid, hipStream_t s) {
    if (kv == PA_DTYPE_BF16) launch<D, PA_DTYPE_BF16>(a, qf32, grid, s);
    else launch<D, PA_DTYPE_INT8>(a, qf32, grid, s);
}

}  // namespace
}  // namespace pa

extern "C" pa_status pa_chunked_prefill(pa_stream* stream, const pa_config* cfg, float* out, const void* q,
                                        const int32_t* q_start_loc, const int32_t* prefix_lens,
                                        const void* k_cache, const void* v_cache, const float* k_scale,
                                        const float* v_scale, const int32_t* block_tables, int32_t num_seqs,
                                        int32_t max_blocks_per_seq, int32_t max_chunk_len) {
    pa_status st = pa::check_config(cfg, "pa_chunked_prefill");
    if (st != PA_SUCCESS) return st;
    if (num_seqs < 0 || max_blocks_per_seq < 0 || max_chunk_len < 0)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_chunked_prefill: negative size");
    if (num_seqs == 0 || max_chunk_len == 0) return pa::clear_error();
    if (num_seqs > 65535) return pa::set_error(PA_ERROR_UNSUPPORTED, "pa_chunked_prefill: num_seqs > 65535");
    if (max_blocks_per_seq == 0)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_chunked_prefill: chunks need at least one block per sequence");
    if (!out || !q || !q_start_loc || !prefix_lens || !k_cache || !v_cache || !block_tables)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_chunked_prefill: null pointer");
    if (cfg->kv_dtype == PA_DTYPE_FP32)
        return pa::set_error(PA_ERROR_UNSUPPORTED, "pa_chunked_prefill: the cache must be BF16 or INT8");
    if (cfg->kv_dtype == PA_DTYPE_INT8 && (!k_scale || !v_scale))
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_chunked_prefill: int8 cache needs k_scale and v_scale");
    if (cfg->num_kv_heads > 65535) return pa::set_error(PA_ERROR_UNSUPPORTED, "pa_chunked_prefill: too many KV heads");
    const uint32_t masks = cfg->flags & (PA_FLAG_REFERENCE_LITERAL_MASK | PA_FLAG_NO_MASK);
    if (masks == (PA_FLAG_REFERENCE_LITERAL_MASK | PA_FLAG_NO_MASK))
        return pa::set_error(PA_ERROR_INVALID_CONFIG, "pa_chunked_prefill: conflicting mask flags");

    pa::PrefillArgs a{};
    a.out = out;
    a.q = q;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.k_scale = k_scale;
    a.v_scale = v_scale;
    a.q_start_loc = q_start_loc;
    a.prefix_lens = prefix_lens;
    a.block_tables = block_tables;
    a.num_kv_heads = cfg->num_kv_heads;
    a.group = cfg->num_q_heads / cfg->num_kv_heads;
    a.max_blocks_per_seq = max_blocks_per_seq;
    a.num_blocks = cfg->num_blocks;
    a.mask_mode = (cfg->flags & PA_FLAG_NO_MASK) ? 2 : ((cfg->flags & PA_FLAG_REFERENCE_LITERAL_MASK) ? 1 : 0);
    a.scale = pa::resolve_scale(cfg);

    dim3 grid((max_chunk_len + 15) / 16, cfg->num_kv_heads, num_seqs);
    hipStream_t s = pa::native(stream);
    const bool qf32 = cfg->q_dtype == PA_DTYPE_FP32;
    switch (cfg->head_dim) {
        case 64: pa::launch_kv<64>(a, cfg->kv_dtype, qf32, grid, s); break;
        case 128: pa::launch_kv<128>(a, cfg->kv_dtype, qf32, grid, s); break;
        default: pa::launch_kv<256>(a, cfg->kv_dtype, qf32, grid, s); break;
    }
    PA_HIP_CHECK(hipGetLastError());
    return pa::clear_error();
}
