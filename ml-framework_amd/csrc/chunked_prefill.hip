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
// Work decomposition: one workgroup per (16-query tile, KV head, sequence). Its 4 waves split the
// key blocks (wave w takes blocks w, w + 4, ...) and each wave runs every query head of the KV
// head's group on each block it loads (HG heads per pass), so a K/V tile is read from memory once
// per workgroup and each loaded operand feeds HG heads' MFMAs. Per 16-key block and head:
// S^T[16 keys][16 queries] = K . Q^T on v_mfma_f32_16x16x32_bf16, online softmax per query in fp32
// with the causal limit per query, O[16 queries][D] += P . V on v_mfma_f32_16x16x16_bf16 with P
// split into bf16 high and low parts. These are the decode kernel's operand layouts with the 16
// MFMA rows holding 16 queries instead of (padded) heads. The 4 waves' (max, sum, O) are combined
// through LDS at the end, head by head.
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

// Heads per pass: bounded by the accumulators (HG x D / 16 x 4 registers) and Q operands.
template <int D, bool QF32> constexpr int prefill_heads_per_pass() { return D > 128 ? 1 : (QF32 ? 2 : 4); }

template <int D, int KV, bool QF32, int HG>
__global__ __launch_bounds__(256, 1) void chunked_prefill_kernel(const PrefillArgs a) {
    using Raw = MfmaRaw<KV>;
    constexpr int ELT = Raw::kElt;
    constexpr int NSLAB = D / 32;
    constexpr int NT = D / 16;
    constexpr int TILE = 16 * D;
    using KR = typename Raw::K;
    using VR = typename Raw::V;
    __shared__ float s_m[4][HG][16], s_l[4][HG][16];
    __shared__ float s_x[2][D][16];

    const int qt = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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
    const int nb = nkb > wave ? (nkb - wave + 3) / 4 : 0;  // this wave's blocks: wave + 4j
    // this lane's query (column n of S^T) sees keys [0, klim)
    const bool qvalid = n < nq;
    const int klim = causal ? min(T, P + i0 + n + 1) : T;

    const int32_t* table = a.block_tables + static_cast<int64_t>(seq) * a.max_blocks_per_seq;
    const char* kc = static_cast<const char*>(a.k_cache);
    const char* vc = static_cast<const char*>(a.v_cache);
    const int k_lane_off = (n * D + 8 * q4) * ELT;
    const int v_lane_off = (n * 16 + 4 * q4) * ELT;

    for (int g0 = 0; g0 < G; g0 += HG) {
        // Q^T operands: lane (q4, n) holds query i0 + n of head kvh*G + g0 + h, dims 32s + 8q4 .. +8.
        bf16x8_t qhi[HG][NSLAB], qlo[QF32 ? HG : 1][QF32 ? NSLAB : 1];
#pragma unroll
        for (int h = 0; h < HG; h++) {
            const int head = kvh * G + g0 + h;
            const int64_t qrow = (static_cast<int64_t>(q0 + i0 + (qvalid ? n : 0)) * Hq + head) * D;
#pragma unroll
            for (int s = 0; s < NSLAB; s++) {
                const int d0 = 32 * s + 8 * q4;
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
                    qhi[h][s] = __builtin_bit_cast(bf16x8_t, make_uint4(hh[0], hh[1], hh[2], hh[3]));
                    qlo[h][s] = __builtin_bit_cast(bf16x8_t, make_uint4(ll[0], ll[1], ll[2], ll[3]));
                } else {
                    const uint4 raw = qvalid
                        ? *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.q) + qrow + d0)
                        : make_uint4(0, 0, 0, 0);
                    qhi[h][s] = __builtin_bit_cast(bf16x8_t, raw);
                }
            }
        }

        // This wave's key blocks go in windows of 64: lane j holds the id (and int8 scales) of
        // block wave + 4 (w0 + j), loaded once per window, so the streaming loop issues only the
        // K/V loads (a table load inside it would make the wave wait for every load before it).
        int my_bid = -1;
        float my_ks = 0.0f, my_vs = 0.0f;
        auto load = [&](KR (&kr)[NSLAB], VR (&vr)[NT], int j, int nbw) {
            int bid = j < nbw ? __builtin_amdgcn_readlane(my_bid, j) : -1;
            bid = bid < a.num_blocks ? bid : -1;
            const int64_t tile = bid >= 0 ? (static_cast<int64_t>(bid) * Hkv + kvh) * TILE * ELT : 0;
            const int bytes = bid >= 0 ? TILE * ELT : 0;
            const __amdgpu_buffer_rsrc_t rk =
                __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(kc + tile), 0, bytes, kBufferFlags);
            const __amdgpu_buffer_rsrc_t rv =
                __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(vc + tile), 0, bytes, kBufferFlags);
#pragma unroll
            for (int s = 0; s < NSLAB; s++) kr[s] = buffer_load<KR>(rk, k_lane_off + 32 * s * ELT);
#pragma unroll
            for (int t = 0; t < NT; t++) vr[t] = buffer_load<VR>(rv, v_lane_off + 256 * t * ELT);
        };

        float m_run[HG], l_run[HG];
        f32x4_t acc[HG][NT];
#pragma unroll
        for (int h = 0; h < HG; h++) {
            m_run[h] = -INFINITY;
            l_run[h] = 0.0f;
#pragma unroll
            for (int t = 0; t < NT; t++) acc[h][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }

        auto compute = [&](const KR (&kr)[NSLAB], const VR (&vr)[NT], int j, int lb) {
            float ks = 1.0f, vfac = 1.0f;
            if constexpr (KV == PA_DTYPE_INT8) {  // an invalid block's tile reads as zeros, scale 0
                const int bid = __builtin_amdgcn_readlane(my_bid, j);
                const bool ok = bid >= 0 && bid < a.num_blocks;
                ks = ok ? readlane_f(my_ks, j) : 0.0f;
                vfac = ok ? readlane_f(my_vs, j) : 0.0f;
            }
            bf16x8_t kop[NSLAB];
#pragma unroll
            for (int sl = 0; sl < NSLAB; sl++) kop[sl] = k_operand(kr[sl]);
            s16x4_t vop[NT];
#pragma unroll
            for (int t = 0; t < NT; t++) vop[t] = v_operand(vr[t]);
            const int kbase = lb * 16 + 4 * q4;
#pragma unroll
            for (int h = 0; h < HG; h++) {
                f32x4_t s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int sl = 0; sl < NSLAB; sl++) {
                    s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[sl], qhi[h][sl], s, 0, 0, 0);
                    if constexpr (QF32) s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[sl], qlo[h][sl], s, 0, 0, 0);
                }
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
                const bool grow = bm > m_run[h] + kPrefillRescaleThreshold;
                if (__any(grow)) {
                    const float m_new = grow ? bm : m_run[h];
                    // 0 from -inf; 1 for a query whose max stays -inf (nothing accumulated yet)
                    const float alpha = m_new == -INFINITY ? 1.0f : __expf(m_run[h] - m_new);
                    l_run[h] *= alpha;
                    m_run[h] = m_new;
                    float ar[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) ar[i] = __shfl(alpha, 4 * q4 + i, 64);
#pragma unroll
                    for (int t = 0; t < NT; t++)
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[h][t][i] *= ar[i];
                }
                // A wave sees only every 4th block: all of them may be masked for a query, whose
                // max then stays -inf; its probabilities are 0, not exp(-inf + inf).
                float p[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    p[i] = sc[i] == -INFINITY ? 0.0f : __expf(sc[i] - m_run[h]);
                    l_run[h] += p[i];
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
                    acc[h][t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(phi, vop[t], acc[h][t], 0, 0, 0);
                    acc[h][t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(plo, vop[t], acc[h][t], 0, 0, 0);
                }
            }
        };

        for (int w0 = 0; w0 < nb; w0 += 64) {
            const int nbw = min(64, nb - w0);
            my_bid = lane < nbw ? table[wave + 4 * (w0 + lane)] : -1;
            if constexpr (KV == PA_DTYPE_INT8) {  // unconditional loads (index clamped)
                const int sb = my_bid >= 0 && my_bid < a.num_blocks ? my_bid : 0;
                my_ks = a.k_scale[static_cast<int64_t>(sb) * Hkv + kvh];
                my_vs = a.v_scale[static_cast<int64_t>(sb) * Hkv + kvh];
            }
            KR ka[NSLAB], kb[NSLAB], kx[NSLAB];
            VR va[NT], vb[NT], vx[NT];
            int j = 0;
            load(ka, va, 0, nbw);
            load(kb, vb, 1, nbw);
            while (j < nbw) {
                load(kx, vx, j + 2, nbw);
                compute(ka, va, j, wave + 4 * (w0 + j));
                if (++j >= nbw) break;
                load(ka, va, j + 2, nbw);
                compute(kb, vb, j, wave + 4 * (w0 + j));
                if (++j >= nbw) break;
                load(kb, vb, j + 2, nbw);
                compute(kx, vx, j, wave + 4 * (w0 + j));
                ++j;
            }
        }

        // ---- combine the 4 waves per head: weights exp(m_w - M), then a 2-level tree in LDS ----
#pragma unroll
        for (int h = 0; h < HG; h++) {
            const float l_tot = rows_sum(l_run[h]);
            if (q4 == 0) {
                s_m[wave][h][n] = m_run[h];
                s_l[wave][h][n] = l_tot;
            }
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < HG; h++) {
            float M[4], f_own[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = 4 * q4 + i;
                M[i] = fmaxf(fmaxf(s_m[0][h][r], s_m[1][h][r]), fmaxf(s_m[2][h][r], s_m[3][h][r]));
                // 0 for a wave that saw no unmasked key of query r (or no block at all)
                f_own[i] = s_m[wave][h][r] == -INFINITY ? 0.0f : __expf(s_m[wave][h][r] - M[i]);
            }
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[h][t][i] *= f_own[i];
            if (wave >= 2) {
#pragma unroll
                for (int t = 0; t < NT; t++)
                    *reinterpret_cast<f32x4_t*>(&s_x[wave - 2][16 * t + n][4 * q4]) = acc[h][t];
            }
            __syncthreads();
            if (wave < 2) {
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    f32x4_t* slot = reinterpret_cast<f32x4_t*>(&s_x[wave][16 * t + n][4 * q4]);
                    acc[h][t] += *slot;
                    if (wave == 1) *slot = acc[h][t];
                }
            }
            __syncthreads();
            if (wave == 0) {
                float L[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = 4 * q4 + i;
                    L[i] = 0.0f;
#pragma unroll
                    for (int w = 0; w < 4; w++)
                        L[i] += s_m[w][h][r] == -INFINITY ? 0.0f : s_l[w][h][r] * __expf(s_m[w][h][r] - M[i]);
                }
                const int head = kvh * G + g0 + h;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int qi = 4 * q4 + i;
                    if (qi < nq) {
                        const float inv = 1.0f / L[i];
                        float* o = a.out + (static_cast<int64_t>(q0 + i0 + qi) * Hq + head) * D;
#pragma unroll
                        for (int t = 0; t < NT; t++) {
                            const f32x4_t other = *reinterpret_cast<const f32x4_t*>(&s_x[1][16 * t + n][4 * q4]);
                            o[16 * t + n] = (acc[h][t][i] + other[i]) * inv;
                        }
                    }
                }
            }
            __syncthreads();  // s_x reuse by the next head
        }
    }
}

template <int D, int KV>
void launch(const PrefillArgs& a, bool qf32, dim3 grid, hipStream_t s) {
    // the heads per pass must divide the group; other group sizes run one head per pass
    if (qf32) {
        constexpr int HG = prefill_heads_per_pass<D, true>();
        if (a.group % HG == 0) chunked_prefill_kernel<D, KV, true, HG><<<grid, 256, 0, s>>>(a);
        else chunked_prefill_kernel<D, KV, true, 1><<<grid, 256, 0, s>>>(a);
    } else {
        constexpr int HG = prefill_heads_per_pass<D, false>();
        if (a.group % HG == 0) chunked_prefill_kernel<D, KV, false, HG><<<grid, 256, 0, s>>>(a);
        else if (HG > 2 && a.group % 2 == 0) chunked_prefill_kernel<D, KV, false, (HG > 2 ? 2 : 1)><<<grid, 256, 0, s>>>(a);
        else chunked_prefill_kernel<D, KV, false, 1><<<grid, 256, 0, s>>>(a);
    }
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
