// decode_fp32.h -- the fp32-cache paged-decode kernel (VALU).
#pragma once

#include "decode_common.h"

namespace pa {

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
    static_assert(CH >= 8 && CH <= 64, "fp32 kernel covers head_dim 32..256");

    __shared__ float s_logits[G][PART];
    __shared__ float s_red[4][G];
    __shared__ float s_o[4][G][D];

    const int part = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int Hkv = a.num_kv_heads, Hq = Hkv * G;

    const int T = clamp_len(a, a.context_lens[seq]);
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

}  // namespace pa
