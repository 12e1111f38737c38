// decode_mfma.h -- the bf16 / int8 paged-decode kernel (MFMA, persistent workgroups).
//
// Work item = (sequence, KV head, partition of `a.part` tokens). A persistent workgroup (4 waves)
// walks the compacted item list with a stride of gridDim.x; each item's 16-token blocks are dealt
// to the waves round-robin (block lb0 + wave + 4j). While an item streams, the next item's block
// ids are already in flight, so an item starts with one memory round trip (its first K/V blocks).
//
// Per block and wave: S^T[16 tokens][16 heads] = K . Q^T on v_mfma_f32_16x16x32_bf16 (query heads
// padded to 16 rows), online softmax in fp32, O[16 heads][D] += P . V on v_mfma_f32_16x16x16_bf16
// with P split into bf16 high and low parts (~16 significant bits). The score layout the first
// MFMA leaves in registers (lane = (token group q4, head n)) is the A-operand layout of the second,
// so P never leaves registers. Three rotating register buffers keep two blocks in flight while a
// third is consumed. The four waves' (max, sum, O) are combined through LDS at the item's end.
#pragma once

#include "decode_common.h"

namespace pa {

// Online-softmax rescaling is deferred until a block's max exceeds the running max by more than
// this (natural-log units): probabilities then stay below e^8 and fp32 sums stay exact enough,
// while the O accumulators are rescaled on few blocks instead of on most of them.
constexpr float kRescaleThreshold = 8.0f;

struct MfmaShared {
    float m[4][16];
    float l[4][16];
    int pref[kMaxPersistentSeqs + 1];  // items (partitions) before sequence s
    int lens[kMaxPersistentSeqs];      // clamped context length of sequence s
};

struct ItemMeta {
    int seq, kvh, part, T;
};

// Ids of this wave's blocks of an item: lane j holds block lb0 + wave + 4j (or -1: beyond the
// item, or outside [0, num_blocks)).
__device__ __forceinline__ int load_block_ids(const DecodeArgs& a, const ItemMeta& m, int wave, int lane) {
    if (m.T <= 0) return -1;
    const int tok0 = m.part * a.part;
    const int tok_end = min(m.T, tok0 + a.part);
    const int nblk = (tok_end - tok0 + 15) / 16;
    const int nb = nblk > wave ? (nblk - wave + 3) / 4 : 0;
    int id = -1;
    if (lane < nb) {
        id = a.block_tables[static_cast<int64_t>(m.seq) * a.max_blocks_per_seq + tok0 / 16 + wave + 4 * lane];
        if (id >= a.num_blocks) id = -1;
    }
    return id;
}

// One work item. Called by all 256 threads of a workgroup; my_bid from load_block_ids.
template <int D, int KV, bool QF32, bool APPEND>
__device__ __forceinline__ void mfma_item(const DecodeArgs& a, const ItemMeta& im, int my_bid, MfmaShared& sh,
                                          float (*s_x)[D][16]) {
    using Raw = MfmaRaw<KV>;
    constexpr int ELT = Raw::kElt;
    constexpr int NSLAB = D / 32;  // QK MFMAs (k = 32 dims each)
    constexpr int NT = D / 16;     // PV n-tiles of 16 dims
    constexpr int TILE = 16 * D;   // elements per (block, KV head) tile
    constexpr int NPL = D / 64;    // appended-token values per lane

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q4 = lane >> 4;  // token group (QK C rows) / k group of the MFMA operands
    const int n = lane & 15;   // head column of S^T / row of P / dim within a PV tile
    const int G = a.group, Hkv = a.num_kv_heads;
    const int seq = im.seq, kvh = im.kvh, part = im.part, T = im.T;

    if (T <= 0) {
        for (int idx = tid; idx < G * D; idx += 256)
            a.out[(static_cast<int64_t>(seq) * Hkv * G + kvh * G) * D + idx] = 0.0f;
        return;
    }
    const int tok0 = part * a.part;
    const int tok_end = min(T, tok0 + a.part);
    const int nparts = (T + a.part - 1) / a.part;
    const int lb0 = tok0 / 16;
    const int nblk = (tok_end - tok0 + 15) / 16;
    const int nb = nblk > wave ? (nblk - wave + 3) / 4 : 0;

    float my_ks = 0.0f, my_vs = 0.0f;
    if constexpr (KV == PA_DTYPE_INT8) {
        if (my_bid >= 0) {
            my_ks = a.k_scale[static_cast<int64_t>(my_bid) * Hkv + kvh];
            my_vs = a.v_scale[static_cast<int64_t>(my_bid) * Hkv + kvh];
        }
    }

    // Fused append: the sequence's last block belongs to wave (rel & 3) at iteration rel >> 2.
    // That wave fetches the new token now (lane l: dims l*NPL ..) and, for int8, the block's
    // running statistics, so the patch costs no extra round trip later.
    int j_app = -1;
    float new_k[NPL], new_v[NPL];
    Int8Stats old{};
    if constexpr (APPEND) {
        const int rel = (T - 1) / 16 - lb0;
        if (part == nparts - 1 && (rel & 3) == wave) j_app = rel >> 2;
        if (j_app >= 0) {
            const int64_t src = (static_cast<int64_t>(seq) * Hkv + kvh) * D + lane * NPL;
#pragma unroll
            for (int e = 0; e < NPL; e++) {
                new_k[e] = act_at(a.k_new, QF32, src + e);
                new_v[e] = act_at(a.v_new, QF32, src + e);
            }
            if constexpr (KV == PA_DTYPE_INT8) {
                const int bid = __builtin_amdgcn_readlane(my_bid, j_app);
                if (bid >= 0) {
                    const int64_t sidx = static_cast<int64_t>(bid) * Hkv + kvh;
                    old = Int8Stats{a.k_absmax[sidx], a.k_scale[sidx], a.v_absmax[sidx], a.v_scale[sidx]};
                }
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
    const int k_lane_off = (n * D + 8 * q4) * ELT;   // K row n, dims 8q4 .. (+32 per slab)
    const int v_lane_off = (n * 16 + 4 * q4) * ELT;  // V dim n, tokens 4q4 .. (+16 dims per tile)
    // Loads go through per-block buffer descriptors: a block past the wave's list or with an
    // invalid id gets a zero-sized descriptor, so its loads return zeros without touching memory.
    // The load sequence is therefore identical on every iteration (no branches), which lets the
    // compiler wait for exactly the oldest block instead of draining every load in flight.
    auto load = [&](KR (&kr)[NSLAB], VR (&vr)[NT], int j) {
        const int bid = j < nb ? __builtin_amdgcn_readlane(my_bid, j & 63) : -1;
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
                // Stage the new token in LDS (free during streaming: the previous item's combine
                // ended with a barrier, this item's starts with one), then patch the tile.
                float* s_new = &s_x[0][0][0];
#pragma unroll
                for (int e = 0; e < NPL; e++) {
                    s_new[lane * NPL + e] = new_k[e];
                    s_new[D + lane * NPL + e] = new_v[e];
                }
                __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the stores have landed in LDS
                __builtin_amdgcn_wave_barrier();
                const int64_t tile = (static_cast<int64_t>(bid) * Hkv + kvh) * TILE;
                const int r = (T - 1) & 15;
                if constexpr (KV == PA_DTYPE_INT8)
                    append_int8_regs<D>(a, tile, static_cast<int64_t>(bid) * Hkv + kvh, s_new, r, q4, n, old, kr, vr,
                                        ks, vfac);
                else
                    append_bf16_regs<D>(a, tile, s_new, r, q4, n, kr, vr);
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
        const float bm = rows_max(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
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
        // Three rotating register buffers: two blocks in flight while a third is consumed. Loads
        // past the wave's list are zero-sized (no memory traffic), so they are issued regardless.
        KR ka[NSLAB], kb[NSLAB], kx[NSLAB];
        VR va[NT], vb[NT], vx[NT];
        int j = 0;
        load(ka, va, 0);
        load(kb, vb, 1);
        while (j < nb) {
            load(kx, vx, j + 2);
            compute(ka, va, j);
            if (++j >= nb) break;
            load(ka, va, j + 2);
            compute(kb, vb, j);
            if (++j >= nb) break;
            load(kb, vb, j + 2);
            compute(kx, vx, j);
            ++j;
        }
    }

    // ---- combine the 4 waves: weights exp(m_w - M) per head, then a 2-level tree in LDS ----
    const float l_tot = rows_sum(l_run);
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

// Persistent mode: gridDim.x workgroups walk the compacted list of non-empty items
// (sequence s owns items pref[s]*Hkv .. pref[s+1]*Hkv - 1, KV head fastest), item w, w + grid, ...
// Every workgroup leaves its loop after a bounded number of items.
template <int D, int KV, bool QF32, bool APPEND>
__global__ __launch_bounds__(256, D > 128 ? 1 : 2) void paged_decode_mfma_persistent_kernel(const DecodeArgs a, int32_t num_seqs) {
    __shared__ MfmaShared sh;
    __shared__ float s_x[2][D][16];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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
            sh.lens[s] = T;
            c = T <= 0 ? 1 : (T + a.part - 1) / a.part;
        }
        cnt[k] = c;
        local += c;
    }
    int incl = local;  // block-wide exclusive scan of `local`
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
    int seq = 0;  // items only increase, so the owning sequence is found by scanning forward
    auto meta_of = [&](int64_t item) -> ItemMeta {
        const int pi = static_cast<int>(item / Hkv);
        const int kvh = static_cast<int>(item - static_cast<int64_t>(pi) * Hkv);
        while (seq + 1 < num_seqs && sh.pref[seq + 1] <= pi) seq++;
        return ItemMeta{seq, kvh, pi - sh.pref[seq], sh.lens[seq]};
    };
    int64_t item = blockIdx.x;
    if (item >= total) return;
    ItemMeta cur = meta_of(item);
    int cur_bid = load_block_ids(a, cur, wave, lane);
    for (;;) {
        const int64_t next = item + gridDim.x;
        const bool has_next = next < total;
        ItemMeta nxt{0, 0, 0, 0};
        int nxt_bid = -1;
        if (has_next) {  // issued before this item's K/V loads, consumed by the next iteration
            nxt = meta_of(next);
            nxt_bid = load_block_ids(a, nxt, wave, lane);
        }
        mfma_item<D, KV, QF32, APPEND>(a, cur, cur_bid, sh, s_x);
        if (!has_next) break;
        item = next;
        cur = nxt;
        cur_bid = nxt_bid;
    }
}

}  // namespace pa
