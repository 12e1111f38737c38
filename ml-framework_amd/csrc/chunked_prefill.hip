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
// Work decomposition: the units are (16-query tile, query head) pairs of one KV head. A
// workgroup of 4 waves takes 2 (G = 4) or more consecutive query tiles of one (sequence, KV head)
// -- all of them on one XCD, the heaviest first -- and each wave computes two units on the same
// K/V operands. The workgroup streams the key blocks through LDS two at a time: the pair's K and
// V tiles go from memory straight into one of three LDS slots (16-byte buffer loads with the LDS
// bit, issued two pairs ahead), and after one barrier every wave reads its MFMA operands from
// that slot, so a K/V tile crosses from memory once per workgroup and never through registers. The LDS tiles are stored with
// XOR swizzles of 16-byte chunks (and the pair's second tile a quarter of a bank line further) so
// the bf16 operand reads are free of bank conflicts. Per pair of blocks and unit:
// S^T[32 keys][16 queries] = K . Q^T on two v_mfma_f32_16x16x32_bf16 per 32 dims, whose rows are
// permuted so every lane ends up with 8 consecutive keys of one block; online softmax per query
// in fp32 (log2 domain, rescale only past a 2^12 margin, mask only on the pairs at the causal
// edge); O[16 queries][D] += P . V on v_mfma_f32_16x16x32_f16 with one fp16 P and the lane's 8
// keys as the k range, the V operand one 16-byte LDS read (bf16 tiles converted to fp16 in LDS by
// the wave that loaded them; int8 codes converted in registers); the row sums of P from the same
// MFMA against ones. With one P operand instead of bf16 high and low parts the D = 128 kernel fits
// three workgroups per CU.
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
    int32_t qtiles_per_wg;  // 16-query tiles per workgroup: max(1, kPrefillUnits / group)
    int32_t num_qgroups;    // workgroups per (sequence, KV head): tiles of the longest chunk / QT
    int32_t num_groups;     // num_seqs * num_kv_heads
};

// LDS-direct loads of a wave's run of HS segments of one block's K tile (LDS base m0k) and of its
// V tile (m0v), 16 bytes a lane: segment j of a run at immediate offset 1024 j, which advances
// both the memory and the LDS address; off[2j] / off[2j + 1] are the lane's register offsets of
// K / V segment j. M0 is saved and restored once around all of them.
template <int HS>
__device__ __forceinline__ void lds_load_runs(u32x4_t rk, u32x4_t rv, const uint32_t* off, uint32_t m0k,
                                              uint32_t m0v) {
    uint32_t saved;
    if constexpr (HS == 1) {
        asm volatile(
            "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
            "buffer_load_dwordx4 %5, %1, 0 offen lds\n\t"
            "s_mov_b32 m0, %4\n\ts_nop 0\n\t"
            "buffer_load_dwordx4 %6, %2, 0 offen lds\n\t"
            "s_mov_b32 m0, %0"
            : "=&s"(saved)
            : "s"(rk), "s"(rv), "s"(m0k), "s"(m0v), "v"(off[0]), "v"(off[1])
            : "memory");
    } else if constexpr (HS == 2) {
        asm volatile(
            "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
            "buffer_load_dwordx4 %5, %1, 0 offen lds\n\t"
            "buffer_load_dwordx4 %6, %1, 0 offen offset:1024 lds\n\t"
            "s_mov_b32 m0, %4\n\ts_nop 0\n\t"
            "buffer_load_dwordx4 %7, %2, 0 offen lds\n\t"
            "buffer_load_dwordx4 %8, %2, 0 offen offset:1024 lds\n\t"
            "s_mov_b32 m0, %0"
            : "=&s"(saved)
            : "s"(rk), "s"(rv), "s"(m0k), "s"(m0v), "v"(off[0]), "v"(off[2]), "v"(off[1]), "v"(off[3])
            : "memory");
    } else {
        static_assert(HS == 4, "runs of 1, 2 or 4 segments");
        asm volatile(
            "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
            "buffer_load_dwordx4 %5, %1, 0 offen lds\n\t"
            "buffer_load_dwordx4 %6, %1, 0 offen offset:1024 lds\n\t"
            "buffer_load_dwordx4 %7, %1, 0 offen offset:2048 lds\n\t"
            "buffer_load_dwordx4 %8, %1, 0 offen offset:3072 lds\n\t"
            "s_mov_b32 m0, %4\n\ts_nop 0\n\t"
            "buffer_load_dwordx4 %9, %2, 0 offen lds\n\t"
            "buffer_load_dwordx4 %10, %2, 0 offen offset:1024 lds\n\t"
            "buffer_load_dwordx4 %11, %2, 0 offen offset:2048 lds\n\t"
            "buffer_load_dwordx4 %12, %2, 0 offen offset:3072 lds\n\t"
            "s_mov_b32 m0, %0"
            : "=&s"(saved)
            : "s"(rk), "s"(rv), "s"(m0k), "s"(m0v), "v"(off[0]), "v"(off[2]), "v"(off[4]), "v"(off[6]),
              "v"(off[1]), "v"(off[3]), "v"(off[5]), "v"(off[7])
            : "memory");
    }
}

// The running maximum (log2 units) is raised only when a block's maximum exceeds it by more than
// this, so unnormalised probabilities stay below 2^12 and the rescale of the accumulators is rare.
constexpr float kPrefillRescaleLog2 = 12.0f;
// int8 caches: the exponent of a block's probabilities includes log2 of its V scale, floored here
// (a zero scale, an invalid block): P then enters the row sum as (P 2^lv) 2^-lv, with 2^-lv <= 2^64
// keeping the sum finite, and a block whose scale is below 2^-64 contributes P 2^-64 code
// instead of P scale code (an absolute error below 127 2^-64 of the output).
constexpr float kMinLog2VScale = -64.0f;

// Waves per workgroup; each computes two (query tile, query head) units.
constexpr int kPrefillWaves = 4;
constexpr int kPrefillThreads = 64 * kPrefillWaves;
constexpr int kPrefillUnits = 2 * kPrefillWaves;  // units per workgroup round

// LDS geometry of one staged block (K tile then V tile) for head_dim D and element size ELT.
// gfx950's LDS serves 256 bytes a clock (64 banks of 4 bytes). A 16-byte read (ds_read_b128) of a
// wave takes 4 clocks of 16 lanes each, the lanes of one clock being the quads (4 consecutive
// lanes) of one half-wave whose quad index (0..7) has the same bit parity: {0, 3, 5, 6} and
// {1, 2, 4, 7}. Two lanes of one clock on the same 16-byte position of a 256-byte line (at
// different addresses) cost a clock more. The layouts below give each clock 16 distinct positions.
template <int D, int ELT> struct PrefillTile {
    static constexpr int RC = D * ELT / 16;             // 16-byte chunks per K row
    static constexpr int K_CHUNKS = 16 * RC;             // K tile [16][D]
    static constexpr int VRC = ELT;                      // 16-byte chunks per V row (16 tokens)
    static constexpr int CHUNKS = 2 * K_CHUNKS;          // K + V tiles, same size
    static constexpr int SPT = K_CHUNKS / 64;            // 64-chunk segments (one wave's load) per tile
    // K row r's chunk c is stored at chunk r * RC + kswz(r, c). A QK operand read takes one chunk
    // column c = 4 sl + q4 (q4 = lane / 16) of rows (n & 3) + 8 (n >> 3) (+ 4) of tile (n >> 2) & 1
    // (n = lane % 16); the second tile sits 4 positions further. In one clock, lane groups q4 and
    // q4 ^ 1 meet with 2 quads each, one of each tile: the low 2 bits (row & 3) separate the lanes of
    // a quad, and the quads get distinct high 2 bits from the tile offset plus, for bf16 rows of 16
    // or more chunks, bit 3 flipped by the column's bit 0 (q4 & 1); 128-byte rows (D = 64) get that
    // spread from the row parity. int8 keeps the row-only swizzle.
    __device__ static constexpr int kswz(int r, int c) {
        return c ^ (r & 3) ^ (ELT == 2 && RC >= 16 ? (c & 1) << 3 : 0);
    }
    __device__ static constexpr int kpos(int r, int c) { return r * RC + kswz(r, c); }
    // Memory chunk of the K tile stored at LDS position p (the inverse of kpos).
    __device__ static constexpr int ksrc(int p) {
        const int r = p / RC, x = p % RC;
        const int c0 = (x ^ r) & 1;  // bit 0 of the column (kswz keeps it up to the row's bit 0)
        return r * RC + (x ^ (r & 3) ^ (ELT == 2 && RC >= 16 ? c0 << 3 : 0));
    }
    // Chunk offset of block b of slot `slot` in the LDS ring: block 1 sits 4 chunks (64 bytes)
    // further, a quarter of a bank line.
    static constexpr int SLOT = 2 * CHUNKS + 8;
    __device__ static constexpr int base(int slot, int b) { return slot * SLOT + b * (CHUNKS + 4); }
    // LDS chunk of V row d, half h, in block b of the pair. A bf16 PV operand read takes half
    // q4 >> 1 of 8 consecutive rows from each tile (b = q4 & 1) in one clock: the half stored first
    // is h ^ b, so the two tiles' rows land on even and odd positions.
    __device__ static constexpr int vpos(int d, int h, int b) {
        return K_CHUNKS + d * VRC + (VRC == 2 ? (h ^ b) : h);
    }
    // Memory chunk of block b's V tile stored at position p of the V area (the inverse of vpos).
    __device__ static constexpr int vsrc(int p, int b) { return VRC == 2 ? p ^ b : p; }
};

// Attention of one unit (query head `head`, queries qrow0 .. qrow0 + nq - 1 of the call, whose
// first sits at absolute position pos0) over a bf16 cache, in fp32 throughout: lane l holds dims
// l + 64 j; per key the wave sums q.k across lanes, then updates a running (max, sum, O) with
// expf. The prefill's fallback when its fp16 V operand cannot hold the cache's values; slow (one
// key at a time) and exact up to the order of the sums.
template <int D, bool QF32>
__device__ void prefill_exact_unit(const PrefillArgs& a, const int32_t* table, int kvh, int head,
                                                int qrow0, int nq, int pos0, int T, bool causal) {
    constexpr int DPL = D / 64;
    const int lane = threadIdx.x & 63;
    const int Hq = a.num_kv_heads * a.group;
    const uint16_t* kc = static_cast<const uint16_t*>(a.k_cache);
    const uint16_t* vc = static_cast<const uint16_t*>(a.v_cache);
    for (int qi = 0; qi < nq; qi++) {
        const int64_t qoff = (static_cast<int64_t>(qrow0 + qi) * Hq + head) * D;
        float qv[DPL];
#pragma unroll
        for (int j = 0; j < DPL; j++) {
            const int d = lane + 64 * j;
            qv[j] = QF32 ? static_cast<const float*>(a.q)[qoff + d]
                         : pa::bf16_to_f32(static_cast<const uint16_t*>(a.q)[qoff + d]);
        }
        const int klim = causal ? min(T, pos0 + qi + 1) : T;
        float m = -INFINITY, l = 0.0f, o[DPL];
#pragma unroll
        for (int j = 0; j < DPL; j++) o[j] = 0.0f;
        for (int t = 0; t < klim; t++) {
            int id = table[t >> 4];
            id = id >= 0 && id < a.num_blocks ? id : -1;
            float s = 0.0f, vv[DPL];
            const int64_t tile = (static_cast<int64_t>(id >= 0 ? id : 0) * a.num_kv_heads + kvh) * 16 * D;
#pragma unroll
            for (int j = 0; j < DPL; j++) {
                const int d = lane + 64 * j;
                const float kx = id >= 0 ? pa::bf16_to_f32(kc[tile + (t & 15) * D + d]) : 0.0f;
                vv[j] = id >= 0 ? pa::bf16_to_f32(vc[tile + d * 16 + (t & 15)]) : 0.0f;
                s = __builtin_fmaf(qv[j], kx, s);
            }
            s = wave_sum(s) * a.scale;
            const float mn = fmaxf(m, s);
            const float alpha = expf(m - mn);  // 0 on the first key
            const float p = expf(s - mn);
            l = l * alpha + p;
#pragma unroll
            for (int j = 0; j < DPL; j++) o[j] = o[j] * alpha + p * vv[j];
            m = mn;
        }
        const float inv = 1.0f / l;
#pragma unroll
        for (int j = 0; j < DPL; j++) a.out[qoff + lane + 64 * j] = o[j] * inv;
    }
}

// The units of round u0 of this workgroup that this wave computes (the kernel's decomposition,
// rederived from the arguments so that nothing stays live across the stream for this rare path),
// through prefill_exact_unit.
template <int D, bool QF32>
__device__ void prefill_exact_round(const PrefillArgs& a, int u0) {
    int lid = blockIdx.x;
    asm volatile("" : "+s"(lid));  // recomputed here, not kept from the kernel's start
    const int wk = lid >> 3;
    const int m = wk / a.num_qgroups;
    const int qg = a.num_qgroups - 1 - (wk - m * a.num_qgroups);
    const int gi = (lid & 7) + 8 * m;
    const int seq = gi / a.num_kv_heads, kvh = gi - seq * a.num_kv_heads;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int G = a.group;
    const int q0 = a.q_start_loc[seq];
    const int Lc = a.q_start_loc[seq + 1] - q0;
    const int P = max(a.prefix_lens[seq], 0);
    const int i0w = qg * a.qtiles_per_wg * 16;
    const int T = min(P + Lc, a.max_blocks_per_seq * 16);
    const bool causal = a.mask_mode == 0 || (a.mask_mode == 1 && P > 0);
    const int32_t* table = a.block_tables + static_cast<int64_t>(seq) * a.max_blocks_per_seq;
    const int U = a.qtiles_per_wg * G;
    for (int k = 0; k < 2; k++) {
        const int u = u0 + 2 * wave + k;
        if (u >= U) break;
        const int qtl = u / G;
        const int i0 = i0w + 16 * qtl;
        const int nq = max(0, min(16, Lc - i0));
        if (nq > 0) prefill_exact_unit<D, QF32>(a, table, kvh, kvh * G + (u - qtl * G), q0 + i0, nq, P + i0, T, causal);
    }
}

// Work units are (16-query tile, query head) pairs of one KV head. A workgroup takes QT =
// max(1, kPrefillUnits / G) consecutive query tiles, i.e. QT * G units, kPrefillUnits at a time:
// wave w computes units 2w and 2w + 1 of the round on the same K/V operands (each LDS operand
// read feeds both).
template <int D, int KV, bool QF32>
__global__ __launch_bounds__(kPrefillThreads, D > 128 ? 1 : (D > 64 && QF32 ? 2 : 3)) void chunked_prefill_kernel(const PrefillArgs a) {
    using Raw = MfmaRaw<KV>;
    constexpr int ELT = Raw::kElt;
    constexpr int NSLAB = D / 32;
    constexpr int NT = D / 16;
    constexpr int TILE = 16 * D;
    using KR = typename Raw::K;
    using TL = PrefillTile<D, ELT>;
    constexpr int NSLOT = 3;  // LDS slots: the pair being computed and two in flight
    constexpr int NSEG = 4 * TL::SPT / kPrefillWaves;  // 64-chunk loads per wave per pair (4 tiles)
    static_assert((4 * TL::SPT) % kPrefillWaves == 0, "a pair's tiles must split evenly over the waves");
    __shared__ __align__(16) uint4 s_tile[NSLOT * TL::SLOT];  // NSLOT slots x 2 blocks (TL::base)

    // Workgroup -> (query-tile group, KV head, sequence). Workgroup ids are dispatched to the 8
    // XCDs in turn (id mod 8); every query-tile group of (sequence, KV head) group gi runs on XCD
    // gi mod 8, so the workgroups that read the same K/V blocks share one L2, and within a group
    // the ones with the most keys (the last ones) start first.
    const int lid = blockIdx.x;
    const int wk = lid >> 3;
    const int m = wk / a.num_qgroups;
    const int qg = a.num_qgroups - 1 - (wk - m * a.num_qgroups);
    const int gi = (lid & 7) + 8 * m;
    if (gi >= a.num_groups) return;
    const int seq = gi / a.num_kv_heads, kvh = gi - seq * a.num_kv_heads;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Which tile each of the wave's load segments belongs to follows from the wave index; with
    // the range known, the compiler resolves it at compile time where the tile size allows.
    __builtin_assume(wave >= 0 && wave < kPrefillWaves);
    const int q4 = lane >> 4, n = lane & 15;
    const int G = a.group, Hkv = a.num_kv_heads, Hq = Hkv * G;
    const int QT = a.qtiles_per_wg;

    const int q0 = a.q_start_loc[seq];
    const int Lc = a.q_start_loc[seq + 1] - q0;
    const int P = max(a.prefix_lens[seq], 0);
    const int i0w = qg * QT * 16;  // the workgroup's queries are [i0w, iew) of the chunk
    if (i0w >= Lc) return;
    const int iew = min(Lc, i0w + QT * 16);
    const int T = min(P + Lc, a.max_blocks_per_seq * 16);
    const bool causal = a.mask_mode == 0 || (a.mask_mode == 1 && P > 0);
    const int kmax = causal ? min(T, P + iew) : T;  // keys any query of the workgroup may see
    const int nkb = (kmax + 15) / 16;
    const int klim_lo = causal ? min(T, P + i0w + 1) : T;  // every query of it sees [0, klim_lo)
    const float c2 = a.scale * 1.4426950408889634f;       // scores in log2 units
    // QK operand row of this lane (see compute) and the keys it holds after QK (for P and V)
    const int krow0 = (n & 3) + 8 * (n >> 3), kblk = (n >> 2) & 1;
    const int pblk = q4 & 1, ptok = 8 * (q4 >> 1);
    const f16x8_t ones16 = __builtin_bit_cast(f16x8_t, make_uint4(0x3c003c00u, 0x3c003c00u, 0x3c003c00u, 0x3c003c00u));

    const int32_t* table = a.block_tables + static_cast<int64_t>(seq) * a.max_blocks_per_seq;
    const char* kc = static_cast<const char*>(a.k_cache);
    const char* vc = static_cast<const char*>(a.v_cache);

    // This wave's loads of a pair. The pair's 64-chunk segments are ordered block by block, K and
    // V alternating (K seg 0, V seg 0, K seg 1, ..); wave w loads the NSEG of them from w NSEG on:
    // with two or more segments per tile, the same segments of one block's K and V tiles, so one
    // block id, one tile offset and two descriptors serve all of a wave's loads. Lane l fills LDS
    // position 64 i + l of segment i of its tile and therefore loads the memory chunk the layout
    // puts there.
    constexpr int HS = NSEG >= 2 ? NSEG / 2 : 1;  // segments per tile and wave
    const int seg_blk = (wave * NSEG) / (2 * TL::SPT);            // the wave's block of the pair
    const int seg_v0 = NSEG >= 2 ? 0 : wave & 1;                   // one segment per wave: K or V
    const int seg_i0 = ((wave * NSEG) % (2 * TL::SPT)) >> 1;       // its first segment of the tile
    // Loads of one tile issue from one LDS base (M0): segment j of the wave's run sits 1024 bytes
    // further in LDS and in the load's immediate offset, which the hardware adds to both
    // addresses, so the lane's register offset for it is its chunk's offset less 1024 j.
    uint32_t seg_off[NSEG];  // k = 2j (K) and 2j + 1 (V) for NSEG >= 2; k = 0 otherwise
#pragma unroll
    for (int k = 0; k < NSEG; k++) {
        const int j = NSEG >= 2 ? k >> 1 : 0;
        const bool is_v = NSEG >= 2 ? (k & 1) : seg_v0;
        const int pos = (seg_i0 + j) * 64 + lane;
        seg_off[k] = 16 * (is_v ? TL::vsrc(pos, seg_blk) : TL::ksrc(pos)) - 1024 * j;
    }
    // Block ids (and int8 scales) of up to KCH key blocks at a time, in LDS.
    constexpr int KCH = D > 64 ? 512 : 1024;  // 3 workgroups per CU at D = 128 fit the LDS with 512
    __shared__ int s_ids[KCH];
    // int8: K scale, log2 of the V scale (clamped at kMinLog2VScale) and 2^-that
    __shared__ float s_ksc[KV == PA_DTYPE_INT8 ? KCH + 4 : 1], s_vlg[KV == PA_DTYPE_INT8 ? KCH + 4 : 1],
        s_vrc[KV == PA_DTYPE_INT8 ? KCH + 4 : 1];
    // bf16: bit r set when round r (u0 = 8 r; bit 31: round 31 or later) met a V value outside
    // fp16's range in any wave's conversion
    __shared__ int s_sat;
    if constexpr (ELT == 2) {
        if (tid == 0) s_sat = 0;  // published by the first barrier of the stream
    }
    const uint32_t tile_lds = lds_address(s_tile);
    // Loads of the pair of blocks jl, jl + 1 (of the current chunk of the table) into slot `slot`.
    // A block past the chunk or with an invalid id gets a zero-sized descriptor and reads as zeros,
    // so every wave issues the same NSEG loads per pair and one vmcnt value covers them all.
    // Block ids are read from a register that holds 64 of them (lane l: id of block 64w + l of the
    // chunk), refilled from LDS when the stream enters the next 64 blocks, so an issue does not
    // wait for an LDS read; each block's tile offset is computed once for its K and V descriptors.
    int ids_win = -1, ids_v = -1;
    auto block_id = [&](int j, int nkc) -> int {  // j wave-uniform
        if (j >= nkc) return -1;
        if ((j >> 6) != ids_win) {
            ids_win = j >> 6;
            const int jj = (ids_win << 6) + lane;
            ids_v = jj < nkc ? s_ids[jj] : -1;
        }
        return __builtin_amdgcn_readlane(ids_v, j & 63);
    };
    const uint32_t seg_lds = tile_lds + 16 * (TL::base(0, seg_blk) + 64 * seg_i0);  // the K run in slot 0
    auto issue = [&](int jl, int nkc, int slot) {
        const int id = block_id(jl + seg_blk, nkc);
        const int64_t tile = (static_cast<int64_t>(id >= 0 ? id : 0) * Hkv + kvh) * TILE * ELT;
        const uint32_t bytes = id >= 0 ? TILE * ELT : 0;
        const uint32_t m0k = seg_lds + 16 * TL::SLOT * slot;
        if constexpr (NSEG >= 2) {
            lds_load_runs<HS>(buffer_rsrc_words(kc + tile, bytes), buffer_rsrc_words(vc + tile, bytes), seg_off, m0k,
                              m0k + 16 * TL::K_CHUNKS);
        } else {
            lds_load16(buffer_rsrc_words((seg_v0 ? vc : kc) + tile, bytes), seg_off[0],
                       m0k + (seg_v0 ? 16 * TL::K_CHUNKS : 0));
        }
    };

    const int U = QT * G;
    for (int u0 = 0; u0 < U; u0 += kPrefillUnits) {
        // This wave's two units. A unit past U repeats unit u0 and a query tile past the chunk has
        // no valid query: both are computed like the others (no branch) and never stored.
        int head[2], i0[2], nq[2], klim[2];
        bool store[2];
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int u = u0 + 2 * wave + k;
            const int uu = u < U ? u : u0;
            const int qtl = uu / G;
            head[k] = kvh * G + (uu - qtl * G);
            i0[k] = i0w + 16 * qtl;
            nq[k] = max(0, min(16, Lc - i0[k]));
            store[k] = u < U && nq[k] > 0;
            klim[k] = causal ? min(T, P + i0[k] + n + 1) : T;  // query n sees keys [0, klim)
        }
        // Q^T operands: lane (q4, n) holds query i0 + n of the unit's head, dims 32s + 8q4 .. +8.
        bf16x8_t qhi[2][NSLAB], qlo[2][QF32 ? NSLAB : 1];
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const bool qvalid = n < nq[k];
            const int64_t qrow = (static_cast<int64_t>(q0 + i0[k] + (qvalid ? n : 0)) * Hq + head[k]) * D;
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
                    qhi[k][sl] = __builtin_bit_cast(bf16x8_t, make_uint4(hh[0], hh[1], hh[2], hh[3]));
                    qlo[k][sl] = __builtin_bit_cast(bf16x8_t, make_uint4(ll[0], ll[1], ll[2], ll[3]));
                } else {
                    const uint4 raw = qvalid
                        ? *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.q) + qrow + d0)
                        : make_uint4(0, 0, 0, 0);
                    qhi[k][sl] = __builtin_bit_cast(bf16x8_t, raw);
                }
            }
        }

        // The Q loads land here, once, rather than behind a wait inside the stream loop (the
        // compiler does not count the slot loads, so it cannot tell them apart there).
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        float m_run[2] = {-INFINITY, -INFINITY};  // log2 units, query n
        float m_thr[2] = {-INFINITY, -INFINITY};  // scores (as computed, before the log2 scale) above
                                                  // this may raise m_run past its rescale margin
        float l_run[2] = {0.0f, 0.0f};            // int8: sum of P for query n over this lane's keys
        f32x4_t acc_l[2], acc[2][NT];             // bf16: row sums of P; outputs (queries 4q4 + i)
#pragma unroll
        for (int k = 0; k < 2; k++) {
            acc_l[k] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < NT; t++) acc[k][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }

        // bf16 caches: this wave's V segments of the pair in `slot` (landed: the caller waited for
        // them) become fp16 in place, same positions. Round toward zero: exact for every bf16 value
        // fp16 represents (|v| <= 65280 among bf16 values; subnormal fp16 below 2^-14 keeps an
        // absolute error under 2^-24); larger magnitudes would saturate at 65504, so the largest
        // |v| converted is kept in v_big and a round that met one is computed again exactly (see
        // the end of the round). The barrier before the pair is computed publishes the fp16 tiles.
        uint64_t v_big = 0;
        // The wave's V chunks of the slot are all read before any is written back, so their LDS
        // latencies overlap (written chunk by chunk, each read waited for the previous write).
        auto convert_v = [&](int slot) {
            constexpr int NV = NSEG >= 2 ? NSEG / 2 : 1;
            if (NSEG >= 2 || seg_v0) {
                uint4* c[NV];
                uint4 x[NV];
#pragma unroll
                for (int j = 0; j < NV; j++) {
                    c[j] = s_tile + (TL::base(slot, seg_blk) + TL::K_CHUNKS + (seg_i0 + j) * 64 + lane);
                    x[j] = *c[j];
                }
#pragma unroll
                for (int j = 0; j < NV; j++) {
                    const uint32_t w[4] = {x[j].x, x[j].y, x[j].z, x[j].w};
                    uint32_t o[4];
                    float mx = 0.0f;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float lo = __uint_as_float(w[e] << 16), hi = __uint_as_float(w[e] & 0xffff0000u);
                        mx = fmaxf(mx, fmaxf(fabsf(lo), fabsf(hi)));
                        o[e] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
                    }
                    v_big |= __builtin_amdgcn_ballot_w64(mx >= 65536.0f);  // 65536: the least bf16 above 65504
                    *c[j] = make_uint4(o[0], o[1], o[2], o[3]);
                }
            }
        };

        // One pair of blocks (keys lb*16 .. lb*16 + 31), lanes (q4, n): the two QK MFMAs h = 0, 1 take
        // as row r key 8 (r >> 3) + 4h + (r & 3) of block (r >> 2) & 1, so lane (q4, n) receives, for
        // query n, scores e = 4h + i of keys ptok + e of block pblk: 8 consecutive keys of one block.
        // That is exactly the k range the lane feeds the PV MFMA (v_mfma_f32_16x16x32_bf16, k = 8q4 +
        // e), in P and in V, where the V operand is then one 16-byte LDS read. Row sums come from a
        // third MFMA against ones, in the accumulators' own layout. Scores are kept in log2 units
        // (scale * log2(e) folded in); pairs with every key below every query's causal limit skip
        // the mask. Both units use the same K and V operands.
        auto compute = [&](bool masked, int kend, int slot, int next_slot, int lb, int jl) {
            const char* tk = reinterpret_cast<const char*>(s_tile + TL::base(slot, kblk));
            const char* tv = reinterpret_cast<const char*>(s_tile + TL::base(slot, pblk));
            // QK per half h (its 16-row K operands are then dead), V operands after QK
            float v[2][8];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int r = krow0 + 4 * h;
                bf16x8_t kop[NSLAB];
#pragma unroll
                for (int sl = 0; sl < NSLAB; sl++) {
                    if constexpr (ELT == 2) {  // 8 bf16 = one 16-byte chunk
                        const int cc = 4 * sl + q4;
                        kop[sl] = k_operand(*reinterpret_cast<const KR*>(tk + TL::kpos(r, cc) * 16));
                    } else {  // 8 int8 codes = half a chunk
                        const int cc = 2 * sl + (q4 >> 1);
                        kop[sl] = k_operand(*reinterpret_cast<const KR*>(tk + TL::kpos(r, cc) * 16 + (q4 & 1) * 8));
                    }
                }
                __builtin_amdgcn_s_setprio(2);
#pragma unroll
                for (int k = 0; k < 2; k++) {
                    f32x4_t sacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int sl = 0; sl < NSLAB; sl++) {
                        sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[sl], qhi[k][sl], sacc, 0, 0, 0);
                        if constexpr (QF32) sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[sl], qlo[k][sl], sacc, 0, 0, 0);
                    }
#pragma unroll
                    for (int i = 0; i < 4; i++) v[k][4 * h + i] = sacc[i];
                }
                __builtin_amdgcn_s_setprio(0);
            }
            if constexpr (ELT == 2) {
                // While the QK MFMAs run: the next pair's V (its loads, older than the NSEG just
                // issued, have landed) turns into fp16 for the barrier before that pair.
                asm volatile("s_waitcnt vmcnt(%0)" : : "n"(NSEG) : "memory");
                convert_v(next_slot);
            }
            if constexpr (KV == PA_DTYPE_INT8) {
                // log2 units plus log2 of the block's V scale: exp2(v - m_run) is then P times the V
                // scale, at most 2^kPrefillRescaleLog2 whatever the scale, the fp16 P operand
                const float mult = c2 * s_ksc[jl + pblk];  // 0 for an invalid block
                const float lvb = s_vlg[jl + pblk];
#pragma unroll
                for (int k = 0; k < 2; k++)
#pragma unroll
                    for (int e = 0; e < 8; e++) v[k][e] = __builtin_fmaf(v[k][e], mult, lvb);
            }
            if (masked) {  // wave-uniform; only the pairs at the causal edge or past the end
                const int kq = (lb + pblk) * 16 + ptok;
#pragma unroll
                for (int k = 0; k < 2; k++) {
                    const int lim = min(klim[k], kend) - kq;
#pragma unroll
                    for (int e = 0; e < 8; e++) v[k][e] = e < lim ? v[k][e] : -INFINITY;
                }
            }
            // The lane's own maximum against the row's threshold decides whether the row maxima
            // are needed at all: a row can only grow if one of its lanes holds a score above it.
            float bl[2];
            bool over = false;
#pragma unroll
            for (int k = 0; k < 2; k++) {
                bl[k] = fmaxf(fmaxf(fmaxf(v[k][0], v[k][1]), fmaxf(v[k][2], v[k][3])),
                              fmaxf(fmaxf(v[k][4], v[k][5]), fmaxf(v[k][6], v[k][7])));
                over = over || bl[k] > m_thr[k];
            }
            if (__any(over)) {
#pragma unroll
                for (int k = 0; k < 2; k++) {
                    float bm = rows_max(bl[k]);
                    if constexpr (KV != PA_DTYPE_INT8) bm *= c2;
                    const bool grow = bm > m_run[k] + kPrefillRescaleLog2;
                    const float m_new = grow ? bm : m_run[k];
                    const float alpha = __builtin_amdgcn_exp2f(m_run[k] - m_new);  // 0 on the first update
                    m_run[k] = m_new;
                    m_thr[k] = KV != PA_DTYPE_INT8 ? (m_new + kPrefillRescaleLog2) / c2 : m_new + kPrefillRescaleLog2;
                    l_run[k] *= alpha;
                    float ar[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) ar[i] = __shfl(alpha, 4 * q4 + i, 64);
#pragma unroll
                    for (int i = 0; i < 4; i++) acc_l[k][i] *= ar[i];
#pragma unroll
                    for (int t = 0; t < NT; t++)
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[k][t][i] *= ar[i];
                }
            }
            // One fp16 P per probability (rounded to nearest, relative error <= 2^-11; at most 2^12
            // by the rescale margin; int8: P times the block's V scale, by the exponent) against V in
            // fp16: bf16 caches' tiles were converted in LDS when they landed, int8 codes are
            // converted here (exact). One PV MFMA per unit and 16-dim tile; bf16 row sums from one
            // more MFMA against ones, int8 row sums in l_run (P without the V scale). The P of both
            // units first, then each V operand is read right before the MFMAs that use it, except
            // (bf16 caches) the first one, read before the exponentials so that its LDS latency
            // passes while those issue (two measured slower: the extra operand's registers cost
            // moves).
            constexpr int NVPF = ELT == 2 ? 1 : 0;
            uint4 vpf[NVPF > 0 ? NVPF : 1];
            if constexpr (ELT == 2) {
#pragma unroll
                for (int t = 0; t < NVPF; t++)
                    vpf[t] = *reinterpret_cast<const uint4*>(tv + TL::vpos(16 * t + n, q4 >> 1, pblk) * 16);
            }
            f16x8_t pf[2];
#pragma unroll
            for (int k = 0; k < 2; k++) {
                float p[8];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    if constexpr (KV == PA_DTYPE_INT8) p[e] = __builtin_amdgcn_exp2f(v[k][e] - m_run[k]);
                    else p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(v[k][e], c2, -m_run[k]));
                }
                if constexpr (KV == PA_DTYPE_INT8) {
                    // p holds P times the V scale; the row sum takes P
                    const float rv = s_vrc[jl + pblk];
#pragma unroll
                    for (int e = 0; e < 8; e++) l_run[k] = __builtin_fmaf(p[e], rv, l_run[k]);
                }
                uint32_t w[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const half2_t h = {static_cast<_Float16>(p[2 * e]), static_cast<_Float16>(p[2 * e + 1])};
                    w[e] = __builtin_bit_cast(uint32_t, h);
                }
                pf[k] = __builtin_bit_cast(f16x8_t, make_uint4(w[0], w[1], w[2], w[3]));
            }
            __builtin_amdgcn_s_setprio(2);
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const int d = 16 * t + n;
                f16x8_t vop;
                if constexpr (ELT == 2) {
                    if (t < NVPF) vop = __builtin_bit_cast(f16x8_t, vpf[t < NVPF ? t : 0]);
                    else vop = __builtin_bit_cast(f16x8_t, *reinterpret_cast<const uint4*>(tv + TL::vpos(d, q4 >> 1, pblk) * 16));
                } else {
                    const uint2 c = *reinterpret_cast<const uint2*>(tv + TL::vpos(d, 0, pblk) * 16 + (q4 >> 1) * 8);
                    uint32_t o[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const uint32_t x = e < 2 ? c.x : c.y;
                        o[e] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(pa::i8_at(x, 2 * (e & 1)),
                                                                                         pa::i8_at(x, 2 * (e & 1) + 1)));
                    }
                    vop = __builtin_bit_cast(f16x8_t, make_uint4(o[0], o[1], o[2], o[3]));
                }
#pragma unroll
                for (int k = 0; k < 2; k++) acc[k][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pf[k], vop, acc[k][t], 0, 0, 0);
            }
            if constexpr (KV != PA_DTYPE_INT8) {
#pragma unroll
                for (int k = 0; k < 2; k++) acc_l[k] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pf[k], ones16, acc_l[k], 0, 0, 0);
            }
            __builtin_amdgcn_s_setprio(0);
        };

        // Stream, a pair of blocks per step: pair j (blocks 2j, 2j + 1 of the chunk) was loaded
        // into slot j % 3 two steps earlier. Every wave has waited for its own loads of pair j
        // (at most pair j + 1's NSEG loads outstanding; loads complete in order): bf16 caches
        // inside compute(j - 1), after its QK MFMAs, where it also converts its V segments of pair
        // j to fp16 (pair 0 before the loop); int8 caches at the top of step j. Step j ends the
        // wave's LDS accesses and meets the other waves at a barrier; then it loads pair j + 2
        // into slot (j + 2) % 3, whose last reader, compute(j - 1), every wave has finished, and
        // computes pair j. Loads past the chunk's end write zeros into slots nobody reads.
        for (int c0 = 0; c0 < nkb; c0 += KCH) {
            const int nkc = min(KCH, nkb - c0);
            const int npair = (nkc + 1) / 2;
            const int kend = (c0 + nkc) * 16;        // keys of this chunk of the table end here
            const int kend_lo = min(klim_lo, kend);  // pairs reaching past it need the mask
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's slot loads have landed
            __syncthreads();  // the previous chunk's ids and the slots are no longer read or written
            for (int i = tid; i < nkc; i += kPrefillThreads) {
                int id = table[c0 + i];
                id = id < a.num_blocks ? id : -1;
                s_ids[i] = id;
                if constexpr (KV == PA_DTYPE_INT8) {
                    s_ksc[i] = id >= 0 ? a.k_scale[static_cast<int64_t>(id) * Hkv + kvh] : 0.0f;
                    const float vsc = id >= 0 ? a.v_scale[static_cast<int64_t>(id) * Hkv + kvh] : 0.0f;
                    const float lv = fmaxf(__log2f(vsc), kMinLog2VScale);  // log2(0) = -inf -> the floor
                    s_vlg[i] = lv;
                    s_vrc[i] = __builtin_amdgcn_exp2f(-lv);
                }
            }
            if constexpr (KV == PA_DTYPE_INT8) {  // blocks past the end (an odd chunk's partner, a step
                if (tid < 4) {                      // past the end): scale 0, keys masked
                    s_ksc[nkc + tid] = 0.0f;
                    s_vlg[nkc + tid] = kMinLog2VScale;
                    s_vrc[nkc + tid] = __builtin_amdgcn_exp2f(-kMinLog2VScale);
                }
            }
            __syncthreads();
            ids_win = -1;
            issue(0, nkc, 0);
            issue(2, nkc, 1);
            if constexpr (ELT == 2) {
                asm volatile("s_waitcnt vmcnt(%0)" : : "n"(NSEG) : "memory");  // pair 0's segments landed
                convert_v(0);
            }
            int slot = 0, load_slot = 2;  // slots of pair jp and of pair jp + 2
            for (int jp = 0; jp < npair; jp++) {
                static_assert(NSEG <= 15, "vmcnt immediate");
                if constexpr (ELT == 2) {
                    // every wave's V segments of pair jp are fp16 (converted during compute(jp - 1))
                    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory");
                } else {
                    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(NSEG) : "memory");
                }
                issue(2 * (jp + 2), nkc, load_slot);
                const int lb = c0 + 2 * jp;
                compute((lb + 2) * 16 > kend_lo, kend, slot, slot == NSLOT - 1 ? 0 : slot + 1, lb, 2 * jp);
                slot = slot == NSLOT - 1 ? 0 : slot + 1;
                load_slot = load_slot == NSLOT - 1 ? 0 : load_slot + 1;
            }
        }
        if constexpr (ELT == 2) {
            if (v_big != 0 && lane == 0) atomicOr(&s_sat, 1 << min(u0 / kPrefillUnits, 31));
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();  // the slots are reused by the next round

        // rows of acc are queries 4q4 + i (int8: their sums live in lanes n = 4q4 + i)
#pragma unroll
        for (int k = 0; k < 2; k++) {
            float li[4];
            if constexpr (KV == PA_DTYPE_INT8) {
                const float l_tot = rows_sum(l_run[k]);
#pragma unroll
                for (int i = 0; i < 4; i++) li[i] = __shfl(l_tot, 4 * q4 + i, 64);
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) li[i] = acc_l[k][i];
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int qi = 4 * q4 + i;
                if (store[k] && qi < nq[k]) {
                    const float inv = 1.0f / li[i];
                    float* o = a.out + (static_cast<int64_t>(q0 + i0[k] + qi) * Hq + head[k]) * D;
#pragma unroll
                    for (int t = 0; t < NT; t++) o[16 * t + n] = acc[k][t][i] * inv;
                }
            }
        }
    }
    if constexpr (ELT == 2) {
        // A round whose V tiles held |v| > 65504, which the fp16 operand cannot carry, is computed
        // again in fp32 from the cache by the same waves (their later stores replace the first
        // ones). Rare: activations that large do not occur in ordinary models. s_sat is final: the
        // last round's barrier follows every wave's flag.
        const int sat = s_sat;
        if (sat != 0) {
            for (int u0 = 0; u0 < QT * G; u0 += kPrefillUnits)
                if (sat & (1 << min(u0 / kPrefillUnits, 31))) prefill_exact_round<D, QF32>(a, u0);
        }
    }
}

template <int D, int KV>
void launch(const PrefillArgs& a, bool qf32, dim3 grid, hipStream_t s) {
    if (qf32) chunked_prefill_kernel<D, KV, true><<<grid, kPrefillThreads, 0, s>>>(a);
    else chunked_prefill_kernel<D, KV, false><<<grid, kPrefillThreads, 0, s>>>(a);
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
    const uint32_t masks = cfg->flags & (PA_FLAG_REFERENCE_LITERAL_MASK | PA_FLAG_NO_MASK);
    if (masks == (PA_FLAG_REFERENCE_LITERAL_MASK | PA_FLAG_NO_MASK))
        return pa::set_error(PA_ERROR_INVALID_CONFIG, "pa_chunked_prefill: conflicting mask flags");
    const int32_t mask_mode = (cfg->flags & PA_FLAG_NO_MASK) ? 2 : ((cfg->flags & PA_FLAG_REFERENCE_LITERAL_MASK) ? 1 : 0);
    if (cfg->kv_dtype == PA_DTYPE_FP32)
        return pa::launch_chunked_prefill_fp32(pa::native(stream), cfg, out, q, q_start_loc, prefix_lens,
                                               static_cast<const float*>(k_cache), static_cast<const float*>(v_cache),
                                               block_tables, num_seqs, max_blocks_per_seq, max_chunk_len, mask_mode);
    if (cfg->head_dim < 64)
        return pa::set_error(PA_ERROR_UNSUPPORTED, "pa_chunked_prefill: bf16 and int8 caches take head_dim 64, 128 or 256");
    if (cfg->kv_dtype == PA_DTYPE_INT8 && (!k_scale || !v_scale))
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_chunked_prefill: int8 cache needs k_scale and v_scale");

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
    a.mask_mode = mask_mode;
    a.scale = pa::resolve_scale(cfg);

    a.qtiles_per_wg = a.group >= pa::kPrefillUnits ? 1 : pa::kPrefillUnits / a.group;
    a.num_qgroups = ((max_chunk_len + 15) / 16 + a.qtiles_per_wg - 1) / a.qtiles_per_wg;
    const int64_t ng = static_cast<int64_t>(num_seqs) * cfg->num_kv_heads;
    const int64_t nwg = static_cast<int64_t>(a.num_qgroups) * ((ng + 7) / 8) * 8;
    if (nwg > 0x7fffffff) return pa::set_error(PA_ERROR_UNSUPPORTED, "pa_chunked_prefill: grid too large");
    a.num_groups = static_cast<int32_t>(ng);
    const dim3 grid(static_cast<uint32_t>(nwg));
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
