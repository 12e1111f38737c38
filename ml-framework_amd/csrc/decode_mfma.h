// decode_mfma.h -- the bf16 / int8 paged-decode kernel (MFMA, persistent waves, balanced split).
//
// Work split: the batch's sequences, as runs of 16-token blocks, are laid end to end and cut into
// ranges of equal block count. A unit is (range, KV head) and belongs to one wave (a worker): the
// launch's waves are numbered blockIdx.x * 4 + wave, and unit u = range * Hkv + kvh goes to worker
// u (workers walk units with a stride of the worker count when there are more units). The 4 waves
// of a workgroup thus take 4 KV heads of one range (or 4 ranges when Hkv is 1 or 2) and read
// neighbouring bytes of the same physical blocks. A range covers the tail of one sequence, whole
// sequences and the head of another; each part, for the unit's KV head, is a row portion. A
// portion that is a whole row (sequence, KV head) writes the normalised output directly; the (at
// most two) partial portions of a unit write (max, sum, unnormalised O) to workspace slots
// 2 * unit + {0: first, 1: last}, and paged_decode_merge_split_kernel combines the slots of every
// split row. Every worker streams the same number of K/V bytes whatever the mix of context lengths,
// and no wave ever waits for another: there is no barrier after the prefix table is built.
//
// A portion is streamed in pieces of at most 64 blocks (lane j holds the id of the piece's block
// j); the running (max, sum, O) carry over from piece to piece and are written when the portion
// ends. Block ids are loaded two pieces ahead. Kernels with head_dim <= 128 and bf16 queries or
// int8 caches also carry the pipeline across pieces: a piece issues the next one's Q and scales at
// its start and its first two blocks in its last two iterations, so a piece or row boundary does
// not drain the blocks in flight. The others start a piece with its own loads (one memory round
// trip).
//
// Fused append (pa_paged_decode_append, bf16 caches): a row streams its first T - 1 cached tokens
// only; the new token (position T - 1, from k_new / v_new) joins the softmax as one more element at
// the end of the row portion that holds the row's last streamed block. No block is patched in
// registers, so the fused kernel streams with the same loop (and carry) as the plain decode. The
// token is written into the cache by the split-merge kernel that follows the decode
// (append_in_merge): written here, among the decode's reads, the V column (one line per dim of
// the tile) cost the step about 3 us whatever the form of the stores. Without a merge launch
// (a single range) the owning wave writes it: its K row as is, its V column by rewriting the
// whole V tile, fetched into LDS when the piece starts, patched there and stored back.
//
// Per block: S^T[16 tokens][16 heads] = K . Q^T on v_mfma_f32_16x16x32_bf16 (query heads padded
// to 16 rows), online softmax in fp32, O[16 heads][D] += P . V on v_mfma_f32_16x16x16_bf16 with P
// split into bf16 high and low parts (~16 significant bits) for bf16 caches, one rounded bf16 P for
// int8 caches. The score layout the first MFMA
// leaves in registers (lane = (token group q4, head n)) is the A-operand layout of the second, so
// P never leaves registers. Three rotating register buffers keep two blocks in flight while a
// third is consumed.
#pragma once

#include "decode_common.h"

namespace pa {

// Online-softmax rescaling is deferred until a block's max exceeds the running max by more than
// this (natural-log units): probabilities then stay below e^8 and fp32 sums stay exact enough,
// while the O accumulators are rescaled on few blocks instead of on most of them.
constexpr float kRescaleThreshold = 8.0f;

template <bool SHARED>
struct MfmaShared {
    int pref[kMaxPersistentSeqs + 1];  // blocks (per KV head row) before row r
    int lens[kMaxPersistentSeqs];      // token bound of row r's blocks (clamped context length)
};
// Shared-prefix decode rows: row r starts at block boff[r] of sequence seq0[r]'s table and its
// query columns are the heads of sequences seq0[r] .. seq0[r] + nmem - 1 (qinfo = seq0 | nmem << 16
// | grouped << 24; grouped rows always leave partials).
template <>
struct MfmaShared<true> {
    int pref[kMaxPersistentSeqs + 1];
    int lens[kMaxPersistentSeqs];
    int boff[kMaxPersistentSeqs];
    int qinfo[kMaxPersistentSeqs];
};

// Blocks [b0, b1) of row (seq, kvh), at most kPieceBlocks of them. slot < 0: the portion the
// piece belongs to is the whole row (final output), else its workspace slot; last: the piece ends
// the portion (its results are written).
struct Piece {
    int seq, kvh, b0, b1, T, slot;
    bool last;
    int nmem;  // shared-prefix decode: query columns are the heads of sequences seq .. seq + nmem - 1
};

constexpr int kPieceBlocks = 64;  // one block id per lane

// Register buffers of a wave's block pipeline (blocks in flight + the one being consumed).
#ifndef PA_INT8_DECODE_BUFFERS
#define PA_INT8_DECODE_BUFFERS 3
#endif
__host__ __device__ constexpr int decode_buffers(int kv) { return kv == PA_DTYPE_INT8 ? PA_INT8_DECODE_BUFFERS : 3; }

// Ids of a piece's blocks: lane j holds block b0 + j (-1 beyond the piece). Ids are range-checked
// where they are used (valid_bid): a check here would make the wave wait for the table load at the
// point of issue instead of when the id is needed. With `extra`, lane b1 - b0 holds the id of
// block b1 as well.
__device__ __forceinline__ int piece_ids(const DecodeArgs& a, const Piece& g, int lane, bool extra = false) {
    const int b = g.b0 + lane;
    int id = -1;
    if (b < g.b1 || (extra && b == g.b1)) id = a.block_tables[static_cast<int64_t>(g.seq) * a.max_blocks_per_seq + b];
    return id;
}
__device__ __forceinline__ int valid_bid(const DecodeArgs& a, int id) { return id < a.num_blocks ? id : -1; }

// Running (max, sum, O) of one row portion; lane (q4, n): head n's max, its share of head n's sum,
// and O rows 4q4 .. 4q4 + 3 of dims 16t + n.
template <int NT>
struct RowState {
    float m_run;  // reference max of head n (exceeded by at most kRescaleThreshold)
    float l_run;  // this lane's share of the running sum of head n
    f32x4_t acc[NT];
    __device__ __forceinline__ void reset() {
        m_run = -INFINITY;
        l_run = 0.0f;
#pragma unroll
        for (int t = 0; t < NT; t++) acc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
};

// Values a piece needs besides its K/V blocks: Q (lane (q4, n): head n's dims of each slab, bf16
// words, or fp32 values in two 16-byte words per slab), the int8 scales of the lane's block (lane
// j: block j of the piece) and the appended token's raw bits.
template <int D, bool QF32>
struct PieceSide {
    static constexpr int NPL = D >= 64 ? D / 64 : 1;  // appended-token values per lane
    static constexpr int NW = QF32 ? NPL : (NPL + 1) / 2;
    uint4 q[QF32 ? D / 16 : D / 32];
    float ks, vs;
    uint32_t nk[NW], nv[NW];
};

// The three rotating register buffers of a wave's block pipeline (two blocks in flight while a
// third is consumed). They outlive a piece: the last iterations of one piece load the first two
// blocks of the next (carry), so a piece boundary does not drain the pipeline.
template <int D, int KV>
struct PipeBufs {
    typename MfmaRaw<KV>::K k[3][D / 32];
    typename MfmaRaw<KV>::V v[3][D / 16];
};

// Vector memory instructions load_block issues per block.
template <int D, int KV>
__host__ __device__ constexpr int decode_block_loads() {
    return KV == PA_DTYPE_INT8 ? D / 64 + D / 64 : D / 32 + D / 32;
}
// s_waitcnt operand: wait until at most N vector memory operations are outstanding (no wait on
// the other counters).
template <int N>
__host__ __device__ constexpr int vmcnt_keep() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    return (N & 15) | 0x7 << 4 | 0xf << 8 | (N >> 4) << 14;
}

// Carry across pieces (head_dim <= 128 with bf16 queries, or with int8 caches, whose K/V buffers
// are half the size): elsewhere the extra registers (the next piece's Q) would spill, so those
// kernels start every piece with its own loads.
template <int D, int KV, bool QF32, bool APPEND>
__host__ __device__ constexpr bool decode_carry() {
    return decode_buffers(KV) == 3 && (!QF32 || KV == PA_DTYPE_INT8) && D <= 128;
}

// Leading empty iterations of a carried piece of nb blocks: its iteration count nb + lead is a
// multiple of 3, the unroll of the three-buffer loop.
__device__ __forceinline__ int piece_lead(int nb) { return (3 - nb % 3) % 3; }

// Fused append (pa_paged_decode_append, bf16 caches): Piece::T counts the streamed tokens, the
// new token sits at position T; the piece that ends the portion holding the row's last streamed
// block appends it.
template <bool APPEND>
__device__ __forceinline__ bool piece_owns_new(const Piece& g) {
    if constexpr (!APPEND) return false;
    return g.last && g.b1 == (g.T + 15) / 16;
}
// The block ids a piece loads: its own, plus for the owning piece whose new token starts a block
// (T % 16 == 0) that block's id in lane b1 - b0 (when the piece has fewer than 64 blocks).
template <bool APPEND>
__device__ __forceinline__ int piece_ids_of(const DecodeArgs& a, const Piece& g, int lane) {
    return piece_ids(a, g, lane, piece_owns_new<APPEND>(g) && (g.T & 15) == 0);
}

// Side loads of piece g (ids: its block ids, lane j = block j): Q, the appended token and, when
// `scales`, the int8 scales (those need the ids, which may still be in flight).
template <int D, int KV, bool QF32, bool APPEND, bool SHARED>
__device__ __forceinline__ void load_side(const DecodeArgs& a, const Piece& g, int ids, bool scales,
                                          PieceSide<D, QF32>& sd) {
    constexpr int NSLAB = D / 32;
    constexpr int NPL = PieceSide<D, QF32>::NPL;
    constexpr int NW = PieceSide<D, QF32>::NW;
    const int lane = threadIdx.x & 63;
    const int q4 = lane >> 4, n = lane & 15;
    const int G = a.group, Hkv = a.num_kv_heads;
    // Column n's query head: head n of the sequence, or (shared-prefix rows) head n % G of member
    // n / G.
    const int ncol = SHARED ? g.nmem * G : G;
    const bool hv = n < ncol;
    const int mi = SHARED && hv ? n / G : 0;
    const int64_t qrow = (static_cast<int64_t>(g.seq + mi) * Hkv * G + g.kvh * G + (hv ? n - mi * G : 0)) * D;
    // Every lane loads (a lane without a head reads head 0 of the row, which exists); the consumer
    // zeroes the columns without a head when it builds the operands (masking here would wait for
    // the load at its issue; a conditional load is compiled into a pointer select through a stack
    // copy).
#pragma unroll
    for (int s = 0; s < NSLAB; s++) {
        const int d0 = k_dim0<D, KV>(s, q4);
        if constexpr (QF32) {
            const uint4* qp = reinterpret_cast<const uint4*>(static_cast<const float*>(a.q) + qrow + d0);
            sd.q[2 * s] = qp[0];
            sd.q[2 * s + 1] = qp[1];
        } else {
            sd.q[s] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.q) + qrow + d0);
        }
    }
    if constexpr (KV == PA_DTYPE_INT8) {  // unconditional: an invalid block's scales are never used
        if (scales) {
            const int sb = ids >= 0 && ids < a.num_blocks ? ids : 0;
            sd.ks = a.k_scale[static_cast<int64_t>(sb) * Hkv + g.kvh];
            sd.vs = a.v_scale[static_cast<int64_t>(sb) * Hkv + g.kvh];
        }
    }
    if constexpr (APPEND) {
        if (piece_owns_new<APPEND>(g) && lane * NPL < D) {
            const int64_t src = (static_cast<int64_t>(g.seq) * Hkv + g.kvh) * D + lane * NPL;
#pragma unroll
            for (int w = 0; w < NW; w++) {
                if constexpr (QF32) {
                    sd.nk[w] = static_cast<const uint32_t*>(a.k_new)[src + w];
                    sd.nv[w] = static_cast<const uint32_t*>(a.v_new)[src + w];
                } else if constexpr (NPL == 1) {
                    sd.nk[w] = static_cast<const uint16_t*>(a.k_new)[src];
                    sd.nv[w] = static_cast<const uint16_t*>(a.v_new)[src];
                } else {
                    sd.nk[w] = static_cast<const uint32_t*>(a.k_new)[(src >> 1) + w];
                    sd.nv[w] = static_cast<const uint32_t*>(a.v_new)[(src >> 1) + w];
                }
            }
        }
    }
}

// Tokens 4 tok_group(q4) .. + 3 of a block are the QK MFMA rows (S^T) and PV MFMA k values of lane
// group q4. bf16 caches exchange groups 1 and 2 (bf16_v_exchange), so their K rows are loaded in
// that order as well.
template <int KV>
__device__ __forceinline__ int tok_group(int q4) {
    return KV == PA_DTYPE_BF16 ? ((q4 & 1) << 1) | (q4 >> 1) : q4;
}

// Loads of block bid (K/V tile of KV head kv) into a pipeline buffer, lane (q4, n): K row n (the
// lane's dims of each slab; bf16: row 4 tok_group(n / 4) + n % 4), V dim n of tokens 4q4 .. 4q4 + 3
// (every 16th dim; loaded 16 bytes per lane, the words put in that order by bf16_v_exchange() /
// int8_v_transpose(), bf16 with tok_group). Loads go through
// per-block buffer descriptors: bid < 0 (past a list, or an invalid id) gives a zero-sized
// descriptor, so its loads return zeros without touching memory. The load sequence is therefore
// identical on every iteration (no branches), which lets the compiler wait for exactly the oldest
// block instead of draining every load in flight.
template <int D, int KV>
__device__ __forceinline__ void load_block(const DecodeArgs& a, typename MfmaRaw<KV>::K (&kr)[D / 32],
                                           typename MfmaRaw<KV>::V (&vr)[D / 16], int bid, int kv) {
    using KR = typename MfmaRaw<KV>::K;
    constexpr int ELT = MfmaRaw<KV>::kElt;
    constexpr int NSLAB = D / 32, TILE = 16 * D;
    static_assert(KV != PA_DTYPE_INT8 || D >= 64, "int8 caches take head_dim 64, 128 or 256");
    // Cache policy: non-temporal for V (each tile is read once) and, for int8 caches, for K too
    // (bf16 K with it measured slower).
    constexpr int kCPK = KV == PA_DTYPE_INT8 ? kLoadNonTemporal : kLoadDefault;
    constexpr int kCPV = kLoadNonTemporal;
    const int lane = threadIdx.x & 63;
    const int q4 = lane >> 4, n = lane & 15;
    const int krow = KV == PA_DTYPE_BF16 ? 4 * tok_group<KV>(n >> 2) + (n & 3) : n;
    const int k_row_off = krow * D * ELT;            // K row krow; slab s of this lane starts at dim k_dim0(s, q4)
    const int64_t tile = bid >= 0 ? (static_cast<int64_t>(bid) * a.num_kv_heads + kv) * TILE * ELT : 0;
    const int bytes = bid >= 0 ? TILE * ELT : 0;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(static_cast<const char*>(a.k_cache) + tile), 0, bytes, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(static_cast<const char*>(a.v_cache) + tile), 0, bytes, kBufferFlags);
    if constexpr (ELT == 1) {  // int8: two slabs (16 codes) per 16-byte load
#pragma unroll
        for (int s = 0; s < NSLAB; s += 2) {
            const uint4 w = buffer_load<uint4, kCPK>(rk, k_row_off + k_dim0<D, KV>(s, q4));
            kr[s] = make_uint2(w.x, w.y);
            kr[s + 1] = make_uint2(w.z, w.w);
        }
    } else {
#pragma unroll
        for (int s = 0; s < NSLAB; s++) kr[s] = buffer_load<KR, kCPK>(rk, k_row_off + k_dim0<D, KV>(s, q4) * ELT);
    }
    if constexpr (KV == PA_DTYPE_BF16) {
        // bf16: load u of lane (q4, n) is tokens 8 (q4 % 2) .. + 7 of dim 32u + 16 (q4 / 2) + n
        // (one contiguous KiB per instruction, two tiles: half the instructions of 8-byte loads);
        // bf16_v_exchange() turns vr[2u], vr[2u + 1] into tiles 2u, 2u + 1.
#pragma unroll
        for (int u = 0; u < D / 32; u++) {
            const uint4 w = buffer_load<uint4, kCPV>(rv, (32 * u + 16 * (q4 >> 1) + n) * 32 + 16 * (q4 & 1));
            vr[2 * u] = make_uint2(w.x, w.y);
            vr[2 * u + 1] = make_uint2(w.z, w.w);
        }
    } else {
        // int8 (D >= 64): load u of lane (q4, n) is all 16 tokens of dim 16 (q4 + 4u) + n (one
        // contiguous KiB per instruction, a quarter of the instructions of 4-byte loads);
        // int8_v_transpose() turns words vr[4u .. 4u + 3] into tiles 4u .. 4u + 3.
#pragma unroll
        for (int u = 0; u < D / 64; u++) {
            const uint4 w = buffer_load<uint4, kCPV>(rv, (16 * (q4 + 4 * u) + n) * 16);
            vr[4 * u] = w.x;
            vr[4 * u + 1] = w.y;
            vr[4 * u + 2] = w.z;
            vr[4 * u + 3] = w.w;
        }
    }
}

// int8 V words after a wide load: lane (q4, n) holds, in w[k], tokens 4k .. 4k + 3 of dim
// 16 (q4 + 4u) + n. The PV MFMA of tile 4u + t needs tokens 4 q4 .. 4 q4 + 3 of dim 16 (4u + t) + n
// in lane (q4, n): word q4 of row group t, i.e. a 4 x 4 transpose of words across the four rows of
// 16 lanes. v_permlane32_swap exchanges rows 2, 3 of its first operand with rows 0, 1 of its second,
// v_permlane16_swap the odd rows of the first with the even rows of the second.
__device__ __forceinline__ void int8_v_transpose(uint32_t& w0, uint32_t& w1, uint32_t& w2, uint32_t& w3) {
    const auto a = __builtin_amdgcn_permlane32_swap(w0, w2, false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(w1, w3, false, false);
    const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
    const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
    w0 = c[0];
    w1 = c[1];
    w2 = d[0];
    w3 = d[1];
}

// bf16 V after a wide load: lane group q4 holds, in (x0, x1), tokens 8 (q4 % 2) .. + 3 and
// 8 (q4 % 2) + 4 .. + 7 of tile 2u (q4 < 2) or 2u + 1 (q4 >= 2). One exchange of rows 2, 3 of x0
// with rows 0, 1 of x1 (per 32-bit word) leaves tile 2u in x0 and tile 2u + 1 in x1, each with
// tokens 4 tok_group(q4) .. + 3 in lane group q4 (groups 1 and 2 exchanged).
__device__ __forceinline__ void bf16_v_exchange(uint2& x0, uint2& x1) {
    const auto a = __builtin_amdgcn_permlane32_swap(x0.x, x1.x, false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(x0.y, x1.y, false, false);
    x0 = make_uint2(a[0], b[0]);
    x1 = make_uint2(a[1], b[1]);
}

// One piece, streamed by one wave; my_bid = piece_ids(..). has_next, nxt, nxt_ids: the next piece
// of the worker and its block ids (loaded during the previous piece). With carry
// (decode_carry()), the piece's first two blocks and side loads were issued before it (by the
// previous piece, or for a worker's first piece by the worker), and it issues the next piece's
// side loads at its start and its first two blocks in its last two iterations. prefetch_next() is
// called once, after the piece's first loads, to start the id loads of the piece after the next.
// s_new: this wave's LDS staging of the appended token (2 * D floats); s_vt: its V tile staging
// (16 D bf16).
template <int D, int KV, bool QF32, bool APPEND, bool SHARED, typename Prefetch>
__device__ __forceinline__ void mfma_piece(const DecodeArgs& a, const Piece& g, int my_bid,
                                           PieceSide<D, QF32>& side, PipeBufs<D, KV>& bufs, RowState<D / 16>& st,
                                           float* s_new, uint4* s_vt, const bool& has_next, const Piece& nxt,
                                           const int& nxt_ids,
                                           PieceSide<D, QF32>& nside, Prefetch&& prefetch_next) {
    using Raw = MfmaRaw<KV>;
    constexpr int NSLAB = D / 32;  // QK MFMAs (k = 32 dims each)
    constexpr int NT = D / 16;     // PV n-tiles of 16 dims
    constexpr int TILE = 16 * D;   // elements per (block, KV head) tile
    constexpr int NPL = PieceSide<D, QF32>::NPL;
    constexpr int NW = PieceSide<D, QF32>::NW;
    constexpr bool CARRY = decode_carry<D, KV, QF32, APPEND>();

    const int lane = threadIdx.x & 63;
    const int q4 = lane >> 4;  // token group (QK C rows) / k group of the MFMA operands
    const int n = lane & 15;   // head column of S^T / row of P / dim within a PV tile
    const int G = a.group, Hkv = a.num_kv_heads;
    const int seq = g.seq, kvh = g.kvh, T = g.T;
    const int nb = g.b1 - g.b0;

    // Loads issued at the piece's start, in this order: its first two K/V blocks and its side loads
    // (without carry), the ids of the piece after the next (prefetch callback) and the next piece's
    // side loads (with carry). Memory returns in order, so the K/V requests go out first; none of the other values is
    // used right after its load (that would stall the wave on the load's latency).
    // Fused append (bf16 caches; int8 caches are appended by a separate launch first): the piece
    // that ends the row's owning portion fetches the new token with its side loads (lane l: dims
    // l*NPL ..); the token's raw bits (fp32, or bf16 packed two per word) are decoded at the end.
    static_assert(!(APPEND && KV == PA_DTYPE_INT8), "int8 caches are appended before the decode");
    auto entry = [](int j) { return j; };
    auto new_val = [&](const uint32_t (&raw)[NW], int e) -> float {
        if constexpr (QF32) return __uint_as_float(raw[e]);
        else if constexpr (NPL == 1) return __uint_as_float(raw[0] << 16);
        else return __uint_as_float((e & 1) ? (raw[e >> 1] & 0xffff0000u) : (raw[e >> 1] << 16));
    };
    // Q^T operand: lane (q4, n) holds head n, dims k_dim0(s, q4) .. +8 of slab s (zero rows for n >= G).
    bf16x8_t qhi[NSLAB], qlo[QF32 ? NSLAB : 1];
    // int8 caches: the K codes go to v_mfma_i32_16x16x64_i8 as they are, against Q as a 16-bit fixed
    // point number in two int8 digits: q ~ q_sq * (256 hi + lo), q_sq = max|q| of the head / 32639,
    // so S = q_sq (256 K.hi + K.lo) exactly in int32 (per score an error of at most q_sq / 2 per
    // dim times |code|, about 2e-5 of max|q| 127 sqrt(D)). Slab t covers the lane's dims
    // k_dim0(2t, q4) .. +16, i.e. K registers 2t and 2t + 1.
    constexpr int NI8 = NSLAB / 2;
    i32x4_t qdh[KV == PA_DTYPE_INT8 ? NI8 : 1], qdl[KV == PA_DTYPE_INT8 ? NI8 : 1];
    float q_sq_scaled = 0.0f;  // q_sq times the softmax scale
    auto int8_q_digits = [&](const float (&x)[NSLAB][8]) {
        float mx = 0.0f;
#pragma unroll
        for (int sl = 0; sl < NSLAB; sl++)
#pragma unroll
            for (int e = 0; e < 8; e++) mx = fmaxf(mx, fabsf(x[sl][e]));
        mx = rows_max(mx);  // max |q| of head n
        q_sq_scaled = mx * (1.0f / 32639.0f) * a.scale;
        const float inv = mx > 0.0f ? 32639.0f / mx : 0.0f;
#pragma unroll
        for (int t = 0; t < NI8; t++) {
            uint32_t wh[4], wl[4];
#pragma unroll
            for (int w = 0; w < 4; w++) {
                wh[w] = 0;
                wl[w] = 0;
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const int e = 4 * w + b;  // dim e of the slab's 16
                    const int q16 = static_cast<int>(__builtin_rintf(x[2 * t + (e >> 3)][e & 7] * inv));
                    const int lo = ((q16 + 128) & 255) - 128;
                    const int hi = (q16 - lo) >> 8;
                    wh[w] |= (static_cast<uint32_t>(hi) & 255u) << (8 * b);
                    wl[w] |= (static_cast<uint32_t>(lo) & 255u) << (8 * b);
                }
            }
            qdh[t] = __builtin_bit_cast(i32x4_t, make_uint4(wh[0], wh[1], wh[2], wh[3]));
            qdl[t] = __builtin_bit_cast(i32x4_t, make_uint4(wl[0], wl[1], wl[2], wl[3]));
        }
    };
    const int ncol = SHARED ? g.nmem * G : G;
    // Q words of the side loads, zero in the columns without a head (n >= ncol).
    const uint32_t qmask = n < ncol ? 0xffffffffu : 0u;
    auto qword = [&](int i) {
        const uint4 w = side.q[i];
        return make_uint4(w.x & qmask, w.y & qmask, w.z & qmask, w.w & qmask);
    };
    // Slab s of Q as 8 floats.
    auto q_floats = [&](int s, float (&x)[8]) {
        if constexpr (QF32) {
            const uint4 w0 = qword(2 * s), w1 = qword(2 * s + 1);
            const uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int e = 0; e < 8; e++) x[e] = __uint_as_float(w[e]);
        } else {
            const uint4 raw = qword(s);
            const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
            for (int e = 0; e < 8; e++) x[e] = __uint_as_float((e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16));
        }
    };
    // Q operands from the side loads.
    auto prep_q = [&]() {
        if constexpr (KV == PA_DTYPE_INT8) {
            float x[NSLAB][8];
#pragma unroll
            for (int s = 0; s < NSLAB; s++) q_floats(s, x[s]);
            int8_q_digits(x);
        } else {
#pragma unroll
            for (int s = 0; s < NSLAB; s++) {
                if constexpr (QF32) {
                    float x[8];
                    q_floats(s, x);
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
                    qhi[s] = __builtin_bit_cast(bf16x8_t, qword(s));
                }
            }
        }
    };

    // The next piece (carry): its block count and this piece's iteration count nbp, a multiple of 3
    // (the loop is unrolled over the three buffers). A piece is padded at its front: its first
    // `lead` = piece_lead(nb) iterations compute nothing and iteration j computes block j - lead,
    // so the last two iterations compute the piece's last blocks while loading the next piece's
    // iterations 0 and 1 (item nbp + k, buffer k): the pipeline stays full across the boundary.
    // (Padded at the end instead, a piece of 3k + 1 or 3k + 2 blocks issued the next piece's first
    // loads only after its last compute: a memory latency per boundary.) The next piece's side
    // loads go out at this piece's start (its ids were loaded during the previous piece).
    const int lead = CARRY ? piece_lead(nb) : 0;
    const int nbp = nb + lead;
    const int nnb = CARRY && has_next ? nxt.b1 - nxt.b0 : 0;
    const int nlead = piece_lead(nnb);
    auto side_next = [&]() {
        if constexpr (CARRY) {
            if (has_next) load_side<D, KV, QF32, APPEND, SHARED>(a, nxt, nxt_ids, true, nside);
        }
    };

    using KR = typename Raw::K;
    using VR = typename Raw::V;
    // Item i (iteration i's block): block i - lead of this piece (lead <= i < nbp), nothing (the
    // lead), or the next piece's iteration i - nbp (its block i - nbp - nlead; zero-sized past
    // its list).
    auto load = [&](KR (&kr)[NSLAB], VR (&vr)[NT], int i) {
        int bid = -1, kv = kvh;
        if (i >= lead && i < nbp) {
            bid = valid_bid(a, __builtin_amdgcn_readlane(my_bid, entry(i - lead) & 63));
        } else if (CARRY && i >= nbp + nlead && i - nbp - nlead < nnb) {
            bid = valid_bid(a, __builtin_amdgcn_readlane(nxt_ids, i - nbp - nlead));
            kv = nxt.kvh;
        }
        load_block<D, KV>(a, kr, vr, bid, kv);
    };

    float& m_run = st.m_run;
    float& l_run = st.l_run;
    f32x4_t(&acc)[NT] = st.acc;

    auto compute = [&](KR (&kr)[NSLAB], VR (&vr)[NT], int j) {
        const int e = entry(j);
        const int bid = valid_bid(a, __builtin_amdgcn_readlane(my_bid, e));
        float ks = 1.0f, vfac = 1.0f;
        if constexpr (KV == PA_DTYPE_INT8) {
            ks = bid >= 0 ? readlane_f(side.ks, e) : 0.0f;
            vfac = bid >= 0 ? readlane_f(side.vs, e) : 0.0f;
        }
        // S^T[token 4 tok_group(q4) + i][head n]
        f32x4_t s = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (KV == PA_DTYPE_INT8) {
            i32x4_t ch = {0, 0, 0, 0}, cl = {0, 0, 0, 0};
#pragma unroll
            for (int t = 0; t < NI8; t++) {
                const i32x4_t kop = __builtin_bit_cast(i32x4_t, make_uint4(kr[2 * t].x, kr[2 * t].y, kr[2 * t + 1].x,
                                                                            kr[2 * t + 1].y));
                ch = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop, qdh[t], ch, 0, 0, 0);
                cl = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop, qdl[t], cl, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
                s[i] = static_cast<float>(ch[i] * 256 + cl[i]);  // |.| < 127 * 32639 * D < 2^31
        } else {
#pragma unroll
            for (int sl = 0; sl < NSLAB; sl++) {
                const bf16x8_t kop = k_operand(kr[sl]);
                s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qhi[sl], s, 0, 0, 0);
                if constexpr (QF32) s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qlo[sl], s, 0, 0, 0);
            }
        }
        // int8: (Q16 . code) times q_sq k_scale scale, one factor per block and head
        const float sf = KV == PA_DTYPE_INT8 ? ks * q_sq_scaled : a.scale;
        float sc[4];
#pragma unroll
        for (int i = 0; i < 4; i++) sc[i] = s[i] * sf;
        // only a row's last block can hold tokens past T (a uniform test: no per-score compare
        // on the others)
        if ((g.b0 + e + 1) * 16 > T) {
            const int lim = T - ((g.b0 + e) * 16 + 4 * tok_group<KV>(q4));
#pragma unroll
            for (int i = 0; i < 4; i++) sc[i] = i < lim ? sc[i] : -INFINITY;
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
        if constexpr (KV == PA_DTYPE_INT8) {
#pragma unroll
            for (int u = 0; u < D / 64; u++) int8_v_transpose(vr[4 * u], vr[4 * u + 1], vr[4 * u + 2], vr[4 * u + 3]);
            // int8 caches (bar 2e-2): one bf16 P, rounded to nearest even (relative error <= 2^-9;
            // v_cvt_pk_bf16_f32), half the PV MFMAs of the split below. p is finite and non-negative.
            uint32_t pr[2];
#pragma unroll
            for (int e = 0; e < 2; e++) pr[e] = pack_bf16_rne(p[2 * e], p[2 * e + 1]);
            const s16x4_t pb = __builtin_bit_cast(s16x4_t, make_uint2(pr[0], pr[1]));
#pragma unroll
            for (int t = 0; t < NT; t++)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pb, v_operand(vr[t]), acc[t], 0, 0, 0);
        } else {
#pragma unroll
            for (int u = 0; u < D / 32; u++) bf16_v_exchange(vr[2 * u], vr[2 * u + 1]);
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
        }
    };

    // Fused append: the owning piece's new-token block (the last streamed one, or when the token
    // starts a block the one after it, whose id the piece loaded in lane nb when it has one) and
    // the prefetch of its V tile into this wave's LDS area s_vt (LDS-direct loads: no registers
    // held across the loop; a zero-sized descriptor for an invalid id writes zeros, never stored).
    int abid = -1;
    auto prefetch_vtile = [&]() {
        if constexpr (APPEND) {
            if (piece_owns_new<APPEND>(g) && !a.append_in_merge) {
                if ((T & 15) != 0) {
                    abid = __builtin_amdgcn_readlane(my_bid, nb - 1);
                } else if (nb < kPieceBlocks) {
                    abid = __builtin_amdgcn_readlane(my_bid, nb);
                } else {  // a piece of 64 blocks has no lane for it: a table load here (rare)
                    int zero = 0;
                    asm volatile("" : "+v"(zero));  // a vector load (vmcnt), not a scalar one
                    abid = __builtin_amdgcn_readfirstlane(
                        a.block_tables[static_cast<int64_t>(seq) * a.max_blocks_per_seq + T / 16 + zero]);
                }
                abid = valid_bid(a, abid);
                constexpr uint32_t kTileBytes = TILE * 2;
                const int64_t tile = abid >= 0 ? (static_cast<int64_t>(abid) * Hkv + kvh) * kTileBytes : 0;
                const u32x4_t rv = buffer_rsrc_words(static_cast<const char*>(a.v_cache) + tile,
                                                     abid >= 0 ? kTileBytes : 0u);
                const uint32_t base = lds_address(s_vt);
#pragma unroll
                for (uint32_t i = 0; i < (kTileBytes + 1023) / 1024; i++)
                    lds_load16(rv, 16 * lane + 1024 * i, base + 1024 * i);
            }
        }
    };

    if constexpr (decode_buffers(KV) != 3) {
        // NB rotating register buffers: NB - 1 blocks in flight while one is consumed (int8 blocks
        // carry half the bytes of bf16 ones, so more of them are kept in flight). No carry.
        constexpr int NB = decode_buffers(KV);
        KR kbuf[NB][NSLAB];
        VR vbuf[NB][NT];
#pragma unroll
        for (int i = 0; i < NB - 1; i++) load(kbuf[i], vbuf[i], i);
        load_side<D, KV, QF32, APPEND, SHARED>(a, g, my_bid, true, side);
        prefetch_next();
        prep_q();
        int j = 0;
        while (j < nb) {
#pragma unroll
            for (int b = 0; b < NB; b++) {
                load(kbuf[(b + NB - 1) % NB], vbuf[(b + NB - 1) % NB], j + NB - 1);
                compute(kbuf[b], vbuf[b], j);
                if (++j >= nb) break;
            }
        }
    } else {
        // Three rotating register buffers (A, B, X = bufs 0, 1, 2): two blocks in flight while a
        // third is consumed. Loads of items past the piece (or of the next piece's blocks past its
        // list) are zero-sized (no memory traffic), so they are issued regardless.
        auto& ka = bufs.k[0];
        auto& kb = bufs.k[1];
        auto& kx = bufs.k[2];
        auto& va = bufs.v[0];
        auto& vb = bufs.v[1];
        auto& vx = bufs.v[2];
        int j = 0;
        if constexpr (CARRY) {
            // Items 0, 1 are in A, B and the side loads in `side` (issued by the previous piece,
            // or for a worker's first piece before it); the loop's last two iterations issue the
            // next piece's first two blocks.
            prefetch_vtile();
            prefetch_next();
            side_next();
            prep_q();
            // The ids of this piece and the next were loaded a piece ago: wait for them here, not
            // inside the loop (where a first use would make every iteration drain the loads).
            asm volatile("" ::"v"(my_bid), "v"(nxt_ids));
            do {
                load(kx, vx, j + 2);
                if (j >= lead) compute(ka, va, j - lead);
                ++j;
                load(ka, va, j + 2);
                if (j >= lead) compute(kb, vb, j - lead);
                ++j;
                load(kb, vb, j + 2);
                if (j >= lead) compute(kx, vx, j - lead);
                ++j;
            } while (j < nbp);
            // Every vector memory access but the next piece's two blocks (the last 2 * LPI) has
            // completed by now. Waiting on that explicitly (free) tells the compiler so: the ids
            // and side values loaded before the loop are then known to be in registers, and the
            // next piece does not drain its carried loads to use them.
            __builtin_amdgcn_s_waitcnt(vmcnt_keep<2 * decode_block_loads<D, KV>()>());
        } else {
            load(ka, va, 0);
            load(kb, vb, 1);
            load_side<D, KV, QF32, APPEND, SHARED>(a, g, my_bid, true, side);
            prefetch_vtile();
            prefetch_next();
            prep_q();
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
            // the V tile prefetch (older than the blocks just computed) has landed in LDS
            if constexpr (APPEND) __builtin_amdgcn_s_waitcnt(vmcnt_keep<0>());
        }
    }

    if (!g.last) return;
    if constexpr (APPEND) {
        if (piece_owns_new<APPEND>(g)) {
            // The new token joins the softmax with the values the cache holds after the append
            // (bf16 by truncation), staged in LDS so every lane can read the dims it needs.
            float kx[NPL], vx[NPL];
#pragma unroll
            for (int e = 0; e < NPL; e++) {
                kx[e] = __uint_as_float(__float_as_uint(new_val(side.nk, e)) & 0xffff0000u);
                vx[e] = __uint_as_float(__float_as_uint(new_val(side.nv, e)) & 0xffff0000u);
            }
            uint16_t* vt16 = reinterpret_cast<uint16_t*>(s_vt);
            const int r = T & 15;
            if (lane * NPL < D) {
#pragma unroll
                for (int e = 0; e < NPL; e++) {
                    s_new[lane * NPL + e] = kx[e];
                    s_new[D + lane * NPL + e] = vx[e];
                    vt16[(lane * NPL + e) * 16 + r] = static_cast<uint16_t>(__float_as_uint(vx[e]) >> 16);
                }
            }
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the stores have landed in LDS
            __builtin_amdgcn_wave_barrier();
            // Score of head n: q . k over this lane's dims of every slab, summed over the four
            // lane groups of column n, then the scale (Q as the MFMA operands hold it).
            float dot = 0.0f;
#pragma unroll
            for (int sl = 0; sl < NSLAB; sl++) {
                const int d0 = k_dim0<D, KV>(sl, q4);
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    float x = static_cast<float>(qhi[sl][e]);
                    if constexpr (QF32) x += static_cast<float>(qlo[sl][e]);
                    dot = __builtin_fmaf(x, s_new[d0 + e], dot);
                }
            }
            const float sc = rows_sum(dot) * a.scale;
            const float m_new = fmaxf(m_run, sc);
            const float alpha = __expf(m_run - m_new);
            const float pn = __expf(sc - m_new);
            l_run = l_run * alpha + (q4 == 0 ? pn : 0.0f);
            m_run = m_new;
            float ar[4], pr[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                ar[i] = __shfl(alpha, 4 * q4 + i, 64);
                pr[i] = __shfl(pn, 4 * q4 + i, 64);
            }
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const float vv = s_new[D + 16 * t + n];
#pragma unroll
                for (int i = 0; i < 4; i++) acc[t][i] = __builtin_fmaf(pr[i], vv, acc[t][i] * ar[i]);
            }
            // The cache (unless the merge kernel writes the token): K row r as is, the V tile
            // (patched in LDS above) in full lines.
            if (abid >= 0 && !a.append_in_merge) {
                const int64_t tile = (static_cast<int64_t>(abid) * Hkv + kvh) * TILE;
                uint16_t* kc = static_cast<uint16_t*>(const_cast<void*>(a.k_cache)) + tile + r * D;
                if (lane * NPL < D) {
#pragma unroll
                    for (int e = 0; e < NPL; e++)
                        kc[lane * NPL + e] = static_cast<uint16_t>(__float_as_uint(kx[e]) >> 16);
                }
                uint4* vg = reinterpret_cast<uint4*>(static_cast<uint16_t*>(const_cast<void*>(a.v_cache)) + tile);
                const uint4* vl = reinterpret_cast<const uint4*>(s_vt);
#pragma unroll
                for (int i = 0; i < (TILE * 2 + 1023) / 1024; i++)
                    if (lane + 64 * i < TILE * 2 / 16) vg[lane + 64 * i] = vl[lane + 64 * i];
            }
        }
    }
    // ---- the portion ends: write it (lane (q4, n) holds O rows 4q4 .. 4q4 + 3, dims 16t + n) ----
    const float l_tot = rows_sum(l_run);  // head n's sum, in every lane of column n
    float M[4], L[4];                     // of head 4q4 + i, read from lane 4q4 + i (column 4q4 + i)
#pragma unroll
    for (int i = 0; i < 4; i++) {
        M[i] = __shfl(m_run, 4 * q4 + i, 64);
        L[i] = __shfl(l_tot, 4 * q4 + i, 64);
    }
    if (4 * q4 < ncol) {
        const int64_t row0 = static_cast<int64_t>(seq) * Hkv * G + kvh * G;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int h = 4 * q4 + i;
            if (h >= ncol) break;
            if (g.slot < 0) {
                const float inv = 1.0f / L[i];
#pragma unroll
                for (int t = 0; t < NT; t++) a.out[(row0 + h) * D + 16 * t + n] = acc[t][i] * inv;
            } else {
                const int64_t pidx = static_cast<int64_t>(g.slot) * (SHARED ? kPrefixSlotRows : G) + h;
#pragma unroll
                for (int t = 0; t < NT; t++) a.ws_o[pidx * D + 16 * t + n] = acc[t][i];
                if (n == 0) {
                    a.ws_m[pidx] = M[i];
                    a.ws_l[pidx] = L[i];
                }
            }
        }
    }
    st.reset();
}

// Persistent decode kernel over at most kMaxPersistentSeqs - 1 rows: the sequences, or (SHARED)
// the plan's prefix rows followed by one suffix row per sequence.
template <int D, int KV, bool QF32, bool APPEND, bool SHARED>
__global__ __launch_bounds__(64 * decode_waves(D), D > 128 ? 1 : 2) void paged_decode_mfma_persistent_kernel(const DecodeArgs a,
                                                                                             int32_t num_seqs) {
    static_assert(!(APPEND && SHARED), "the shared-prefix decode does not append");
    constexpr int WAVES = decode_waves(D);
    constexpr int THREADS = 64 * WAVES;
    __shared__ MfmaShared<SHARED> sh;
    __shared__ float s_app[APPEND ? WAVES : 1][2 * D];  // per wave: the appended token's K and V values
    __shared__ uint4 s_vtile[APPEND ? WAVES : 1][APPEND ? D * 16 * 2 / 16 : 1];  // per wave: a V tile
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Blocks per row of each sequence; exclusive prefix over sequences, built by the workgroup.
    // All PER lengths are loaded before any is used, so the loads overlap (a use between them would
    // serialise PER memory round trips).
    constexpr int PER = (kMaxPersistentSeqs + THREADS - 1) / THREADS;
    const int NG = SHARED ? a.num_groups : 0;
    const int R = NG + num_seqs;  // rows
    const int G = a.group;
    // Row r's record: the context length (and, SHARED, the sequence's {group, shared blocks}), or
    // a prefix row's group {first sequence, members, shared blocks}.
    int raw[PER], x1[PER], x2[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int r = min(tid * PER + k, R - 1);
        x1[k] = 0;
        x2[k] = 0;
        if (SHARED && r < NG) {
            const int32_t* gr = a.plan + static_cast<int64_t>(r) * kPlanGroupInts;
            raw[k] = gr[0];
            x1[k] = gr[1];
            x2[k] = gr[2];
        } else {
            raw[k] = a.context_lens[r - NG];
            if constexpr (SHARED) {
                const int32_t* si = a.plan + static_cast<int64_t>(NG) * kPlanGroupInts +
                                    static_cast<int64_t>(r - NG) * kPlanSeqInts;
                x1[k] = si[0];
                x2[k] = si[1];
            }
        }
    }
    int cnt[PER];
    int local = 0;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int r = tid * PER + k;
        int c = 0;
        if (r < R) {
            if (SHARED && r < NG) {
                // A record that does not fit the call (members beyond num_seqs, more columns than
                // one MFMA tile, no shared block) gives an empty row.
                const int first = raw[k], nm = x1[k];
                const bool ok = first >= 0 && nm >= 2 && nm * G <= 16 && first <= num_seqs - nm && x2[k] > 0;
                const int T = ok ? clamp_len(a, min(x2[k], a.max_blocks_per_seq) * 16) : 0;
                sh.lens[r] = T;
                c = T <= 0 ? 0 : (T + 15) / 16;
                if constexpr (SHARED) {
                    sh.boff[r] = 0;
                    sh.qinfo[r] = (ok ? first : 0) | (ok ? nm : 1) << 16 | 1 << 24;
                }
            } else {
                // Fused append: the row streams its first T - 1 tokens; the new token at T - 1
                // joins at the end (T == 1: nothing streamed, see below).
                const int T = clamp_len(a, raw[k]) - (APPEND ? 1 : 0);
                sh.lens[r] = T;
                c = T <= 0 ? 0 : (T + 15) / 16;
                if constexpr (SHARED) {
                    const bool grouped = x1[k] >= 0 && x1[k] < NG;
                    const int skip = grouped ? min(max(x2[k], 0), c) : 0;
                    c -= skip;
                    sh.boff[r] = skip;
                    sh.qinfo[r] = (r - NG) | 1 << 16 | (grouped ? 1 : 0) << 24;
                }
            }
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
    __syncthreads();
    int run = wave_off + incl - local;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int r = tid * PER + k;
        if (r <= R) {
            sh.pref[r] = run;
            if (blockIdx.x == 0) a.ws_pref[r] = run;  // read by the merge kernel
        }
        run += cnt[k];
    }
    __syncthreads();

    const int Hkv = a.num_kv_heads;
    // Sequences with no context produce zeros. Fused append: a sequence whose only token is the new
    // one (context length 1) produces that token's V (bf16 by truncation) in every head of its KV
    // head, and the token is written into row 0 of its first block.
    for (int s = blockIdx.x; s < num_seqs; s += gridDim.x) {
        if (sh.lens[NG + s] > 0) continue;
        const int n = Hkv * a.group * D;
        if (APPEND && sh.lens[NG + s] == 0) {
            const bool f32 = !a.q_bf16;
            for (int idx = tid; idx < n; idx += THREADS) {
                const int kvh = idx / (a.group * D), d = idx % D;
                const float v = act_at(a.v_new, f32, (static_cast<int64_t>(s) * Hkv + kvh) * D + d);
                a.out[static_cast<int64_t>(s) * n + idx] = __uint_as_float(__float_as_uint(v) & 0xffff0000u);
            }
            const int bid = a.block_tables[static_cast<int64_t>(s) * a.max_blocks_per_seq];
            if (bid >= 0 && bid < a.num_blocks) {
                uint16_t* kc = static_cast<uint16_t*>(const_cast<void*>(a.k_cache));
                uint16_t* vc = static_cast<uint16_t*>(const_cast<void*>(a.v_cache));
                for (int idx = tid; idx < Hkv * D; idx += THREADS) {
                    const int kvh = idx / D, d = idx % D;
                    const int64_t src = (static_cast<int64_t>(s) * Hkv + kvh) * D + d;
                    const int64_t tile = (static_cast<int64_t>(bid) * Hkv + kvh) * 16 * D;
                    kc[tile + d] = pa::bf16_trunc(act_at(a.k_new, f32, src));
                    vc[tile + d * 16] = pa::bf16_trunc(act_at(a.v_new, f32, src));
                }
            }
            continue;
        }
        for (int idx = tid; idx < n; idx += THREADS) a.out[static_cast<int64_t>(s) * n + idx] = 0.0f;
    }

    // Units u = range * Hkv + kvh; unit u walks blocks [range * C, (range + 1) * C) of the
    // sequence-major block list for KV head kvh, on worker u (mod the worker count W). Workers
    // u .. u + Hkv - 1 run together and read the same physical blocks (all KV heads of a block are
    // one contiguous Hkv * 16 * D run). From here on every wave works alone.
    const int64_t total = sh.pref[R];
    if (total == 0) return;
    const int64_t W = a.split_grid;
    const int64_t C = split_range_blocks(a, total);
    // Per-sequence split (a.num_splits = P > 0, not for the shared-prefix decode): unit u =
    // ((seq * P) + k) * Hkv + kvh takes partition k of row (seq, kvh), blocks [k c, (k + 1) c) of
    // the row with c = ceil(blocks / P); its partial goes to slot 2u.
    const int NSP = SHARED ? 0 : a.num_splits;
    const int64_t units = NSP > 0 ? static_cast<int64_t>(num_seqs) * NSP * Hkv : (total + C - 1) / C * Hkv;
    // int8 caches: workgroup b runs on XCD b % 8, and consecutive logical workgroups are placed on
    // one XCD, so the KV heads of a range (and neighbouring ranges) are read from one L2 at about
    // the same time (C4 134.8 -> 132.2 us; bf16 caches measured slower with it, 53.3 -> 54.9 us).
    int lb = static_cast<int>(blockIdx.x);
    if constexpr (KV == PA_DTYPE_INT8) {
        const int nwg = static_cast<int>(gridDim.x);
        if (nwg % 8 == 0) lb = static_cast<int>((blockIdx.x % 8) * (nwg / 8) + blockIdx.x / 8);
    }
    int64_t u = static_cast<int64_t>(lb) * WAVES + wave;
    if (u >= W || u >= units) return;
    int64_t r = u / Hkv;
    int kvh = static_cast<int>(u - r * Hkv);
    int64_t p = r * C, end = min(total, p + C);
    // Per-sequence split: unit u's block range in the sequence-major list (empty when the row has
    // fewer than k + 1 partitions' worth of blocks).
    auto split_range = [&](int64_t su, int64_t& pp, int64_t& ee) {
        const int64_t sr = su / Hkv;
        const int ns = NSP > 0 ? NSP : 1;  // only called with NSP > 0
        const int sq = static_cast<int>(sr / ns), k = static_cast<int>(sr - static_cast<int64_t>(sq) * ns);
        const int nbr = sh.pref[sq + 1] - sh.pref[sq];
        const int c = (nbr + ns - 1) / ns;
        pp = sh.pref[sq] + min(nbr, k * c);
        ee = sh.pref[sq] + min(nbr, (k + 1) * c);
    };
    if (NSP > 0) {
        // the worker's first non-empty unit
        for (;;) {
            split_range(u, p, end);
            if (p < end) break;
            u += W;
            if (u >= units) return;
        }
        r = u / Hkv;
        kvh = static_cast<int>(u - r * Hkv);
    }
    // Sequence holding block position pos (pref[s] <= pos < pref[s + 1]; pos < total): a binary
    // search, so a worker whose range lies far into the batch does not start late behind a chain of
    // dependent LDS reads.
    auto locate = [&](int64_t pos) {
        int lo = 0, hi = R;  // pref[lo] <= pos < pref[hi]
        while (hi - lo > 1) {
            const int h = (lo + hi) >> 1;
            if (sh.pref[h] <= pos) lo = h;
            else hi = h;
        }
        return lo;
    };
    int seq = locate(p);  // then scanned forward while positions increase
    bool mid = false;     // the next piece continues the current row portion
    int prow_end = 0;     // block (within the row) where the unit's portion of the row ends
    int pslot = -1;       // the portion's output: -1 the whole row, else its workspace slot
    auto next_piece = [&](Piece& g) -> bool {
        if (!mid) {
            if (p >= end) {
                do {
                    u += W;
                    if (u >= units) return false;
                    r = u / Hkv;
                    kvh = static_cast<int>(u - r * Hkv);
                    if (NSP > 0) {
                        split_range(u, p, end);
                    } else {
                        p = r * C;
                        end = min(total, p + C);
                    }
                } while (p >= end);
                seq = locate(p);
            }
            while (sh.pref[seq + 1] <= p) seq++;
            const int nbr = sh.pref[seq + 1] - sh.pref[seq];
            const int pb0 = static_cast<int>(p - sh.pref[seq]);
            prow_end = static_cast<int>(min(static_cast<int64_t>(nbr), pb0 + (end - p)));
            bool grouped = false;
            if constexpr (SHARED) grouped = (sh.qinfo[seq] >> 24) != 0;
            if (pb0 == 0 && prow_end == nbr) pslot = grouped ? a.row_slot_base + seq * Hkv + kvh : -1;  // whole row
            else pslot = static_cast<int>(2 * u + (NSP == 0 && p != r * C ? 1 : 0));
        }
        const int b0 = static_cast<int>(p - sh.pref[seq]);
        const int b1 = min(prow_end, b0 + kPieceBlocks);
        mid = b1 < prow_end;
        if constexpr (SHARED) {
            const int qi = sh.qinfo[seq], bo = sh.boff[seq];
            g = Piece{qi & 0xffff, kvh, bo + b0, bo + b1, sh.lens[seq], pslot, !mid, (qi >> 16) & 0xff};
        } else {
            g = Piece{seq, kvh, b0, b1, sh.lens[seq], pslot, !mid, 1};
        }
        p += b1 - b0;
        return true;
    };
    RowState<D / 16> st;
    st.reset();
    float* s_new = &s_app[APPEND ? wave : 0][0];
    uint4* s_vt = &s_vtile[APPEND ? wave : 0][0];
    PipeBufs<D, KV> bufs;
    PieceSide<D, QF32> side, nside;
    // Pieces in flight: cur (streaming), nxt (ids loaded during the previous piece) and nxt2 (ids
    // loaded during this one).
    Piece cur, nxt;
    next_piece(cur);
    int cur_ids = piece_ids_of<APPEND>(a, cur, lane);
    bool has_next = next_piece(nxt);
    int nxt_ids = has_next ? piece_ids_of<APPEND>(a, nxt, lane) : -1;
    // The first piece waits for its ids anyway; waiting for both here lets the compiler treat the
    // ids a piece receives as loaded on every path into the loop.
    asm volatile("" ::"v"(cur_ids), "v"(nxt_ids));
    if constexpr (decode_carry<D, KV, QF32, APPEND>()) {
        // The first piece's carried loads: its side loads, then its first two blocks. Waiting for
        // all but the blocks here puts the side values in registers on every path into the loop,
        // so no later piece waits on them (with its carried blocks in flight).
        // Iterations 0 and 1 of the piece: blocks 0 - lead and 1 - lead (nothing for the lead).
        const int nb0 = cur.b1 - cur.b0, lead0 = piece_lead(nb0);
        load_side<D, KV, QF32, APPEND, SHARED>(a, cur, cur_ids, true, side);
        load_block<D, KV>(a, bufs.k[0], bufs.v[0], lead0 == 0 ? valid_bid(a, __builtin_amdgcn_readlane(cur_ids, 0)) : -1,
                          cur.kvh);
        load_block<D, KV>(a, bufs.k[1], bufs.v[1],
                          lead0 <= 1 && 1 - lead0 < nb0 ? valid_bid(a, __builtin_amdgcn_readlane(cur_ids, 1 - lead0)) : -1,
                          cur.kvh);
        __builtin_amdgcn_s_waitcnt(vmcnt_keep<2 * decode_block_loads<D, KV>()>());
    }
    for (;;) {
        Piece nxt2;
        bool has_next2 = false;
        int nxt2_ids = -1;
        mfma_piece<D, KV, QF32, APPEND, SHARED>(a, cur, cur_ids, side, bufs, st, s_new, s_vt, has_next, nxt,
                                                nxt_ids, nside, [&]() {
                                                    if (has_next) has_next2 = next_piece(nxt2);
                                                    if (has_next2) nxt2_ids = piece_ids_of<APPEND>(a, nxt2, lane);
                                                });
        if (!has_next) break;
        cur = nxt;
        cur_ids = nxt_ids;
        has_next = has_next2;
        nxt = nxt2;
        nxt_ids = nxt2_ids;
        if constexpr (decode_carry<D, KV, QF32, APPEND>()) side = nside;
    }
}

}  // namespace pa
