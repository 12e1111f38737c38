// kv_append.hip -- slot mapping and KV-cache append/scatter for gfx950.
//
// Fills the no-op placeholders of the reference's append path: PagedAttentionLayer.UpdateKVCache /
// CopyTensorToBlock (src/MLFramework/Inference/PagedAttention/Layers/PagedAttentionLayer.cs:244-327).
// Cache layout per layer (the reference's [num_blocks][num_kv_heads][block][head_dim] block tensor,
// PagedAttentionLayer.cs:315, with V transposed per tile): K tile [16 tokens][head_dim], V tile
// [head_dim][16 tokens], one tile per (block, KV head). The append kernels are HBM-bound scatters;
// the int8 one also owns the per-(block, KV head) scale and running absmax.
#include <string>
#include <type_traits>

#include "append_int8.h"
#include "pa_internal.h"

namespace {

// Slot of new token j of sequence s: table[s][p / 16] * 16 + p % 16 with p = start_pos[s] + j.
__global__ __launch_bounds__(256) void slot_mapping_kernel(
    const int32_t* __restrict__ block_tables, int32_t max_blocks_per_seq,
    const int32_t* __restrict__ start_pos, const int32_t* __restrict__ num_new,
    const int32_t* __restrict__ token_offset, int64_t* __restrict__ slot_mapping) {
    const int s = blockIdx.x;
    const int n = num_new[s];
    const int64_t p0 = start_pos[s];
    const int64_t dst0 = token_offset[s];
    for (int j = blockIdx.y * blockDim.x + threadIdx.x; j < n; j += gridDim.y * blockDim.x) {
        const int64_t p = p0 + j;
        const int64_t lb = p / pa::kBlockSize;
        int64_t slot = -1;
        if (p >= 0 && lb < max_blocks_per_seq) {
            const int32_t blk = block_tables[static_cast<int64_t>(s) * max_blocks_per_seq + lb];
            if (blk >= 0) slot = static_cast<int64_t>(blk) * pa::kBlockSize + p % pa::kBlockSize;
        }
        slot_mapping[dst0 + j] = slot;
    }
}

// Eight consecutive activation values (fp32 or bf16) as fp32; `i` is a multiple of 8 and the
// buffer 16-byte aligned.
template <bool IN_BF16>
__device__ __forceinline__ void load8(const void* __restrict__ p, int64_t i, float (&x)[8]) {
    if constexpr (IN_BF16) {
        const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            x[2 * k] = pa::bf16_lo(ws[k]);
            x[2 * k + 1] = pa::bf16_hi(ws[k]);
        }
    } else {
        const float4 a = reinterpret_cast<const float4*>(static_cast<const float*>(p) + i)[0];
        const float4 b = reinterpret_cast<const float4*>(static_cast<const float*>(p) + i)[1];
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    }
}

// Two fp32 values truncated to bf16 and packed (lo in the low half).
__device__ __forceinline__ uint32_t pack2_trunc(float lo, float hi) {
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// Stores eight values as cache elements (bf16 truncation or fp32) at element `i` of `p`, 16-byte aligned.
template <bool CACHE_BF16>
__device__ __forceinline__ void store8(void* __restrict__ p, int64_t i, const float (&x)[8]) {
    if constexpr (CACHE_BF16) {
        *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p) + i) =
            make_uint4(pack2_trunc(x[0], x[1]), pack2_trunc(x[2], x[3]), pack2_trunc(x[4], x[5]),
                       pack2_trunc(x[6], x[7]));
    } else {
        float4* q = reinterpret_cast<float4*>(static_cast<float*>(p) + i);
        q[0] = make_float4(x[0], x[1], x[2], x[3]);
        q[1] = make_float4(x[4], x[5], x[6], x[7]);
    }
}

// fp32 / bf16 caches with 16-byte aligned operands: one wave per (group of 16 consecutive tokens
// of the call, KV head). A block whose 16 tokens arrive as 16 consecutive slots, starting at a
// token of the group, is written as whole tiles: K rows in 16-byte pieces, V staged in LDS as
// [token][dim] and stored as the tile's [dim][16] rows, so every store is a 16-byte piece of one
// contiguous tile (at most one such block starts in 16 consecutive tokens). The group's other
// tokens (blocks that arrive partly or out of order, tokens of blocks that started in an earlier
// group excepted) go four lanes per token: K rows in 16-byte pieces, V as element stores down
// the tile's column. Lane l first reads the slot of token 16 g - 16 + l: a block starting at
// token b is whole when slots b .. b + 15 are consecutive and the first is a block's row 0.
template <int D, bool IN_BF16, bool CACHE_BF16>
__global__ __launch_bounds__(64) void append_tiles_kernel(
    const void* __restrict__ k_new, const void* __restrict__ v_new, const int64_t* __restrict__ slot_mapping,
    int32_t n_tok, void* __restrict__ k_cache, void* __restrict__ v_cache, int32_t num_kv_heads, int64_t capacity,
    int64_t tok_stride) {
    using CT = std::conditional_t<CACHE_BF16, uint16_t, float>;
    constexpr int kRow = D + 16 / static_cast<int>(sizeof(CT));  // LDS row of the V stage, padded by 16 bytes
    __shared__ __align__(16) CT s_v[16 * kRow];
    const int lane = threadIdx.x;
    const int64_t g = blockIdx.x;
    const int h = blockIdx.y;
    const int64_t u = 16 * g - 16 + lane;
    int64_t sl = -1;
    if (u >= 0 && u < n_tok) sl = slot_mapping[u];
    const bool valid = sl >= 0 && sl < capacity;
    const int64_t nxt = __shfl_down(sl, 1, 64);
    const uint64_t cont = __ballot(valid && lane < 63 && nxt == sl + 1);
    const uint64_t starts = __ballot(valid && (sl & 15) == 0 && lane <= 48 && ((cont >> lane) & 0x7fffull) == 0x7fffull);
    const int off = static_cast<int>(sl & 15);
    const bool mine = valid && lane >= 16 && lane < 32;  // the group's own tokens
    const bool covered = mine && ((starts >> (lane - off)) & 1ull);
    const uint32_t loose = static_cast<uint32_t>(__ballot(mine && !covered) >> 16) & 0xffffu;
    const uint64_t here = starts & 0xffff0000ull;
    const int64_t head_elems = static_cast<int64_t>(h) * D;

    if (here) {
        const int li = __builtin_ctzll(here);
        const int64_t b0 = 16 * g - 16 + li;
        const int64_t tile = (__shfl(sl, li, 64) / 16 * num_kv_heads + h) * 16 * D;
        constexpr int kPer = 2 * D / 64;  // 8-element pieces per lane: 16 tokens x D / 8 over 64 lanes
        float xk[kPer][8], xv[kPer][8];
#pragma unroll
        for (int i = 0; i < kPer; i++) {
            const int p = lane + 64 * i, t = p / (D / 8), d = (p % (D / 8)) * 8;
            const int64_t src = (b0 + t) * tok_stride + head_elems + d;
            load8<IN_BF16>(k_new, src, xk[i]);
            load8<IN_BF16>(v_new, src, xv[i]);
        }
#pragma unroll
        for (int i = 0; i < kPer; i++) {
            const int p = lane + 64 * i, t = p / (D / 8), d = (p % (D / 8)) * 8;
            store8<CACHE_BF16>(k_cache, tile + t * D + d, xk[i]);
            store8<CACHE_BF16>(s_v, t * kRow + d, xv[i]);
        }
        __syncthreads();
        if constexpr (CACHE_BF16) {
            // piece q: dim q / 2, tokens 8 (q % 2) .. + 7 (16 bytes)
#pragma unroll
            for (int i = 0; i < 2 * D / 64; i++) {
                const int q = lane + 64 * i, d = q >> 1, t0 = (q & 1) * 8;
                uint32_t w[4];
#pragma unroll
                for (int k = 0; k < 4; k++)
                    w[k] = static_cast<uint32_t>(s_v[(t0 + 2 * k) * kRow + d]) |
                           (static_cast<uint32_t>(s_v[(t0 + 2 * k + 1) * kRow + d]) << 16);
                *reinterpret_cast<uint4*>(static_cast<uint16_t*>(v_cache) + tile + d * 16 + t0) =
                    make_uint4(w[0], w[1], w[2], w[3]);
            }
        } else {
            // piece q: dim q / 4, tokens 4 (q % 4) .. + 3 (16 bytes)
#pragma unroll
            for (int i = 0; i < 4 * D / 64; i++) {
                const int q = lane + 64 * i, d = q >> 2, t0 = (q & 3) * 4;
                *reinterpret_cast<float4*>(static_cast<float*>(v_cache) + tile + d * 16 + t0) =
                    make_float4(s_v[t0 * kRow + d], s_v[(t0 + 1) * kRow + d], s_v[(t0 + 2) * kRow + d],
                                s_v[(t0 + 3) * kRow + d]);
            }
        }
    }

    if (loose) {
        // token j = lane / 4 of the group, dims [c D / 4, (c + 1) D / 4) with c = lane % 4
        const int j = lane >> 2, c = lane & 3;
        const int64_t s = __shfl(sl, 16 + j, 64);
        if ((loose >> j) & 1u) {
            const int64_t tok = 16 * g + j;
            const int o = static_cast<int>(s & 15);
            const int64_t tile = (s / 16 * num_kv_heads + h) * 16 * D;
            constexpr int kPer = D / 32;  // 8-element pieces per lane
            float xk[kPer][8], xv[kPer][8];
#pragma unroll
            for (int i = 0; i < kPer; i++) {
                const int64_t src = tok * tok_stride + head_elems + c * (D / 4) + 8 * i;
                load8<IN_BF16>(k_new, src, xk[i]);
                load8<IN_BF16>(v_new, src, xv[i]);
            }
#pragma unroll
            for (int i = 0; i < kPer; i++) {
                const int d = c * (D / 4) + 8 * i;
                store8<CACHE_BF16>(k_cache, tile + o * D + d, xk[i]);
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    if constexpr (CACHE_BF16)
                        static_cast<uint16_t*>(v_cache)[tile + (d + k) * 16 + o] = pa::bf16_trunc(xv[i][k]);
                    else
                        static_cast<float*>(v_cache)[tile + (d + k) * 16 + o] = xv[i][k];
                }
            }
        }
    }
}

// fp32 / bf16 caches, any alignment: one workgroup per token, blockIdx.y selects K (0) or V (1). K rows are
// contiguous per token. A V tile is [D][16]: one token's values are a column, so writing them one
// by one is D scattered element stores. When the 16 tokens of a block arrive as 16 consecutive
// slots of this call (a prefill chunk's whole blocks), the 16 workgroups of the block write the
// tile by dim rows instead (each row one contiguous 16-token run, written in 8- or 16-byte
// pieces); tokens of partly filled blocks keep the element stores.
__global__ __launch_bounds__(256) void append_plain_kernel(
    const void* __restrict__ k_new, const void* __restrict__ v_new, bool in_bf16,
    const int64_t* __restrict__ slot_mapping, int32_t n_tok, void* __restrict__ k_cache, void* __restrict__ v_cache,
    bool cache_bf16, int32_t num_kv_heads, int32_t head_dim, int64_t capacity, int64_t tok_stride) {
    // Token t's values for (head h, dim d) are at t * tok_stride + h * head_dim + d of k_new / v_new.
    const int i = blockIdx.x;
    const int64_t slot = slot_mapping[i];
    if (slot < 0 || slot >= capacity) return;
    const bool is_v = blockIdx.y != 0;
    const void* src = is_v ? v_new : k_new;
    void* dst = is_v ? v_cache : k_cache;
    const int64_t blk = slot / pa::kBlockSize, off = slot % pa::kBlockSize;
    const int n = num_kv_heads * head_dim;
    if (is_v) {
        // Does token i's block arrive whole, as tokens i - off .. i - off + 15 with consecutive slots?
        __shared__ int s_full;
        if (threadIdx.x < 64) {
            const int t = threadIdx.x;
            const int64_t j = static_cast<int64_t>(i) - off + t;
            bool ok = true;
            if (t < pa::kBlockSize) ok = j >= 0 && j < n_tok && slot_mapping[j] == slot - off + t;
            const bool all = __all(ok);
            if (t == 0) s_full = all ? 1 : 0;
        }
        __syncthreads();
        if (s_full) {
            // The 16 workgroups of the block share its tile: workgroup `off` writes dim rows
            // [off * n / 16, (off + 1) * n / 16) (all heads' rows, row = h * D + d), four threads
            // per row, each taking 4 consecutive tokens (one 8-byte bf16 / 16-byte fp32 store).
            const int per = n / pa::kBlockSize;  // rows per workgroup (D is a multiple of 16)
            const int64_t tok0 = static_cast<int64_t>(i) - off;
            const int q = threadIdx.x & 3;
            for (int r = threadIdx.x >> 2; r < per; r += blockDim.x >> 2) {
                const int idx = static_cast<int>(off) * per + r;
                const int h = idx / head_dim, d = idx - h * head_dim;
                float x[4];
#pragma unroll
                for (int k = 0; k < 4; k++) x[k] = pa::load_act(src, in_bf16, (tok0 + 4 * q + k) * tok_stride + idx);
                const int64_t row = ((blk * num_kv_heads + h) * head_dim + d) * pa::kBlockSize;  // V row d of the tile
                if (cache_bf16) {
                    const uint32_t w0 = static_cast<uint32_t>(pa::bf16_trunc(x[0])) | (static_cast<uint32_t>(pa::bf16_trunc(x[1])) << 16);
                    const uint32_t w1 = static_cast<uint32_t>(pa::bf16_trunc(x[2])) | (static_cast<uint32_t>(pa::bf16_trunc(x[3])) << 16);
                    reinterpret_cast<uint2*>(static_cast<uint16_t*>(dst) + row)[q] = make_uint2(w0, w1);
                } else {
                    reinterpret_cast<float4*>(static_cast<float*>(dst) + row)[q] = make_float4(x[0], x[1], x[2], x[3]);
                }
            }
            return;
        }
    }
    for (int idx = threadIdx.x; idx < n; idx += blockDim.x) {
        const int h = idx / head_dim, d = idx - h * head_dim;
        const float x = pa::load_act(src, in_bf16, static_cast<int64_t>(i) * tok_stride + idx);
        const int64_t tile = (blk * num_kv_heads + h) * pa::kBlockSize * head_dim;
        // K tiles are [16][D] (token rows); V tiles are [D][16] (dim rows).
        const int64_t o = is_v ? tile + static_cast<int64_t>(d) * pa::kBlockSize + off : tile + off * head_dim + d;
        if (cache_bf16) static_cast<uint16_t*>(dst)[o] = pa::bf16_trunc(x);
        else static_cast<float*>(dst)[o] = x;
    }
}

// int8 caches: one workgroup per token of the call; the workgroup of the first token that lands in
// a block applies all of that block's segments (append_int8_block), one wave per (KV head, K|V).
template <int D>
__global__ __launch_bounds__(pa::kAppendMaxThreads) void append_int8_kernel(
    const void* __restrict__ k_new, const void* __restrict__ v_new, bool in_bf16,
    const int64_t* __restrict__ slot_mapping, int32_t n_tok, int8_t* __restrict__ k_cache,
    int8_t* __restrict__ v_cache, float* __restrict__ k_scale, float* __restrict__ v_scale,
    float* __restrict__ k_absmax, float* __restrict__ v_absmax, int32_t num_kv_heads, int64_t capacity,
    int64_t tok_stride) {
    pa::append_int8_block<D>(k_new, v_new, in_bf16, tok_stride, [&](int t) { return slot_mapping[t]; },
                             static_cast<int32_t>(blockIdx.x), n_tok, k_cache, v_cache, k_scale, v_scale, k_absmax,
                             v_absmax, num_kv_heads, capacity);
}

}  // namespace

extern "C" {

pa_status pa_build_slot_mapping(pa_stream* stream, const pa_config* cfg,
                                const int32_t* block_tables, int32_t max_blocks_per_seq,
                                const int32_t* start_pos, const int32_t* num_new,
                                const int32_t* token_offset, int32_t num_seqs,
                                int32_t max_new_per_seq, int64_t* slot_mapping) {
    if (!cfg) return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_build_slot_mapping: cfg is null");
    if (cfg->block_size != pa::kBlockSize)
        return pa::set_error(PA_ERROR_UNSUPPORTED, "pa_build_slot_mapping: block_size must be 16");
    if (num_seqs < 0 || max_blocks_per_seq < 0 || max_new_per_seq < 0)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_build_slot_mapping: negative size");
    if (num_seqs == 0 || max_new_per_seq == 0) return pa::clear_error();
    if (!block_tables || !start_pos || !num_new || !token_offset || !slot_mapping)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_build_slot_mapping: null pointer");
    const int per = 256;
    int gy = (max_new_per_seq + per - 1) / per;
    if (gy > 65535) gy = 65535;
    dim3 grid(num_seqs, gy);
    slot_mapping_kernel<<<grid, per, 0, pa::native(stream)>>>(block_tables, max_blocks_per_seq, start_pos,
                                                              num_new, token_offset, slot_mapping);
    PA_HIP_CHECK(hipGetLastError());
    return pa::clear_error();
}
}  // extern "C"

namespace pa {

pa_status launch_kv_append(const char* f, hipStream_t s, const pa_config* cfg, const void* k_new, const void* v_new,
                           bool in_bf16, int64_t tok_stride, const int64_t* slot_mapping, int32_t n_tok,
                           void* k_cache, void* v_cache, float* k_scale, float* v_scale, float* k_absmax,
                           float* v_absmax) {
    const std::string fn(f);
    if (n_tok < 0) return set_error(PA_ERROR_INVALID_ARGUMENT, fn + ": n_tok < 0");
    if (n_tok == 0) return clear_error();
    if (!k_new || !v_new || !slot_mapping || !k_cache || !v_cache)
        return set_error(PA_ERROR_INVALID_ARGUMENT, fn + ": null pointer");
    const int64_t capacity = static_cast<int64_t>(cfg->num_blocks) * kBlockSize;
    const bool aligned = ((reinterpret_cast<uintptr_t>(k_new) | reinterpret_cast<uintptr_t>(v_new) |
                           reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) % 16 == 0) &&
                         (tok_stride * (in_bf16 ? 2 : 4)) % 16 == 0;
    if (cfg->kv_dtype != PA_DTYPE_INT8 && aligned && cfg->num_kv_heads <= 65535) {  // grid y: one row per KV head
        const dim3 grid((n_tok + 15) / 16, cfg->num_kv_heads);
        const bool cb = cfg->kv_dtype == PA_DTYPE_BF16;
        auto go = [&](auto kern) {
            kern<<<grid, 64, 0, s>>>(k_new, v_new, slot_mapping, n_tok, k_cache, v_cache, cfg->num_kv_heads, capacity,
                                     tok_stride);
        };
        switch (cfg->head_dim) {
#define PA_APPEND_TILES(DD)                                                                   \
    case DD:                                                                                  \
        if (in_bf16) go(cb ? append_tiles_kernel<DD, true, true> : append_tiles_kernel<DD, true, false>); \
        else go(cb ? append_tiles_kernel<DD, false, true> : append_tiles_kernel<DD, false, false>);       \
        break;
            PA_APPEND_TILES(32)
            PA_APPEND_TILES(64)
            PA_APPEND_TILES(128)
            PA_APPEND_TILES(256)
#undef PA_APPEND_TILES
            default:
                return set_error(PA_ERROR_UNSUPPORTED, fn + ": head_dim must be 32, 64, 128 or 256");
        }
    } else if (cfg->kv_dtype != PA_DTYPE_INT8) {
        dim3 grid(n_tok, 2);
        append_plain_kernel<<<grid, 256, 0, s>>>(k_new, v_new, in_bf16, slot_mapping, n_tok, k_cache, v_cache,
                                                  cfg->kv_dtype == PA_DTYPE_BF16, cfg->num_kv_heads, cfg->head_dim,
                                                  capacity, tok_stride);
    } else {
        if (!k_scale || !v_scale || !k_absmax || !v_absmax)
            return set_error(PA_ERROR_INVALID_ARGUMENT, fn + ": int8 cache needs scales and absmax");
        const int threads = append_int8_threads(cfg->num_kv_heads);
        auto* kc = static_cast<int8_t*>(k_cache);
        auto* vc = static_cast<int8_t*>(v_cache);
        switch (cfg->head_dim) {
            case 64:
                append_int8_kernel<64><<<n_tok, threads, 0, s>>>(k_new, v_new, in_bf16, slot_mapping, n_tok, kc, vc,
                                                                 k_scale, v_scale, k_absmax, v_absmax,
                                                                 cfg->num_kv_heads, capacity, tok_stride);
                break;
            case 128:
                append_int8_kernel<128><<<n_tok, threads, 0, s>>>(k_new, v_new, in_bf16, slot_mapping, n_tok, kc, vc,
                                                                  k_scale, v_scale, k_absmax, v_absmax,
                                                                  cfg->num_kv_heads, capacity, tok_stride);
                break;
            default:
                append_int8_kernel<256><<<n_tok, threads, 0, s>>>(k_new, v_new, in_bf16, slot_mapping, n_tok, kc, vc,
                                                                  k_scale, v_scale, k_absmax, v_absmax,
                                                                  cfg->num_kv_heads, capacity, tok_stride);
                break;
        }
    }
    PA_HIP_CHECK(hipGetLastError());
    return clear_error();
}

}  // namespace pa

extern "C" {

pa_status pa_kv_append(pa_stream* stream, const pa_config* cfg, const void* k_new, const void* v_new,
                       const int64_t* slot_mapping, int32_t n_tok, void* k_cache, void* v_cache,
                       float* k_scale, float* v_scale, float* k_absmax, float* v_absmax) {
    pa_status st = pa::check_config(cfg, "pa_kv_append");
    if (st != PA_SUCCESS) return st;
    return pa::launch_kv_append("pa_kv_append", pa::native(stream), cfg, k_new, v_new, cfg->q_dtype == PA_DTYPE_BF16,
                                static_cast<int64_t>(cfg->num_kv_heads) * cfg->head_dim, slot_mapping, n_tok,
                                k_cache, v_cache, k_scale, v_scale, k_absmax, v_absmax);
}

}  // extern "C"
