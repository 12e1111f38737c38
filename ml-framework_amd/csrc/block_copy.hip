// block_copy.hip -- whole-block moves of the paged KV cache for gfx950: copy-on-write copies,
// swap-out / swap-in through a packed buffer, and the fp32 view of one block.
//
// The reference's block sharing leaves the copy to a comment (BeamSearchBlockSharing.
// OnBeamDivergence, src/MLFramework/Inference/PagedAttention/Sharing/BeamSearchBlockSharing.cs:
// 69-79: "at divergence ... allocate unique blocks for this beam"; refcounts in BlockShareManager.cs:
// 34-105), and its cache interface moves block data as float arrays (IPagedAttentionCache.
// GetBlockData / StoreBlockData, ContinuousBatching/KVCache/IPagedAttentionCache.cs:40-47;
// CacheBlockData.cs:7-12) with no implementation. These kernels are those moves on the device
// layout: per block, K is [Hkv][16][D] and V is [Hkv][D][16] (each one contiguous run of
// Hkv * 16 * D elements), plus for int8 the [Hkv] scales and running absmax.
//
// All of it is HBM-bound byte movement: 16-byte non-temporal vector loads and stores, kSplit
// workgroups per (block, part), part 0 K, 1 V, 2 the int8 statistics.
#include <string>

#include "append_int8.h"
#include "pa_internal.h"

namespace {

constexpr int kCopyThreads = 256;
// Workgroups per part (K or V of one block): a part is Hkv * 16 * D elements, a multiple of
// 16 * 64 bytes, so 4 pieces of it stay 16-byte multiples.
constexpr int kSplit = 4;

// Bytes of K (or of V) of one block, all KV heads.
int64_t part_bytes(const pa_config* cfg) {
    const int64_t elt = cfg->kv_dtype == PA_DTYPE_FP32 ? 4 : cfg->kv_dtype == PA_DTYPE_BF16 ? 2 : 1;
    return static_cast<int64_t>(cfg->num_kv_heads) * pa::kBlockSize * cfg->head_dim * elt;
}
// int8 statistics of one block: k_scale, v_scale, k_absmax, v_absmax, [Hkv] floats each.
int64_t stats_bytes(const pa_config* cfg) {
    return cfg->kv_dtype == PA_DTYPE_INT8 ? 4 * static_cast<int64_t>(cfg->num_kv_heads) * 4 : 0;
}
// One packed record: K bytes, V bytes, then the statistics; a multiple of 16 bytes.
int64_t record_bytes(const pa_config* cfg) { return 2 * part_bytes(cfg) + stats_bytes(cfg); }

struct CacheRefs {
    char* k;
    char* v;
    float* stat[4];  // k_scale, v_scale, k_absmax, v_absmax (int8)
    int64_t part;    // bytes of K (of V) per block
    int32_t hkv;
    int32_t num_blocks;
    bool int8;
};

// Moved data is not read again soon: non-temporal loads and stores (measured faster than
// ordinary ones on scattered 32 KiB runs).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void copy16(char* dst, const char* src, int64_t bytes) {
    for (int64_t o = static_cast<int64_t>(threadIdx.x) * 16; o < bytes; o += kCopyThreads * 16)
        __builtin_nontemporal_store(__builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + o)),
                                    reinterpret_cast<u32x4*>(dst + o));
}

// Copy-on-write: pairs[i] = (src, dst); every part of block src is copied into block dst. Pairs
// with an id outside [0, num_blocks) or src == dst are skipped.
__global__ __launch_bounds__(kCopyThreads) void copy_blocks_kernel(CacheRefs c, const int32_t* __restrict__ pairs) {
    const int32_t src = pairs[2 * blockIdx.x], dst = pairs[2 * blockIdx.x + 1];
    if (src < 0 || src >= c.num_blocks || dst < 0 || dst >= c.num_blocks || src == dst) return;
    const int part = blockIdx.y / kSplit, piece = blockIdx.y % kSplit;
    if (part < 2) {
        char* base = part == 0 ? c.k : c.v;
        const int64_t len = c.part / kSplit, off = piece * len;
        copy16(base + dst * c.part + off, base + src * c.part + off, len);
    } else if (c.int8 && piece == 0) {
        const int n = 4 * c.hkv;
        for (int i = threadIdx.x; i < n; i += kCopyThreads) {
            float* s = c.stat[i / c.hkv];
            const int h = i % c.hkv;
            s[static_cast<int64_t>(dst) * c.hkv + h] = s[static_cast<int64_t>(src) * c.hkv + h];
        }
    }
}

// Swap-out (to_packed) or swap-in: record i of `packed` <-> block ids[i]. Ids outside
// [0, num_blocks) are skipped (their records are neither written nor read).
__global__ __launch_bounds__(kCopyThreads) void move_blocks_kernel(CacheRefs c, const int32_t* __restrict__ ids,
                                                                  char* packed, int64_t record, bool to_packed) {
    const int32_t b = ids[blockIdx.x];
    if (b < 0 || b >= c.num_blocks) return;
    char* rec = packed + static_cast<int64_t>(blockIdx.x) * record;
    const int part = blockIdx.y / kSplit, piece = blockIdx.y % kSplit;
    if (part < 2) {
        const int64_t len = c.part / kSplit, off = piece * len;
        char* blk = (part == 0 ? c.k : c.v) + b * c.part + off;
        char* r = rec + part * c.part + off;
        if (to_packed) copy16(r, blk, len);
        else copy16(blk, r, len);
    } else if (c.int8 && piece == 0) {
        float* r = reinterpret_cast<float*>(rec + 2 * c.part);
        const int n = 4 * c.hkv;
        for (int i = threadIdx.x; i < n; i += kCopyThreads) {
            float* s = c.stat[i / c.hkv] + static_cast<int64_t>(b) * c.hkv + i % c.hkv;
            if (to_packed) r[i] = *s;
            else *s = r[i];
        }
    }
}

// fp32 view of tokens [0, tokens) of one block: out[t][h][d] (K, or V for part 1). int8 values
// are code * scale (the reference's Dequantize); bf16 widens exactly.
__global__ __launch_bounds__(kCopyThreads) void read_block_f32_kernel(CacheRefs c, int32_t block, int32_t tokens,
                                                                     int32_t head_dim, float* __restrict__ k_out,
                                                                     float* __restrict__ v_out, int32_t kv_dtype) {
    const bool is_v = blockIdx.y != 0;
    const int h = blockIdx.x, D = head_dim;
    float* out = is_v ? v_out : k_out;
    const int64_t tile = (static_cast<int64_t>(block) * c.hkv + h) * pa::kBlockSize * D;
    const float scale = c.int8 ? c.stat[is_v ? 1 : 0][static_cast<int64_t>(block) * c.hkv + h] : 1.0f;
    const char* base = is_v ? c.v : c.k;
    for (int idx = threadIdx.x; idx < tokens * D; idx += kCopyThreads) {
        const int t = idx / D, d = idx - t * D;
        const int64_t e = tile + (is_v ? static_cast<int64_t>(d) * pa::kBlockSize + t : static_cast<int64_t>(t) * D + d);
        float x;
        if (kv_dtype == PA_DTYPE_FP32) x = reinterpret_cast<const float*>(base)[e];
        else if (kv_dtype == PA_DTYPE_BF16) x = pa::bf16_to_f32(reinterpret_cast<const uint16_t*>(base)[e]);
        else x = static_cast<float>(static_cast<int32_t>(reinterpret_cast<const int8_t*>(base)[e])) * scale;
        out[(static_cast<int64_t>(t) * c.hkv + h) * D + d] = x;
    }
}

// Tokens [0, tokens) of one block from fp32 in[t][h][d]: what pa_kv_append does with fp32 input
// at slots block * 16 + t. fp32 / bf16 caches: one workgroup per (head, K|V), elementwise.
__global__ __launch_bounds__(kCopyThreads) void write_block_plain_kernel(CacheRefs c, int32_t block, int32_t tokens,
                                                                        int32_t head_dim, const float* __restrict__ k_in,
                                                                        const float* __restrict__ v_in, bool bf16) {
    const bool is_v = blockIdx.y != 0;
    const int h = blockIdx.x, D = head_dim;
    const float* in = is_v ? v_in : k_in;
    const int64_t tile = (static_cast<int64_t>(block) * c.hkv + h) * pa::kBlockSize * D;
    char* base = is_v ? c.v : c.k;
    for (int idx = threadIdx.x; idx < tokens * D; idx += kCopyThreads) {
        const int t = idx / D, d = idx - t * D;
        const int64_t e = tile + (is_v ? static_cast<int64_t>(d) * pa::kBlockSize + t : static_cast<int64_t>(t) * D + d);
        const float x = in[(static_cast<int64_t>(t) * c.hkv + h) * D + d];
        if (bf16) reinterpret_cast<uint16_t*>(base)[e] = pa::bf16_trunc(x);
        else reinterpret_cast<float*>(base)[e] = x;
    }
}

// int8 caches: the quantising append of pa_kv_append (one segment: the block's tokens, row 0
// included, so the block starts afresh), one wave per (head, K|V).
template <int D>
__global__ __launch_bounds__(64) void write_block_int8_kernel(CacheRefs c, int32_t block, int32_t tokens,
                                                             const float* __restrict__ k_in,
                                                             const float* __restrict__ v_in) {
    const bool is_v = blockIdx.y != 0;
    float amax = 0.0f, scale = 0.0f;
    bool have = false;
    pa::append_int8_apply<D>(is_v ? static_cast<const void*>(v_in) : static_cast<const void*>(k_in), false,
                             static_cast<int64_t>(c.hkv) * D,
                             [&](int t) { return static_cast<int64_t>(block) * pa::kBlockSize + t; }, 0, tokens, block,
                             reinterpret_cast<int8_t*>(is_v ? c.v : c.k), c.stat[is_v ? 1 : 0], c.stat[is_v ? 3 : 2],
                             static_cast<int>(blockIdx.x), c.hkv, is_v, amax, scale, have);
}

// Checks shared by the entry points; fills `c`. need_absmax: int8 needs the running absmax too
// (every entry point but the read).
pa_status refs_for(const std::string& f, const pa_config* cfg, void* k_cache, void* v_cache, float* k_scale,
                   float* v_scale, float* k_absmax, float* v_absmax, CacheRefs* c, bool need_absmax = true) {
    pa_status st = pa::check_config(cfg, f.c_str());
    if (st != PA_SUCCESS) return st;
    if (!k_cache || !v_cache) return pa::set_error(PA_ERROR_INVALID_ARGUMENT, f + ": null cache pointer");
    if ((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) & 15)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, f + ": cache pointers must be 16-byte aligned");
    const bool int8 = cfg->kv_dtype == PA_DTYPE_INT8;
    if (int8 && (!k_scale || !v_scale || (need_absmax && (!k_absmax || !v_absmax))))
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT,
                             f + (need_absmax ? ": int8 cache needs scales and absmax" : ": int8 cache needs scales"));
    *c = CacheRefs{static_cast<char*>(k_cache), static_cast<char*>(v_cache), {k_scale, v_scale, k_absmax, v_absmax},
                   part_bytes(cfg), cfg->num_kv_heads, cfg->num_blocks, int8};
    return PA_SUCCESS;
}

}  // namespace

extern "C" {

pa_status pa_block_bytes(const pa_config* cfg, size_t* bytes) {
    pa_status st = pa::check_config(cfg, "pa_block_bytes");
    if (st != PA_SUCCESS) return st;
    if (!bytes) return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_block_bytes: bytes is null");
    *bytes = static_cast<size_t>(record_bytes(cfg));
    return pa::clear_error();
}

pa_status pa_copy_blocks(pa_stream* stream, const pa_config* cfg, void* k_cache, void* v_cache, float* k_scale,
                         float* v_scale, float* k_absmax, float* v_absmax, const int32_t* block_pairs,
                         int32_t num_pairs) {
    CacheRefs c;
    pa_status st = refs_for("pa_copy_blocks", cfg, k_cache, v_cache, k_scale, v_scale, k_absmax, v_absmax, &c);
    if (st != PA_SUCCESS) return st;
    if (num_pairs < 0) return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_copy_blocks: num_pairs < 0");
    if (num_pairs == 0) return pa::clear_error();
    if (!block_pairs) return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_copy_blocks: block_pairs is null");
    dim3 grid(num_pairs, (c.int8 ? 3 : 2) * kSplit);
    copy_blocks_kernel<<<grid, kCopyThreads, 0, pa::native(stream)>>>(c, block_pairs);
    PA_HIP_CHECK(hipGetLastError());
    return pa::clear_error();
}

static pa_status move_blocks(const char* f, pa_stream* stream, const pa_config* cfg, void* k_cache, void* v_cache,
                             float* k_scale, float* v_scale, float* k_absmax, float* v_absmax,
                             const int32_t* block_ids, int32_t n, void* packed, bool to_packed) {
    CacheRefs c;
    pa_status st = refs_for(f, cfg, k_cache, v_cache, k_scale, v_scale, k_absmax, v_absmax, &c);
    if (st != PA_SUCCESS) return st;
    if (n < 0) return pa::set_error(PA_ERROR_INVALID_ARGUMENT, std::string(f) + ": n < 0");
    if (n == 0) return pa::clear_error();
    if (!block_ids || !packed) return pa::set_error(PA_ERROR_INVALID_ARGUMENT, std::string(f) + ": null pointer");
    if (reinterpret_cast<uintptr_t>(packed) & 15)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, std::string(f) + ": packed buffer must be 16-byte aligned");
    dim3 grid(n, (c.int8 ? 3 : 2) * kSplit);
    move_blocks_kernel<<<grid, kCopyThreads, 0, pa::native(stream)>>>(c, block_ids, static_cast<char*>(packed),
                                                                      record_bytes(cfg), to_packed);
    PA_HIP_CHECK(hipGetLastError());
    return pa::clear_error();
}

pa_status pa_gather_blocks(pa_stream* stream, const pa_config* cfg, const void* k_cache, const void* v_cache,
                           const float* k_scale, const float* v_scale, const float* k_absmax, const float* v_absmax,
                           const int32_t* block_ids, int32_t n, void* packed) {
    return move_blocks("pa_gather_blocks", stream, cfg, const_cast<void*>(k_cache), const_cast<void*>(v_cache),
                       const_cast<float*>(k_scale), const_cast<float*>(v_scale), const_cast<float*>(k_absmax),
                       const_cast<float*>(v_absmax), block_ids, n, packed, true);
}

pa_status pa_scatter_blocks(pa_stream* stream, const pa_config* cfg, void* k_cache, void* v_cache, float* k_scale,
                            float* v_scale, float* k_absmax, float* v_absmax, const int32_t* block_ids, int32_t n,
                            const void* packed) {
    return move_blocks("pa_scatter_blocks", stream, cfg, k_cache, v_cache, k_scale, v_scale, k_absmax, v_absmax,
                       block_ids, n, const_cast<void*>(packed), false);
}

pa_status pa_read_block_f32(pa_stream* stream, const pa_config* cfg, const void* k_cache, const void* v_cache,
                            const float* k_scale, const float* v_scale, int32_t block, int32_t tokens, float* k_out,
                            float* v_out) {
    CacheRefs c;
    pa_status st = refs_for("pa_read_block_f32", cfg, const_cast<void*>(k_cache), const_cast<void*>(v_cache),
                            const_cast<float*>(k_scale), const_cast<float*>(v_scale), nullptr, nullptr, &c, false);
    if (st != PA_SUCCESS) return st;
    if (block < 0 || block >= cfg->num_blocks)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_read_block_f32: block out of range");
    if (tokens < 0 || tokens > pa::kBlockSize)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_read_block_f32: tokens must be in [0, 16]");
    if (tokens == 0) return pa::clear_error();
    if (!k_out || !v_out) return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_read_block_f32: null output");
    dim3 grid(cfg->num_kv_heads, 2);
    read_block_f32_kernel<<<grid, kCopyThreads, 0, pa::native(stream)>>>(c, block, tokens, cfg->head_dim, k_out, v_out,
                                                                         cfg->kv_dtype);
    PA_HIP_CHECK(hipGetLastError());
    return pa::clear_error();
}

pa_status pa_write_block_f32(pa_stream* stream, const pa_config* cfg, void* k_cache, void* v_cache, float* k_scale,
                             float* v_scale, float* k_absmax, float* v_absmax, int32_t block, int32_t tokens,
                             const float* k_in, const float* v_in) {
    CacheRefs c;
    pa_status st = refs_for("pa_write_block_f32", cfg, k_cache, v_cache, k_scale, v_scale, k_absmax, v_absmax, &c);
    if (st != PA_SUCCESS) return st;
    if (block < 0 || block >= cfg->num_blocks)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_write_block_f32: block out of range");
    if (tokens < 0 || tokens > pa::kBlockSize)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_write_block_f32: tokens must be in [0, 16]");
    if (tokens == 0) return pa::clear_error();
    if (!k_in || !v_in) return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_write_block_f32: null input");
    if (cfg->num_kv_heads > 65535)
        return pa::set_error(PA_ERROR_INVALID_CONFIG, "pa_write_block_f32: too many KV heads");
    hipStream_t s = pa::native(stream);
    dim3 grid(cfg->num_kv_heads, 2);
    if (!c.int8) {
        write_block_plain_kernel<<<grid, kCopyThreads, 0, s>>>(c, block, tokens, cfg->head_dim, k_in, v_in,
                                                               cfg->kv_dtype == PA_DTYPE_BF16);
    } else {
        switch (cfg->head_dim) {
            case 64: write_block_int8_kernel<64><<<grid, 64, 0, s>>>(c, block, tokens, k_in, v_in); break;
            case 128: write_block_int8_kernel<128><<<grid, 64, 0, s>>>(c, block, tokens, k_in, v_in); break;
            default: write_block_int8_kernel<256><<<grid, 64, 0, s>>>(c, block, tokens, k_in, v_in); break;
        }
    }
    PA_HIP_CHECK(hipGetLastError());
    return pa::clear_error();
}

}  // extern "C"
