// paged_decode.hip -- ragged paged decode for gfx950 (wave64).
//
// Replaces the reference's per-sequence decode loop (DecodeOrchestrator.BatchDecode /
// ComputeDecodeAttention, src/MLFramework/Inference/PagedAttention/Phases/DecodeOrchestrator.cs:64-109,
// which gathers each sequence's K/V and calls StandardPagedAttentionKernel once per sequence,
// Kernels/StandardPagedAttentionKernel.cs:21-84) with one launch over the whole ragged batch.
//
// bf16 / int8 caches (decode_mfma.h, paged_decode_mfma_persistent_kernel): persistent workgroups
// cut the batch's blocks into equal ranges, one (range, KV head) unit each, so every workgroup
// streams the same bytes whatever the mix of context lengths; rows (sequence, KV head) split
// between ranges leave (max, sum, unnormalised O) partials that paged_decode_merge_split_kernel
// combines with a log-sum-exp reduction. The G = Hq / Hkv query heads of a KV head share every
// K/V byte loaded (GQA): QK and PV run on MFMA with the heads as the 16 MFMA rows.
// fp32 caches (decode_fp32.h): one workgroup per (partition, KV head, sequence), VALU dot products
// reduced across lanes with DPP, a partition-wide softmax in LDS, VALU P.V, and the same kind of
// merge over fixed 256/512-token partitions (paged_decode_merge_kernel).
#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "append_int8.h"
#include "decode_common.h"

namespace pa {

int device_cus() {
    // CU count per device ordinal, queried once (read-only afterwards).
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

}  // namespace pa

namespace {

using pa::DecodeArgs;

// Largest pa_config.num_splits accepted (partitions per sequence).
constexpr int kMaxNumSplits = 256;
using pa::clamp_len;
using pa::act_at;

// Split length for this call. fp32 caches use partitions of 256 or 512 tokens (VALU kernel
// templates). bf16/int8 caches: 0 lets the kernel cut the batch's blocks into one equal range per
// resident workgroup; otherwise the ranges are `partition_size` tokens (multiple of 64).
int resolve_part(const pa_config* cfg, std::string* err) {
    const int req = cfg->partition_size;
    if (cfg->num_splits < 0 || cfg->num_splits > kMaxNumSplits) {
        *err = "num_splits must be in [0, " + std::to_string(kMaxNumSplits) + "]";
        return -1;
    }
    if (cfg->num_splits > 0 && (cfg->kv_dtype == PA_DTYPE_FP32 || req != 0)) {
        *err = cfg->kv_dtype == PA_DTYPE_FP32 ? "num_splits applies to bf16 / int8 caches only"
                                              : "num_splits and partition_size are exclusive";
        return -1;
    }
    if (cfg->kv_dtype == PA_DTYPE_FP32) {
        if (req == 0) return 256;
        if (req == 256 || req == 512) return req;
        *err = "partition_size must be 0, 256 or 512 for an fp32 cache";
        return -1;
    }
    if (req == 0) return 0;
    if (req < 64 || req > 4096 || req % 64 != 0) {
        *err = "partition_size must be 0 or a multiple of 64 in [64, 4096]";
        return -1;
    }
    return req;
}

// Units (range, KV head) an MFMA launch over (at most) this shape can produce: the bound the
// workspace is sized for. By default there are at most nr ranges (nr = workers / Hkv, workers <=
// kMaxDecodeWorkers) of at least 4 blocks each; with num_splits P, P units per (sequence, KV head).
int64_t mfma_max_units(const pa_config* cfg, int32_t num_seqs, int32_t max_len, int part, int splits) {
    const int64_t seqs = num_seqs < pa::kMaxPersistentSeqs - 1 ? num_seqs : pa::kMaxPersistentSeqs - 1;
    const int64_t wmax = seqs * ((static_cast<int64_t>(max_len) + 15) / 16);
    const int64_t hkv = cfg->num_kv_heads;
    if (wmax <= 0) return 0;
    if (splits > 0) return seqs * splits * hkv;
    if (part > 0) return (wmax + part / 16 - 1) / (part / 16) * hkv;
    const int64_t workers = pa::kMaxDecodeWorkers;
    const int64_t nr = workers >= hkv ? workers / hkv : 1;
    const int64_t by_min_len = (wmax + 3) / 4;
    return (nr < by_min_len ? nr : by_min_len) * hkv;
}

size_t workspace_bytes_for(const pa_config* cfg, int32_t num_seqs, int32_t max_len, int part) {
    if (num_seqs <= 0) return 0;
    if (cfg->kv_dtype == PA_DTYPE_FP32) {
        const int64_t max_parts = (static_cast<int64_t>(max_len) + part - 1) / part;
        if (max_parts <= 1) return 0;
        const int64_t rows = static_cast<int64_t>(num_seqs) * cfg->num_q_heads * max_parts;
        return static_cast<size_t>(rows) * (cfg->head_dim + 2) * sizeof(float);
    }
    const int64_t seqs = num_seqs < pa::kMaxPersistentSeqs - 1 ? num_seqs : pa::kMaxPersistentSeqs - 1;
    const int64_t rows = 2 * mfma_max_units(cfg, num_seqs, max_len, part, cfg->num_splits) * (cfg->num_q_heads / cfg->num_kv_heads);
    // partials (o, max, sum), sequence offsets
    return static_cast<size_t>(rows) * (cfg->head_dim + 2) * sizeof(float) + static_cast<size_t>(seqs + 1) * 4;
}

int32_t effective_max_len(int32_t max_context_len, int32_t max_blocks_per_seq) {
    // Tokens beyond the table are never read, so the grid only needs to cover what the table holds.
    const int64_t table_tokens = static_cast<int64_t>(max_blocks_per_seq) * pa::kBlockSize;
    return max_context_len > table_tokens ? static_cast<int32_t>(table_tokens) : max_context_len;
}


// fp32 caches, fused entry point: append the token at position context_len - 1 of every
// sequence (one workgroup per sequence, K row and V column of every KV head), before the decode.
__global__ __launch_bounds__(256) void append_last_token_fp32_kernel(const DecodeArgs a, int32_t head_dim) {
    const int seq = blockIdx.x;
    const int T = clamp_len(a, a.context_lens[seq]);
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

// int8 caches, pa_paged_decode_append: the new token of every sequence (position T - 1, T the
// clamped context length) is appended by the quantising append of pa_kv_append, as token i = seq
// i of one call, before the decode reads the cache: one workgroup per sequence, the owner of each
// block applying its tokens, one wave per (KV head, K|V). (Done inside the decode kernel instead,
// the requantisation stalls the wave that owns each row's last block mid-stream; a separate launch
// costs less.)
template <int D>
__global__ __launch_bounds__(pa::kAppendMaxThreads) void append_last_token_int8_kernel(const DecodeArgs a,
                                                                                      int32_t num_seqs) {
    const int64_t capacity = static_cast<int64_t>(a.num_blocks) * pa::kBlockSize;
    const int i = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int Hkv = a.num_kv_heads;
    // Wave p < 2 Hkv: KV head p / 2, K (p even) or V. Its token values first: they do not depend on
    // the slot, so they are in flight with the slot lookups below.
    const int h = wave >> 1;
    const bool is_v = (wave & 1) != 0;
    float x[D / 64];
    if (wave < 2 * Hkv) {
        const int64_t src = (static_cast<int64_t>(i) * Hkv + h) * D;
#pragma unroll
        for (int k = 0; k < D / 64; k++) x[k] = pa::load_act(is_v ? a.v_new : a.k_new, a.q_bf16 != 0, src + lane + 64 * k);
    }
    auto last_slot = [&](int t) -> int64_t {
        const int T = clamp_len(a, a.context_lens[t]);
        if (T <= 0) return -1;
        const int32_t bid = a.block_tables[static_cast<int64_t>(t) * a.max_blocks_per_seq + (T - 1) / pa::kBlockSize];
        return bid >= 0 ? static_cast<int64_t>(bid) * pa::kBlockSize + (T - 1) % pa::kBlockSize : -1;
    };
    // Every sequence's slot, looked up once by the workgroup (two dependent loads each, all in
    // flight together): the ownership checks read LDS.
    __shared__ int64_t s_slot[pa::kMaxPersistentSeqs];
    __shared__ __align__(16) int8_t s_stage[pa::kAppendMaxThreads / 64][D];
    for (int t = tid; t < num_seqs; t += blockDim.x) s_slot[t] = last_slot(t);
    __syncthreads();
    auto slot_at = [&](int t) -> int64_t { return s_slot[t]; };
    // The usual case: no other token of the call lands in this token's block, which is then
    // appended by append_int8_one_token; otherwise the general owner path (append_int8_block).
    const int64_t my = s_slot[i];
    const bool valid = my >= 0 && my < capacity;
    bool shared = false;
    if (valid) {
        for (int t = tid; t < num_seqs; t += blockDim.x) {
            const int64_t sl = s_slot[t];
            shared |= t != i && sl >= 0 && sl < capacity && sl / pa::kBlockSize == my / pa::kBlockSize;
        }
    }
    if (__syncthreads_or(shared)) {
        pa::append_int8_block<D>(a.k_new, a.v_new, a.q_bf16 != 0, static_cast<int64_t>(Hkv) * D, slot_at,
                                 static_cast<int32_t>(blockIdx.x), num_seqs,
                                 static_cast<int8_t*>(const_cast<void*>(a.k_cache)),
                                 static_cast<int8_t*>(const_cast<void*>(a.v_cache)), const_cast<float*>(a.k_scale),
                                 const_cast<float*>(a.v_scale), a.k_absmax, a.v_absmax, Hkv, capacity);
        return;
    }
    if (!valid) return;
    const int nwaves = static_cast<int>(blockDim.x) >> 6;
    for (int p = wave; p < 2 * Hkv; p += nwaves) {  // more than 8 KV heads: a wave takes several
        const int hp = p >> 1;
        const bool vp = (p & 1) != 0;
        if (p != wave) {
            const int64_t src = (static_cast<int64_t>(i) * Hkv + hp) * D;
#pragma unroll
            for (int k = 0; k < D / 64; k++) x[k] = pa::load_act(vp ? a.v_new : a.k_new, a.q_bf16 != 0, src + lane + 64 * k);
        }
        pa::append_int8_one_token<D>(x, my, static_cast<int8_t*>(const_cast<void*>(vp ? a.v_cache : a.k_cache)),
                                     const_cast<float*>(vp ? a.v_scale : a.k_scale), vp ? a.v_absmax : a.k_absmax, hp,
                                     Hkv, vp, &s_stage[wave][0]);
    }
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
    const int part = resolve_part(cfg, &err);
    if (part < 0) return pa::set_error(PA_ERROR_UNSUPPORTED, "pa_decode_workspace_size: " + err);
    *bytes = workspace_bytes_for(cfg, num_seqs, max_context_len, part);
    return pa::clear_error();
}

}  // extern "C"

namespace {

pa_status decode_chunk(const char* fn, bool append, pa_stream* stream, const pa_config* cfg, float* out,
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
    const int part = resolve_part(cfg, &err);
    if (part < 0) return pa::set_error(PA_ERROR_UNSUPPORTED, f + ": " + err);
    const bool fp32 = cfg->kv_dtype == PA_DTYPE_FP32;
    const int32_t max_parts = fp32 && max_len > 0 ? (max_len + part - 1) / part : 1;
    // max_len <= max_context_len, so a workspace sized by pa_decode_workspace_size suffices.
    const size_t need = workspace_bytes_for(cfg, num_seqs, max_len, part);
    if (need > 0 && (!workspace || workspace_bytes < need))
        return pa::set_error(PA_ERROR_WORKSPACE_TOO_SMALL,
                             f + ": workspace of " + std::to_string(need) + " bytes required");

    pa::DecodeArgs a{};
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
    a.split_blocks = fp32 ? 0 : part / 16;
    a.num_splits = fp32 ? 0 : cfg->num_splits;
    a.q_bf16 = cfg->q_dtype == PA_DTYPE_BF16;
    a.scale = pa::resolve_scale(cfg);
    const int64_t max_units = fp32 ? 0 : mfma_max_units(cfg, num_seqs, max_len, part, cfg->num_splits);
    a.max_units = max_units;
    if (need > 0) {
        const int64_t rows = fp32 ? static_cast<int64_t>(num_seqs) * cfg->num_q_heads * max_parts : 2 * max_units * G;
        a.ws_o = static_cast<float*>(workspace);
        a.ws_m = a.ws_o + rows * cfg->head_dim;
        a.ws_l = a.ws_m + rows;
        a.ws_pref = reinterpret_cast<int32_t*>(a.ws_l + rows);
    }

    hipStream_t s = pa::native(stream);
    if (cfg->kv_dtype == PA_DTYPE_FP32) {
        if (append) append_last_token_fp32_kernel<<<num_seqs, 256, 0, s>>>(a, cfg->head_dim);
        dim3 grid(max_parts, cfg->num_kv_heads, num_seqs);
        if (!pa::launch_decode_fp32(a, cfg->head_dim, grid, s))
            return pa::set_error(PA_ERROR_UNSUPPORTED, f + ": configuration not compiled");
        PA_HIP_CHECK(hipGetLastError());
        if (max_parts > 1) {
            dim3 mgrid(cfg->num_kv_heads, num_seqs);
            switch (cfg->head_dim) {
                case 32: pa::paged_decode_merge_kernel<32><<<mgrid, 256, 0, s>>>(a); break;
                case 64: pa::paged_decode_merge_kernel<64><<<mgrid, 256, 0, s>>>(a); break;
                case 128: pa::paged_decode_merge_kernel<128><<<mgrid, 256, 0, s>>>(a); break;
                default: pa::paged_decode_merge_kernel<256><<<mgrid, 256, 0, s>>>(a); break;
            }
            PA_HIP_CHECK(hipGetLastError());
        }
        return pa::clear_error();
    }
    const bool qf32 = cfg->q_dtype == PA_DTYPE_FP32;
    const int64_t max_grid = max_units > 0 ? max_units : 1;
    // The merge kernel runs when there is more than one range (a row may span two); a fused bf16
    // append then has it write the new tokens into the cache.
    const bool merge = max_units > cfg->num_kv_heads;
    a.append_in_merge = append && cfg->kv_dtype == PA_DTYPE_BF16 && merge ? 1 : 0;
    if (append && cfg->kv_dtype == PA_DTYPE_INT8 && num_seqs > 0) {
        const int threads = pa::append_int8_threads(cfg->num_kv_heads);
        switch (cfg->head_dim) {
            case 64: append_last_token_int8_kernel<64><<<num_seqs, threads, 0, s>>>(a, num_seqs); break;
            case 128: append_last_token_int8_kernel<128><<<num_seqs, threads, 0, s>>>(a, num_seqs); break;
            default: append_last_token_int8_kernel<256><<<num_seqs, threads, 0, s>>>(a, num_seqs); break;
        }
        PA_HIP_CHECK(hipGetLastError());
        append = false;  // the decode below reads the appended cache
    }
    switch (cfg->head_dim) {
        case 32: pa::launch_decode_mfma<32>(a, cfg->kv_dtype, qf32, append, false, num_seqs, max_grid, s); break;
        case 64: pa::launch_decode_mfma<64>(a, cfg->kv_dtype, qf32, append, false, num_seqs, max_grid, s); break;
        case 128: pa::launch_decode_mfma<128>(a, cfg->kv_dtype, qf32, append, false, num_seqs, max_grid, s); break;
        default: pa::launch_decode_mfma<256>(a, cfg->kv_dtype, qf32, append, false, num_seqs, max_grid, s); break;
    }
    PA_HIP_CHECK(hipGetLastError());
    if (merge) {
        dim3 mgrid(cfg->num_kv_heads, num_seqs);
        const int mthreads = pa::kMergeThreads + (a.append_in_merge ? 64 : 0);
        switch (cfg->head_dim) {
            case 32: pa::paged_decode_merge_split_kernel<32><<<mgrid, mthreads, 0, s>>>(a, num_seqs); break;
            case 64: pa::paged_decode_merge_split_kernel<64><<<mgrid, mthreads, 0, s>>>(a, num_seqs); break;
            case 128: pa::paged_decode_merge_split_kernel<128><<<mgrid, mthreads, 0, s>>>(a, num_seqs); break;
            default: pa::paged_decode_merge_split_kernel<256><<<mgrid, mthreads, 0, s>>>(a, num_seqs); break;
        }
        PA_HIP_CHECK(hipGetLastError());
    }
    return pa::clear_error();
}

// Calls with more sequences than one launch takes (the persistent kernel's prefix table for bf16 /
// int8 caches, the grid's z extent for fp32 caches) are issued in chunks of sequences (each chunk
// is an independent ragged batch on the same stream and workspace).
pa_status decode_impl(const char* fn, bool append, pa_stream* stream, const pa_config* cfg, float* out,
                      const void* q, const void* k_new, const void* v_new, const void* k_cache,
                      const void* v_cache, const float* k_scale, const float* v_scale, float* k_absmax,
                      float* v_absmax, const int32_t* block_tables, const int32_t* context_lens,
                      int32_t num_seqs, int32_t max_blocks_per_seq, int32_t max_context_len, void* workspace,
                      size_t workspace_bytes) {
    // MFMA kernels: the persistent kernel's per-sequence tables; fp32: the grid's z extent.
    const int32_t kChunk = cfg && cfg->kv_dtype == PA_DTYPE_FP32 ? 65535 : pa::kMaxPersistentSeqs - 1;
    if (!cfg || num_seqs <= kChunk)
        return decode_chunk(fn, append, stream, cfg, out, q, k_new, v_new, k_cache, v_cache, k_scale, v_scale,
                            k_absmax, v_absmax, block_tables, context_lens, num_seqs, max_blocks_per_seq,
                            max_context_len, workspace, workspace_bytes);
    const size_t q_elt = cfg->q_dtype == PA_DTYPE_BF16 ? 2 : 4;
    const int64_t qrow = static_cast<int64_t>(cfg->num_q_heads) * cfg->head_dim;
    const int64_t krow = static_cast<int64_t>(cfg->num_kv_heads) * cfg->head_dim;
    for (int32_t s0 = 0; s0 < num_seqs; s0 += kChunk) {
        const int32_t n = num_seqs - s0 < kChunk ? num_seqs - s0 : kChunk;
        auto off = [&](const void* p, int64_t elems) -> const void* {
            return p ? static_cast<const char*>(p) + elems * q_elt : nullptr;
        };
        pa_status st = decode_chunk(fn, append, stream, cfg, out + s0 * qrow, off(q, s0 * qrow),
                                    off(k_new, s0 * krow), off(v_new, s0 * krow), k_cache, v_cache, k_scale,
                                    v_scale, k_absmax, v_absmax,
                                    block_tables ? block_tables + static_cast<int64_t>(s0) * max_blocks_per_seq : nullptr,
                                    context_lens ? context_lens + s0 : nullptr, n, max_blocks_per_seq,
                                    max_context_len, workspace, workspace_bytes);
        if (st != PA_SUCCESS) return st;
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

// ---- decode without a caller workspace ----
//
// pa_paged_decode_noalloc runs pa_paged_decode with the split-K workspace in `scratch`, a
// file-scope device array of PA_NOALLOC_SCRATCH_BYTES. Every device the library runs on holds its
// own copy until the process ends; host code reaches a device's copy only through the address
// hipGetSymbolAddress returns with that device current (kept per device in g_scratch_ptr). The
// decode reads nothing from the workspace that the same call did not write first, so no clearing
// is needed; calls that overlap on one device share the array and race.

namespace {

static __device__ __align__(256) unsigned char scratch[PA_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on device `ordinal`, resolved once per device.
pa_status scratch_address(const std::string& f, int ordinal, void** ptr) {
    if (ordinal < 0 || ordinal >= kMaxScratchDevices)
        return pa::set_error(PA_ERROR_UNSUPPORTED, f + ": device ordinal beyond the scratch table");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[ordinal]) {
        int prev = -1;
        PA_HIP_CHECK(hipGetDevice(&prev));
        if (prev != ordinal) PA_HIP_CHECK(hipSetDevice(ordinal));
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (prev != ordinal) (void)hipSetDevice(prev);
        if (e != hipSuccess) return pa::set_hip_error(e, "hipGetSymbolAddress(scratch)");
        if (!p) return pa::set_error(PA_ERROR_HIP, f + ": hipGetSymbolAddress returned a null scratch address");
        g_scratch_ptr[ordinal] = p;
    }
    *ptr = g_scratch_ptr[ordinal];
    return PA_SUCCESS;
}

}  // namespace

namespace pa {
// Called by pa_device_open, the library's per-device set-up.
pa_status init_decode_scratch(int ordinal) {
    void* p = nullptr;
    return scratch_address("pa_device_open", ordinal, &p);
}
}  // namespace pa

extern "C" {

pa_status pa_paged_decode_noalloc(pa_stream* stream, const pa_config* cfg, float* out, const void* q,
                                  const void* k_cache, const void* v_cache, const float* k_scale,
                                  const float* v_scale, const int32_t* block_tables, const int32_t* context_lens,
                                  int32_t num_seqs, int32_t max_blocks_per_seq, int32_t max_context_len) {
    const std::string f = "pa_paged_decode_noalloc";
    pa_status st = pa::check_config(cfg, f.c_str());
    if (st != PA_SUCCESS) return st;
    if (num_seqs < 0 || max_blocks_per_seq < 0 || max_context_len < 0)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, f + ": negative size");
    if (num_seqs == 0) return pa::clear_error();
    std::string err;
    const int part = resolve_part(cfg, &err);
    if (part < 0) return pa::set_error(PA_ERROR_UNSUPPORTED, f + ": " + err);
    // The workspace a pa_paged_decode call of this shape needs (chunks of sequences reuse it).
    const size_t need = workspace_bytes_for(cfg, num_seqs, effective_max_len(max_context_len, max_blocks_per_seq), part);
    if (need > PA_NOALLOC_SCRATCH_BYTES)
        return pa::set_error(PA_ERROR_WORKSPACE_TOO_SMALL,
                             f + ": this call needs " + std::to_string(need) + " bytes of split-K scratch, above the " +
                                 std::to_string(static_cast<size_t>(PA_NOALLOC_SCRATCH_BYTES)) +
                                 " the library holds per device; use pa_paged_decode with a workspace");
    int ordinal = 0;
    if (stream) ordinal = stream->ordinal;
    else PA_HIP_CHECK(hipGetDevice(&ordinal));
    void* ws = nullptr;
    st = scratch_address(f, ordinal, &ws);
    if (st != PA_SUCCESS) return st;
    return decode_impl(f.c_str(), false, stream, cfg, out, q, nullptr, nullptr, k_cache, v_cache, k_scale, v_scale,
                       nullptr, nullptr, block_tables, context_lens, num_seqs, max_blocks_per_seq, max_context_len,
                       ws, PA_NOALLOC_SCRATCH_BYTES);
}

}  // extern "C"

// ---- shared-prefix decode ----
//
// Sequences forked from one parent keep the parent's first blocks in their tables (copy-on-write
// sharing). pa_paged_decode reads those blocks once per sequence; this entry point reads them once
// per group of up to 16 / G sequences: the group's query heads fill the 16 MFMA columns of one
// pass over the shared blocks (a prefix row), each sequence's own blocks form a suffix row, and a
// merge combines the two per sequence with the usual log-sum-exp reduction. The result is the same
// attention as pa_paged_decode's over the whole context.

namespace {

// Groups the host-side link counts: shared_with_prev[s] = leading table entries sequence s has in
// common with sequence s - 1 (entry 0 ignored). A run of linked sequences shares the minimum of
// its links; runs are cut into groups of at most 16 / G members, and a group of one is no group.
std::vector<int32_t> build_plan_host(int32_t num_seqs, int G, const int32_t* shared_with_prev, int32_t* num_groups) {
    const int cap = 16 / G;
    std::vector<int32_t> groups, seqinfo(static_cast<size_t>(num_seqs) * pa::kPlanSeqInts, 0);
    for (int32_t s = 0; s < num_seqs; s++) seqinfo[static_cast<size_t>(s) * pa::kPlanSeqInts] = -1;
    int32_t s = 0;
    while (s < num_seqs) {
        int32_t e = s + 1;  // run [s, e)
        while (e < num_seqs && shared_with_prev[e] > 0) e++;
        for (int32_t c0 = s; c0 < e; c0 += cap) {
            const int32_t c1 = c0 + cap < e ? c0 + cap : e;
            if (c1 - c0 < 2) continue;
            int32_t shared = INT32_MAX;
            for (int32_t t = c0 + 1; t < c1; t++) shared = shared_with_prev[t] < shared ? shared_with_prev[t] : shared;
            const int32_t g = static_cast<int32_t>(groups.size() / pa::kPlanGroupInts);
            groups.push_back(c0);
            groups.push_back(c1 - c0);
            groups.push_back(shared);
            for (int32_t t = c0; t < c1; t++) {
                seqinfo[static_cast<size_t>(t) * pa::kPlanSeqInts] = g;
                seqinfo[static_cast<size_t>(t) * pa::kPlanSeqInts + 1] = shared;
            }
        }
        s = e;
    }
    *num_groups = static_cast<int32_t>(groups.size() / pa::kPlanGroupInts);
    groups.insert(groups.end(), seqinfo.begin(), seqinfo.end());
    return groups;
}

size_t plan_bytes_for(int32_t num_seqs) {
    return (static_cast<size_t>(num_seqs / 2) * pa::kPlanGroupInts + static_cast<size_t>(num_seqs) * pa::kPlanSeqInts) *
           sizeof(int32_t);
}

// Slots of 16 rows: 2 per unit, then one per (row, KV head) of the decode's list (num_seqs +
// num_groups rows, num_groups <= num_seqs / 2); and a block prefix over the rows.
int64_t prefix_slots(const pa_config* cfg, int32_t num_seqs, int32_t max_len) {
    return 2 * mfma_max_units(cfg, num_seqs, max_len, 0, 0) +
           (static_cast<int64_t>(num_seqs) + num_seqs / 2) * cfg->num_kv_heads;
}
size_t prefix_workspace_bytes_for(const pa_config* cfg, int32_t num_seqs, int32_t max_len) {
    if (num_seqs <= 0) return 0;
    const int64_t rows = prefix_slots(cfg, num_seqs, max_len) * pa::kPrefixSlotRows;
    const int64_t prefs = static_cast<int64_t>(num_seqs) + num_seqs / 2 + 1;
    return static_cast<size_t>(rows) * (cfg->head_dim + 2) * sizeof(float) + static_cast<size_t>(prefs) * 4;
}

}  // namespace

extern "C" {

pa_status pa_prefix_plan_bytes(int32_t num_seqs, size_t* bytes) {
    if (!bytes || num_seqs < 0) return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_prefix_plan_bytes: bad argument");
    *bytes = plan_bytes_for(num_seqs);
    return pa::clear_error();
}

pa_status pa_prefix_plan_fill(const pa_config* cfg, int32_t num_seqs, const int32_t* shared_with_prev,
                              int32_t* plan_host, size_t plan_bytes, int32_t* num_groups) {
    const std::string f = "pa_prefix_plan_fill";
    pa_status st = pa::check_config(cfg, f.c_str());
    if (st != PA_SUCCESS) return st;
    if (num_seqs < 0 || !num_groups || (num_seqs > 0 && (!shared_with_prev || !plan_host)))
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, f + ": bad argument");
    const int G = cfg->num_q_heads / cfg->num_kv_heads;
    if (G < 1 || G > 16) return pa::set_error(PA_ERROR_UNSUPPORTED, f + ": unsupported Hq / Hkv ratio");
    if (plan_bytes < plan_bytes_for(num_seqs))
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, f + ": plan buffer smaller than pa_prefix_plan_bytes");
    *num_groups = 0;
    if (num_seqs == 0) return pa::clear_error();
    for (int32_t s = 1; s < num_seqs; s++)
        if (shared_with_prev[s] < 0) return pa::set_error(PA_ERROR_INVALID_ARGUMENT, f + ": negative shared count");
    int32_t ng = 0;
    const std::vector<int32_t> host = build_plan_host(num_seqs, G, shared_with_prev, &ng);
    std::copy(host.begin(), host.end(), plan_host);
    *num_groups = ng;
    return pa::clear_error();
}

pa_status pa_prefix_plan_build(pa_stream* stream, const pa_config* cfg, int32_t num_seqs,
                               const int32_t* shared_with_prev, void* plan, size_t plan_bytes, int32_t* num_groups) {
    const std::string f = "pa_prefix_plan_build";
    if (num_seqs < 0 || !num_groups || (num_seqs > 0 && !plan))
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, f + ": bad argument");
    *num_groups = 0;
    std::vector<int32_t> host(plan_bytes_for(num_seqs) / sizeof(int32_t) + 1);
    int32_t ng = 0;
    pa_status st = pa_prefix_plan_fill(cfg, num_seqs, shared_with_prev, host.data(), plan_bytes, &ng);
    if (st != PA_SUCCESS) return st;
    if (num_seqs == 0) return pa::clear_error();
    host.resize(static_cast<size_t>(ng) * pa::kPlanGroupInts + static_cast<size_t>(num_seqs) * pa::kPlanSeqInts);
    hipStream_t s = pa::native(stream);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    PA_HIP_CHECK(hipStreamIsCapturing(s, &cs));
    if (cs != hipStreamCaptureStatusNone)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, f + ": the stream is capturing a graph");
    // The host vector dies with this call: the copy is waited for.
    PA_HIP_CHECK(hipMemcpyAsync(plan, host.data(), host.size() * sizeof(int32_t), hipMemcpyHostToDevice, s));
    PA_HIP_CHECK(hipStreamSynchronize(s));
    *num_groups = ng;
    return pa::clear_error();
}

pa_status pa_prefix_workspace_size(const pa_config* cfg, int32_t num_seqs, int32_t max_context_len, size_t* bytes) {
    pa_status st = pa::check_config(cfg, "pa_prefix_workspace_size");
    if (st != PA_SUCCESS) return st;
    if (!bytes || num_seqs < 0 || max_context_len < 0)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_prefix_workspace_size: bad argument");
    *bytes = prefix_workspace_bytes_for(cfg, num_seqs, max_context_len);
    return pa::clear_error();
}

pa_status pa_paged_decode_prefix(pa_stream* stream, const pa_config* cfg, float* out, const void* q,
                                 const void* k_cache, const void* v_cache, const float* k_scale,
                                 const float* v_scale, const int32_t* block_tables, const int32_t* context_lens,
                                 int32_t num_seqs, int32_t max_blocks_per_seq, int32_t max_context_len,
                                 const void* plan, int32_t num_groups, void* workspace, size_t workspace_bytes) {
    const std::string f = "pa_paged_decode_prefix";
    pa_status st = pa::check_config(cfg, f.c_str());
    if (st != PA_SUCCESS) return st;
    if (num_seqs < 0 || max_blocks_per_seq < 0 || max_context_len < 0 || num_groups < 0)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, f + ": negative size");
    if (num_seqs == 0) return pa::clear_error();
    if (cfg->kv_dtype == PA_DTYPE_FP32)
        return pa::set_error(PA_ERROR_UNSUPPORTED, f + ": bf16 or int8 caches only");
    if (num_groups > num_seqs / 2) return pa::set_error(PA_ERROR_INVALID_ARGUMENT, f + ": more groups than pairs");
    if (num_seqs + num_groups > pa::kMaxPersistentSeqs - 1)
        return pa::set_error(PA_ERROR_UNSUPPORTED, f + ": num_seqs + num_groups above " +
                                                       std::to_string(pa::kMaxPersistentSeqs - 1));
    if (!out || !q || !k_cache || !v_cache || !block_tables || !context_lens || !plan)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, f + ": null pointer");
    if (cfg->kv_dtype == PA_DTYPE_INT8 && (!k_scale || !v_scale))
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, f + ": int8 cache needs k_scale and v_scale");
    const int G = cfg->num_q_heads / cfg->num_kv_heads;
    if (!(G == 1 || G == 2 || G == 4 || G == 8 || G == 16))
        return pa::set_error(PA_ERROR_UNSUPPORTED, f + ": unsupported Hq / Hkv ratio");
    if (cfg->num_kv_heads > 65535) return pa::set_error(PA_ERROR_UNSUPPORTED, f + ": too many KV heads");
    const int32_t max_len = effective_max_len(max_context_len, max_blocks_per_seq);
    const size_t need = prefix_workspace_bytes_for(cfg, num_seqs, max_len);
    if (!workspace || workspace_bytes < need)
        return pa::set_error(PA_ERROR_WORKSPACE_TOO_SMALL,
                             f + ": workspace of " + std::to_string(need) + " bytes required");
    pa::DecodeArgs a{};
    a.out = out;
    a.q = q;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.k_scale = k_scale;
    a.v_scale = v_scale;
    a.block_tables = block_tables;
    a.context_lens = context_lens;
    a.num_kv_heads = cfg->num_kv_heads;
    a.group = G;
    a.max_blocks_per_seq = max_blocks_per_seq;
    a.num_blocks = cfg->num_blocks;
    a.max_context_len = max_len;
    a.max_parts = 1;
    a.split_blocks = 0;  // equal ranges per worker (partition_size and num_splits do not apply here)
    a.num_splits = 0;
    a.q_bf16 = cfg->q_dtype == PA_DTYPE_BF16;
    a.scale = pa::resolve_scale(cfg);
    a.plan = static_cast<const int32_t*>(plan);
    a.num_groups = num_groups;
    const int64_t max_units = mfma_max_units(cfg, num_seqs, max_len, 0, 0);
    a.max_units = max_units;
    const int64_t rows = prefix_slots(cfg, num_seqs, max_len) * pa::kPrefixSlotRows;
    a.row_slot_base = static_cast<int32_t>(2 * max_units);
    a.ws_o = static_cast<float*>(workspace);
    a.ws_m = a.ws_o + rows * cfg->head_dim;
    a.ws_l = a.ws_m + rows;
    a.ws_pref = reinterpret_cast<int32_t*>(a.ws_l + rows);
    hipStream_t s = pa::native(stream);
    const bool qf32 = cfg->q_dtype == PA_DTYPE_FP32;
    const int64_t max_grid = max_units > 0 ? max_units : 1;
    switch (cfg->head_dim) {
        case 32: pa::launch_decode_mfma<32>(a, cfg->kv_dtype, qf32, false, true, num_seqs, max_grid, s); break;
        case 64: pa::launch_decode_mfma<64>(a, cfg->kv_dtype, qf32, false, true, num_seqs, max_grid, s); break;
        case 128: pa::launch_decode_mfma<128>(a, cfg->kv_dtype, qf32, false, true, num_seqs, max_grid, s); break;
        default: pa::launch_decode_mfma<256>(a, cfg->kv_dtype, qf32, false, true, num_seqs, max_grid, s); break;
    }
    PA_HIP_CHECK(hipGetLastError());
    dim3 mgrid(cfg->num_kv_heads, num_seqs, G);
    switch (cfg->head_dim) {
        case 32: pa::paged_decode_merge_prefix_kernel<32><<<mgrid, 256, 0, s>>>(a, num_seqs); break;
        case 64: pa::paged_decode_merge_prefix_kernel<64><<<mgrid, 256, 0, s>>>(a, num_seqs); break;
        case 128: pa::paged_decode_merge_prefix_kernel<128><<<mgrid, 256, 0, s>>>(a, num_seqs); break;
        default: pa::paged_decode_merge_prefix_kernel<256><<<mgrid, 256, 0, s>>>(a, num_seqs); break;
    }
    PA_HIP_CHECK(hipGetLastError());
    return pa::clear_error();
}

}  // extern "C"
