// paged_decode.hip -- ragged paged decode for gfx950 (wave64).
//
// Replaces the reference's per-sequence decode loop (DecodeOrchestrator.BatchDecode /
// ComputeDecodeAttention, src/MLFramework/Inference/PagedAttention/Phases/DecodeOrchestrator.cs:64-109,
// which gathers each sequence's K/V and calls StandardPagedAttentionKernel once per sequence,
// Kernels/StandardPagedAttentionKernel.cs:21-84) with one launch over the whole ragged batch.
//
// Work decomposition: one workgroup (256 threads = 4 waves) per (partition, KV head, sequence).
// A partition is PART consecutive tokens (PART / 16 blocks) of one sequence; sequences that fit in
// one partition are finished in place, longer ones write per-partition (max, sum, unnormalised
// output) to the workspace and a second kernel merges them with a log-sum-exp reduction.
// The G = Hq / Hkv query heads of a KV head share every K/V byte loaded (GQA).
//
// Per wave and 16-token block, each lane loads 16-byte chunks: lane = (token-in-group ti, chunk ch),
// CH = D * elt / 16 chunks per token row, TPI = 64 / CH tokens per load instruction, so every load
// instruction of a wave reads 1 KiB of contiguous cache. q.k partial dots are summed across the CH
// lanes of a token with DPP; scores go to LDS, the partition's softmax statistics are block-reduced,
// and P.V accumulates per lane in fp32, reduced across token groups and waves at the end.
#include <string>

#include "pa_internal.h"

namespace {

template <int KV> struct KvT;
template <> struct KvT<PA_DTYPE_FP32> { static constexpr int kElt = 4; };
template <> struct KvT<PA_DTYPE_BF16> { static constexpr int kElt = 2; };
template <> struct KvT<PA_DTYPE_INT8> { static constexpr int kElt = 1; };

template <int KV, int EPC>
__device__ __forceinline__ void unpack(const uint4& r, float (&f)[EPC]) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
    if constexpr (KV == PA_DTYPE_FP32) {
#pragma unroll
        for (int k = 0; k < 4; k++) f[k] = __uint_as_float(w[k]);
    } else if constexpr (KV == PA_DTYPE_BF16) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            f[2 * k] = pa::bf16_lo(w[k]);
            f[2 * k + 1] = pa::bf16_hi(w[k]);
        }
    } else {
#pragma unroll
        for (int k = 0; k < 4; k++)
#pragma unroll
            for (int b = 0; b < 4; b++) f[4 * k + b] = pa::i8_at(w[k], b);
    }
}

struct DecodeArgs {
    float* out;
    const void* q;
    const void* k_cache;
    const void* v_cache;
    const float* k_scale;
    const float* v_scale;
    const int32_t* block_tables;
    const int32_t* context_lens;
    float* ws_o;  // [num_seqs][Hq][max_parts][D]
    float* ws_m;  // [num_seqs][Hq][max_parts]
    float* ws_l;  // [num_seqs][Hq][max_parts]
    int32_t num_kv_heads;
    int32_t max_blocks_per_seq;
    int32_t num_blocks;
    int32_t max_context_len;
    int32_t max_parts;
    int32_t q_bf16;
    float scale;
};

__device__ __forceinline__ int clamp_len(const DecodeArgs& a, int seq) {
    int T = a.context_lens[seq];
    T = min(T, a.max_blocks_per_seq * pa::kBlockSize);
    T = min(T, a.max_context_len);
    return T;
}

template <int D, int KV, int G, int PART>
__global__ __launch_bounds__(256) void paged_decode_kernel(const DecodeArgs a) {
    constexpr int ELT = KvT<KV>::kElt;
    constexpr int CH = D * ELT / 16;  // 16-byte chunks per token row
    constexpr int EPC = 16 / ELT;     // elements per chunk
    constexpr int TPI = 64 / CH;      // tokens per wave load instruction
    constexpr int LPB = 16 / TPI;     // load instructions per block per lane
    constexpr int NBP = PART / 16;    // blocks per partition
    constexpr int NBW = NBP / 4;      // blocks per wave
    constexpr int TPT = PART / 256;   // softmax tokens per thread
    // Loads are hoisted ahead of the math while they fit in registers (bytes in flight hide HBM
    // latency); wider rows (fp32 D >= 128, D = 256) load block by block instead.
    constexpr bool kPreloadK = NBW * LPB <= 32;
    constexpr bool kPreloadV = NBW * LPB <= 16;
    static_assert(CH >= 4 && CH <= 64, "unsupported head_dim / dtype combination");
    static_assert(PART % 256 == 0, "PART must be a multiple of 256");

    __shared__ float s_logits[G][PART];
    __shared__ float s_red[4][G];
    __shared__ float s_o[4][G][D];

    const int part = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int Hkv = a.num_kv_heads, Hq = Hkv * G;

    const int T = clamp_len(a, seq);
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

    // This lane's slice of the G query heads.
    float qf[G][EPC];
    {
        const int64_t qb = (static_cast<int64_t>(seq) * Hq + kvh * G) * D + ch * EPC;
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int e = 0; e < EPC; e++)
                qf[g][e] = a.q_bf16 ? pa::bf16_to_f32(static_cast<const uint16_t*>(a.q)[qb + g * D + e])
                                    : static_cast<const float*>(a.q)[qb + g * D + e];
    }

    // Physical block ids of this wave's blocks (wave-uniform).
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

    const char* kc = static_cast<const char*>(a.k_cache);
    const char* vc = static_cast<const char*>(a.v_cache);
    auto chunk_off = [&](int b, int j) -> int64_t {
        return ((static_cast<int64_t>(b) * Hkv + kvh) * 16 + j * TPI + ti) * (D * ELT) + ch * 16;
    };

    auto load = [&](const char* base, int b, int j) -> uint4 {
        return b >= 0 ? *reinterpret_cast<const uint4*>(base + chunk_off(b, j)) : make_uint4(0, 0, 0, 0);
    };
    uint4 kr[kPreloadK ? NBW : 1][LPB];
    uint4 vr[kPreloadV ? NBW : 1][LPB];
#pragma unroll
    for (int i = 0; i < NBW; i++)
#pragma unroll
        for (int j = 0; j < LPB; j++) {
            if constexpr (kPreloadK) kr[i][j] = load(kc, bid[i], j);
            if constexpr (kPreloadV) vr[i][j] = load(vc, bid[i], j);
        }

    // ---- scores: s = (q . k) * scale  (int8: (q . k_code) * k_scale * scale) ----
#pragma unroll
    for (int i = 0; i < NBW; i++) {
        float ks = 1.0f;
        if constexpr (KV == PA_DTYPE_INT8) ks = bid[i] >= 0 ? a.k_scale[static_cast<int64_t>(bid[i]) * Hkv + kvh] : 0.0f;
#pragma unroll
        for (int j = 0; j < LPB; j++) {
            uint4 raw;
            if constexpr (kPreloadK) raw = kr[i][j];
            else raw = load(kc, bid[i], j);
            float kf[EPC];
            unpack<KV, EPC>(raw, kf);
            float dot[G];
#pragma unroll
            for (int g = 0; g < G; g++) {
                float acc = 0.0f;
#pragma unroll
                for (int e = 0; e < EPC; e++) acc += qf[g][e] * kf[e];
                dot[g] = pa::group_sum<CH>(acc);
            }
            const int lt = (i * 4 + wave) * 16 + j * TPI + ti;
            if (ch == 0) {
#pragma unroll
                for (int g = 0; g < G; g++) {
                    float sc = dot[g];
                    if constexpr (KV == PA_DTYPE_INT8) sc = sc * ks;
                    s_logits[g][lt] = lt < ntok ? sc * a.scale : -INFINITY;
                }
            }
        }
    }
    __syncthreads();

    // ---- partition softmax statistics: m = max s, p = exp(s - m), l = sum p ----
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

    // ---- o = sum_t p_t * v_t ----
    float acc[G][EPC];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < EPC; e++) acc[g][e] = 0.0f;
#pragma unroll
    for (int i = 0; i < NBW; i++) {
        float vs = 1.0f;
        if constexpr (KV == PA_DTYPE_INT8) vs = bid[i] >= 0 ? a.v_scale[static_cast<int64_t>(bid[i]) * Hkv + kvh] : 0.0f;
#pragma unroll
        for (int j = 0; j < LPB; j++) {
            uint4 raw;
            if constexpr (kPreloadV) raw = vr[i][j];
            else raw = load(vc, bid[i], j);
            float vf[EPC];
            unpack<KV, EPC>(raw, vf);
            const int lt = (i * 4 + wave) * 16 + j * TPI + ti;
#pragma unroll
            for (int g = 0; g < G; g++) {
                float p = s_logits[g][lt];
                if constexpr (KV == PA_DTYPE_INT8) p = p * vs;
#pragma unroll
                for (int e = 0; e < EPC; e++) acc[g][e] += p * vf[e];
            }
        }
    }
    // Sum the TPI token groups of the wave (lanes ch, ch + CH, ...).
#pragma unroll
    for (int off = CH; off < 64; off <<= 1)
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int e = 0; e < EPC; e++) acc[g][e] += __shfl_xor(acc[g][e], off, 64);
    if (ti == 0)
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int e = 0; e < EPC; e++) s_o[wave][g][ch * EPC + e] = acc[g][e];
    __syncthreads();

    for (int idx = tid; idx < G * D; idx += 256) {
        const int g = idx / D, d = idx - g * D;
        const float o = (s_o[0][g][d] + s_o[1][g][d]) + (s_o[2][g][d] + s_o[3][g][d]);
        const int64_t row = static_cast<int64_t>(seq) * Hq + kvh * G + g;
        if (nparts == 1) {
            a.out[row * D + d] = o / l[g];
        } else {
            const int64_t pidx = row * a.max_parts + part;
            a.ws_o[pidx * D + d] = o;
            if (d == 0) {
                a.ws_m[pidx] = m[g];
                a.ws_l[pidx] = l[g];
            }
        }
    }
}

// Log-sum-exp merge of the partitions of one (sequence, query head).
template <int D>
__global__ __launch_bounds__(256) void paged_decode_merge_kernel(const DecodeArgs a, int32_t part_size) {
    const int h = blockIdx.x, seq = blockIdx.y, Hq = gridDim.x;
    const int T = clamp_len(a, seq);
    if (T <= 0) return;
    const int nparts = (T + part_size - 1) / part_size;
    if (nparts <= 1) return;
    const int64_t row = static_cast<int64_t>(seq) * Hq + h;
    const int64_t base = row * a.max_parts;
    float M = -INFINITY;
    for (int p = 0; p < nparts; p++) M = fmaxf(M, a.ws_m[base + p]);
    float L = 0.0f;
    for (int p = 0; p < nparts; p++) L += a.ws_l[base + p] * __expf(a.ws_m[base + p] - M);
    const float inv = 1.0f / L;
    for (int d = threadIdx.x; d < D; d += blockDim.x) {
        float o = 0.0f;
        for (int p = 0; p < nparts; p++) o += a.ws_o[(base + p) * D + d] * __expf(a.ws_m[base + p] - M);
        a.out[row * D + d] = o * inv;
    }
}

constexpr int kDefaultPart = 256;

template <int D, int KV, int G>
void launch_decode(const DecodeArgs& a, int part, dim3 grid, hipStream_t s) {
    if (part == 512) paged_decode_kernel<D, KV, G, 512><<<grid, 256, 0, s>>>(a);
    else paged_decode_kernel<D, KV, G, 256><<<grid, 256, 0, s>>>(a);
}

template <int D, int KV>
bool dispatch_g(int G, const DecodeArgs& a, int part, dim3 grid, hipStream_t s) {
    switch (G) {
        case 1: launch_decode<D, KV, 1>(a, part, grid, s); return true;
        case 2: launch_decode<D, KV, 2>(a, part, grid, s); return true;
        case 4: launch_decode<D, KV, 4>(a, part, grid, s); return true;
        case 8: launch_decode<D, KV, 8>(a, part, grid, s); return true;
        default: return false;
    }
}

template <int D>
bool dispatch_kv(int kv, int G, const DecodeArgs& a, int part, dim3 grid, hipStream_t s) {
    switch (kv) {
        case PA_DTYPE_FP32: return dispatch_g<D, PA_DTYPE_FP32>(G, a, part, grid, s);
        case PA_DTYPE_BF16: return dispatch_g<D, PA_DTYPE_BF16>(G, a, part, grid, s);
        case PA_DTYPE_INT8: return dispatch_g<D, PA_DTYPE_INT8>(G, a, part, grid, s);
        default: return false;
    }
}

int resolve_part(const pa_config* cfg) { return cfg->partition_size > 0 ? cfg->partition_size : kDefaultPart; }

size_t workspace_bytes_for(const pa_config* cfg, int32_t num_seqs, int32_t max_context_len) {
    const int part = resolve_part(cfg);
    const int64_t max_parts = (static_cast<int64_t>(max_context_len) + part - 1) / part;
    if (max_parts <= 1 || num_seqs <= 0) return 0;
    const int64_t rows = static_cast<int64_t>(num_seqs) * cfg->num_q_heads * max_parts;
    return static_cast<size_t>(rows) * (cfg->head_dim + 2) * sizeof(float);
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
    const int part = resolve_part(cfg);
    if (part != 256 && part != 512)
        return pa::set_error(PA_ERROR_UNSUPPORTED, "pa_decode_workspace_size: partition_size must be 256 or 512");
    *bytes = workspace_bytes_for(cfg, num_seqs, max_context_len);
    return pa::clear_error();
}

pa_status pa_paged_decode(pa_stream* stream, const pa_config* cfg, float* out, const void* q,
                          const void* k_cache, const void* v_cache, const float* k_scale,
                          const float* v_scale, const int32_t* block_tables, const int32_t* context_lens,
                          int32_t num_seqs, int32_t max_blocks_per_seq, int32_t max_context_len,
                          void* workspace, size_t workspace_bytes) {
    pa_status st = pa::check_config(cfg, "pa_paged_decode");
    if (st != PA_SUCCESS) return st;
    if (num_seqs < 0 || max_blocks_per_seq < 0 || max_context_len < 0)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_paged_decode: negative size");
    if (num_seqs == 0) return pa::clear_error();
    if (num_seqs > 65535) return pa::set_error(PA_ERROR_UNSUPPORTED, "pa_paged_decode: num_seqs > 65535");
    if (!out || !q || !k_cache || !v_cache || !block_tables || !context_lens)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_paged_decode: null pointer");
    if (cfg->kv_dtype == PA_DTYPE_INT8 && (!k_scale || !v_scale))
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_paged_decode: int8 cache needs k_scale and v_scale");
    const int part = resolve_part(cfg);
    if (part != 256 && part != 512)
        return pa::set_error(PA_ERROR_UNSUPPORTED, "pa_paged_decode: partition_size must be 256 or 512");
    const int G = cfg->num_q_heads / cfg->num_kv_heads;
    if (G != 1 && G != 2 && G != 4 && G != 8)
        return pa::set_error(PA_ERROR_UNSUPPORTED, "pa_paged_decode: Hq / Hkv must be 1, 2, 4 or 8");
    if (cfg->num_kv_heads > 65535) return pa::set_error(PA_ERROR_UNSUPPORTED, "pa_paged_decode: too many KV heads");

    // Tokens beyond the table are never read, so the grid only needs to cover what the table holds.
    int32_t max_len = max_context_len;
    const int64_t table_tokens = static_cast<int64_t>(max_blocks_per_seq) * pa::kBlockSize;
    if (max_len > table_tokens) max_len = static_cast<int32_t>(table_tokens);
    const int32_t max_parts = max_len > 0 ? (max_len + part - 1) / part : 1;
    const size_t need = workspace_bytes_for(cfg, num_seqs, max_len);
    if (need > 0 && (!workspace || workspace_bytes < need))
        return pa::set_error(PA_ERROR_WORKSPACE_TOO_SMALL,
                             "pa_paged_decode: workspace of " + std::to_string(need) + " bytes required");

    DecodeArgs a{};
    a.out = out;
    a.q = q;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.k_scale = k_scale;
    a.v_scale = v_scale;
    a.block_tables = block_tables;
    a.context_lens = context_lens;
    a.num_kv_heads = cfg->num_kv_heads;
    a.max_blocks_per_seq = max_blocks_per_seq;
    a.num_blocks = cfg->num_blocks;
    a.max_context_len = max_len;
    a.max_parts = max_parts;
    a.q_bf16 = cfg->q_dtype == PA_DTYPE_BF16;
    a.scale = pa::resolve_scale(cfg);
    if (need > 0) {
        const int64_t rows = static_cast<int64_t>(num_seqs) * cfg->num_q_heads * max_parts;
        a.ws_o = static_cast<float*>(workspace);
        a.ws_m = a.ws_o + rows * cfg->head_dim;
        a.ws_l = a.ws_m + rows;
    }

    hipStream_t s = pa::native(stream);
    dim3 grid(max_parts, cfg->num_kv_heads, num_seqs);
    bool ok = false;
    switch (cfg->head_dim) {
        case 64: ok = dispatch_kv<64>(cfg->kv_dtype, G, a, part, grid, s); break;
        case 128: ok = dispatch_kv<128>(cfg->kv_dtype, G, a, part, grid, s); break;
        case 256: ok = dispatch_kv<256>(cfg->kv_dtype, G, a, part, grid, s); break;
    }
    if (!ok) return pa::set_error(PA_ERROR_UNSUPPORTED, "pa_paged_decode: configuration not compiled");
    PA_HIP_CHECK(hipGetLastError());
    if (max_parts > 1) {
        dim3 mgrid(cfg->num_q_heads, num_seqs);
        const int threads = cfg->head_dim;
        switch (cfg->head_dim) {
            case 64: paged_decode_merge_kernel<64><<<mgrid, threads, 0, s>>>(a, part); break;
            case 128: paged_decode_merge_kernel<128><<<mgrid, threads, 0, s>>>(a, part); break;
            default: paged_decode_merge_kernel<256><<<mgrid, threads, 0, s>>>(a, part); break;
        }
        PA_HIP_CHECK(hipGetLastError());
    }
    return pa::clear_error();
}

}  // extern "C"
