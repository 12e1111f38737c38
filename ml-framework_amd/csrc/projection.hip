// projection.hip -- the Q/K/V and output projections either side of paged attention, gfx950.
//
// The reference layer projects the hidden states with three bias-free Linear layers, stores the
// new K/V in the cache and projects the attention output with a fourth
// (PagedAttentionLayer.ComputeAttention, src/MLFramework/Inference/PagedAttention/Layers/
// PagedAttentionLayer.cs:112-142; Linear.Forward y = x W^T, src/MLFramework/Modules/Linear.cs:
// 81-110). Here the three input projections are one GEMM against the stacked weight
// [(Hq + 2 Hkv) * D][hidden] (bf16 operands, fp32 accumulation), followed by an epilogue that
// writes Q in the activation dtype and appends K/V into the paged cache exactly as pa_kv_append
// does with fp32 input (the GEMM rows are read in place with a token stride). The output
// projection truncates the fp32 attention output to bf16 and multiplies by W_o^T.
//
// Decode-sized batches (at most kSkinnyMaxTok tokens) run on skinny_gemm_kernel: the weight is
// read once from HBM in 16-byte pieces straight into MFMA operands, the whole batch of tokens
// rides along as the other operand, and the k range is split over workgroups so that the chip has
// enough loads in flight; a small kernel adds the split partials in a fixed order. Larger batches
// (prefill chunks) are compute-bound and go to rocBLAS.
#include <mutex>
#include <string>
#include <unordered_map>

#include <rocblas/rocblas.h>

#include "decode_common.h"

namespace {

using pa::bf16x8_t;
using pa::f32x4_t;

// ---- weight-streaming GEMM for decode-sized batches --------------------------------------------
//
// part[s][t][c] = sum over k in split s of a[t][k] * w[c][k], t < n <= 64, c < cols.
// A workgroup owns 64 output columns (64 weight rows) and one split's k range, and streams it in
// stages of 64 k: each stage brings the 64 rows' next 128-byte lines (8 KB) and the activations'
// matching pieces into LDS with LDS-direct loads, 8 rows x one full line per instruction (reading
// weight rows in whole lines streams at the chip's bandwidth; 64-byte pieces of 16 rows per
// instruction, what MFMA operands loaded straight into registers would need, measured 30% slower).
// Wave w multiplies all 64 rows by tokens 16w .. 16w + 15 (v_mfma_f32_16x16x32_bf16, four 16-row
// tiles), so no partials are exchanged inside the workgroup. The weight is the only operand read
// from HBM; the activations (at most 1 MB) come from the L2.
constexpr int kSkinnyMaxTok = 64;  // tokens per launch: one 16-token MFMA column tile per wave
constexpr int kSkinnyCols = 64;    // output columns (weight rows) per workgroup
constexpr int kSkinnyChunk = 64;   // k per stage: one 128-byte line of each bf16 weight row
constexpr int kSkinnyMaxSplits = 8;

struct SkinnyArgs {
    const void* a;      // [n][k], bf16 or fp32 (truncated to bf16 on use), row stride k
    const uint16_t* w;  // [cols][k] bf16
    float* slab0;       // split 0's partial, [n][cols]
    float* slabs;       // splits 1 ..: [splits - 1][n][cols]
    int32_t n, cols, k;
    int32_t krw;        // k per workgroup (per split), a multiple of kSkinnyChunk
};

// LDS stage layout: weight rows [64][128 B], then activation rows [64][128 B] (bf16) or [64][256 B]
// (fp32). The 16-byte pieces of a row are stored XOR-swizzled by the row's bits 1..3 (bf16) or
// 0..3 (fp32): a ds_read_b128 of an MFMA operand (lane (r, g) reads row r, piece 4s + g) then hits
// 16 distinct bank groups in each of the 16-lane sets gfx950 serves together (quads {0,3,5,6} and
// {1,2,4,7} of each half-wave).
template <bool AF32> struct SkinnyStage {
    static constexpr int kAE = AF32 ? 4 : 2;                             // bytes per activation element
    static constexpr int kWBytes = kSkinnyCols * kSkinnyChunk * 2;       // 8 KB
    static constexpr int kABytes = kSkinnyMaxTok * kSkinnyChunk * kAE;   // 8 or 16 KB
    static constexpr int kBytes = kWBytes + kABytes;
    static constexpr int kSlots = AF32 ? 3 : 4;                          // stages resident (72 / 64 KB)
    static constexpr int kALoads = kABytes / 4096;                       // per wave per stage
    static constexpr int kLoads = 2 + kALoads;                           // + 2 weight loads
};

__device__ __forceinline__ uint32_t trunc_pair(float lo, float hi) {
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

template <bool AF32>
__global__ __launch_bounds__(256, 2) void skinny_gemm_kernel(const SkinnyArgs p) {
    using L = SkinnyStage<AF32>;
    __shared__ __attribute__((aligned(16))) char lds[L::kSlots * L::kBytes];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: LDS addresses go to M0
    const int tiles = (p.cols + kSkinnyCols - 1) / kSkinnyCols;
    const int tile = blockIdx.x % tiles, split = blockIdx.x / tiles;
    const int c0 = tile * kSkinnyCols;
    const int kbeg = split * p.krw;
    const int nst = p.krw / kSkinnyChunk;
    const uint32_t base = pa::lds_address(lds);

    // LDS-direct sources at stage 0 (byte offsets). Weight load i of wave w: rows 16w + 8i .. + 7,
    // lane l -> row 16w + 8i + l / 8, LDS piece l % 8 holding memory piece (l % 8) ^ ((row >> 1) & 7).
    // Rows past cols and tokens past n read the last row / token (never stored).
    int wsrc[2], asrc[L::kALoads];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int row = 16 * wave + 8 * i + (lane >> 3);
        const int mem = (lane & 7) ^ ((row >> 1) & 7);
        wsrc[i] = (min(c0 + row, p.cols - 1) * p.k + kbeg + 8 * mem) * 2;
    }
#pragma unroll
    for (int i = 0; i < L::kALoads; i++) {
        if constexpr (AF32) {  // tokens 16w + 4i .. + 3, 16 pieces per 256-byte row
            const int tok = 16 * wave + 4 * i + (lane >> 4);
            const int mem = (lane & 15) ^ (tok & 15);
            asrc[i] = (min(tok, p.n - 1) * p.k + kbeg) * 4 + 16 * mem;
        } else {  // tokens 16w + 8i .. + 7, like the weight rows
            const int tok = 16 * wave + 8 * i + (lane >> 3);
            const int mem = (lane & 7) ^ ((tok >> 1) & 7);
            asrc[i] = (min(tok, p.n - 1) * p.k + kbeg + 8 * mem) * 2;
        }
    }
    const uint32_t wbytes = static_cast<uint32_t>(p.cols) * p.k * 2;
    const uint32_t abytes = static_cast<uint32_t>(p.n) * p.k * L::kAE;

    // Stage st into slot sl; stages past the end load through zero-sized descriptors (zeros, no
    // memory traffic) so that every stage issues the same number of loads.
    auto issue = [&](int st, int sl) {
        const bool live = st < nst;
        const pa::u32x4_t rw = pa::buffer_rsrc_words(p.w, live ? wbytes : 0u);
        const pa::u32x4_t ra = pa::buffer_rsrc_words(p.a, live ? abytes : 0u);
        const uint32_t dst = base + sl * L::kBytes;
#pragma unroll
        for (int i = 0; i < 2; i++)
            pa::lds_load16(rw, wsrc[i] + st * kSkinnyChunk * 2, dst + (2 * wave + i) * 1024);
#pragma unroll
        for (int i = 0; i < L::kALoads; i++)
            pa::lds_load16(ra, asrc[i] + st * kSkinnyChunk * L::kAE,
                           dst + L::kWBytes + (L::kALoads * wave + i) * 1024);
    };

    // MFMA operand layout (16x16x32): lane (r, g) holds row / column r and k elements 8g .. 8g + 7
    // of each 32-wide step; the accumulator holds rows 4g .. 4g + 3 of column r.
    const int r = lane & 15, g = lane >> 4;
    const int sw3 = (r >> 1) & 7;  // swizzle of weight row 16 rb + r and bf16 token row 16 w + r
    f32x4_t acc[4];
#pragma unroll
    for (int rb = 0; rb < 4; rb++) acc[rb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // All of a stage's operand reads are issued before its MFMAs (one LDS latency per stage, not
    // one per MFMA).
    auto compute = [&](int sl) {
        const char* ws = lds + sl * L::kBytes;
        const char* as = ws + L::kWBytes;
        uint4 wv[2][4], av[2][L::kAE / 2];
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const int c = 4 * s + g;  // 16-byte piece of the 128-byte line
            if constexpr (AF32) {
                const char* row = as + (16 * wave + r) * 256;
                av[s][0] = *reinterpret_cast<const uint4*>(row + 16 * ((2 * c) ^ r));
                av[s][1] = *reinterpret_cast<const uint4*>(row + 16 * ((2 * c + 1) ^ r));
            } else {
                av[s][0] = *reinterpret_cast<const uint4*>(as + (16 * wave + r) * 128 + 16 * (c ^ sw3));
            }
#pragma unroll
            for (int rb = 0; rb < 4; rb++)
                wv[s][rb] = *reinterpret_cast<const uint4*>(ws + (16 * rb + r) * 128 + 16 * (c ^ sw3));
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < 2; s++) {
            bf16x8_t bop;
            if constexpr (AF32) {
                const uint4 x = av[s][0], y = av[s][1];
                bop = __builtin_bit_cast(bf16x8_t, make_uint4(trunc_pair(__uint_as_float(x.x), __uint_as_float(x.y)),
                                                              trunc_pair(__uint_as_float(x.z), __uint_as_float(x.w)),
                                                              trunc_pair(__uint_as_float(y.x), __uint_as_float(y.y)),
                                                              trunc_pair(__uint_as_float(y.z), __uint_as_float(y.w))));
            } else {
                bop = __builtin_bit_cast(bf16x8_t, av[s][0]);
            }
#pragma unroll
            for (int rb = 0; rb < 4; rb++)
                acc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, wv[s][rb]), bop, acc[rb],
                                                                  0, 0, 0);
        }
    };

    // kSlots - 1 stages in flight. Before stage st: this wave's loads of stage st have landed (the
    // kSlots - 2 later stages may still be in flight), its LDS reads are done, and the barrier makes
    // that true for all waves, so stage st is complete in LDS and the slot of stage st - 1 is free.
    // The waits are explicit: the compiler does not see the LDS-direct loads, and __syncthreads()
    // would wait for every load.
#pragma unroll
    for (int i = 0; i < L::kSlots - 1; i++) issue(i, i);
    for (int st = 0; st < nst; st++) {
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(L::kLoads * (L::kSlots - 2)) : "memory");
        issue(st + L::kSlots - 1, (st + L::kSlots - 1) % L::kSlots);
        compute(st % L::kSlots);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no LDS-direct write may outlive the workgroup

    const int t = 16 * wave + r;
    float* dst = split == 0 ? p.slab0 : p.slabs + static_cast<int64_t>(split - 1) * p.n * p.cols;
    if (t < p.n) {
#pragma unroll
        for (int rb = 0; rb < 4; rb++) {
            const int c = c0 + 16 * rb + 4 * g;
            if (c < p.cols) *reinterpret_cast<f32x4_t*>(dst + static_cast<int64_t>(t) * p.cols + c) = acc[rb];
        }
    }
}

// Epilogue of the skinny GEMMs, one workgroup per (token row of y [n][cols], 1024 columns):
// y = slab0 + slabs[0] + ... + slabs[rest - 1] (in that order, written back into slab0), 4 columns
// per thread. With q_out, columns below nq also go to q_out [n][nq] as bf16 (truncation), and with
// an fp32 / bf16 cache (`cache` 1 / 2; 0: none) the K columns [nq, nq + nkv) and V columns
// [nq + nkv, nq + 2 nkv) are stored at the row's slot exactly as pa_kv_append stores fp32 input: K
// tiles [16][D] (4 consecutive dims per thread: one 8- or 16-byte store), V tiles [D][16] (element
// stores). A slot outside [0, capacity) skips the row's append.
__global__ __launch_bounds__(256) void skinny_epilogue_kernel(float* __restrict__ slab0, const float* __restrict__ slabs,
                                                              int32_t rest, int32_t n, int32_t cols, int32_t nq,
                                                              uint16_t* __restrict__ q_out, int32_t cache,
                                                              const int64_t* __restrict__ slot_mapping,
                                                              void* __restrict__ k_cache, void* __restrict__ v_cache,
                                                              int32_t num_kv_heads, int32_t head_dim, int64_t capacity) {
    const int t = blockIdx.x;
    const int64_t plane = static_cast<int64_t>(n) * cols;
    const int nkv = num_kv_heads * head_dim;
    int64_t slot = -1;
    if (cache) slot = slot_mapping[t];
    const bool app = cache && slot >= 0 && slot < capacity;
    const int64_t blk = slot / pa::kBlockSize, off = slot % pa::kBlockSize;
    const int c = 1024 * blockIdx.y + 4 * threadIdx.x;
    if (c < cols) {
        const int64_t i = static_cast<int64_t>(t) * cols + c;
        f32x4_t v = *reinterpret_cast<const f32x4_t*>(slab0 + i);
        for (int s = 0; s < rest; s++) v += *reinterpret_cast<const f32x4_t*>(slabs + s * plane + i);
        if (rest > 0) *reinterpret_cast<f32x4_t*>(slab0 + i) = v;
        if (c < nq) {
            if (q_out)
                *reinterpret_cast<uint2*>(q_out + static_cast<int64_t>(t) * nq + c) =
                    make_uint2(trunc_pair(v[0], v[1]), trunc_pair(v[2], v[3]));
        } else if (app && c < nq + 2 * nkv) {
            const bool is_v = c >= nq + nkv;
            const int j = c - nq - (is_v ? nkv : 0);
            const int h = j / head_dim, d = j - h * head_dim;
            const int64_t tile = (blk * num_kv_heads + h) * pa::kBlockSize * head_dim;
            if (!is_v) {
                const int64_t o = tile + off * head_dim + d;
                if (cache == 2)
                    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(k_cache) + o) =
                        make_uint2(trunc_pair(v[0], v[1]), trunc_pair(v[2], v[3]));
                else
                    *reinterpret_cast<f32x4_t*>(static_cast<float*>(k_cache) + o) = v;
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int64_t o = tile + static_cast<int64_t>(d + e) * pa::kBlockSize + off;
                    if (cache == 2) static_cast<uint16_t*>(v_cache)[o] = pa::bf16_trunc(v[e]);
                    else static_cast<float*>(v_cache)[o] = v[e];
                }
            }
        }
    }
}

// Splits of the k range for a skinny GEMM with `cols` output columns: at most 384 workgroups (one
// or two per CU of a 256-CU device, all resident), as many as that allows up to kSkinnyMaxSplits.
// Measured at k = 4096 (cold weights): 6144 columns 15.6 us at 4 splits against 16.0 / 17.2 at 2 /
// 8; 4096 columns 12.3 us at 4 against 13.5 at 8 (each split adds a partial plane to write and
// add). Depends on cols only, so the workspace sizes need no k.
int skinny_splits(int64_t cols) {
    const int64_t tiles = (cols + kSkinnyCols - 1) / kSkinnyCols;
    int s = 1;
    while (s < kSkinnyMaxSplits && tiles * 2 * s <= 384) s *= 2;
    return s;
}

// The skinny path takes n <= 64 tokens, k a multiple of 64 (whole stages), cols a multiple of 16,
// operands under 2 GiB (32-bit buffer offsets) and 16-byte aligned.
bool skinny_fits(int32_t n, int64_t cols, int32_t k, const void* a, const void* w, const void* out0,
                 const void* out1) {
    auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    return n > 0 && n <= kSkinnyMaxTok && k > 0 && k % kSkinnyChunk == 0 && cols % 16 == 0 &&
           cols * k * 2 < (int64_t{1} << 31) && al(a) && al(w) && al(out0) && (!out1 || al(out1));
}

// Launches the skinny GEMM: partial 0 into slab0, the others into slabs [splits - 1][n][cols].
// Returns the split count used (at most skinny_splits(cols)).
int launch_skinny(hipStream_t s, const void* a, bool a_f32, const uint16_t* w, float* slab0, float* slabs,
                  int32_t n, int32_t cols, int32_t k) {
    int splits = skinny_splits(cols);
    while (splits > 1 && k % (splits * kSkinnyChunk) != 0) splits /= 2;
    const SkinnyArgs p{a, w, slab0, slabs, n, cols, k, k / splits};
    const dim3 grid(static_cast<unsigned>(((cols + kSkinnyCols - 1) / kSkinnyCols) * splits));
    if (a_f32) skinny_gemm_kernel<true><<<grid, 256, 0, s>>>(p);
    else skinny_gemm_kernel<false><<<grid, 256, 0, s>>>(p);
    return splits;
}

void launch_epilogue(hipStream_t s, float* slab0, const float* slabs, int rest, int32_t n, int32_t cols, int32_t nq,
                     uint16_t* q_out, int32_t cache, const int64_t* slot_mapping, void* k_cache, void* v_cache,
                     int32_t num_kv_heads, int32_t head_dim, int64_t capacity) {
    const dim3 grid(static_cast<unsigned>(n), static_cast<unsigned>((cols + 1023) / 1024));
    skinny_epilogue_kernel<<<grid, 256, 0, s>>>(slab0, slabs, rest, n, cols, nq, q_out, cache, slot_mapping, k_cache,
                                                v_cache, num_kv_heads, head_dim, capacity);
}

// ---- rocBLAS, for batches past the skinny path -------------------------------------------------

// One rocBLAS handle per device, created on first use and kept for the life of the process
// (destroying it at exit would race the runtime's own teardown). Calls serialise on the mutex
// around the handle's stream binding and launch.
struct BlasHandles {
    std::mutex mu;
    std::unordered_map<int, rocblas_handle> by_device;
};
BlasHandles& blas() {
    static BlasHandles* h = new BlasHandles;
    return *h;
}

const char* blas_status(rocblas_status st) { return rocblas_status_to_string(st); }

// y[n][o] (fp32, row-major) = a[n][k] (bf16) . w[o][k]^T (bf16), on stream s.
pa_status gemm_bf16_nt(const std::string& f, hipStream_t s, const void* a, const void* w, float* y, int32_t n,
                       int32_t o, int32_t k) {
    int dev = 0;
    if (s) PA_HIP_CHECK(hipStreamGetDevice(s, &dev));
    else PA_HIP_CHECK(hipGetDevice(&dev));
    int cur = 0;
    PA_HIP_CHECK(hipGetDevice(&cur));
    if (cur != dev) PA_HIP_CHECK(hipSetDevice(dev));  // the handle and its launches belong to dev
    struct Restore {
        int d;
        bool on;
        ~Restore() {
            if (on) (void)hipSetDevice(d);
        }
    } restore{cur, cur != dev};
    BlasHandles& b = blas();
    std::lock_guard<std::mutex> lock(b.mu);
    auto it = b.by_device.find(dev);
    if (it == b.by_device.end()) {
        rocblas_handle h = nullptr;
        const rocblas_status st = rocblas_create_handle(&h);
        if (st != rocblas_status_success)
            return pa::set_error(PA_ERROR_HIP, f + ": rocblas_create_handle: " + blas_status(st));
        it = b.by_device.emplace(dev, h).first;
    }
    rocblas_handle h = it->second;
    rocblas_status st = rocblas_set_stream(h, s);
    if (st != rocblas_status_success) return pa::set_error(PA_ERROR_HIP, f + ": rocblas_set_stream: " + blas_status(st));
    const float alpha = 1.0f, beta = 0.0f;
    // Column-major view: y^T (o x n) = w (k x o, transposed) . a^T (k x n).
    st = (rocblas_gemm_ex)(h, rocblas_operation_transpose, rocblas_operation_none, o, n, k, &alpha, w,
                           rocblas_datatype_bf16_r, k, a, rocblas_datatype_bf16_r, k, &beta, y, rocblas_datatype_f32_r, o,
                           y, rocblas_datatype_f32_r, o, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
    if (st != rocblas_status_success) return pa::set_error(PA_ERROR_HIP, f + ": rocblas_gemm_ex: " + blas_status(st));
    return PA_SUCCESS;
}

// q_out[t][j] = y[t][j] for j < nq (the Q columns of the stacked GEMM output, row stride `stride`),
// in the activation dtype (bf16 by truncation); total = n_tok * nq elements.
__global__ __launch_bounds__(256) void q_from_rows_kernel(const float* __restrict__ y, int64_t stride, int32_t nq,
                                                         int64_t total, uint16_t* __restrict__ q_out) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t t = i / nq, j = i - t * nq;
        q_out[i] = pa::bf16_trunc(y[t * stride + j]);
    }
}

// a[i] = bf16(x[i]) by truncation.
__global__ __launch_bounds__(256) void to_bf16_kernel(const float* __restrict__ x, int64_t n, uint16_t* __restrict__ a) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256)
        a[i] = pa::bf16_trunc(x[i]);
}

int64_t qkv_cols(const pa_config* cfg) {
    return static_cast<int64_t>(cfg->num_q_heads + 2 * cfg->num_kv_heads) * cfg->head_dim;
}

pa_status check_proj(const std::string& f, const pa_config* cfg, int32_t hidden, int32_t n_tok) {
    pa_status st = pa::check_config(cfg, f.c_str());
    if (st != PA_SUCCESS) return st;
    if (cfg->q_dtype != PA_DTYPE_BF16)
        return pa::set_error(PA_ERROR_UNSUPPORTED, f + ": projections take bf16 activations (q_dtype BF16)");
    if (hidden <= 0 || n_tok < 0) return pa::set_error(PA_ERROR_INVALID_ARGUMENT, f + ": bad hidden / n_tok");
    return PA_SUCCESS;
}

// Workspace of the Q/K/V projection: the skinny path's split partials [splits][n][cols] (split 0 is
// then summed in place into y), or rocBLAS's y [n][cols].
size_t qkv_ws_bytes(const pa_config* cfg, int32_t n_tok) {
    const int64_t cols = qkv_cols(cfg);
    const int64_t slabs = n_tok <= kSkinnyMaxTok ? skinny_splits(cols) : 1;
    return static_cast<size_t>(slabs * n_tok * cols) * sizeof(float);
}

// Workspace of the output projection: room for the skinny path's partials of splits 1 ..
// ([splits - 1][n][hidden]; split 0 goes to y) and for the bf16 copy of the attention output that
// rocBLAS multiplies (the path the call takes depends on the operands' alignment too).
size_t o_ws_bytes(const pa_config* cfg, int32_t hidden, int32_t n_tok) {
    const size_t copy = static_cast<size_t>(n_tok) * cfg->num_q_heads * cfg->head_dim * sizeof(uint16_t);
    if (n_tok > kSkinnyMaxTok) return copy;
    const size_t part = static_cast<size_t>((skinny_splits(hidden) - 1) * static_cast<int64_t>(n_tok) * hidden) * sizeof(float);
    return part > copy ? part : copy;
}

}  // namespace

extern "C" {

pa_status pa_qkv_workspace_size(const pa_config* cfg, int32_t n_tok, size_t* bytes) {
    pa_status st = pa::check_config(cfg, "pa_qkv_workspace_size");
    if (st != PA_SUCCESS) return st;
    if (!bytes || n_tok < 0) return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_qkv_workspace_size: bad argument");
    *bytes = qkv_ws_bytes(cfg, n_tok);
    return pa::clear_error();
}

pa_status pa_qkv_project_append(pa_stream* stream, const pa_config* cfg, const void* x, const void* w_qkv,
                                int32_t hidden, int32_t n_tok, const int64_t* slot_mapping, void* q_out, void* k_cache,
                                void* v_cache, float* k_scale, float* v_scale, float* k_absmax, float* v_absmax,
                                void* workspace, size_t workspace_bytes) {
    const std::string f = "pa_qkv_project_append";
    pa_status st = check_proj(f, cfg, hidden, n_tok);
    if (st != PA_SUCCESS) return st;
    if (n_tok == 0) return pa::clear_error();
    if (!x || !w_qkv || !slot_mapping || !q_out || !k_cache || !v_cache || !workspace)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, f + ": null pointer");
    const int64_t cols = qkv_cols(cfg);
    if (workspace_bytes < qkv_ws_bytes(cfg, n_tok))
        return pa::set_error(PA_ERROR_WORKSPACE_TOO_SMALL, f + ": workspace smaller than pa_qkv_workspace_size");
    if (cols > INT32_MAX) return pa::set_error(PA_ERROR_UNSUPPORTED, f + ": too many heads");
    hipStream_t s = pa::native(stream);
    float* y = static_cast<float*>(workspace);
    const int32_t nq = cfg->num_q_heads * cfg->head_dim;
    const int64_t kv = static_cast<int64_t>(cfg->num_kv_heads) * cfg->head_dim;
    if (skinny_fits(n_tok, cols, hidden, x, w_qkv, y, q_out)) {
        const int splits = launch_skinny(s, x, false, static_cast<const uint16_t*>(w_qkv), y, y + n_tok * cols, n_tok,
                                         static_cast<int32_t>(cols), hidden);
        PA_HIP_CHECK(hipGetLastError());
        // fp32 / bf16 caches take the new K/V in the epilogue; int8 caches in their append kernel
        const int32_t cache = cfg->kv_dtype == PA_DTYPE_BF16 ? 2 : (cfg->kv_dtype == PA_DTYPE_FP32 ? 1 : 0);
        launch_epilogue(s, y, y + n_tok * cols, splits - 1, n_tok, static_cast<int32_t>(cols), nq,
                        static_cast<uint16_t*>(q_out), cache, slot_mapping, k_cache, v_cache, cfg->num_kv_heads,
                        cfg->head_dim, static_cast<int64_t>(cfg->num_blocks) * pa::kBlockSize);
        PA_HIP_CHECK(hipGetLastError());
        if (cache) return pa::clear_error();
    } else {
        st = gemm_bf16_nt(f, s, x, w_qkv, y, n_tok, static_cast<int32_t>(cols), hidden);
        if (st != PA_SUCCESS) return st;
        const int64_t total = static_cast<int64_t>(n_tok) * nq, qblocks = (total + 255) / 256;
        q_from_rows_kernel<<<static_cast<unsigned>(qblocks < 65536 ? qblocks : 65536), 256, 0, s>>>(
            y, cols, nq, total, static_cast<uint16_t*>(q_out));
        PA_HIP_CHECK(hipGetLastError());
    }
    return pa::launch_kv_append(f.c_str(), s, cfg, y + nq, y + nq + kv, false, cols, slot_mapping, n_tok, k_cache,
                                v_cache, k_scale, v_scale, k_absmax, v_absmax);
}

pa_status pa_o_workspace_size(const pa_config* cfg, int32_t hidden, int32_t n_tok, size_t* bytes) {
    pa_status st = pa::check_config(cfg, "pa_o_workspace_size");
    if (st != PA_SUCCESS) return st;
    if (!bytes || n_tok < 0 || hidden <= 0)
        return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_o_workspace_size: bad argument");
    *bytes = o_ws_bytes(cfg, hidden, n_tok);
    return pa::clear_error();
}

pa_status pa_o_project(pa_stream* stream, const pa_config* cfg, const float* attn, const void* w_o, int32_t hidden,
                       int32_t n_tok, float* y, void* workspace, size_t workspace_bytes) {
    const std::string f = "pa_o_project";
    pa_status st = check_proj(f, cfg, hidden, n_tok);
    if (st != PA_SUCCESS) return st;
    if (n_tok == 0) return pa::clear_error();
    if (!attn || !w_o || !y || !workspace) return pa::set_error(PA_ERROR_INVALID_ARGUMENT, f + ": null pointer");
    if (workspace_bytes < o_ws_bytes(cfg, hidden, n_tok))
        return pa::set_error(PA_ERROR_WORKSPACE_TOO_SMALL, f + ": workspace smaller than pa_o_workspace_size");
    const int64_t in = static_cast<int64_t>(cfg->num_q_heads) * cfg->head_dim;
    if (in > INT32_MAX) return pa::set_error(PA_ERROR_UNSUPPORTED, f + ": too many heads");
    hipStream_t s = pa::native(stream);
    float* rest = static_cast<float*>(workspace);
    if (skinny_fits(n_tok, hidden, static_cast<int32_t>(in), attn, w_o, y, rest)) {
        const int splits = launch_skinny(s, attn, true, static_cast<const uint16_t*>(w_o), y, rest, n_tok, hidden,
                                         static_cast<int32_t>(in));
        PA_HIP_CHECK(hipGetLastError());
        if (splits > 1) {
            launch_epilogue(s, y, rest, splits - 1, n_tok, hidden, 0, nullptr, 0, nullptr, nullptr, nullptr, 0, 0, 0);
            PA_HIP_CHECK(hipGetLastError());
        }
        return pa::clear_error();
    }
    const int64_t n = static_cast<int64_t>(n_tok) * in;
    uint16_t* a = static_cast<uint16_t*>(workspace);
    const int64_t blocks = (n + 255) / 256;
    to_bf16_kernel<<<static_cast<unsigned>(blocks < 65536 ? blocks : 65536), 256, 0, s>>>(attn, n, a);
    PA_HIP_CHECK(hipGetLastError());
    st = gemm_bf16_nt(f, s, a, w_o, y, n_tok, hidden, static_cast<int32_t>(in));
    if (st != PA_SUCCESS) return st;
    return pa::clear_error();
}

}  // extern "C"
