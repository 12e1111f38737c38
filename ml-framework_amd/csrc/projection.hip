// projection.hip -- the Q/K/V and output projections either side of paged attention, gfx950.
//
// The reference layer projects the hidden states with three bias-free Linear layers, stores the
// new K/V in the cache and projects the attention output with a fourth
// (PagedAttentionLayer.ComputeAttention, src/MLFramework/Inference/PagedAttention/Layers/
// PagedAttentionLayer.cs:112-142; Linear.Forward y = x W^T, src/MLFramework/Modules/Linear.cs:
// 81-110). Here the three input projections are one GEMM against the stacked weight
// [(Hq + 2 Hkv) * D][hidden] (bf16 operands, fp32 accumulation, rocBLAS: a plain library GEMM),
// followed by an epilogue that writes Q in the activation dtype and appends K/V into the paged
// cache exactly as pa_kv_append does with fp32 input (the GEMM rows are read in place with a token
// stride). The output projection truncates the fp32 attention output to bf16 and multiplies by
// W_o^T. Decode-sized GEMMs are weight-bound (HBM).
#include <mutex>
#include <string>
#include <unordered_map>

#include <rocblas/rocblas.h>

#include "pa_internal.h"

namespace {

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

}  // namespace

extern "C" {

pa_status pa_qkv_workspace_size(const pa_config* cfg, int32_t n_tok, size_t* bytes) {
    pa_status st = pa::check_config(cfg, "pa_qkv_workspace_size");
    if (st != PA_SUCCESS) return st;
    if (!bytes || n_tok < 0) return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_qkv_workspace_size: bad argument");
    *bytes = static_cast<size_t>(n_tok) * qkv_cols(cfg) * sizeof(float);
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
    if (workspace_bytes < static_cast<size_t>(n_tok) * cols * sizeof(float))
        return pa::set_error(PA_ERROR_WORKSPACE_TOO_SMALL, f + ": workspace smaller than pa_qkv_workspace_size");
    if (cols > INT32_MAX) return pa::set_error(PA_ERROR_UNSUPPORTED, f + ": too many heads");
    hipStream_t s = pa::native(stream);
    float* y = static_cast<float*>(workspace);
    st = gemm_bf16_nt(f, s, x, w_qkv, y, n_tok, static_cast<int32_t>(cols), hidden);
    if (st != PA_SUCCESS) return st;
    const int32_t nq = cfg->num_q_heads * cfg->head_dim;
    const int64_t total = static_cast<int64_t>(n_tok) * nq, qblocks = (total + 255) / 256;
    q_from_rows_kernel<<<static_cast<unsigned>(qblocks < 65536 ? qblocks : 65536), 256, 0, s>>>(
        y, cols, nq, total, static_cast<uint16_t*>(q_out));
    PA_HIP_CHECK(hipGetLastError());
    const int64_t kv = static_cast<int64_t>(cfg->num_kv_heads) * cfg->head_dim;
    return pa::launch_kv_append(f.c_str(), s, cfg, y + nq, y + nq + kv, false, cols, slot_mapping, n_tok, k_cache,
                                v_cache, k_scale, v_scale, k_absmax, v_absmax);
}

pa_status pa_o_workspace_size(const pa_config* cfg, int32_t n_tok, size_t* bytes) {
    pa_status st = pa::check_config(cfg, "pa_o_workspace_size");
    if (st != PA_SUCCESS) return st;
    if (!bytes || n_tok < 0) return pa::set_error(PA_ERROR_INVALID_ARGUMENT, "pa_o_workspace_size: bad argument");
    *bytes = static_cast<size_t>(n_tok) * cfg->num_q_heads * cfg->head_dim * sizeof(uint16_t);
    return pa::clear_error();
}

pa_status pa_o_project(pa_stream* stream, const pa_config* cfg, const float* attn, const void* w_o, int32_t hidden,
                       int32_t n_tok, float* y, void* workspace, size_t workspace_bytes) {
    const std::string f = "pa_o_project";
    pa_status st = check_proj(f, cfg, hidden, n_tok);
    if (st != PA_SUCCESS) return st;
    if (n_tok == 0) return pa::clear_error();
    if (!attn || !w_o || !y || !workspace) return pa::set_error(PA_ERROR_INVALID_ARGUMENT, f + ": null pointer");
    const int64_t in = static_cast<int64_t>(cfg->num_q_heads) * cfg->head_dim;
    const int64_t n = static_cast<int64_t>(n_tok) * in;
    if (workspace_bytes < static_cast<size_t>(n) * sizeof(uint16_t))
        return pa::set_error(PA_ERROR_WORKSPACE_TOO_SMALL, f + ": workspace smaller than pa_o_workspace_size");
    hipStream_t s = pa::native(stream);
    uint16_t* a = static_cast<uint16_t*>(workspace);
    const int64_t blocks = (n + 255) / 256;
    to_bf16_kernel<<<static_cast<unsigned>(blocks < 65536 ? blocks : 65536), 256, 0, s>>>(attn, n, a);
    PA_HIP_CHECK(hipGetLastError());
    st = gemm_bf16_nt(f, s, a, w_o, y, n_tok, hidden, static_cast<int32_t>(in));
    if (st != PA_SUCCESS) return st;
    return pa::clear_error();
}

}  // extern "C"
