// hip_paged_attention.h -- C++ host side of the MI355X paged-attention backend, above the C-ABI.
//
// Mirrors the reference's operator interface for this path, IPagedAttentionKernel
// (src/MLFramework/Inference/PagedAttention/Kernels/IPagedAttentionKernel.cs:11-34): the same
// method names, argument meanings and defaults, so a host written against that interface finds the
// same calls here. Errors are C++ exceptions mapped from the library's status codes the way the
// reference maps CudaError to exceptions (HAL/CUDA/CudaDevice.cs:15-21):
//   PA_ERROR_INVALID_ARGUMENT              -> std::invalid_argument   (ArgumentException)
//   PA_ERROR_INVALID_CONFIG / UNSUPPORTED  -> pa_host::NotSupported   (NotImplementedException)
//   anything else                          -> pa_host::PagedAttentionError (InvalidOperationException)
// Every computation runs on the GPU through libpa_hip.so; there is no CPU fallback.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "paged_attn.h"

namespace pa_host {

// Phases/AttentionPhase.cs:6-17
enum class AttentionPhase { Prefill = 0, Decode = 1 };

// HAL/DeviceType.cs
enum class DeviceType { CPU, CUDA, ROCm, Metal };

// MLFramework.Core.Device (Core/Device.cs): type and ordinal.
struct Device {
    DeviceType type = DeviceType::CPU;
    int index = 0;
};

// Dense fp32 host tensor, row-major: the reference Tensor's Data and Shape
// (RitterFramework.Core/Tensor.cs:40-45).
struct Tensor {
    std::vector<float> data;
    std::vector<int> shape;
    Tensor() = default;
    Tensor(std::vector<float> d, std::vector<int> s) : data(std::move(d)), shape(std::move(s)) {}
};

class PagedAttentionError : public std::runtime_error {
public:
    PagedAttentionError(pa_status status, const std::string& what) : std::runtime_error(what), status_(status) {}
    pa_status status() const { return status_; }

private:
    pa_status status_;
};

class NotSupported : public std::logic_error {
public:
    NotSupported(pa_status status, const std::string& what) : std::logic_error(what), status_(status) {}
    pa_status status() const { return status_; }

private:
    pa_status status_;
};

// Throws the exception that corresponds to a non-success status (with the library's last error).
void check(pa_status st, const char* call);

// IPagedAttentionKernel.cs:11-34
class IPagedAttentionKernel {
public:
    virtual ~IPagedAttentionKernel() = default;
    // query [batch, numQueries, numHeads, headDim]; cachedKeys/cachedValues [batch, numCached,
    // numHeads, headDim]; returns [batch, numQueries, numHeads, headDim]. scale <= 0 selects the
    // kernel's default 1/sqrt(headDim).
    virtual Tensor ComputePagedAttention(const Tensor& query, const Tensor& cachedKeys, const Tensor& cachedValues,
                                         AttentionPhase phase, float scale = -1.0f) = 0;
    virtual bool SupportsDevice(const Device& device) const = 0;
};

// Flattens per-sequence physical block lists (BlockTable.GetSequenceBlocks, BlockTable.cs:50-58)
// into the int32 [num_seqs][max_blocks_per_seq] table the kernels take, padded with -1.
std::vector<int32_t> FlattenBlockTables(const std::vector<std::vector<int>>& sequence_blocks,
                                        int32_t* max_blocks_per_seq);

// Device buffers of one ragged decode batch over a paged cache (all device pointers).
struct PagedDecodeBatch {
    const void* query = nullptr;          // [num_seqs][Hq][D] of config.q_dtype
    const void* k_cache = nullptr;        // [num_blocks][Hkv][16][D]
    const void* v_cache = nullptr;        // [num_blocks][Hkv][D][16]
    const float* k_scale = nullptr;       // int8 caches: [num_blocks][Hkv]
    const float* v_scale = nullptr;
    const int32_t* block_tables = nullptr;  // [num_seqs][max_blocks_per_seq]
    const int32_t* context_lens = nullptr;  // [num_seqs]
    int32_t num_seqs = 0;
    int32_t max_blocks_per_seq = 0;
    int32_t max_context_len = 0;
};

// The HIP kernel behind IPagedAttentionKernel, plus the paged overload the backend exists for.
class HipPagedAttentionKernel : public IPagedAttentionKernel {
public:
    // headDim sets the default scale 1/sqrtf(headDim) (StandardPagedAttentionKernel.cs:16-19);
    // opens GPU `ordinal` (throws PagedAttentionError with PA_ERROR_NO_DEVICE without one).
    explicit HipPagedAttentionKernel(int headDim, int ordinal = 0);
    ~HipPagedAttentionKernel() override;
    HipPagedAttentionKernel(const HipPagedAttentionKernel&) = delete;
    HipPagedAttentionKernel& operator=(const HipPagedAttentionKernel&) = delete;

    // Dense interface: the caller's K/V become an identity-paged fp32 cache (batch element b owns
    // blocks [b * nb, (b + 1) * nb)) and every (batch, query) row is one ragged decode sequence whose
    // context length implements the reference's mask: phase Decode with numCached > numQueries
    // masks query i to keys 0 .. numCached - numQueries + i (StandardPagedAttentionKernel.cs:57-66,
    // 219-255); otherwise every query sees all keys. Synchronous, returns a new tensor.
    Tensor ComputePagedAttention(const Tensor& query, const Tensor& cachedKeys, const Tensor& cachedValues,
                                 AttentionPhase phase, float scale = -1.0f) override;

    // DeviceType.ROCm only (the reference's CUDA kernel answers DeviceType.CUDA,
    // CudaPagedAttentionKernel.cs:39-42).
    bool SupportsDevice(const Device& device) const override { return device.type == DeviceType::ROCm; }

    // Paged overload: ragged decode over a paged cache already in device memory, asynchronous on
    // `stream` (nullptr: the library's default stream). `out` is device memory [num_seqs][Hq][D]
    // fp32. The workspace is kept by the object and grown on demand (allocation happens only
    // when a larger shape arrives).
    void ComputePagedAttention(const pa_config& config, const PagedDecodeBatch& batch, float* out,
                               pa_stream* stream = nullptr);

    pa_device* device() const { return device_; }
    float default_scale() const { return default_scale_; }

private:
    void* ensure_workspace(size_t bytes);

    pa_device* device_ = nullptr;
    pa_stream* stream_ = nullptr;
    float default_scale_;
    void* workspace_ = nullptr;
    size_t workspace_bytes_ = 0;
};

}  // namespace pa_host
