// hip_paged_attention.cpp -- C++ host side above the C-ABI (see hip_paged_attention.h).
#include "hip_paged_attention.h"

#include <cmath>
#include <cstring>

namespace pa_host {

void check(pa_status st, const char* call) {
    if (st == PA_SUCCESS) return;
    char buf[1024] = {0};
    pa_get_last_error(buf, sizeof(buf));
    std::string msg = std::string(call) + ": " + pa_status_string(st) + (buf[0] ? std::string(" (") + buf + ")" : "");
    switch (st) {
        case PA_ERROR_INVALID_ARGUMENT: throw std::invalid_argument(msg);
        case PA_ERROR_INVALID_CONFIG:
        case PA_ERROR_UNSUPPORTED: throw NotSupported(st, msg);
        default: throw PagedAttentionError(st, msg);
    }
}

std::vector<int32_t> FlattenBlockTables(const std::vector<std::vector<int>>& sequence_blocks,
                                        int32_t* max_blocks_per_seq) {
    size_t mb = 0;
    for (const auto& s : sequence_blocks) mb = s.size() > mb ? s.size() : mb;
    std::vector<int32_t> flat(sequence_blocks.size() * mb, -1);
    for (size_t i = 0; i < sequence_blocks.size(); i++)
        for (size_t j = 0; j < sequence_blocks[i].size(); j++) flat[i * mb + j] = sequence_blocks[i][j];
    if (max_blocks_per_seq) *max_blocks_per_seq = static_cast<int32_t>(mb);
    return flat;
}

HipPagedAttentionKernel::HipPagedAttentionKernel(int headDim, int ordinal)
    : default_scale_(1.0f / std::sqrt(static_cast<float>(headDim))) {
    if (headDim <= 0) throw std::invalid_argument("HipPagedAttentionKernel: headDim must be positive");
    check(pa_device_open(ordinal, &device_), "pa_device_open");
    pa_status st = pa_stream_create(device_, &stream_);
    if (st != PA_SUCCESS) {
        pa_device_close(device_);
        device_ = nullptr;
        check(st, "pa_stream_create");
    }
}

HipPagedAttentionKernel::~HipPagedAttentionKernel() {
    if (workspace_) pa_free(device_, workspace_);
    if (stream_) pa_stream_destroy(stream_);
    if (device_) pa_device_close(device_);
}

void* HipPagedAttentionKernel::ensure_workspace(size_t bytes) {
    if (bytes <= workspace_bytes_) return workspace_;
    if (workspace_) check(pa_free(device_, workspace_), "pa_free");
    workspace_ = nullptr;
    workspace_bytes_ = 0;
    check(pa_alloc(device_, bytes, &workspace_), "pa_alloc");
    workspace_bytes_ = bytes;
    return workspace_;
}

namespace {

// Device allocation released on scope exit.
struct DeviceBuffer {
    pa_device* dev;
    void* ptr = nullptr;
    DeviceBuffer(pa_device* d, size_t bytes) : dev(d) { check(pa_alloc(d, bytes ? bytes : 4, &ptr), "pa_alloc"); }
    ~DeviceBuffer() {
        if (ptr) pa_free(dev, ptr);
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
};

void require_4d(const Tensor& t, const char* name) {
    if (t.shape.size() != 4) throw std::invalid_argument(std::string(name) + " must be 4-dimensional");
    size_t n = 1;
    for (int s : t.shape) {
        if (s < 0) throw std::invalid_argument(std::string(name) + " has a negative dimension");
        n *= static_cast<size_t>(s);
    }
    if (n != t.data.size()) throw std::invalid_argument(std::string(name) + ": data size does not match the shape");
}

}  // namespace

Tensor HipPagedAttentionKernel::ComputePagedAttention(const Tensor& query, const Tensor& cachedKeys,
                                                      const Tensor& cachedValues, AttentionPhase phase, float scale) {
    require_4d(query, "query");
    require_4d(cachedKeys, "cachedKeys");
    require_4d(cachedValues, "cachedValues");
    const int B = query.shape[0], Q = query.shape[1], H = query.shape[2], D = query.shape[3];
    const int C = cachedKeys.shape[1];
    if (cachedKeys.shape != cachedValues.shape || cachedKeys.shape[0] != B || cachedKeys.shape[2] != H ||
        cachedKeys.shape[3] != D)
        throw std::invalid_argument("ComputePagedAttention: cachedKeys/cachedValues must be [batch, numCached, "
                                    "numHeads, headDim] matching the query");
    Tensor out(std::vector<float>(query.data.size(), 0.0f), query.shape);
    if (B == 0 || Q == 0 || H == 0) return out;

    // Identity-paged fp32 cache: K tile [16][D], V tile [D][16] per (block, head).
    const int nbb = (C + 15) / 16;
    const int nb = B * nbb;
    const size_t tile = static_cast<size_t>(16) * D;
    std::vector<float> kc(static_cast<size_t>(nb) * H * tile, 0.0f), vc(kc.size(), 0.0f);
    for (int b = 0; b < B; b++)
        for (int t = 0; t < C; t++)
            for (int h = 0; h < H; h++) {
                const size_t src = ((static_cast<size_t>(b) * C + t) * H + h) * D;
                const size_t blk = static_cast<size_t>(b) * nbb + t / 16, r = t % 16;
                float* kt = kc.data() + (blk * H + h) * tile;
                float* vt = vc.data() + (blk * H + h) * tile;
                for (int d = 0; d < D; d++) {
                    kt[r * D + d] = cachedKeys.data[src + d];
                    vt[static_cast<size_t>(d) * 16 + r] = cachedValues.data[src + d];
                }
            }
    pa_config cfg{};
    cfg.block_size = 16;
    cfg.num_q_heads = H;
    cfg.num_kv_heads = H;
    cfg.head_dim = D;
    cfg.kv_dtype = PA_DTYPE_FP32;
    cfg.q_dtype = PA_DTYPE_FP32;
    cfg.num_blocks = nb;
    cfg.scale = scale > 0 ? scale : default_scale_;
    cfg.partition_size = 0;
    const int mbps = nbb > 0 ? nbb : 1;
    DeviceBuffer dq(device_, query.data.size() * 4), dk(device_, kc.size() * 4), dv(device_, vc.size() * 4),
        dout(device_, out.data.size() * 4);
    check(pa_memcpy(dq.ptr, query.data.data(), query.data.size() * 4, PA_MEMCPY_HOST_TO_DEVICE, stream_), "pa_memcpy");
    check(pa_memcpy(dk.ptr, kc.data(), kc.size() * 4, PA_MEMCPY_HOST_TO_DEVICE, stream_), "pa_memcpy");
    check(pa_memcpy(dv.ptr, vc.data(), vc.size() * 4, PA_MEMCPY_HOST_TO_DEVICE, stream_), "pa_memcpy");

    if (Q > 1 && C >= Q) {
        // Several queries over at least as many keys: one chunked-prefill launch in which the queries
        // of a batch entry are its chunk, at positions C - Q .. C - 1. The reference masks only in the
        // Decode phase and only when C > Q (StandardPagedAttentionKernel.cs:57-66): the literal mask
        // rule, or no mask at all in the Prefill phase.
        cfg.flags = phase == AttentionPhase::Decode ? PA_FLAG_REFERENCE_LITERAL_MASK : PA_FLAG_NO_MASK;
        std::vector<int32_t> q_start(B + 1), prefix(B, C - Q), tables(static_cast<size_t>(B) * nbb);
        for (int b = 0; b <= B; b++) q_start[b] = b * Q;
        for (int b = 0; b < B; b++)
            for (int j = 0; j < nbb; j++) tables[static_cast<size_t>(b) * nbb + j] = b * nbb + j;
        DeviceBuffer dqs(device_, q_start.size() * 4), dp(device_, prefix.size() * 4), dt(device_, tables.size() * 4);
        check(pa_memcpy(dqs.ptr, q_start.data(), q_start.size() * 4, PA_MEMCPY_HOST_TO_DEVICE, stream_), "pa_memcpy");
        check(pa_memcpy(dp.ptr, prefix.data(), prefix.size() * 4, PA_MEMCPY_HOST_TO_DEVICE, stream_), "pa_memcpy");
        check(pa_memcpy(dt.ptr, tables.data(), tables.size() * 4, PA_MEMCPY_HOST_TO_DEVICE, stream_), "pa_memcpy");
        check(pa_chunked_prefill(stream_, &cfg, static_cast<float*>(dout.ptr), dq.ptr,
                                 static_cast<const int32_t*>(dqs.ptr), static_cast<const int32_t*>(dp.ptr), dk.ptr,
                                 dv.ptr, nullptr, nullptr, static_cast<const int32_t*>(dt.ptr), B, mbps, Q),
              "pa_chunked_prefill");
        check(pa_memcpy(out.data.data(), dout.ptr, out.data.size() * 4, PA_MEMCPY_DEVICE_TO_HOST, stream_), "pa_memcpy");
        check(pa_stream_synchronize(stream_), "pa_stream_synchronize");
        return out;
    }

    // One query, or more queries than keys: one decode sequence per (batch, query), the reference's
    // mask becoming its context length.
    const int S = B * Q;
    const bool masked = phase == AttentionPhase::Decode && C > Q;
    std::vector<int32_t> lens(S), tables(static_cast<size_t>(S) * mbps, -1);
    for (int b = 0; b < B; b++)
        for (int i = 0; i < Q; i++) {
            const int s = b * Q + i;
            lens[s] = masked ? C - Q + i + 1 : C;
            for (int j = 0; j < nbb; j++) tables[static_cast<size_t>(s) * mbps + j] = b * nbb + j;
        }
    cfg.flags = 0;
    size_t wsb = 0;
    check(pa_decode_workspace_size(&cfg, S, C, &wsb), "pa_decode_workspace_size");
    DeviceBuffer dt(device_, tables.size() * 4), dl(device_, lens.size() * 4);
    void* ws = wsb ? ensure_workspace(wsb) : nullptr;
    check(pa_memcpy(dt.ptr, tables.data(), tables.size() * 4, PA_MEMCPY_HOST_TO_DEVICE, stream_), "pa_memcpy");
    check(pa_memcpy(dl.ptr, lens.data(), lens.size() * 4, PA_MEMCPY_HOST_TO_DEVICE, stream_), "pa_memcpy");
    check(pa_paged_decode(stream_, &cfg, static_cast<float*>(dout.ptr), dq.ptr, dk.ptr, dv.ptr, nullptr, nullptr,
                          static_cast<const int32_t*>(dt.ptr), static_cast<const int32_t*>(dl.ptr), S, mbps, C, ws, wsb),
          "pa_paged_decode");
    check(pa_memcpy(out.data.data(), dout.ptr, out.data.size() * 4, PA_MEMCPY_DEVICE_TO_HOST, stream_), "pa_memcpy");
    check(pa_stream_synchronize(stream_), "pa_stream_synchronize");
    return out;
}

void HipPagedAttentionKernel::ComputePagedAttention(const pa_config& config, const PagedDecodeBatch& batch, float* out,
                                                    pa_stream* stream) {
    size_t wsb = 0;
    check(pa_decode_workspace_size(&config, batch.num_seqs, batch.max_context_len, &wsb), "pa_decode_workspace_size");
    void* ws = wsb ? ensure_workspace(wsb) : nullptr;
    check(pa_paged_decode(stream ? stream : stream_, &config, out, batch.query, batch.k_cache, batch.v_cache,
                          batch.k_scale, batch.v_scale, batch.block_tables, batch.context_lens, batch.num_seqs,
                          batch.max_blocks_per_seq, batch.max_context_len, ws, wsb),
          "pa_paged_decode");
}

}  // namespace pa_host
