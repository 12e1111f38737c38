// decode_mfma_launch.h -- the launcher of the MFMA paged-decode kernel, templated on head_dim.
// Each decode_mfma_d<D>.hip instantiates it for one head_dim, so the kernel instances of the
// head_dims compile in parallel.
#pragma once

#include "decode_mfma.h"

namespace pa {

namespace {

template <int D, int KV, bool QF32, bool APPEND, bool SHARED>
void launch_one(DecodeArgs& a, int num_seqs, int64_t max_grid, hipStream_t s) {
    auto kern = paged_decode_mfma_persistent_kernel<D, KV, QF32, APPEND, SHARED>;
    // Resident workgroups per CU for this instance (queried once; read-only afterwards).
    constexpr int waves = decode_waves(D);
    static const int per_cu = [&] {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, 64 * waves, 0) != hipSuccess || n < 1) n = 1;
        return n;
    }();
    int64_t workers = static_cast<int64_t>(device_cus()) * per_cu * waves;
    if (workers > kMaxDecodeWorkers) workers = kMaxDecodeWorkers;
    if (workers >= a.num_kv_heads) workers -= workers % a.num_kv_heads;  // whole ranges (one unit per KV head)
    if (workers > max_grid) workers = max_grid;
    if (workers < 1) workers = 1;
    a.split_grid = static_cast<int32_t>(workers);
    const int64_t nwg = (workers + waves - 1) / waves;
    kern<<<static_cast<unsigned>(nwg), 64 * waves, 0, s>>>(a, num_seqs);
}

template <int D, int KV, bool QF32>
void pick(DecodeArgs& a, bool append, bool shared, int num_seqs, int64_t max_grid, hipStream_t s) {
    if (shared) launch_one<D, KV, QF32, false, true>(a, num_seqs, max_grid, s);
    else if (append) launch_one<D, KV, QF32, true, false>(a, num_seqs, max_grid, s);
    else launch_one<D, KV, QF32, false, false>(a, num_seqs, max_grid, s);
}

}  // namespace

template <int D>
void launch_decode_mfma(DecodeArgs& a, int kv_dtype, bool q_f32, bool append, bool shared, int num_seqs,
                        int64_t max_grid, hipStream_t s) {
    if (kv_dtype == PA_DTYPE_BF16) {
        if (q_f32) pick<D, PA_DTYPE_BF16, true>(a, append, shared, num_seqs, max_grid, s);
        else pick<D, PA_DTYPE_BF16, false>(a, append, shared, num_seqs, max_grid, s);
    } else if constexpr (D < 64) {
        // int8 caches need head_dim >= 64 (refused on the host): no instances.
    } else if (shared) {
        if (q_f32) launch_one<D, PA_DTYPE_INT8, true, false, true>(a, num_seqs, max_grid, s);
        else launch_one<D, PA_DTYPE_INT8, false, false, true>(a, num_seqs, max_grid, s);
    } else {  // int8 caches are appended by a separate launch before the decode
        if (q_f32) launch_one<D, PA_DTYPE_INT8, true, false, false>(a, num_seqs, max_grid, s);
        else launch_one<D, PA_DTYPE_INT8, false, false, false>(a, num_seqs, max_grid, s);
    }
}

}  // namespace pa
