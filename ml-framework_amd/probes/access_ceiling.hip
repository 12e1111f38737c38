// Measures the HBM ceiling of the C2 decode step's access pattern, without attention math.
//
// A C2 step reads every block of the batch's tables once: per block, one contiguous 32 KiB run of
// K (8 KV heads x 16 tokens x 128 dims, bf16) and one of V, the blocks in a random order over a
// pool of 1.1x the blocks needed. Two pools alternate, so no step finds its blocks in the 256 MiB
// last-level cache. Patterns:
//   runs   one workgroup reads a block's whole K run and V run (1 or 2 blocks at a time);
//   tiles  the decode's own split: wave w of unit (range, KV head) reads its 4 KiB K tile and 4 KiB
//          V tile of every block of its range, in batches of 1, 2 or 3 blocks, or as a rolling
//          pipeline of NB register buffers (NB - 1 blocks in flight while one is read);
//   seq    a sequential read of the same byte count (calibration).
// V is read non-temporal and K with default caching, as the decode does. Each pattern: 20 warm-up
// steps, then 200 timed with hipEvents. Usage: access_ceiling [blocks] (default 4420, C2's).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#define CHECK(x)                                                                     \
    do {                                                                             \
        hipError_t e_ = (x);                                                         \
        if (e_ != hipSuccess) {                                                      \
            std::fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
            std::exit(1);                                                            \
        }                                                                            \
    } while (0)

namespace {

constexpr int kRun = 32768;  // bytes per block per cache
constexpr int kTile = 4096;  // bytes per block per cache and KV head
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4 load_nt(const u32x4* p) { return __builtin_nontemporal_load(p); }

template <int PER>
__global__ __launch_bounds__(256) void runs_kernel(const char* kc, const char* vc, const int* order, int nblk,
                                                   unsigned* sink) {
    const int t = threadIdx.x;
    unsigned acc = 0;
    for (int i = blockIdx.x * PER; i < nblk; i += gridDim.x * PER) {
        u32x4 x[PER][16];
#pragma unroll
        for (int k = 0; k < PER; k++) {
            const int b = i + k < nblk ? order[i + k] : order[0];
            const u32x4* pk = reinterpret_cast<const u32x4*>(kc + static_cast<size_t>(b) * kRun);
            const u32x4* pv = reinterpret_cast<const u32x4*>(vc + static_cast<size_t>(b) * kRun);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                x[k][j] = pk[j * 256 + t];
                x[k][8 + j] = load_nt(pv + j * 256 + t);
            }
        }
#pragma unroll
        for (int k = 0; k < PER; k++)
#pragma unroll
            for (int j = 0; j < 16; j++) acc ^= x[k][j][0] ^ x[k][j][3];
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;  // keeps the loads; practically never taken
}

// One block's 4 KiB K tile and 4 KiB V tile of KV head h into d (4 + 4 loads of 16 B per lane).
__device__ __forceinline__ void load_tiles(u32x4 (&d)[8], const char* kc, const char* vc, int b, int h, int lane) {
    const u32x4* pk = reinterpret_cast<const u32x4*>(kc + static_cast<size_t>(b) * kRun + h * kTile);
    const u32x4* pv = reinterpret_cast<const u32x4*>(vc + static_cast<size_t>(b) * kRun + h * kTile);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        d[j] = pk[j * 64 + lane];
        d[4 + j] = load_nt(pv + j * 64 + lane);
    }
}

template <int BATCH>
__global__ __launch_bounds__(256, 2) void tiles_batch_kernel(const char* kc, const char* vc, const int* order, int nblk,
                                                             int range, int units, unsigned* sink) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    unsigned acc = 0;
    for (int u = blockIdx.x * 4 + wave; u < units; u += gridDim.x * 4) {
        const int b0 = (u >> 3) * range, b1 = min(nblk, b0 + range), h = u & 7;
        for (int b = b0; b < b1; b += BATCH) {
            u32x4 x[BATCH][8];
#pragma unroll
            for (int k = 0; k < BATCH; k++) load_tiles(x[k], kc, vc, b + k < b1 ? order[b + k] : order[b0], h, lane);
#pragma unroll
            for (int k = 0; k < BATCH; k++)
#pragma unroll
                for (int j = 0; j < 8; j++) acc ^= x[k][j][0] ^ x[k][j][3];
        }
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;
}

template <int NB>
__global__ __launch_bounds__(256, 2) void tiles_rolling_kernel(const char* kc, const char* vc, const int* order,
                                                               int nblk, int range, int units, unsigned* sink) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    unsigned acc = 0;
    for (int u = blockIdx.x * 4 + wave; u < units; u += gridDim.x * 4) {
        const int b0 = (u >> 3) * range, n = min(nblk, b0 + range) - b0, h = u & 7;
        u32x4 x[NB][8];
        // item i: block b0 + i of the range, or (past its end) block b0 again, never read
        auto item = [&](int i) { return order[b0 + (i < n ? i : 0)]; };
#pragma unroll
        for (int k = 0; k < NB - 1; k++) load_tiles(x[k], kc, vc, item(k), h, lane);
        for (int i = 0; i < n; i += NB) {
#pragma unroll
            for (int k = 0; k < NB; k++) {
                load_tiles(x[(k + NB - 1) % NB], kc, vc, item(i + k + NB - 1), h, lane);
#pragma unroll
                for (int j = 0; j < 8; j++) acc ^= x[k][j][0] ^ x[k][j][3];
            }
        }
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;
}

__global__ __launch_bounds__(256) void seq_kernel(const u32x4* p, const u32x4* q, size_t n16, unsigned* sink) {
    unsigned acc = 0;  // n16 / 2 16-byte words from each of p and q
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n16 / 2;
         i += static_cast<size_t>(gridDim.x) * 256) {
        const u32x4 x = load_nt(p + i), y = load_nt(q + i);
        acc ^= x[0] ^ y[3];
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;
}

}  // namespace

int main(int argc, char** argv) {
    const int nblk = argc > 1 ? std::atoi(argv[1]) : 4420;
    if (nblk < 1 || nblk > 1 << 20) {
        std::fprintf(stderr, "blocks must be in [1, 2^20]\n");
        return 2;
    }
    const int pool = static_cast<int>(std::ceil(nblk * 1.1));
    std::mt19937 rng(7);
    std::vector<int> perm(pool);
    for (int i = 0; i < pool; i++) perm[i] = i;
    std::shuffle(perm.begin(), perm.end(), rng);
    const std::vector<int> order(perm.begin(), perm.begin() + nblk);
    char *kc[2], *vc[2];
    int* d_order;
    unsigned* sink;
    for (int p = 0; p < 2; p++) {
        CHECK(hipMalloc(&kc[p], static_cast<size_t>(pool) * kRun));
        CHECK(hipMalloc(&vc[p], static_cast<size_t>(pool) * kRun));
        CHECK(hipMemset(kc[p], 1, static_cast<size_t>(pool) * kRun));
        CHECK(hipMemset(vc[p], 2, static_cast<size_t>(pool) * kRun));
    }
    CHECK(hipMalloc(&d_order, nblk * sizeof(int)));
    CHECK(hipMalloc(&sink, sizeof(unsigned)));
    CHECK(hipMemcpy(d_order, order.data(), nblk * sizeof(int), hipMemcpyHostToDevice));
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    const double bytes = 2.0 * nblk * kRun;
    auto time_it = [&](const char* name, auto launch) {
        for (int i = 0; i < 20; i++) launch(i & 1);
        CHECK(hipDeviceSynchronize());
        constexpr int kSteps = 200;
        CHECK(hipEventRecord(e0));
        for (int i = 0; i < kSteps; i++) launch(i & 1);
        CHECK(hipEventRecord(e1));
        CHECK(hipEventSynchronize(e1));
        float ms = 0.0f;
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        const double us = ms * 1e3 / kSteps;
        std::printf("%-58s %8.2f us %8.1f GB/s  %.3f of 8 TB/s\n", name, us, bytes / (us * 1e-6) / 1e9,
                    bytes / (us * 1e-6) / 8e12);
        std::fflush(stdout);
    };
    std::printf("blocks %d, pool %d, bytes per step %.1f MB\n", nblk, pool, bytes / 1e6);
    char name[96];
    for (int grid : {512, 2048}) {
        std::snprintf(name, sizeof name, "runs: 1 block per workgroup at a time, grid %d", grid);
        time_it(name, [&](int p) { runs_kernel<1><<<grid, 256>>>(kc[p], vc[p], d_order, nblk, sink); });
        std::snprintf(name, sizeof name, "runs: 2 blocks per workgroup at a time, grid %d", grid);
        time_it(name, [&](int p) { runs_kernel<2><<<grid, 256>>>(kc[p], vc[p], d_order, nblk, sink); });
    }
    constexpr int kGrid = 512;  // 2048 waves, as the decode launches on 256 CUs
    const int ranges = kGrid * 4 / 8, range = (nblk + ranges - 1) / ranges, units = ((nblk + range - 1) / range) * 8;
    auto tiles = [&](const char* what, auto kernel) {
        std::snprintf(name, sizeof name, "tiles: %s, %d waves, ranges of %d blocks", what, kGrid * 4, range);
        time_it(name, [&](int p) { kernel<<<kGrid, 256>>>(kc[p], vc[p], d_order, nblk, range, units, sink); });
    };
    tiles("batches of 3 blocks", tiles_batch_kernel<3>);
    tiles("batches of 2 blocks", tiles_batch_kernel<2>);
    tiles("one block at a time", tiles_batch_kernel<1>);
    tiles("rolling, 1 block in flight", tiles_rolling_kernel<2>);
    tiles("rolling, 2 blocks in flight", tiles_rolling_kernel<3>);
    tiles("rolling, 3 blocks in flight", tiles_rolling_kernel<4>);
    for (int grid : {1024, 4096}) {
        std::snprintf(name, sizeof name, "seq: sequential read, grid %d", grid);
        time_it(name, [&](int p) {
            seq_kernel<<<grid, 256>>>(reinterpret_cast<const u32x4*>(kc[p]), reinterpret_cast<const u32x4*>(vc[p]),
                                      static_cast<size_t>(bytes) / 16, sink);
        });
    }
    for (int p = 0; p < 2; p++) {
        CHECK(hipFree(kc[p]));
        CHECK(hipFree(vc[p]));
    }
    CHECK(hipFree(d_order));
    CHECK(hipFree(sink));
    return 0;
}
