// test_host_mirror.cpp -- tests of the C++ host side (ml-framework_amd/host), written like the
// reference's own PagedAttention tests (tests/MLFramework.Tests/Inference/PagedAttention/
// PagedAttentionFunctionalTests.cs): build inputs, call ComputePagedAttention, compare.
//
//   test_host_mirror --cpu   checks that need no GPU (error mapping, table flattening, no device)
//   test_host_mirror --gpu   the HIP kernel behind the interface against the CPU oracle
//
// The oracle (oracle/libpa_oracle.so) is the checker only. Exit status 0 = all passed.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <random>
#include <string>
#include <vector>

#include "hip_paged_attention.h"
#include "pa_oracle.h"

using namespace pa_host;

static int g_failed = 0, g_run = 0;

#define EXPECT(cond, ...)                                                  \
    do {                                                                   \
        if (!(cond)) {                                                     \
            std::printf("  FAIL %s:%d: %s -- ", __FILE__, __LINE__, #cond); \
            std::printf(__VA_ARGS__);                                      \
            std::printf("\n");                                             \
            throw std::runtime_error("expectation failed");               \
        }                                                                  \
    } while (0)

static void run(const char* name, const std::function<void()>& fn) {
    g_run++;
    std::printf("[ RUN  ] %s\n", name);
    std::fflush(stdout);
    try {
        fn();
        std::printf("[  OK  ] %s\n", name);
    } catch (const std::exception& e) {
        g_failed++;
        std::printf("[ FAIL ] %s: %s\n", name, e.what());
    }
    std::fflush(stdout);
}

template <typename E>
static bool throws_as(const std::function<void()>& fn) {
    try {
        fn();
    } catch (const E&) {
        return true;
    } catch (...) {
        return false;
    }
    return false;
}

static std::vector<float> randn(size_t n, uint64_t seed, float s = 1.0f) {
    std::mt19937_64 rng(seed);
    std::normal_distribution<float> nd(0.0f, 1.0f);
    std::vector<float> v(n);
    for (auto& x : v) x = nd(rng) * s;
    return v;
}

// |got - ref| <= 2e-3 + 1e-2 |ref| (the fp32/bf16 parity bar)
static void expect_close(const std::vector<float>& got, const std::vector<float>& ref, const char* what) {
    EXPECT(got.size() == ref.size(), "%s: size %zu vs %zu", what, got.size(), ref.size());
    double worst = 0;
    for (size_t i = 0; i < got.size(); i++) {
        const double err = std::fabs(static_cast<double>(got[i]) - ref[i]);
        EXPECT(std::isfinite(got[i]), "%s: non-finite output at %zu", what, i);
        EXPECT(err <= 2e-3 + 1e-2 * std::fabs(ref[i]), "%s: element %zu got %g ref %g", what, i, got[i], ref[i]);
        worst = err > worst ? err : worst;
    }
    std::printf("  %s: max-abs %.3g over %zu values\n", what, worst, got.size());
}

// ---- CPU-only -------------------------------------------------------------------------------------
static void cpu_tests() {
    run("StatusCodesMapToTheReferenceExceptionKinds", [] {
        EXPECT(throws_as<std::invalid_argument>([] { check(PA_ERROR_INVALID_ARGUMENT, "x"); }), "invalid arg");
        EXPECT(throws_as<NotSupported>([] { check(PA_ERROR_UNSUPPORTED, "x"); }), "unsupported");
        EXPECT(throws_as<NotSupported>([] { check(PA_ERROR_INVALID_CONFIG, "x"); }), "config");
        EXPECT(throws_as<PagedAttentionError>([] { check(PA_ERROR_HIP, "x"); }), "hip");
        check(PA_SUCCESS, "x");  // no throw
    });
    run("FlattenBlockTablesPadsWithMinusOne", [] {
        int32_t mb = -1;
        auto flat = FlattenBlockTables({{5, 2}, {}, {7, 1, 9}}, &mb);
        EXPECT(mb == 3, "max blocks %d", mb);
        const std::vector<int32_t> want = {5, 2, -1, -1, -1, -1, 7, 1, 9};
        EXPECT(flat == want, "flattened table differs");
    });
    run("ConstructorWithoutGpuReportsNoDevice", [] {
        bool ok = false;
        try {
            HipPagedAttentionKernel k(128);
        } catch (const PagedAttentionError& e) {
            ok = e.status() == PA_ERROR_NO_DEVICE;
        }
        EXPECT(ok, "expected PA_ERROR_NO_DEVICE");
    });
    run("ConstructorRejectsNonPositiveHeadDim", [] {
        EXPECT(throws_as<std::invalid_argument>([] { HipPagedAttentionKernel k(0); }), "headDim 0");
    });
}

// ---- GPU ------------------------------------------------------------------------------------------
static void dense_case(HipPagedAttentionKernel& kern, int B, int Q, int C, int H, int D, AttentionPhase phase,
                       float scale, uint64_t seed, const char* name) {
    Tensor q(randn(static_cast<size_t>(B) * Q * H * D, seed), {B, Q, H, D});
    Tensor k(randn(static_cast<size_t>(B) * C * H * D, seed + 1), {B, C, H, D});
    Tensor v(randn(static_cast<size_t>(B) * C * H * D, seed + 2), {B, C, H, D});
    Tensor got = kern.ComputePagedAttention(q, k, v, phase, scale);
    EXPECT(got.shape == q.shape, "%s: output shape", name);
    std::vector<float> ref(q.data.size());
    const float s = scale > 0 ? scale : 1.0f / std::sqrt(static_cast<float>(D));
    EXPECT(orc_sdpa(q.data.data(), k.data.data(), v.data.data(), ref.data(), B, Q, C, H, D,
                    phase == AttentionPhase::Decode ? PA_PHASE_DECODE : PA_PHASE_PREFILL, s, 0) == 0,
           "%s: oracle failed", name);
    expect_close(got.data, ref, name);
}

static void gpu_tests() {
    HipPagedAttentionKernel kern(128);
    run("SupportsRocmOnly", [&] {
        EXPECT(kern.SupportsDevice({DeviceType::ROCm, 0}), "ROCm");
        EXPECT(!kern.SupportsDevice({DeviceType::CUDA, 0}), "CUDA");
        EXPECT(!kern.SupportsDevice({DeviceType::CPU, 0}), "CPU");
    });
    run("DecodeSingleQueryMatchesOracle", [&] {
        dense_case(kern, 3, 1, 37, 8, 128, AttentionPhase::Decode, -1.0f, 11, "decode c=37");
        dense_case(kern, 2, 1, 300, 4, 128, AttentionPhase::Decode, -1.0f, 12, "decode c=300");
    });
    run("DecodePhaseMasksBottomRightWhenCachedExceedsQueries", [&] {
        dense_case(kern, 2, 5, 40, 4, 128, AttentionPhase::Decode, -1.0f, 13, "decode q=5 c=40");
    });
    run("DecodePhaseWithoutExtraKeysIsUnmasked", [&] {
        dense_case(kern, 1, 16, 16, 4, 128, AttentionPhase::Decode, -1.0f, 14, "decode q=c=16");
    });
    run("PrefillPhaseIsUnmasked", [&] {
        dense_case(kern, 2, 20, 20, 8, 128, AttentionPhase::Prefill, -1.0f, 15, "prefill q=c=20");
        dense_case(kern, 1, 7, 50, 8, 128, AttentionPhase::Prefill, -1.0f, 16, "prefill q=7 c=50");
    });
    run("ExplicitScaleOverridesTheDefault", [&] {
        dense_case(kern, 2, 1, 64, 4, 128, AttentionPhase::Decode, 0.3f, 17, "scale 0.3");
    });
    run("OtherHeadDims", [&] {
        // the default scale comes from the constructor's headDim, as in the reference
        HipPagedAttentionKernel k64(64), k256(256);
        dense_case(k64, 2, 3, 33, 8, 64, AttentionPhase::Decode, -1.0f, 18, "D=64");
        dense_case(k256, 1, 1, 100, 2, 256, AttentionPhase::Decode, -1.0f, 19, "D=256");
    });
    run("UnsupportedHeadDimIsNotSupported", [&] {
        HipPagedAttentionKernel k48(48);
        Tensor q(randn(48, 1), {1, 1, 1, 48}), kv(randn(48 * 4, 2), {1, 4, 1, 48});
        EXPECT(throws_as<NotSupported>([&] { k48.ComputePagedAttention(q, kv, kv, AttentionPhase::Decode); }),
               "head_dim 48");
    });
    run("ShapeMismatchIsInvalidArgument", [&] {
        Tensor q(randn(128, 1), {1, 1, 1, 128}), k(randn(256, 2), {1, 2, 1, 128}), v(randn(128, 3), {1, 1, 1, 128});
        EXPECT(throws_as<std::invalid_argument>([&] { kern.ComputePagedAttention(q, k, v, AttentionPhase::Decode); }),
               "K/V shape mismatch");
    });
    run("PagedOverloadMatchesOracleWithBlockManagerTables", [&] {
        // bf16 cache, GQA 4:1, tables from the reference's FIFO block manager (restated by the oracle)
        const int Hq = 16, Hkv = 4, D = 128, nb = 200;
        const std::vector<int> lens = {1, 16, 17, 300, 700, 1000};
        orc_block_manager* bm = orc_bm_create(nb);
        std::vector<std::vector<int>> seq_blocks;
        for (int t : lens) {
            const int need = (t + 15) / 16;
            std::vector<int32_t> ids(need);
            EXPECT(orc_bm_allocate_blocks(bm, need, ids.data()) == need, "pool too small");
            seq_blocks.emplace_back(ids.begin(), ids.end());
        }
        orc_bm_destroy(bm);
        int32_t mb = 0;
        const auto tables = FlattenBlockTables(seq_blocks, &mb);
        const int S = static_cast<int>(lens.size());
        const size_t cache_elems = static_cast<size_t>(nb) * Hkv * 16 * D;
        std::vector<uint16_t> kc(cache_elems), vc(cache_elems), qb(static_cast<size_t>(S) * Hq * D);
        auto kf = randn(cache_elems, 21, 0.5f), vf = randn(cache_elems, 22, 0.5f), qf = randn(qb.size(), 23, 0.5f);
        for (size_t i = 0; i < cache_elems; i++) {
            kc[i] = orc_bf16_from_f32(kf[i]);
            vc[i] = orc_bf16_from_f32(vf[i]);
        }
        for (size_t i = 0; i < qb.size(); i++) qb[i] = orc_bf16_from_f32(qf[i]);
        pa_config cfg{};
        cfg.block_size = 16;
        cfg.num_q_heads = Hq;
        cfg.num_kv_heads = Hkv;
        cfg.head_dim = D;
        cfg.kv_dtype = PA_DTYPE_BF16;
        cfg.q_dtype = PA_DTYPE_BF16;
        cfg.num_blocks = nb;
        cfg.scale = -1.0f;
        std::vector<float> ref(static_cast<size_t>(S) * Hq * D);
        EXPECT(orc_paged_decode(&cfg, ref.data(), qb.data(), kc.data(), vc.data(), nullptr, nullptr, tables.data(),
                                lens.data(), S, mb, 4) == 0,
               "oracle decode");
        pa_device* dev = kern.device();
        void *dq, *dk, *dv, *dt, *dl, *dout;
        check(pa_alloc(dev, qb.size() * 2, &dq), "alloc");
        check(pa_alloc(dev, cache_elems * 2, &dk), "alloc");
        check(pa_alloc(dev, cache_elems * 2, &dv), "alloc");
        check(pa_alloc(dev, tables.size() * 4, &dt), "alloc");
        check(pa_alloc(dev, lens.size() * 4, &dl), "alloc");
        check(pa_alloc(dev, ref.size() * 4, &dout), "alloc");
        check(pa_memcpy(dq, qb.data(), qb.size() * 2, PA_MEMCPY_HOST_TO_DEVICE, nullptr), "memcpy");
        check(pa_memcpy(dk, kc.data(), cache_elems * 2, PA_MEMCPY_HOST_TO_DEVICE, nullptr), "memcpy");
        check(pa_memcpy(dv, vc.data(), cache_elems * 2, PA_MEMCPY_HOST_TO_DEVICE, nullptr), "memcpy");
        check(pa_memcpy(dt, tables.data(), tables.size() * 4, PA_MEMCPY_HOST_TO_DEVICE, nullptr), "memcpy");
        check(pa_memcpy(dl, lens.data(), lens.size() * 4, PA_MEMCPY_HOST_TO_DEVICE, nullptr), "memcpy");
        PagedDecodeBatch batch;
        batch.query = dq;
        batch.k_cache = dk;
        batch.v_cache = dv;
        batch.block_tables = static_cast<const int32_t*>(dt);
        batch.context_lens = static_cast<const int32_t*>(dl);
        batch.num_seqs = S;
        batch.max_blocks_per_seq = mb;
        batch.max_context_len = 1000;
        kern.ComputePagedAttention(cfg, batch, static_cast<float*>(dout));
        std::vector<float> got(ref.size());
        check(pa_device_synchronize(dev), "sync");
        check(pa_memcpy(got.data(), dout, got.size() * 4, PA_MEMCPY_DEVICE_TO_HOST, nullptr), "memcpy");
        check(pa_device_synchronize(dev), "sync");
        for (void* p : {dq, dk, dv, dt, dl, dout}) pa_free(dev, p);
        expect_close(got, ref, "paged overload");
    });
}

int main(int argc, char** argv) {
    const bool gpu = argc > 1 && std::strcmp(argv[1], "--gpu") == 0;
    const bool cpu = argc > 1 && std::strcmp(argv[1], "--cpu") == 0;
    if (!gpu && !cpu) {
        std::printf("usage: %s --cpu | --gpu\n", argv[0]);
        return 2;
    }
    if (cpu) cpu_tests();
    if (gpu) {
        try {
            gpu_tests();
        } catch (const std::exception& e) {
            std::printf("[ FAIL ] setup: %s\n", e.what());
            g_failed++;
        }
    }
    std::printf("%d tests, %d failed\n", g_run, g_failed);
    return g_failed ? 1 : 0;
}
