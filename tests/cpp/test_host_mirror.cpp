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

// Parity bars: |got - ref| <= atol + rtol |ref|. fp32 caches and queries (the dense interface):
// the kernel computes in fp32 throughout, held to about 100 ulps; bf16 caches: the stated bar.
constexpr double kFp32Atol = 1e-5, kFp32Rtol = 1e-4;
constexpr double kBf16Atol = 2e-3, kBf16Rtol = 1e-2;

static void expect_close(const std::vector<float>& got, const std::vector<float>& ref, const char* what,
                         double atol = kFp32Atol, double rtol = kFp32Rtol) {
    EXPECT(got.size() == ref.size(), "%s: size %zu vs %zu", what, got.size(), ref.size());
    double worst = 0;
    for (size_t i = 0; i < got.size(); i++) {
        const double err = std::fabs(static_cast<double>(got[i]) - ref[i]);
        EXPECT(std::isfinite(got[i]), "%s: non-finite output at %zu", what, i);
        EXPECT(err <= atol + rtol * std::fabs(ref[i]), "%s: element %zu got %g ref %g", what, i, got[i], ref[i]);
        worst = err > worst ? err : worst;
    }
    std::printf("  %s: max-abs %.3g over %zu values\n", what, worst, got.size());
}

// Uniform in [-1, 1) times `scale`: the distribution of the reference tests' CreateRandomQuery
// (PagedAttentionFunctionalTests.cs:284-293, .NET Random(42); this generator's own stream).
static std::vector<float> uniform_pm1(size_t n, uint64_t seed, float scale = 1.0f) {
    std::mt19937_64 rng(seed);
    std::uniform_real_distribution<double> u(0.0, 1.0);
    std::vector<float> v(n);
    for (auto& x : v) x = static_cast<float>(u(rng) * 2 - 1) * scale;
    return v;
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

// The reference's PagedAttentionFunctionalTests (tests/MLFramework.Tests/Inference/PagedAttention/
// PagedAttentionFunctionalTests.cs:40-277) replayed through HipPagedAttentionKernel at their shape:
// 4 heads x head_dim 32, blocks of 16, inputs uniform in [-1, 1) (x100 for the stability case).
// Each output is held to the fp32 bar against the oracle (the reference kernel restated), and to
// the closed form or property the reference test asserts.
static Tensor functional_tensor(int b, int t, uint64_t seed, float scale = 1.0f) {
    return Tensor(uniform_pm1(static_cast<size_t>(b) * t * 4 * 32, seed, scale), {b, t, 4, 32});
}

static std::vector<float> oracle_dense(const Tensor& q, const Tensor& k, const Tensor& v, AttentionPhase phase) {
    std::vector<float> ref(q.data.size());
    EXPECT(orc_sdpa(q.data.data(), k.data.data(), v.data.data(), ref.data(), q.shape[0], q.shape[1], k.shape[1],
                    q.shape[2], q.shape[3], phase == AttentionPhase::Decode ? PA_PHASE_DECODE : PA_PHASE_PREFILL,
                    1.0f / std::sqrt(32.0f), 0) == 0,
           "oracle failed");
    return ref;
}

static void functional_tests_head_dim_32() {
    HipPagedAttentionKernel kern(32);  // StandardPagedAttentionKernel(_headDim = 32)
    run("Functional32_MatchesContiguousForSingleToken", [&] {
        Tensor q = functional_tensor(1, 1, 101), k = functional_tensor(1, 1, 102), v = functional_tensor(1, 1, 103);
        Tensor got = kern.ComputePagedAttention(q, k, v, AttentionPhase::Decode);
        expect_close(got.data, oracle_dense(q, k, v, AttentionPhase::Decode), "single token");
        EXPECT(got.data == v.data, "one cached token: the output is that token's value exactly");
    });
    run("Functional32_MatchesContiguousForMultipleTokens", [&] {
        Tensor q = functional_tensor(1, 1, 111), k = functional_tensor(1, 32, 112), v = functional_tensor(1, 32, 113);
        Tensor got = kern.ComputePagedAttention(q, k, v, AttentionPhase::Decode);
        expect_close(got.data, oracle_dense(q, k, v, AttentionPhase::Decode), "32 tokens");
    });
    run("Functional32_MatchesContiguousAcrossMultipleBlocks", [&] {
        Tensor q = functional_tensor(1, 1, 121), k = functional_tensor(1, 48, 122), v = functional_tensor(1, 48, 123);
        Tensor got = kern.ComputePagedAttention(q, k, v, AttentionPhase::Decode);
        expect_close(got.data, oracle_dense(q, k, v, AttentionPhase::Decode), "3 blocks");
    });
    run("Functional32_PrefillPhaseMatchesContiguous", [&] {
        Tensor q = functional_tensor(1, 16, 131), k = functional_tensor(1, 16, 132), v = functional_tensor(1, 16, 133);
        Tensor got = kern.ComputePagedAttention(q, k, v, AttentionPhase::Prefill);
        expect_close(got.data, oracle_dense(q, k, v, AttentionPhase::Prefill), "prefill 16 x 16");
    });
    run("Functional32_MultipleSequencesIndependentResults", [&] {
        Tensor q1 = functional_tensor(1, 1, 141), k1 = functional_tensor(1, 10, 142), v1 = functional_tensor(1, 10, 143);
        Tensor q2 = functional_tensor(1, 1, 144), k2 = functional_tensor(1, 10, 145), v2 = functional_tensor(1, 10, 146);
        Tensor o1 = kern.ComputePagedAttention(q1, k1, v1, AttentionPhase::Decode);
        Tensor o2 = kern.ComputePagedAttention(q2, k2, v2, AttentionPhase::Decode);
        expect_close(o1.data, oracle_dense(q1, k1, v1, AttentionPhase::Decode), "sequence 1");
        expect_close(o2.data, oracle_dense(q2, k2, v2, AttentionPhase::Decode), "sequence 2");
        bool differ = false;
        for (size_t i = 0; i < o1.data.size(); i++) differ |= std::fabs(o1.data[i] - o2.data[i]) > 1e-5f;
        EXPECT(differ, "different inputs gave outputs within 1e-5 of each other");
        // both sequences in one batched call: each row equals its own call (no leakage)
        std::vector<float> qb(q1.data), kb(k1.data), vb(v1.data);
        qb.insert(qb.end(), q2.data.begin(), q2.data.end());
        kb.insert(kb.end(), k2.data.begin(), k2.data.end());
        vb.insert(vb.end(), v2.data.begin(), v2.data.end());
        Tensor ob = kern.ComputePagedAttention(Tensor(qb, {2, 1, 4, 32}), Tensor(kb, {2, 10, 4, 32}),
                                               Tensor(vb, {2, 10, 4, 32}), AttentionPhase::Decode);
        std::vector<float> o12(o1.data);
        o12.insert(o12.end(), o2.data.begin(), o2.data.end());
        EXPECT(ob.data == o12, "batched rows differ from the per-sequence calls");
    });
    run("Functional32_NumericalStabilityLargeValues", [&] {
        Tensor q = functional_tensor(1, 1, 151, 100.0f), k = functional_tensor(1, 10, 152, 100.0f),
               v = functional_tensor(1, 10, 153, 100.0f);
        Tensor got = kern.ComputePagedAttention(q, k, v, AttentionPhase::Decode);
        for (float x : got.data) EXPECT(std::isfinite(x), "NaN or Inf in the output");
        expect_close(got.data, oracle_dense(q, k, v, AttentionPhase::Decode), "x100 inputs");
    });
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
    run("LongPromptIsOneReadOnceLaunch", [&] {
        // more than one query over at least as many keys runs as one chunked-prefill launch
        dense_case(kern, 2, 512, 512, 8, 128, AttentionPhase::Prefill, -1.0f, 21, "prefill q=c=512");
        dense_case(kern, 1, 512, 700, 8, 128, AttentionPhase::Decode, -1.0f, 22, "decode q=512 c=700");
        dense_case(kern, 1, 512, 512, 4, 128, AttentionPhase::Decode, -1.0f, 23, "decode q=c=512");
    });
    run("MoreQueriesThanKeys", [&] {
        dense_case(kern, 2, 20, 10, 4, 128, AttentionPhase::Decode, -1.0f, 24, "decode q=20 c=10");
        dense_case(kern, 1, 9, 4, 4, 128, AttentionPhase::Prefill, -1.0f, 25, "prefill q=9 c=4");
    });
    run("ExplicitScaleOverridesTheDefault", [&] {
        dense_case(kern, 2, 1, 64, 4, 128, AttentionPhase::Decode, 0.3f, 17, "scale 0.3");
    });
    run("OtherHeadDims", [&] {
        // the default scale comes from the constructor's headDim, as in the reference
        HipPagedAttentionKernel k64(64), k256(256);
        dense_case(k64, 2, 3, 33, 8, 64, AttentionPhase::Decode, -1.0f, 18, "D=64");
        dense_case(k256, 1, 1, 100, 2, 256, AttentionPhase::Decode, -1.0f, 19, "D=256");
        dense_case(k64, 2, 40, 40, 4, 64, AttentionPhase::Prefill, -1.0f, 26, "D=64 prefill q=c=40");
        dense_case(k256, 1, 33, 90, 2, 256, AttentionPhase::Decode, -1.0f, 27, "D=256 decode q=33 c=90");
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
        expect_close(got, ref, "paged overload", kBf16Atol, kBf16Rtol);
    });
    run("DenseCallWithMoreRowsThanOneLaunchTakes", [&] {
        // 70000 (batch, query) rows become 70000 decode sequences: the fp32 path issues them in
        // launches of at most 65535 sequences.
        HipPagedAttentionKernel k32(32);
        dense_case(k32, 70000, 1, 3, 1, 32, AttentionPhase::Decode, -1.0f, 31, "70000 rows");
    });
    functional_tests_head_dim_32();
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
