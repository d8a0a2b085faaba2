// Parity tests of the C++ host layer (llmtoy-zig_amd/host/llmtoy_ops.hpp)
// against the CPU oracle, named after the reference's own test blocks.
// Run with a GPU: ./test_host_ops ; without one: ./test_host_ops --list.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "../../llmtoy-zig_amd/host/llmtoy_ops.hpp"
#include "../../oracle/lt_oracle.h"

using namespace llmtoy;

static int failures = 0;
#define EXPECT(cond)                                                          \
    do {                                                                      \
        if (!(cond)) {                                                        \
            std::printf("    FAILED %s:%d: %s\n", __FILE__, __LINE__, #cond); \
            failures++;                                                       \
            return;                                                           \
        }                                                                     \
    } while (0)

struct Rng {  // splitmix64
    uint64_t s;
    uint64_t next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    float uniform() { return (float)((next() >> 40) * (1.0 / (1ull << 24))); }
};

// Random bytes with every f16 super-scale stamped to 0x21CD (~0.012), the
// scheme of the reference's fuzzQuantMatvec (gpu/matvec.zig:4543-4619).
static std::vector<uint8_t> fuzz_matrix(GgmlType t, size_t rows, size_t cols, uint64_t seed) {
    Rng r{seed};
    const size_t rb = rowBytes(t, cols);
    std::vector<uint8_t> m(rows * rb);
    for (auto &b : m) b = (uint8_t)r.next();
    const size_t bb = t == GgmlType::q8_0 ? 34 : t == GgmlType::q4_k ? 144 : 210;
    for (size_t off = 0; off < m.size(); off += bb) {
        const size_t d = t == GgmlType::q6_k ? 208 : 0;
        m[off + d] = 0xCD;
        m[off + d + 1] = 0x21;
        if (t == GgmlType::q4_k) {
            m[off + 2] = 0xCD;
            m[off + 3] = 0x21;
        }
    }
    return m;
}

static double max_rel(const std::vector<float> &a, const std::vector<float> &b) {
    double md = 0, mr = 0;
    for (size_t i = 0; i < a.size(); i++) {
        md = std::fmax(md, std::fabs((double)a[i] - b[i]));
        mr = std::fmax(mr, std::fabs((double)b[i]));
    }
    return md / (mr + 1e-6);
}

static double rel_l2(const std::vector<float> &a, const std::vector<float> &b) {
    double n = 0, d = 0;
    for (size_t i = 0; i < a.size(); i++) {
        n += ((double)a[i] - b[i]) * ((double)a[i] - b[i]);
        d += (double)b[i] * b[i];
    }
    return std::sqrt(n / d);
}

static void test_q8_0_correctness(GpuContext &g) {  // gpu/matvec.zig:3728-3767
    std::vector<uint8_t> m(32 * 34, 0);
    for (int r = 0; r < 32; r++) {
        m[r * 34 + 1] = 0x3C;
        m[r * 34 + 2 + r] = 1;
    }
    std::vector<float> vec(32), out(32);
    for (int i = 0; i < 32; i++) vec[i] = (float)(i + 1);
    auto s = MatvecSession::initFromRaw(g, {m.data(), m.size(), GgmlType::q8_0, 32, 32});
    EXPECT(s.has_value());
    s->run(vec.data(), out.data());
    for (int i = 0; i < 32; i++) EXPECT(std::fabs(out[i] - (float)(i + 1)) < 1e-4);
}

static void test_q4_k_scale(GpuContext &g) {  // gpu/matvec.zig:3877-3908
    std::vector<uint8_t> m(144, 0);
    m[1] = 0x3C;
    m[4] = 1;
    std::memset(&m[16], 0x11, 32);
    std::vector<float> vec(256, 1.0f), out(1);
    quantMatvec(g, out.data(), {m.data(), m.size(), GgmlType::q4_k, 1, 256}, vec.data());
    EXPECT(std::fabs(out[0] - 32.0f) < 1e-4);
}

static void test_q4_k_min(GpuContext &g) {  // gpu/matvec.zig:3910-3939
    std::vector<uint8_t> m(144, 0);
    m[3] = 0x3C;
    m[8] = 2;
    std::vector<float> vec(256, 1.0f), out(1);
    quantMatvec(g, out.data(), {m.data(), m.size(), GgmlType::q4_k, 1, 256}, vec.data());
    EXPECT(std::fabs(out[0] + 64.0f) < 1e-4);
}

static void test_unsupported_type_has_no_session(GpuContext &g) {  // gpu/matvec.zig:564-577
    std::vector<uint8_t> m(64, 0);
    EXPECT(!MatvecSession::initFromRaw(g, {m.data(), m.size(), GgmlType::f16, 1, 32}).has_value());
}

static void fuzz(GpuContext &g, GgmlType t, size_t rows, size_t cols, uint64_t seed) {
    auto m = fuzz_matrix(t, rows, cols, seed);
    Rng r{seed * 7 + 1};
    std::vector<float> vec(cols), out(rows), ref(rows), rowbuf(cols);
    for (auto &v : vec) v = (r.uniform() - 0.5f) * 2.0f;
    quantMatvec(g, out.data(), {m.data(), m.size(), t, rows, cols}, vec.data());
    lto_quant_matvec(ref.data(), m.data(), (uint32_t)t, vec.data(), rows, cols, rowbuf.data());
    EXPECT(max_rel(out, ref) < 1e-4);
}
static void test_q8_0_fuzz(GpuContext &g) { fuzz(g, GgmlType::q8_0, 32, 256, 1); }
static void test_q4_k_fuzz(GpuContext &g) { fuzz(g, GgmlType::q4_k, 64, 2048, 11); }
static void test_q6_k_fuzz(GpuContext &g) { fuzz(g, GgmlType::q6_k, 37, 1024, 17); }

// A small MoE layer: fp32 router ~ U(-0.05, 0.05), Q4_K experts with random
// bytes and stamped super-scales.
struct Layer {
    size_t E = 16, D = 512, F = 256, k = 4;
    std::vector<float> router;
    std::vector<uint8_t> gate_up, down;
    std::vector<float> x;
    explicit Layer(uint64_t seed) {
        Rng r{seed};
        router.resize(E * D);
        for (auto &v : router) v = (r.uniform() - 0.5f) * 0.1f;
        gate_up = fuzz_matrix(GgmlType::q4_k, E * 2 * F, D, seed + 1);
        down = fuzz_matrix(GgmlType::q4_k, E * D, F, seed + 2);
        x.resize(D);
        for (auto &v : x) v = (r.uniform() - 0.5f) * 2.0f;
    }
    RawMatrix R() const { return {(const uint8_t *)router.data(), router.size() * 4, GgmlType::f32, E, D}; }
    RawMatrix GU() const { return {gate_up.data(), gate_up.size(), GgmlType::q4_k, E * 2 * F, D}; }
    RawMatrix DN() const { return {down.data(), down.size(), GgmlType::q4_k, E * D, F}; }
};

// The context caches device copies by host pointer (the reference's "mmap
// outlives the weights" contract), so each test forgets its buffers before
// they are freed.
struct Scoped {
    GpuContext &g;
    const Layer &L;
    ~Scoped() {
        g.forget(L.router.data());
        g.forget(L.gate_up.data());
        g.forget(L.down.data());
    }
};

static void test_moe_forward_accumulates(GpuContext &g) {  // ops/moe.zig:18-77
    Layer L(101);
    Scoped sc{g, L};
    std::vector<float> out(L.D, 0.25f), ref(L.D, 0.25f);
    moeForward(g, out.data(), L.R(), L.GU(), L.DN(), L.x.data(), L.k, L.F);
    int agree = 0;
    EXPECT(lto_moe_forward(ref.data(), L.router.data(), L.E, nullptr, L.gate_up.data(), LTO_Q4_K, L.down.data(),
                           LTO_Q4_K, L.F, L.x.data(), L.D, L.k, L.F, LTO_ACT_SILU, 0, nullptr, nullptr, nullptr,
                           &agree) == 0);
    EXPECT(agree == 1);
    EXPECT(rel_l2(out, ref) < 1e-3);
}

static void test_run_expert_batch(GpuContext &g) {  // gemma4/forward.zig:463-479
    Layer L(202);
    Scoped sc{g, L};
    const std::vector<size_t> top = {3, 11, 0, 7};
    std::vector<float> router_out(L.E, 0.0f), scale(L.E, 1.0f);
    router_out[3] = 0.4f, router_out[11] = 0.3f, router_out[0] = 0.2f, router_out[7] = 0.1f;
    scale[11] = 0.5f;
    std::vector<float> moe(L.D, 0.0f), ref(L.D, 0.0f);
    GpuWeights gw(g, L.GU(), L.DN(), L.E, L.F);
    gw.runExpertBatch(top.data(), top.size(), scale.data(), L.x.data(), router_out.data(), moe.data());
    // CPU expert loop with gelu (the Gemma4 loop), per expert
    std::vector<float> eg(L.F), eu(L.F), ed(L.D), scratch(L.D);
    const size_t gu_rb = rowBytes(GgmlType::q4_k, L.D), dn_rb = rowBytes(GgmlType::q4_k, L.F);
    for (size_t e : top) {
        const uint8_t *gd = L.gate_up.data() + e * 2 * L.F * gu_rb;
        lto_quant_matvec(eg.data(), gd, LTO_Q4_K, L.x.data(), L.F, L.D, scratch.data());
        lto_quant_matvec(eu.data(), gd + L.F * gu_rb, LTO_Q4_K, L.x.data(), L.F, L.D, scratch.data());
        for (size_t j = 0; j < L.F; j++) eg[j] = lto_gelu(eg[j]) * eu[j];
        lto_quant_matvec(ed.data(), L.down.data() + e * L.D * dn_rb, LTO_Q4_K, eg.data(), L.D, L.F, scratch.data());
        const float s = scale[e] * router_out[e];
        for (size_t i = 0; i < L.D; i++) ref[i] += s * ed[i];
    }
    EXPECT(rel_l2(moe, ref) < 1e-3);
}

static void test_expert_not_on_gpu(GpuContext &g) {  // gemma4/forward.zig:434-480
    Layer L(303);
    Scoped sc{g, L};
    std::vector<uint8_t> q8(L.E * L.D * rowBytes(GgmlType::q8_0, L.F), 0);
    GpuWeights gw(g, L.GU(), {q8.data(), q8.size(), GgmlType::q8_0, L.E * L.D, L.F}, L.E, L.F);
    const size_t top[1] = {0};
    std::vector<float> ro(L.E, 1.0f), moe(L.D, 0.0f);
    bool thrown = false;
    try {
        gw.runExpertBatch(top, 1, nullptr, L.x.data(), ro.data(), moe.data());
    } catch (const Exception &e) {
        thrown = e.kind == Error::ExpertNotOnGpu;
    }
    EXPECT(thrown);
}

static void test_rmsnorm_kat(GpuContext &g) {  // ops/math.zig:344-354
    const float x[4] = {1, 2, 3, 4}, w[4] = {1, 1, 1, 1};
    float out[4];
    rmsnorm(g, out, x, w, 4, 1e-8f);
    const float rms = std::sqrt((1.0f + 4.0f + 9.0f + 16.0f) / 4.0f);
    EXPECT(std::fabs(out[0] - x[0] / rms) <= 1e-5f && std::fabs(out[3] - x[3] / rms) <= 1e-5f);
    float wo[4], ro[4], ref_w[4], ref_r[4];
    const float xs[4] = {3, -4, 1, 2}, ww[4] = {0.5f, 1.25f, -0.75f, 2.0f}, sc[4] = {2.0f, 0.25f, -1.0f, 0.5f};
    rmsnormWeightedAndRawScaled(g, wo, ro, xs, ww, sc, 0.125f, 4, 1e-6f, true);  // math.zig:356-376
    lto_rmsnorm_wrs(ref_w, ref_r, xs, ww, sc, 0.125f, 4, 1e-6f);
    EXPECT(std::memcmp(wo, ref_w, sizeof wo) == 0 && std::memcmp(ro, ref_r, sizeof ro) == 0);
}

static void test_run_moe_block(GpuContext &g) {  // gemma4/forward.zig:403-497
    Layer L(404);
    Scoped sc{g, L};
    Rng r{405};
    auto vec = [&](size_t n, float c, float a) {
        std::vector<float> v(n);
        for (auto &t : v) t = c + (r.uniform() - 0.5f) * a;
        return v;
    };
    const std::vector<float> pre = vec(L.D, 1, 0.4f), rs = vec(L.D, 1, 0.2f), ds = vec(L.E, 1, 0.5f),
                             p2 = vec(L.D, 1, 0.4f), p = vec(L.D, 1, 0.4f), dense = vec(L.D, 0, 2);
    const Gemma4MoeNorms nm{pre.data(), rs.data(), ds.data(), p2.data(), p.data()};
    std::vector<float> x = L.x, ref = L.x;
    GpuWeights gw(g, L.GU(), L.DN(), L.E, L.F);
    size_t top[4];
    gw.runMoeBlock(L.R(), nm, L.k, MoeTailParams{1e-6f, x.data(), dense.data(), 0.75f}, top, nullptr,
                   LT_ACT_GELU_TANH, true);
    uint32_t rids[4];
    EXPECT(lto_gemma4_moe_block(ref.data(), dense.data(), L.D, (const uint8_t *)L.router.data(), LTO_F32, L.E,
                                L.gate_up.data(), LTO_Q4_K, L.down.data(), LTO_Q4_K, L.F, L.k, L.F, pre.data(),
                                rs.data(), ds.data(), p2.data(), p.data(), 0.75f, 1e-6f, LTO_ACT_GELU_TANH, nullptr,
                                rids, nullptr) == 0);
    for (size_t i = 0; i < L.k; i++) EXPECT(top[i] == rids[i]);
    EXPECT(rel_l2(x, ref) < 1e-3);
}

int main(int argc, char **argv) {
    const std::vector<std::pair<std::string, std::function<void(GpuContext &)>>> tests = {
        {"gpu matvec Q8_0 correctness", test_q8_0_correctness},
        {"gpu matvec Q4_K scale", test_q4_k_scale},
        {"gpu matvec Q4_K min", test_q4_k_min},
        {"MatvecSession.initFromRaw: unsupported type gives null", test_unsupported_type_has_no_session},
        {"gpu matvec Q8_0 fuzz", test_q8_0_fuzz},
        {"gpu matvec Q4_K fuzz", test_q4_k_fuzz},
        {"gpu matvec Q6_K fuzz", test_q6_k_fuzz},
        {"moeForward: accumulates the weighted experts into out", test_moe_forward_accumulates},
        {"runExpertBatch: matches the CPU expert loop", test_run_expert_batch},
        {"runExpertBatch: non-device experts raise ExpertNotOnGpu", test_expert_not_on_gpu},
        {"rmsnorm: all-ones weight is pure normalisation", test_rmsnorm_kat},
        {"runMoeBlock: matches the Gemma4 CPU block", test_run_moe_block},
    };
    if (argc > 1 && std::strcmp(argv[1], "--list") == 0) {
        for (auto &t : tests) std::printf("%s\n", t.first.c_str());
        return 0;
    }
    try {
        GpuContext g(0);
        for (auto &t : tests) {
            const int before = failures;
            std::printf("test \"%s\" ...\n", t.first.c_str());
            std::fflush(stdout);
            t.second(g);
            std::printf("    %s\n", failures == before ? "ok" : "FAILED");
        }
    } catch (const Exception &e) {
        std::printf("exception: %s\n", e.what());
        return 2;
    }
    std::printf(failures ? "%d FAILED\n" : "ALL PASSED\n", failures);
    return failures ? 1 : 0;
}
