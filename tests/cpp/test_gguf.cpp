// Tests of the GGUF reader (llmtoy-zig_amd/host/gguf_reader.hpp).
//   ./test_gguf --list        test names
//   ./test_gguf --cpu         parser tests that need no device
//   ./test_gguf --dump FILE   canonical dump of a file's header (compared
//                             with the Python reader's by the pytest suite)
//   ./test_gguf --gpu FILE    load MoE layer 0 and the test.* tensors of
//                             FILE, run them on the device through
//                             llmtoy_ops.hpp and check against the oracle
#include <cinttypes>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include <unistd.h>

#include "../../llmtoy-zig_amd/host/gguf_reader.hpp"
#include "../../llmtoy-zig_amd/host/llmtoy_ops.hpp"
#include "../../oracle/lt_oracle.h"

using namespace llmtoy;
using gguf::MetaValueType;

static int failures = 0;
#define EXPECT(cond)                                                          \
    do {                                                                      \
        if (!(cond)) {                                                        \
            std::printf("    FAILED %s:%d: %s\n", __FILE__, __LINE__, #cond); \
            failures++;                                                       \
            return;                                                           \
        }                                                                     \
    } while (0)

// ------------------------------------------------------------ byte builders
struct Buf {
    std::vector<uint8_t> b;
    template <typename T>
    Buf &put(T v) {
        const auto *p = reinterpret_cast<const uint8_t *>(&v);
        b.insert(b.end(), p, p + sizeof(T));
        return *this;
    }
    Buf &str(const std::string &s) {
        put<uint64_t>(s.size());
        b.insert(b.end(), s.begin(), s.end());
        return *this;
    }
    Buf &pad_to(size_t a) {
        while (b.size() % a) b.push_back(0);
        return *this;
    }
};

static gguf::Error parse_error(const std::vector<uint8_t> &b) {
    try {
        gguf::parseBytes(b.data(), b.size());
    } catch (const gguf::Exception &e) {
        return e.kind;
    }
    return (gguf::Error)-1;
}

// gguf/reader.zig:247-297 "parseBytes: synthetic GGUF v3", restated.
static Buf reference_kat(size_t *header_end) {
    Buf w;
    w.put<uint32_t>(0x46554747u).put<uint32_t>(3).put<uint64_t>(1).put<uint64_t>(2);
    w.str("general.architecture").put<uint32_t>(8).str("test_arch");
    w.str("test.context_length").put<uint32_t>(4).put<uint32_t>(256);
    w.str("weight").put<uint32_t>(2).put<uint64_t>(4).put<uint64_t>(4).put<uint32_t>(0).put<uint64_t>(0);
    *header_end = w.b.size();
    w.pad_to(32);
    w.b.insert(w.b.end(), 64, 0);
    return w;
}

static void test_reference_kat() {
    size_t hend;
    const Buf w = reference_kat(&hend);
    const gguf::GgufData g = gguf::parseBytes(w.b.data(), w.b.size());
    EXPECT(g.version == 3);
    EXPECT(g.metadata.size() == 2);
    EXPECT(g.tensors.size() == 1);
    std::string arch;
    uint32_t ctx = 0;
    EXPECT(g.metaString("general.architecture", arch) && arch == "test_arch");
    EXPECT(g.metaU32("test.context_length", ctx) && ctx == 256);
    EXPECT(g.tensors[0].name == "weight");
    EXPECT(g.tensors[0].n_elements() == 16);
    EXPECT(g.tensors[0].type == 0);
    // 24 header + 49 + 35 metadata + 46 tensor info = 154 bytes, aligned to 160
    EXPECT(hend == 154 && g.data_offset == 160);
}

static void test_every_prefix_is_truncated() {
    size_t hend;
    const Buf w = reference_kat(&hend);
    for (size_t n = 0; n < hend; n++) {
        std::vector<uint8_t> cut(w.b.begin(), w.b.begin() + n);
        EXPECT(parse_error(cut) == gguf::Error::Truncated);
    }
    std::vector<uint8_t> whole(w.b.begin(), w.b.begin() + hend);
    EXPECT(parse_error(whole) == (gguf::Error)-1);
}

static void test_magic_and_version() {
    size_t hend;
    Buf w = reference_kat(&hend);
    std::vector<uint8_t> b = w.b;
    b[0] ^= 1;
    EXPECT(parse_error(b) == gguf::Error::InvalidMagic);
    for (uint32_t v : {0u, 4u, 0xffffffffu}) {
        b = w.b;
        std::memcpy(b.data() + 4, &v, 4);
        EXPECT(parse_error(b) == gguf::Error::UnsupportedVersion);
    }
}

static void test_v1_u32_counts() {
    Buf w;
    w.put<uint32_t>(0x46554747u).put<uint32_t>(1).put<uint32_t>(1).put<uint32_t>(1);
    w.str("k").put<uint32_t>(10).put<uint64_t>(0x0123456789abcdefull);
    w.str("t").put<uint32_t>(1).put<uint64_t>(32).put<uint32_t>(8).put<uint64_t>(0);
    const size_t hend = w.b.size();
    w.pad_to(32);
    w.b.insert(w.b.end(), 34, 0);
    const gguf::GgufData g = gguf::parseBytes(w.b.data(), w.b.size());
    uint64_t u = 0;
    EXPECT(g.version == 1 && g.metaU64("k", u) && u == 0x0123456789abcdefull);
    EXPECT(g.tensors.size() == 1 && g.tensors[0].type == 8 && g.tensors[0].byteSize() == 34);
    EXPECT(g.data_offset == (hend + 31) / 32 * 32);
}

static void test_every_value_type() {
    Buf w;
    w.put<uint32_t>(0x46554747u).put<uint32_t>(2).put<uint64_t>(0).put<uint64_t>(14);
    w.str("u8").put<uint32_t>(0).put<uint8_t>(200);
    w.str("i8").put<uint32_t>(1).put<int8_t>(-100);
    w.str("u16").put<uint32_t>(2).put<uint16_t>(60000);
    w.str("i16").put<uint32_t>(3).put<int16_t>(-30000);
    w.str("u32").put<uint32_t>(4).put<uint32_t>(4000000000u);
    w.str("i32").put<uint32_t>(5).put<int32_t>(-2000000000);
    w.str("f32").put<uint32_t>(6).put<float>(-1.5f);
    w.str("bool").put<uint32_t>(7).put<uint8_t>(2);  // any non-zero byte is true
    w.str("str").put<uint32_t>(8).str("h\xc3\xa9llo");
    w.str("u64").put<uint32_t>(10).put<uint64_t>(18000000000000000000ull);
    w.str("i64").put<uint32_t>(11).put<int64_t>(-9000000000000000000ll);
    w.str("f64").put<uint32_t>(12).put<double>(0.1);
    w.str("arr").put<uint32_t>(9).put<uint32_t>(8).put<uint64_t>(2).str("a").str("");
    w.str("nest").put<uint32_t>(9).put<uint32_t>(9).put<uint64_t>(2);
    w.put<uint32_t>(5).put<uint64_t>(1).put<int32_t>(-7);  // [[-7], []]
    w.put<uint32_t>(6).put<uint64_t>(0);
    const gguf::GgufData g = gguf::parseBytes(w.b.data(), w.b.size());
    EXPECT(g.version == 2 && g.metadata.size() == 14);
    EXPECT(g.get("u8")->u == 200 && g.get("i8")->i == -100 && g.get("u16")->u == 60000);
    EXPECT(g.get("i16")->i == -30000 && g.get("u32")->u == 4000000000u && g.get("i32")->i == -2000000000);
    float f;
    bool b;
    std::string s;
    uint64_t u;
    EXPECT(g.metaF32("f32", f) && f == -1.5f);
    EXPECT(g.metaBool("bool", b) && b);
    EXPECT(g.metaString("str", s) && s == "h\xc3\xa9llo");
    EXPECT(g.metaU64("u64", u) && u == 18000000000000000000ull && g.get("i64")->i == -9000000000000000000ll);
    EXPECT(g.get("f64")->f == 0.1);
    const gguf::MetaValue *a = g.metaArray("arr");
    EXPECT(a && a->elem == MetaValueType::string && a->arr.size() == 2 && a->arr[0].s == "a" && a->arr[1].s.empty());
    const gguf::MetaValue *n = g.metaArray("nest");
    EXPECT(n && n->arr.size() == 2 && n->arr[0].arr.size() == 1 && n->arr[0].arr[0].i == -7 && n->arr[1].arr.empty());
    // typed lookups reject other types and missing keys (the reference's null)
    uint32_t u32;
    EXPECT(!g.metaU32("u64", u32) && !g.metaString("u8", s) && !g.metaF32("f64", f) && !g.metaArray("missing"));
    EXPECT(g.metaU64("u32", u) && u == 4000000000u);  // metaU64 also takes uint32
}

static void test_bad_value_type_and_huge_counts() {
    Buf w;
    w.put<uint32_t>(0x46554747u).put<uint32_t>(3).put<uint64_t>(0).put<uint64_t>(1);
    w.str("x").put<uint32_t>(13).put<uint32_t>(0);
    EXPECT(parse_error(w.b) == gguf::Error::BadValueType);
    Buf h;  // an array count far beyond the data is truncation, not an allocation
    h.put<uint32_t>(0x46554747u).put<uint32_t>(3).put<uint64_t>(0).put<uint64_t>(1);
    h.str("x").put<uint32_t>(9).put<uint32_t>(0).put<uint64_t>(1ull << 60);
    EXPECT(parse_error(h.b) == gguf::Error::Truncated);
    Buf t;
    t.put<uint32_t>(0x46554747u).put<uint32_t>(3).put<uint64_t>(1ull << 50).put<uint64_t>(0);
    EXPECT(parse_error(t.b) == gguf::Error::Truncated);
    gguf::TensorInfo big;  // dims whose product overflows 64 bits saturate
    big.type = 12;
    big.dims = {1ull << 40, 1ull << 40};
    EXPECT(big.n_elements() == (1ull << 63) && big.byteSize() > (1ull << 50));
}

// byteSize against each block layout's byte count (d/dmin halves, scale
// bytes, packed quants); gguf/types.zig:138-172 holds the same table.
static void test_byte_size_table() {
    struct Row {
        uint32_t id;
        uint64_t bytes, elems;
    } rows[] = {
        {0, 4, 1}, {1, 2, 1}, {30, 2, 1}, {24, 1, 1}, {25, 2, 1}, {26, 4, 1}, {27, 8, 1},
        {2, 2 + 16, 32},                // q4_0: d, 32 nibbles
        {3, 2 + 2 + 16, 32},            // q4_1: d, m, 32 nibbles
        {6, 2 + 4 + 16, 32},            // q5_0: d, high bits, nibbles
        {7, 2 + 2 + 4 + 16, 32},        // q5_1
        {8, 2 + 32, 32},                // q8_0: d, 32 int8
        {9, 4 + 4 + 32, 32},            // q8_1 as the reference sizes it (f32 d and s)
        {10, 16 + 64 + 2 + 2, 256},     // q2_k: scales, 2-bit quants, d, dmin
        {11, 32 + 64 + 12 + 2, 256},    // q3_k: hmask, quants, scales, d
        {12, 2 + 2 + 12 + 128, 256},    // q4_k
        {13, 2 + 2 + 12 + 32 + 128, 256},  // q5_k
        {14, 128 + 64 + 16 + 2, 256},   // q6_k: ql, qh, scales, d
        {15, 4 + 256 + 32, 256},        // q8_k: f32 d, quants, 16 i16 sums
    };
    for (const Row &r : rows) {
        gguf::TensorInfo t;
        t.type = r.id;
        t.dims = {r.elems * 8, 3};
        EXPECT(t.byteSize() == 24 * r.bytes);
        EXPECT(gguf::block_size(r.id).bytes == r.bytes && gguf::block_size(r.id).elems == r.elems);
    }
    gguf::TensorInfo f64;
    f64.type = 28;
    f64.dims = {5};
    EXPECT(f64.byteSize() == 0);  // f64 has no entry in the reference's table
    // the decode path's rowBytes agrees on its types
    for (GgmlType t : {GgmlType::f32, GgmlType::f16, GgmlType::q8_0, GgmlType::q4_k, GgmlType::q6_k}) {
        gguf::TensorInfo i;
        i.type = (uint32_t)t;
        i.dims = {1024, 5};
        EXPECT(i.byteSize() == 5 * rowBytes(t, 1024) && lto_row_bytes((uint32_t)t, 1024) == rowBytes(t, 1024));
    }
}

// a file on disk: open, tensorBytes, rawMatrix3D bounds, empty file
static void test_reader_file() {
    Buf w;
    w.put<uint32_t>(0x46554747u).put<uint32_t>(3).put<uint64_t>(2).put<uint64_t>(0);
    w.str("e").put<uint32_t>(3).put<uint64_t>(256).put<uint64_t>(2).put<uint64_t>(3).put<uint32_t>(12).put<uint64_t>(0);
    w.str("f").put<uint32_t>(1).put<uint64_t>(8).put<uint32_t>(0).put<uint64_t>(6 * 144);
    w.pad_to(32);
    const size_t data = w.b.size();
    for (size_t i = 0; i < 6 * 144 + 32; i++) w.b.push_back((uint8_t)(i * 7 + 1));
    char tp[] = "/tmp/test_gguf_XXXXXX", te[] = "/tmp/test_gguf_empty_XXXXXX";
    const int fd1 = mkstemp(tp), fd2 = mkstemp(te);
    EXPECT(fd1 >= 0 && fd2 >= 0);
    close(fd1);
    close(fd2);
    const std::string path = tp, empty = te;
    FILE *fp = std::fopen(path.c_str(), "wb");
    EXPECT(fp);
    std::fwrite(w.b.data(), 1, w.b.size(), fp);
    std::fclose(fp);
    {
        gguf::GgufReader r(path);
        size_t nb;
        const uint8_t *p = r.tensorBytes(r.tensor("e"), nb);
        EXPECT(nb == 6 * 144 && p[0] == w.b[data] && p[nb - 1] == w.b[data + nb - 1]);
        const RawMatrix m = r.rawMatrix3D("e", 3, 2, 256);
        EXPECT(m.rows == 6 && m.cols == 256 && m.type == GgmlType::q4_k && m.size == 6 * 144);
        bool threw = false;
        try {
            r.rawMatrix3D("e", 4, 2, 256);  // 8 rows from a 6-row tensor
        } catch (const gguf::Exception &e) {
            threw = e.kind == gguf::Error::Truncated;
        }
        EXPECT(threw);
        threw = false;
        try {
            r.tensor("nope");
        } catch (const gguf::Exception &e) {
            threw = e.kind == gguf::Error::MissingTensor;
        }
        EXPECT(threw);
    }
    {  // mkstemp left it empty
        bool threw = false;
        try {
            gguf::GgufReader r(empty);
        } catch (const gguf::Exception &e) {
            threw = e.kind == gguf::Error::EmptyFile;
        }
        EXPECT(threw);
    }
    {  // a tensor whose bytes run past the end of the file
        std::vector<uint8_t> cut(w.b.begin(), w.b.begin() + data + 6 * 144 + 10);
        fp = std::fopen(path.c_str(), "wb");
        std::fwrite(cut.data(), 1, cut.size(), fp);
        std::fclose(fp);
        gguf::GgufReader r(path);
        size_t nb;
        bool threw = false;
        try {
            r.tensorBytes(r.tensor("f"), nb);
        } catch (const gguf::Exception &e) {
            threw = e.kind == gguf::Error::Truncated;
        }
        EXPECT(threw);
    }
    std::remove(path.c_str());
    std::remove(empty.c_str());
}

// A hostile header: sizes whose products wrap around 64 bits must be
// Error::Truncated, not a small allocation followed by a huge copy.
// E = 1024 experts of d_expert = 2^54 rows (E * F = 2^64 wraps to 0), with
// 1-element F32 gate and up tensors; then a fused gate_up tensor with
// d_expert = 2^63 (2 * F wraps to 0).
static std::string write_temp(const Buf &w) {
    char tp[] = "/tmp/test_gguf_ovf_XXXXXX";
    const int fd = mkstemp(tp);
    if (fd < 0) return "";
    close(fd);
    FILE *fp = std::fopen(tp, "wb");
    if (!fp) return "";
    std::fwrite(w.b.data(), 1, w.b.size(), fp);
    std::fclose(fp);
    return tp;
}

static Buf overflow_file(uint64_t d_expert, bool fused) {
    const uint64_t E = 1024;
    Buf w;
    w.put<uint32_t>(0x46554747u).put<uint32_t>(3).put<uint64_t>(fused ? 3 : 4).put<uint64_t>(4);
    w.str("general.architecture").put<uint32_t>(8).str("qwen3moe");
    w.str("qwen3moe.embedding_length").put<uint32_t>(10).put<uint64_t>(1);
    w.str("qwen3moe.expert_count").put<uint32_t>(10).put<uint64_t>(E);
    w.str("qwen3moe.expert_feed_forward_length").put<uint32_t>(10).put<uint64_t>(d_expert);
    uint64_t off = 0;
    auto tensor = [&](const char *name, std::vector<uint64_t> dims, uint64_t nbytes) {
        w.str(name).put<uint32_t>((uint32_t)dims.size());
        for (uint64_t d : dims) w.put<uint64_t>(d);
        w.put<uint32_t>(0).put<uint64_t>(off);  // F32
        off += (nbytes + 31) / 32 * 32;
    };
    tensor("blk.0.ffn_gate_inp.weight", {1, E}, 4 * E);
    if (fused) {
        tensor("blk.0.ffn_gate_up_exps.weight", {1}, 4);
    } else {
        tensor("blk.0.ffn_gate_exps.weight", {1}, 4);
        tensor("blk.0.ffn_up_exps.weight", {1}, 4);
    }
    tensor("blk.0.ffn_down_exps.weight", {1}, 4);
    w.pad_to(32);
    w.b.insert(w.b.end(), off, 0);
    return w;
}

static void test_moe_layer_size_overflow() {
    for (int fused = 0; fused < 2; fused++) {
        const std::string path = write_temp(overflow_file(fused ? (1ull << 63) : (1ull << 54), fused));
        EXPECT(!path.empty());
        bool threw = false;
        try {
            gguf::GgufReader r(path);
            const gguf::MoeConfig c = gguf::moeConfig(r.data);
            (void)gguf::moeLayer(r, c, 0);
        } catch (const gguf::Exception &e) {
            threw = e.kind == gguf::Error::Truncated;
        }
        std::remove(path.c_str());
        EXPECT(threw);
    }
}

// ------------------------------------------------------------------- dump
static void dump_value(const gguf::MetaValue &v, std::string &o) {
    char tmp[64];
    switch (v.type) {
    case MetaValueType::uint8: case MetaValueType::uint16: case MetaValueType::uint32: case MetaValueType::uint64:
        std::snprintf(tmp, sizeof tmp, "%" PRIu64, v.u);
        break;
    case MetaValueType::int8: case MetaValueType::int16: case MetaValueType::int32: case MetaValueType::int64:
        std::snprintf(tmp, sizeof tmp, "%" PRId64, v.i);
        break;
    case MetaValueType::float32: {
        float f = (float)v.f;
        uint32_t bits;
        std::memcpy(&bits, &f, 4);
        std::snprintf(tmp, sizeof tmp, "f%08x", bits);
        break;
    }
    case MetaValueType::float64: {
        uint64_t bits;
        std::memcpy(&bits, &v.f, 8);
        std::snprintf(tmp, sizeof tmp, "d%016" PRIx64, bits);
        break;
    }
    case MetaValueType::bool_: std::snprintf(tmp, sizeof tmp, "%s", v.b ? "true" : "false"); break;
    case MetaValueType::string:
        o += "s";
        for (unsigned char c : v.s) {
            std::snprintf(tmp, sizeof tmp, "%02x", c);
            o += tmp;
        }
        return;
    case MetaValueType::array:
        std::snprintf(tmp, sizeof tmp, "[%u:", (unsigned)v.elem);
        o += tmp;
        for (size_t i = 0; i < v.arr.size(); i++) {
            if (i) o += ",";
            dump_value(v.arr[i], o);
        }
        o += "]";
        return;
    }
    o += tmp;
}

static uint64_t fnv1a(const uint8_t *p, size_t n) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (size_t i = 0; i < n; i++) h = (h ^ p[i]) * 0x100000001b3ull;
    return h;
}

static int dump(const char *path) {
    gguf::GgufReader r(path);
    std::printf("version %u\ndata_offset %zu\n", r.data.version, r.data.data_offset);
    for (const auto &kv : r.data.metadata) {  // std::map: sorted by key bytes
        std::string o;
        dump_value(kv.second, o);
        std::printf("kv %s %u %s\n", kv.first.c_str(), (unsigned)kv.second.type, o.c_str());
    }
    for (const auto &t : r.data.tensors) {
        std::string dims;
        for (size_t i = 0; i < t.dims.size(); i++) dims += (i ? "," : "") + std::to_string(t.dims[i]);
        size_t nb;
        const uint8_t *p = r.tensorBytes(t, nb);
        std::printf("tensor %s %u %" PRIu64 " %s %" PRIu64 " %" PRIu64 " %016" PRIx64 "\n", t.name.c_str(), t.type,
                    t.offset, dims.c_str(), t.n_elements(), t.byteSize(), fnv1a(p, nb));
    }
    return 0;
}

// -------------------------------------------------------------------- gpu
static double rel_l2(const std::vector<float> &a, const std::vector<float> &b) {
    double n = 0, d = 0;
    for (size_t i = 0; i < a.size(); i++) {
        n += ((double)a[i] - b[i]) * ((double)a[i] - b[i]);
        d += (double)b[i] * b[i];
    }
    return std::sqrt(n / d);
}

static const float *f32_tensor(const gguf::GgufReader &r, const std::string &name, size_t n) {
    const gguf::TensorInfo &t = r.tensor(name);
    if (t.type != 0 || t.n_elements() != n) throw gguf::Exception(gguf::Error::BadValueType, name + " is not F32");
    size_t nb;
    return reinterpret_cast<const float *>(r.tensorBytes(t, nb));
}

// MoE layer 0 of the file through moeForward and GpuWeights, and every 2-D
// test.* weight through quantMatvec, each against the oracle on the same bytes.
static int run_gpu(const char *path) {
    gguf::GgufReader r(path);
    const gguf::MoeConfig c = gguf::moeConfig(r.data);
    gguf::MoeLayer L = gguf::moeLayer(r, c, 0);
    const float *x = f32_tensor(r, "test.x", c.d_model);
    std::printf("%s: %s d_model %zu experts %zu top-%zu d_expert %zu down_cols %zu\n", path, c.arch.c_str(),
                c.d_model, c.n_experts, c.n_experts_used, c.d_expert, L.down_cols);
    GpuContext g(0);
    int bad = 0;
    if (L.router.type == GgmlType::f32) {  // moeForward takes the fp32 router (ops/moe.zig:18-28)
        std::vector<float> out(c.d_model, 0.0f), ref(c.d_model, 0.0f);
        moeForward(g, out.data(), L.router, L.gate_up, L.down, x, c.n_experts_used, c.d_expert, true);
        std::vector<uint32_t> ids(c.n_experts_used);
        int agree = 0;
        const int rc = lto_moe_forward(ref.data(), reinterpret_cast<const float *>(L.router.data), c.n_experts,
                                       nullptr, L.gate_up.data, (uint32_t)L.gate_up.type, L.down.data,
                                       (uint32_t)L.down.type, L.down_cols, x, c.d_model, c.n_experts_used,
                                       c.d_expert, LTO_ACT_SILU, 0, nullptr, ids.data(), nullptr, &agree);
        const double e = rel_l2(out, ref);
        std::printf("moeForward: rel-L2 %.3g vs oracle (rc %d, selection order agrees %d)\n", e, rc, agree);
        bad += !(rc == 0 && agree == 1 && e < 1e-3);
        if (L.down_exps_scale) {  // runExpertBatch with the file's per-expert scale
            std::vector<float> ro(c.n_experts, 0.0f), moe(c.d_model, 0.0f), ref2(c.d_model, 0.0f);
            std::vector<size_t> top(ids.begin(), ids.end());
            for (size_t k = 0; k < top.size(); k++) ro[top[k]] = 1.0f / (float)(k + 1);
            GpuWeights gw(g, L.gate_up, L.down, c.n_experts, c.d_expert);
            gw.runExpertBatch(top.data(), top.size(), L.down_exps_scale, x, ro.data(), moe.data(), LT_ACT_SILU);
            const size_t gu_rb = rowBytes(L.gate_up.type, c.d_model), dn_rb = rowBytes(L.down.type, L.down_cols);
            std::vector<float> eg(c.d_expert), eu(c.d_expert), h(L.down_cols, 0.0f), ed(c.d_model),
                scratch(c.d_model > L.down_cols ? c.d_model : L.down_cols);
            for (size_t e2 : top) {
                const uint8_t *gd = L.gate_up.data + e2 * 2 * c.d_expert * gu_rb;
                lto_quant_matvec(eg.data(), gd, (uint32_t)L.gate_up.type, x, c.d_expert, c.d_model, scratch.data());
                lto_quant_matvec(eu.data(), gd + c.d_expert * gu_rb, (uint32_t)L.gate_up.type, x, c.d_expert,
                                 c.d_model, scratch.data());
                for (size_t j = 0; j < c.d_expert; j++) h[j] = lto_silu(eg[j]) * eu[j];
                lto_quant_matvec(ed.data(), L.down.data + e2 * c.d_model * dn_rb, (uint32_t)L.down.type, h.data(),
                                 c.d_model, L.down_cols, scratch.data());
                const float s = L.down_exps_scale[e2] * ro[e2];
                for (size_t i = 0; i < c.d_model; i++) ref2[i] += s * ed[i];
            }
            const double e3 = rel_l2(moe, ref2);
            std::printf("runExpertBatch with ffn_down_exps.scale: rel-L2 %.3g\n", e3);
            bad += !(e3 < 1e-3);
        }
    }
    if (r.data.find("blk.0.pre_ffw_norm_2.weight")) {  // a Gemma4 block: runMoeBlock against the CPU block
        const gguf::Gemma4Norms nm = gguf::gemma4Norms(r, c, 0);
        const float *dense = f32_tensor(r, "test.dense", c.d_model);
        std::vector<float> xg(x, x + c.d_model), xr(x, x + c.d_model);
        GpuWeights gw(g, L.gate_up, L.down, c.n_experts, c.d_expert);
        std::vector<size_t> top(c.n_experts_used);
        gw.runMoeBlock(L.router, {nm.pre_ffw_norm_2.data(), nm.router_scale.data(), nm.down_exps_scale.data(),
                                  nm.post_ffw_norm_2.data(), nm.post_ffw_norm.data()},
                       c.n_experts_used, MoeTailParams{1e-6f, xg.data(), dense, nm.layer_output_scale}, top.data(),
                       nullptr, LT_ACT_GELU_TANH, true);
        std::vector<uint32_t> rids(c.n_experts_used);
        const int rc = lto_gemma4_moe_block(
            xr.data(), dense, c.d_model, L.router.data, (uint32_t)L.router.type, c.n_experts, L.gate_up.data,
            (uint32_t)L.gate_up.type, L.down.data, (uint32_t)L.down.type, L.down_cols, c.n_experts_used, c.d_expert,
            nm.pre_ffw_norm_2.data(), nm.router_scale.data(), nm.down_exps_scale.data(), nm.post_ffw_norm_2.data(),
            nm.post_ffw_norm.data(), nm.layer_output_scale, 1e-6f, LTO_ACT_GELU_TANH, nullptr, rids.data(), nullptr);
        bool same = rc == 0;
        for (size_t i = 0; i < top.size(); i++) same = same && top[i] == rids[i];
        const double e = rel_l2(xg, xr);
        std::printf("runMoeBlock (Gemma4 block, output scale %g): ids %s, rel-L2 %.3g\n", nm.layer_output_scale,
                    same ? "match" : "DIFFER", e);
        bad += !(same && e < 1e-3);
    }
    for (const gguf::TensorInfo &t : r.data.tensors) {
        if (t.name.rfind("test.", 0) != 0 || t.dims.size() != 2) continue;
        const size_t rows = t.dims[1], cols = t.dims[0];
        const RawMatrix m = r.rawMatrix(t.name, rows, cols);
        const float *v = f32_tensor(r, "test.v" + std::to_string(cols), cols);
        std::vector<float> out(rows), ref(rows), scratch(cols);
        quantMatvec(g, out.data(), m, v);
        const int rc = lto_quant_matvec(ref.data(), m.data, t.type, v, rows, cols, scratch.data());
        const double e = rel_l2(out, ref);
        std::printf("quantMatvec %s (type %u, %zux%zu): rel-L2 %.3g\n", t.name.c_str(), t.type, rows, cols, e);
        bad += !(rc == 0 && e < 1e-3);
        g.forget(m.data);
    }
    std::printf(bad ? "%d FAILED\n" : "ALL PASSED\n", bad);
    return bad ? 1 : 0;
}

int main(int argc, char **argv) {
    const std::vector<std::pair<std::string, std::function<void()>>> tests = {
        {"parseBytes: synthetic GGUF v3", test_reference_kat},
        {"parseBytes: every header prefix is Truncated", test_every_prefix_is_truncated},
        {"parseBytes: InvalidMagic and UnsupportedVersion", test_magic_and_version},
        {"parseBytes: v1 u32 counts", test_v1_u32_counts},
        {"parseBytes: every metadata value type", test_every_value_type},
        {"parseBytes: bad value type and oversized counts", test_bad_value_type_and_huge_counts},
        {"TensorInfo.byteSize: block layouts", test_byte_size_table},
        {"GgufReader: tensorBytes, rawMatrix3D, EmptyFile", test_reader_file},
        {"moeLayer: wrapping size products are Truncated", test_moe_layer_size_overflow},
    };
    const std::string mode = argc > 1 ? argv[1] : "";
    try {
        if (mode == "--list") {
            for (auto &t : tests) std::printf("%s\n", t.first.c_str());
            return 0;
        }
        if (mode == "--dump" && argc > 2) return dump(argv[2]);
        if (mode == "--gpu" && argc > 2) return run_gpu(argv[2]);
        if (mode == "--cpu") {
            for (auto &t : tests) {
                const int before = failures;
                std::printf("test \"%s\" ...\n", t.first.c_str());
                t.second();
                std::printf("    %s\n", failures == before ? "ok" : "FAILED");
            }
            std::printf(failures ? "%d FAILED\n" : "ALL PASSED\n", failures);
            return failures ? 1 : 0;
        }
    } catch (const gguf::Exception &e) {
        std::printf("gguf exception: %s\n", e.what());
        return 2;
    } catch (const Exception &e) {
        std::printf("exception: %s\n", e.what());
        return 2;
    }
    std::fprintf(stderr, "usage: %s --list | --cpu | --dump FILE | --gpu FILE\n", argv[0]);
    return 64;
}
