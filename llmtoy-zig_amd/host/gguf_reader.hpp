// gguf_reader.hpp -- GGUF v1-v3 reader for feeding real tensors to the decode
// path (llmtoy_ops.hpp).  Mirrors llmtoy-zig's parser and its types:
//
//   MAGIC, ALIGNMENT, MetaValueType, GgmlType ids   gguf/types.zig:3-53
//   Array, MetaValue                                gguf/types.zig:86-122
//   TensorInfo (n_elements, byteSize)               gguf/types.zig:125-173
//   GgufData (metaString/U32/Array/Bool/F32/U64)    gguf/reader.zig:7-53
//   parseBytes, readMetaValue                       gguf/reader.zig:56-100, 216-235
//   GgufReader (open: mmap + parse, tensorBytes)    gguf/reader.zig:104-171
//   rawMatrix (a 2-D weight as a RawMatrix)         model/loader.zig:190-204
//   rawMatrix3D (expert tensors as one RawMatrix)   gemma4/loader.zig:275-292
//   moeConfig / moeLayer (MoE keys and tensors)     gemma4/loader.zig:27-83, 152-163
//   loadNorm / gemma4Norms (block vectors)          gemma4/loader.zig:121-163, 182-214
//
// Same layout rules as the reference: little-endian fields; v1 counts are
// u32, v2/v3 counts u64; tensor data starts at the header end rounded up to
// 32 bytes (the reference ignores general.alignment, and so does this
// reader); a tensor's bytes are data_offset + offset .. + byteSize().
// Errors: the reference's error.InvalidMagic / UnsupportedVersion /
// EmptyFile become gguf::Error with the same names.  One deliberate
// difference: every read is bounds-checked and a header or tensor that runs
// past the end of the data is Error::Truncated (the reference indexes the
// mmap without a check, undefined in ReleaseFast).  Header-only, host C++17.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "llmtoy_ops.hpp"

namespace llmtoy {
namespace gguf {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" little-endian
constexpr size_t kAlignment = 32;

enum class MetaValueType : uint32_t {
    uint8 = 0, int8 = 1, uint16 = 2, int16 = 3, uint32 = 4, int32 = 5, float32 = 6,
    bool_ = 7, string = 8, array = 9, uint64 = 10, int64 = 11, float64 = 12,
};

enum class Error {
    InvalidMagic, UnsupportedVersion, EmptyFile,  // the reference's parse/open errors
    MissingTensor, MissingMetadata,              // its loaders' LoadError
    Truncated, BadValueType, Io,
};

class Exception : public std::runtime_error {
   public:
    Exception(Error kind, const std::string &msg) : std::runtime_error(msg), kind(kind) {}
    Error kind;
};

// a * b for sizes taken from a file's metadata or tensor dims; a product
// that does not fit in 64 bits (a corrupt or hostile header) is
// Error::Truncated, since no file can hold that many bytes.
inline size_t checkedMul(size_t a, size_t b, const std::string &what) {
    size_t r;
    if (__builtin_mul_overflow(a, b, &r)) throw Exception(Error::Truncated, "gguf: " + what + " overflows");
    return r;
}

// A metadata value: the member named by type holds it (integers in i / u,
// floats in f, arrays in arr with their element type in elem).
struct MetaValue {
    MetaValueType type = MetaValueType::uint8;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0.0;
    bool b = false;
    std::string s;
    MetaValueType elem = MetaValueType::uint8;
    std::vector<MetaValue> arr;
};

// Bytes per block and elements per block of the GgmlType ids
// (gguf/types.zig:140-172); {0, 0} for a type without a size there.
struct BlockSize {
    uint64_t bytes, elems;
};
inline BlockSize block_size(uint32_t type) {
    switch (type) {
    case 0: return {4, 1};      // f32
    case 1: return {2, 1};      // f16
    case 30: return {2, 1};     // bf16
    case 24: return {1, 1};     // i8
    case 25: return {2, 1};     // i16
    case 26: return {4, 1};     // i32
    case 27: return {8, 1};     // i64
    case 2: return {18, 32};    // q4_0
    case 3: return {20, 32};    // q4_1
    case 6: return {22, 32};    // q5_0
    case 7: return {24, 32};    // q5_1
    case 8: return {34, 32};    // q8_0
    case 9: return {40, 32};    // q8_1
    case 10: return {84, 256};  // q2_k
    case 11: return {110, 256}; // q3_k
    case 12: return {144, 256}; // q4_k
    case 13: return {176, 256}; // q5_k
    case 14: return {210, 256}; // q6_k
    case 15: return {292, 256}; // q8_k
    case 16: return {66, 256};  // iq2_xxs
    case 17: return {74, 256};  // iq2_xs
    case 22: return {82, 256};  // iq2_s
    case 18: return {98, 256};  // iq3_xxs
    case 21: return {110, 256}; // iq3_s
    case 20: return {18, 32};   // iq4_nl
    case 23: return {136, 256}; // iq4_xs
    case 19: return {50, 256};  // iq1_s
    case 29: return {56, 256};  // iq1_m
    default: return {0, 0};     // f64 and unknown ids: byteSize 0, as the reference
    }
}

struct TensorInfo {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0;

    // Product of the dims; a product past 2^63 (a corrupt header) saturates
    // there, so byteSize is then larger than any file and tensorBytes fails.
    uint64_t n_elements() const {
        uint64_t n = 1;
        for (uint64_t d : dims) {
            if (d && n > (1ull << 63) / d) return 1ull << 63;
            n *= d;
        }
        return n;
    }
    // Exact byte size of the stored weights: (n / block elements) * block
    // bytes, integer division as in the reference.
    uint64_t byteSize() const {
        const BlockSize b = block_size(type);
        return b.elems ? (n_elements() / b.elems) * b.bytes : 0;
    }
};

struct GgufData {
    uint32_t version = 0;
    std::map<std::string, MetaValue> metadata;
    std::vector<TensorInfo> tensors;
    size_t data_offset = 0;  // where tensor data begins in the source bytes

    const MetaValue *get(const std::string &key) const {
        auto it = metadata.find(key);
        return it == metadata.end() ? nullptr : &it->second;
    }
    // The typed lookups return false when the key is missing or holds
    // another type (the reference's optional null).
    bool metaString(const std::string &key, std::string &out) const {
        const MetaValue *v = get(key);
        if (!v || v->type != MetaValueType::string) return false;
        out = v->s;
        return true;
    }
    bool metaU32(const std::string &key, uint32_t &out) const {
        const MetaValue *v = get(key);
        if (!v || v->type != MetaValueType::uint32) return false;
        out = (uint32_t)v->u;
        return true;
    }
    bool metaU64(const std::string &key, uint64_t &out) const {  // uint32 or uint64
        const MetaValue *v = get(key);
        if (!v || (v->type != MetaValueType::uint32 && v->type != MetaValueType::uint64)) return false;
        out = v->u;
        return true;
    }
    bool metaBool(const std::string &key, bool &out) const {
        const MetaValue *v = get(key);
        if (!v || v->type != MetaValueType::bool_) return false;
        out = v->b;
        return true;
    }
    bool metaF32(const std::string &key, float &out) const {
        const MetaValue *v = get(key);
        if (!v || v->type != MetaValueType::float32) return false;
        out = (float)v->f;
        return true;
    }
    const MetaValue *metaArray(const std::string &key) const {
        const MetaValue *v = get(key);
        return v && v->type == MetaValueType::array ? v : nullptr;
    }
    const TensorInfo *find(const std::string &name) const {
        for (const TensorInfo &t : tensors)
            if (t.name == name) return &t;
        return nullptr;
    }
};

namespace detail {

struct Cursor {
    const uint8_t *p;
    size_t n, pos;

    void need(size_t k) {
        if (k > n || pos > n - k) throw Exception(Error::Truncated, "gguf: header runs past the end of the data");
    }
    template <typename T>
    T get() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, p + pos, sizeof(T));  // little-endian host (x86-64, the only host here)
        pos += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t len = get<uint64_t>();
        need(len);
        std::string s(reinterpret_cast<const char *>(p + pos), (size_t)len);
        pos += (size_t)len;
        return s;
    }
};

inline MetaValue read_value(Cursor &c, MetaValueType t, int depth) {
    MetaValue v;
    v.type = t;
    switch (t) {
    case MetaValueType::uint8: v.u = c.get<uint8_t>(); break;
    case MetaValueType::int8: v.i = c.get<int8_t>(); break;
    case MetaValueType::uint16: v.u = c.get<uint16_t>(); break;
    case MetaValueType::int16: v.i = c.get<int16_t>(); break;
    case MetaValueType::uint32: v.u = c.get<uint32_t>(); break;
    case MetaValueType::int32: v.i = c.get<int32_t>(); break;
    case MetaValueType::float32: v.f = c.get<float>(); break;
    case MetaValueType::bool_: v.b = c.get<uint8_t>() != 0; break;
    case MetaValueType::string: v.s = c.str(); break;
    case MetaValueType::uint64: v.u = c.get<uint64_t>(); break;
    case MetaValueType::int64: v.i = c.get<int64_t>(); break;
    case MetaValueType::float64: v.f = c.get<double>(); break;
    case MetaValueType::array: {
        if (depth > 8) throw Exception(Error::BadValueType, "gguf: arrays nested too deeply");
        v.elem = (MetaValueType)c.get<uint32_t>();
        const uint64_t count = c.get<uint64_t>();
        // every element takes at least one byte: a count beyond the data is truncation
        c.need(count);
        v.arr.reserve((size_t)count);
        for (uint64_t k = 0; k < count; k++) v.arr.push_back(read_value(c, v.elem, depth + 1));
        break;
    }
    default: throw Exception(Error::BadValueType, "gguf: unknown metadata value type " + std::to_string((uint32_t)t));
    }
    return v;
}

}  // namespace detail

// gguf/reader.zig:55-100
inline GgufData parseBytes(const uint8_t *data, size_t size) {
    detail::Cursor c{data, size, 0};
    if (c.get<uint32_t>() != kMagic) throw Exception(Error::InvalidMagic, "gguf: invalid magic");
    GgufData g;
    g.version = c.get<uint32_t>();
    if (g.version < 1 || g.version > 3)
        throw Exception(Error::UnsupportedVersion, "gguf: unsupported version " + std::to_string(g.version));
    const uint64_t n_tensors = g.version == 1 ? c.get<uint32_t>() : c.get<uint64_t>();
    const uint64_t n_kv = g.version == 1 ? c.get<uint32_t>() : c.get<uint64_t>();
    for (uint64_t k = 0; k < n_kv; k++) {
        std::string key = c.str();
        const auto t = (MetaValueType)c.get<uint32_t>();
        g.metadata[key] = detail::read_value(c, t, 0);  // a repeated key keeps the last value, as put()
    }
    c.need(n_tensors);  // each tensor descriptor is longer than a byte
    g.tensors.resize((size_t)n_tensors);
    for (TensorInfo &t : g.tensors) {
        t.name = c.str();
        const uint32_t n_dims = c.get<uint32_t>();
        c.need((size_t)n_dims * 8);
        t.dims.resize(n_dims);
        for (uint64_t &d : t.dims) d = c.get<uint64_t>();
        t.type = c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
    }
    g.data_offset = (c.pos + kAlignment - 1) / kAlignment * kAlignment;
    return g;
}

// gguf/reader.zig:104-171: the file is mapped read-only and parsed; tensor
// bytes are views into the mapping, valid while the reader lives.
class GgufReader {
   public:
    explicit GgufReader(const std::string &path) {
        fd_ = ::open(path.c_str(), O_RDONLY);
        if (fd_ < 0) throw Exception(Error::Io, "gguf: cannot open " + path);
        struct stat st;
        if (fstat(fd_, &st) != 0) {
            ::close(fd_);
            throw Exception(Error::Io, "gguf: cannot stat " + path);
        }
        size_ = (size_t)st.st_size;
        if (size_ == 0) {
            ::close(fd_);
            throw Exception(Error::EmptyFile, "gguf: empty file " + path);
        }
        void *m = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
        if (m == MAP_FAILED) {
            ::close(fd_);
            throw Exception(Error::Io, "gguf: cannot map " + path);
        }
        map_ = static_cast<const uint8_t *>(m);
        try {
            data = parseBytes(map_, size_);
        } catch (...) {
            munmap(const_cast<uint8_t *>(map_), size_);
            ::close(fd_);
            throw;
        }
    }
    GgufReader(const GgufReader &) = delete;
    GgufReader &operator=(const GgufReader &) = delete;
    ~GgufReader() {
        munmap(const_cast<uint8_t *>(map_), size_);
        ::close(fd_);
    }

    // Raw bytes of a tensor: exactly byteSize() bytes.
    const uint8_t *tensorBytes(const TensorInfo &info, size_t &nbytes) const {
        const uint64_t start = (uint64_t)data.data_offset + info.offset, len = info.byteSize();
        if (start > size_ || len > size_ - start)
            throw Exception(Error::Truncated, "gguf: tensor " + info.name + " runs past the end of the file");
        nbytes = (size_t)len;
        return map_ + start;
    }

    const TensorInfo &tensor(const std::string &name) const {
        const TensorInfo *t = data.find(name);
        if (!t) throw Exception(Error::MissingTensor, "gguf: no tensor " + name);
        return *t;
    }

    // model/loader.zig:190-204: a weight as a RawMatrix of rows x cols, the
    // shape coming from the model config as in the reference.  Unlike the
    // reference, the tensor must hold rows whole rows (Error::Truncated
    // otherwise), so a device upload of rows * rowBytes never reads past it.
    RawMatrix rawMatrix(const std::string &name, size_t rows, size_t cols) const {
        const TensorInfo &t = tensor(name);
        size_t nb;
        const uint8_t *p = tensorBytes(t, nb);
        RawMatrix m{p, nb, (GgmlType)t.type, rows, cols};
        const BlockSize b = block_size(t.type);
        const uint64_t rb = b.elems ? (cols / b.elems) * b.bytes : 0;  // one row; cols < 2^40 in any real file
        if (!b.elems || cols % b.elems || rb == 0 || cols > (1ull << 40) || rows > nb / rb)
            throw Exception(Error::Truncated, "gguf: tensor " + name + " does not hold " + std::to_string(rows) +
                                                  " rows of " + std::to_string(cols));
        return m;
    }

    // gemma4/loader.zig:275-292: an expert tensor stored [cols,
    // rows_per_expert, n_experts] as one RawMatrix of n_experts *
    // rows_per_expert rows.
    RawMatrix rawMatrix3D(const std::string &name, size_t n_experts, size_t rows_per_expert, size_t cols) const {
        return rawMatrix(name, checkedMul(n_experts, rows_per_expert, "expert rows of " + name), cols);
    }

    GgufData data;

   private:
    int fd_ = -1;
    const uint8_t *map_ = nullptr;
    size_t size_ = 0;
};

// The MoE shape keys, read as gemma4/loader.zig:27-75 reads them.
struct MoeConfig {
    std::string arch;
    size_t d_model, n_experts, n_experts_used, d_expert;
};

inline MoeConfig moeConfig(const GgufData &g) {
    MoeConfig c;
    if (!g.metaString("general.architecture", c.arch))
        throw Exception(Error::MissingMetadata, "gguf: no general.architecture");
    auto need = [&](const char *k) -> size_t {
        uint64_t v;
        if (!g.metaU64(c.arch + "." + k, v)) throw Exception(Error::MissingMetadata, "gguf: no " + c.arch + "." + k);
        return (size_t)v;
    };
    c.d_model = need("embedding_length");
    c.n_experts = need("expert_count");
    c.d_expert = need("expert_feed_forward_length");
    uint64_t used;
    c.n_experts_used = g.metaU64(c.arch + ".expert_used_count", used) ? (size_t)used : 8;
    return c;
}

// One layer's MoE tensors as the RawMatrix views moeForward / GpuWeights
// take (gemma4/loader.zig:152-163):
//   blk.L.ffn_gate_inp.weight      router [E, d]
//   blk.L.ffn_gate_up_exps.weight  [d, 2F, E]: per expert F gate rows, F up rows
//   blk.L.ffn_down_exps.weight     [down_cols, d, E]
// A file with separate blk.L.ffn_gate_exps / ffn_up_exps ([d, F, E] each,
// the llama.cpp Qwen3-MoE naming) is accepted too: gate and up rows are
// interleaved per expert into an owned host copy.  The optional F32
// ffn_down_exps.scale [E] and ffn_gate_inp.scale [d] are returned, not applied.
struct MoeLayer {
    MoeLayer() = default;
    MoeLayer(MoeLayer &&) = default;  // moving keeps gate_up_copy's buffer, so gate_up stays valid
    MoeLayer(const MoeLayer &) = delete;
    MoeLayer &operator=(const MoeLayer &) = delete;

    RawMatrix router{}, gate_up{}, down{};
    size_t d_expert = 0, down_cols = 0;
    const float *down_exps_scale = nullptr, *router_scale = nullptr;
    std::vector<uint8_t> gate_up_copy;  // backs gate_up for split gate/up files
};

inline MoeLayer moeLayer(const GgufReader &r, const MoeConfig &c, size_t layer) {
    const std::string p = "blk." + std::to_string(layer) + ".";
    const size_t d = c.d_model, E = c.n_experts, F = c.d_expert;
    MoeLayer L;
    L.d_expert = F;
    L.router = r.rawMatrix(p + "ffn_gate_inp.weight", E, d);
    if (r.data.find(p + "ffn_gate_up_exps.weight")) {
        L.gate_up = r.rawMatrix3D(p + "ffn_gate_up_exps.weight", E, checkedMul(2, F, "2 * d_expert"), d);
    } else {
        const RawMatrix g = r.rawMatrix3D(p + "ffn_gate_exps.weight", E, F, d);
        const RawMatrix u = r.rawMatrix3D(p + "ffn_up_exps.weight", E, F, d);
        if (g.type != u.type) throw Exception(Error::BadValueType, "gguf: gate and up experts differ in type");
        // one expert's gate (or up) bytes; both rawMatrix3D calls above have
        // shown E * F rows fit in the file, the checks only guard the products
        const size_t eb = checkedMul(F, rowBytes(g.type, d), "expert bytes");
        L.gate_up_copy.resize(checkedMul(2, checkedMul(E, eb, "gate/up bytes"), "gate/up bytes"));
        for (size_t e = 0; e < E; e++) {
            std::memcpy(L.gate_up_copy.data() + 2 * e * eb, g.data + e * eb, eb);
            std::memcpy(L.gate_up_copy.data() + (2 * e + 1) * eb, u.data + e * eb, eb);
        }
        L.gate_up = RawMatrix{L.gate_up_copy.data(), L.gate_up_copy.size(), g.type, 2 * E * F, d};
    }
    const TensorInfo &dn = r.tensor(p + "ffn_down_exps.weight");
    L.down_cols = dn.dims.empty() ? F : (size_t)dn.dims[0];
    L.down = r.rawMatrix3D(p + "ffn_down_exps.weight", E, d, L.down_cols);
    auto f32 = [&](const std::string &name, size_t n) -> const float * {
        const TensorInfo *t = r.data.find(name);
        if (!t) return nullptr;
        if (t->type != 0 || t->n_elements() != n) throw Exception(Error::BadValueType, "gguf: " + name + " is not F32");
        size_t nb;
        return reinterpret_cast<const float *>(r.tensorBytes(*t, nb));
    };
    L.down_exps_scale = f32(p + "ffn_down_exps.scale", E);
    L.router_scale = f32(p + "ffn_gate_inp.scale", d);
    return L;
}

// gemma4/loader.zig:182-199 loadNorm: an F32 or F16 vector of n values
// (F16 converted exactly).
inline std::vector<float> loadNorm(const GgufReader &r, const std::string &name, size_t n) {
    const TensorInfo &t = r.tensor(name);
    if (t.n_elements() != n) throw Exception(Error::BadValueType, "gguf: " + name + " has the wrong length");
    size_t nb;
    const uint8_t *p = r.tensorBytes(t, nb);
    std::vector<float> v(n);
    if (t.type == 0) {
        std::memcpy(v.data(), p, n * 4);
    } else if (t.type == 1) {
        for (size_t i = 0; i < n; i++) {
            const uint32_t h = (uint32_t)p[2 * i] | ((uint32_t)p[2 * i + 1] << 8);
            const uint32_t sign = (h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
            float f;
            if (e == 0) {
                f = (float)m * 5.9604644775390625e-08f;  // m * 2^-24, exact
                if (sign) f = -f;
            } else {
                const uint32_t bits = sign | (e == 31 ? 0x7f800000u | (m << 13) : ((e + 112u) << 23) | (m << 13));
                std::memcpy(&f, &bits, 4);
            }
            v[i] = f;
        }
    } else {
        throw Exception(Error::BadValueType, "gguf: " + name + " is neither F32 nor F16");
    }
    return v;
}

// The vectors of a Gemma4 MoE block (gemma4/loader.zig:121-163); a missing
// layer_output_scale is 1, as loadScalar returns (201-214).
struct Gemma4Norms {
    std::vector<float> pre_ffw_norm_2, router_scale, down_exps_scale, post_ffw_norm_2, post_ffw_norm;
    float layer_output_scale = 1.0f;
};

inline Gemma4Norms gemma4Norms(const GgufReader &r, const MoeConfig &c, size_t layer) {
    const std::string p = "blk." + std::to_string(layer) + ".";
    Gemma4Norms g;
    g.pre_ffw_norm_2 = loadNorm(r, p + "pre_ffw_norm_2.weight", c.d_model);
    g.router_scale = loadNorm(r, p + "ffn_gate_inp.scale", c.d_model);
    g.down_exps_scale = loadNorm(r, p + "ffn_down_exps.scale", c.n_experts);
    g.post_ffw_norm_2 = loadNorm(r, p + "post_ffw_norm_2.weight", c.d_model);
    g.post_ffw_norm = loadNorm(r, p + "post_ffw_norm.weight", c.d_model);
    const TensorInfo *t = r.data.find(p + "layer_output_scale.weight");
    if (t && (t->type == 0 || t->type == 1) && t->n_elements() == 1) g.layer_output_scale = loadNorm(r, t->name, 1)[0];
    return g;
}

}  // namespace gguf
}  // namespace llmtoy
