// llmtoy_ops.hpp -- C++ host layer over the C ABI (include/llmtoy_hip.h) that
// mirrors llmtoy-zig's op-level interface on the decode path, so a caller of
// the reference's ops finds the same names, argument meaning and error
// behaviour:
//
//   RawMatrix                      model/model_weights.zig:17-22
//   quantMatvec(out, mat, vec)     ops/math.zig:133-171 (one matvec; the
//                                  device copy of mat is made on first use
//                                  and cached by data pointer, the way
//                                  GpuWeights uploads at load time)
//   moeForward(out, router_w, gate_up, down, x, n_experts_used, d_expert)
//                                  ops/moe.zig:18-77 (accumulates into out)
//   MatvecSession::initFromRaw     gpu/matvec.zig:564-577 (nullopt for a
//                                  type the device path does not cover)
//   GpuWeights::runExpertBatch     gemma4/gpu_weights.zig:2748-3149
//                                  (throws Error::ExpertNotOnGpu when the
//                                  experts are not on the device, which the
//                                  caller answers with its CPU loop,
//                                  gemma4/forward.zig:434-480)
//   rmsnorm, rmsnormWeightedAndRawScaled
//                                  ops/math.zig:19-25, 42-48, 51-82
//   MoeTailParams                  gemma4/gpu_weights.zig:100-109
//   GpuWeights::runMoeBlock        runExpertBatch with the GPU router and
//                                  the MoE residual tail (gpu_weights.zig:
//                                  2748-3149, 3349-3410; the CPU order of
//                                  gemma4/forward.zig:403-497)
//
// Zig error unions become llmtoy::Exception carrying an Error kind; the
// reference's std.debug.panic on an unsupported type (math.zig:206, 223)
// becomes Error::Unsupported.  Header-only; link with -lllmtoy_hip.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

#include "llmtoy_hip.h"

namespace llmtoy {

// GgmlType ids (gguf/types.zig:23-53) of the formats on this path.
enum class GgmlType : uint32_t {
    f32 = 0, f16 = 1, q5_0 = 6, q5_1 = 7, q8_0 = 8, q3_k = 11, q4_k = 12, q6_k = 14, iq4_nl = 20
};

enum class Error { Unsupported, Invalid, NotOnGpu, ExpertNotOnGpu, Device, OutOfMemory };

class Exception : public std::runtime_error {
   public:
    Exception(Error kind, int status, const std::string &msg) : std::runtime_error(msg), kind(kind), status(status) {}
    Error kind;
    int status;
};

inline Error error_of(int status) {
    switch (status) {
    case LT_ERR_UNSUPPORTED: return Error::Unsupported;
    case LT_ERR_INVALID: return Error::Invalid;
    case LT_ERR_OOM: return Error::OutOfMemory;
    default: return Error::Device;
    }
}

// model/model_weights.zig:17-22: a zero-copy view of GGUF tensor bytes.
// For the flattened 3-D expert tensors rows = n_experts * rows_per_expert
// (gemma4/loader.zig:277-292).
struct RawMatrix {
    const uint8_t *data;
    size_t size;  // bytes
    GgmlType type;
    size_t rows;
    size_t cols;
};

// ops/math.zig:194-208
inline size_t rowBytes(GgmlType t, size_t cols) {
    switch (t) {
    case GgmlType::f32: return cols * 4;
    case GgmlType::f16: return cols * 2;
    case GgmlType::q8_0: return (cols / 32) * 34;
    case GgmlType::q4_k: return (cols / 256) * 144;
    case GgmlType::q6_k: return (cols / 256) * 210;
    case GgmlType::q5_0: return (cols / 32) * 22;
    case GgmlType::q5_1: return (cols / 32) * 24;
    case GgmlType::iq4_nl: return (cols / 32) * 18;
    case GgmlType::q3_k: return (cols / 256) * 110;
    }
    throw Exception(Error::Unsupported, LT_ERR_UNSUPPORTED, "unsupported quant type in rowBytes");
}

// One device context (GpuContext, gpu/context.zig:270-).  Owns the device
// copies of the matrices it has seen.
class GpuContext {
   public:
    explicit GpuContext(int device = 0) {
        int rc = lt_init(device, &ctx_);
        if (rc != LT_OK) throw Exception(Error::Device, rc, "lt_init failed (no usable device)");
    }
    ~GpuContext() {
        for (auto &kv : cache_) lt_tensor_free(ctx_, kv.second);
        lt_destroy(ctx_);
    }
    GpuContext(const GpuContext &) = delete;
    GpuContext &operator=(const GpuContext &) = delete;

    lt_ctx *raw() { return ctx_; }

    void check(int rc) const {
        if (rc != LT_OK) throw Exception(error_of(rc), rc, lt_last_error(ctx_));
    }

    // The device copy of m viewed as n_experts matrices of rows/n_experts
    // rows (uploaded on first use, cached by data pointer and shape).  As in
    // the reference (the GGUF mmap must outlive the weights,
    // model/model_weights.zig:11), the host bytes must stay alive and
    // unchanged while the context may use them; call forget() before
    // freeing or rewriting a buffer that was passed in.
    const lt_tensor *tensor(const RawMatrix &m, size_t n_experts = 1) {
        const Key key{m.data, m.rows, m.cols, n_experts};
        auto it = cache_.find(key);
        if (it != cache_.end()) return it->second;
        lt_tensor *t = nullptr;
        check(lt_tensor_upload(ctx_, m.data, m.rows * rowBytes(m.type, m.cols), (uint32_t)m.type, m.rows / n_experts,
                               m.cols, n_experts, &t));
        cache_[key] = t;
        return t;
    }

    // Drops (and frees) every device copy made from host bytes at data.
    void forget(const void *data) {
        for (auto it = cache_.begin(); it != cache_.end();) {
            if (it->first.data == data) {
                lt_tensor_free(ctx_, it->second);
                it = cache_.erase(it);
            } else {
                ++it;
            }
        }
    }

   private:
    struct Key {
        const uint8_t *data;
        size_t rows, cols, n_experts;
        bool operator<(const Key &o) const {
            if (data != o.data) return data < o.data;
            if (rows != o.rows) return rows < o.rows;
            if (cols != o.cols) return cols < o.cols;
            return n_experts < o.n_experts;
        }
    };
    lt_ctx *ctx_ = nullptr;
    std::map<Key, lt_tensor *> cache_;
};

// ops/math.zig:133-171: out[rows] = mat . vec (fp32 activations).  The
// reference's row_buf scratch argument has no device counterpart.
inline void quantMatvec(GpuContext &g, float *out, const RawMatrix &mat, const float *vec) {
    g.check(lt_matvec(g.raw(), out, g.tensor(mat), vec, LT_HOST_IO));
}

// ops/moe.zig:18-77: route x through the top n_experts_used experts and
// accumulate the weighted expert outputs into out (the caller zeroes it).
// Same semantics as the reference: softmax over all router logits, top-k
// with the lowest index winning ties, weights not renormalised, SiLU.
// deterministic: add the expert outputs in slot order (bit-identical run to
// run); otherwise the device adds them in arrival order.
inline void moeForward(GpuContext &g, float *out, const RawMatrix &router_w, const RawMatrix &gate_up,
                       const RawMatrix &down, const float *x, size_t n_experts_used, size_t d_expert,
                       bool deterministic = false) {
    const size_t n_experts = router_w.rows;
    if (gate_up.rows != n_experts * 2 * d_expert || down.rows % n_experts)
        throw Exception(Error::Invalid, LT_ERR_INVALID, "moeForward: expert tensor shapes do not match the router");
    const lt_tensor *r = g.tensor(router_w);
    const lt_tensor *gu = g.tensor(gate_up, n_experts);
    const lt_tensor *dn = g.tensor(down, n_experts);
    g.check(lt_moe_forward(g.raw(), out, x, r, nullptr, gu, dn, nullptr, nullptr, nullptr, (uint32_t)n_experts_used,
                           (uint32_t)d_expert, LT_ACT_SILU,
                           LT_HOST_IO | LT_MOE_ACCUMULATE | (deterministic ? LT_MOE_DETERMINISTIC : 0u), nullptr,
                           nullptr));
}

// ops/math.zig:19-25 (rmsnorm) and 42-48 (rmsnormRaw: weight == nullptr) on
// host vectors of n floats.  precise: the reference's index-order sum of
// squares (bit-exact with the CPU code); otherwise a fixed tree order.
inline void rmsnorm(GpuContext &g, float *out, const float *x, const float *weight, size_t n, float eps,
                    bool precise = false) {
    g.check(lt_rmsnorm(g.raw(), out, x, weight, 1, (uint32_t)n, eps, LT_HOST_IO | (precise ? LT_NORM_PRECISE : 0u)));
}

// ops/math.zig:51-82
inline void rmsnormWeightedAndRawScaled(GpuContext &g, float *weighted_out, float *raw_scaled_out, const float *x,
                                        const float *weight, const float *raw_scale, float raw_global_scale,
                                        size_t n, float eps, bool precise = false) {
    g.check(lt_rmsnorm_weighted_raw_scaled(g.raw(), weighted_out, raw_scaled_out, x, weight, raw_scale,
                                           raw_global_scale, (uint32_t)n, eps,
                                           LT_HOST_IO | (precise ? LT_NORM_PRECISE : 0u)));
}

// gemma4/gpu_weights.zig:100-109: what the MoE residual tail needs.
struct MoeTailParams {
    float eps;
    float *x;                 // residual stream, updated in place
    const float *dense_ffn;   // dense FFN output after post_ffw_norm_1
    float layer_output_scale;
};

// The per-layer vectors of the Gemma4 MoE block (gemma4/weights.zig).
struct Gemma4MoeNorms {
    const float *pre_ffw_norm_2, *router_scale, *down_exps_scale, *post_ffw_norm_2, *post_ffw_norm;
};

// gpu/matvec.zig:497-647: one matrix resident on the device.
class MatvecSession {
   public:
    // nullopt when the device path does not cover the type (the reference
    // returns null and the caller stays on the CPU, matvec.zig:564-577).
    static std::optional<MatvecSession> initFromRaw(GpuContext &g, const RawMatrix &m) {
        switch (m.type) {
        case GgmlType::f32: case GgmlType::q8_0: case GgmlType::q4_k: case GgmlType::q6_k:
        case GgmlType::q5_0: case GgmlType::q5_1: case GgmlType::iq4_nl: case GgmlType::q3_k: break;
        default: return std::nullopt;
        }
        try {
            return MatvecSession(g, g.tensor(m), m.rows);
        } catch (const Exception &e) {
            if (e.kind == Error::Unsupported) return std::nullopt;
            throw;
        }
    }
    void run(const float *vec, float *out) { g_->check(lt_matvec(g_->raw(), out, t_, vec, LT_HOST_IO)); }
    size_t rows() const { return rows_; }

   private:
    MatvecSession(GpuContext &g, const lt_tensor *t, size_t rows) : g_(&g), t_(t), rows_(rows) {}
    GpuContext *g_;
    const lt_tensor *t_;
    size_t rows_;
};

// gemma4/gpu_weights.zig: the expert tensors of one layer on the device.
class GpuWeights {
   public:
    GpuWeights(GpuContext &g, const RawMatrix &gate_up_exps, const RawMatrix &down_exps, size_t n_experts,
               size_t d_expert)
        : g_(&g), n_experts_(n_experts), d_expert_(d_expert), down_cols_(down_exps.cols) {
        try {
            gate_up_ = g.tensor(gate_up_exps, n_experts);
            down_ = g.tensor(down_exps, n_experts);
            auto ok = [](GgmlType t) {
                return t == GgmlType::q4_k || t == GgmlType::q3_k || t == GgmlType::q5_0 || t == GgmlType::q5_1 ||
                       t == GgmlType::iq4_nl;
            };
            on_gpu_ = ok(gate_up_exps.type) && ok(down_exps.type);
        } catch (const Exception &e) {
            if (e.kind != Error::Unsupported) throw;
            on_gpu_ = false;  // stays on the CPU path
        }
    }

    // gpu_weights.zig:2748-2761: run the selected experts for one token and
    // accumulate sum_k down_exps_scale[e_k] * router_out[e_k] * expert_k(moe_in)
    // into moe_buf.  act: LT_ACT_SILU or LT_ACT_GELU_TANH.
    void runExpertBatch(const size_t *top_idx, size_t n, const float *down_exps_scale, const float *moe_in,
                        const float *router_out, float *moe_buf, uint32_t act = LT_ACT_GELU_TANH) {
        if (!on_gpu_) throw Exception(Error::ExpertNotOnGpu, LT_ERR_UNSUPPORTED, "experts are not on the GPU");
        std::vector<uint32_t> ids(n);
        std::vector<float> w(n);
        for (size_t k = 0; k < n; k++) {
            ids[k] = (uint32_t)top_idx[k];
            w[k] = (down_exps_scale ? down_exps_scale[top_idx[k]] : 1.0f) * router_out[top_idx[k]];
        }
        std::vector<float> h(n * down_cols_);
        g_->check(lt_expert_gate_up_id(g_->raw(), gate_up_, moe_in, ids.data(), (uint32_t)n, (uint32_t)d_expert_,
                                       (uint32_t)down_cols_, act, h.data(), LT_HOST_IO));
        g_->check(lt_expert_down_id(g_->raw(), down_, h.data(), ids.data(), w.data(), (uint32_t)n, moe_buf,
                                    LT_HOST_IO | LT_MOE_ACCUMULATE));
    }

    // The whole MoE block of one token on the device: router-input prep,
    // routerTopKSoftmax on router_w, the selected experts scaled by
    // down_exps_scale, and the tail (post_ffw_norm_2, + dense FFN,
    // post_ffw_norm, residual, layer_output_scale) -- runExpertBatch with the
    // GPU router and MoeTailParams.  tail.x is updated in place; top_idx and
    // router_out_sel (may be null) receive the selection and its softmax
    // probabilities.
    void runMoeBlock(const RawMatrix &router_w, const Gemma4MoeNorms &nm, size_t n_experts_used,
                     const MoeTailParams &tail, size_t *top_idx = nullptr, float *router_out_sel = nullptr,
                     uint32_t act = LT_ACT_GELU_TANH, bool precise = false) {
        if (!on_gpu_) throw Exception(Error::ExpertNotOnGpu, LT_ERR_UNSUPPORTED, "experts are not on the GPU");
        std::vector<uint32_t> ids(n_experts_used);
        g_->check(lt_gemma4_moe_block(g_->raw(), tail.x, tail.dense_ffn, g_->tensor(router_w), gate_up_, down_,
                                      nm.pre_ffw_norm_2, nm.router_scale, nm.down_exps_scale, nm.post_ffw_norm_2,
                                      nm.post_ffw_norm, tail.layer_output_scale, tail.eps, (uint32_t)n_experts_used,
                                      (uint32_t)d_expert_, act, LT_HOST_IO | (precise ? LT_NORM_PRECISE : 0u),
                                      ids.data(), router_out_sel));
        if (top_idx)
            for (size_t i = 0; i < n_experts_used; i++) top_idx[i] = ids[i];
    }

   private:
    GpuContext *g_;
    const lt_tensor *gate_up_ = nullptr, *down_ = nullptr;
    size_t n_experts_, d_expert_, down_cols_;
    bool on_gpu_ = false;
};

}  // namespace llmtoy
