// lt_internal.h -- shared definitions of the gfx950 decode path.
//
// Device layout of an uploaded tensor ("planar": the GGUF block fields are
// split into separate planes so that every lane load is a naturally aligned,
// fully coalesced 16-byte vector; total bytes equal the GGUF byte count):
//
//   Q4_K  (144 B / 256 elements, quant/dequant.zig:136-155)
//         hdr plane  [R][nsb][16]  = d(f16) dmin(f16) scales[12]
//         qs  plane  [R][nsb][128] = 4-bit quants, ggml order
//   Q8_0  (34 B / 32 elements, dequant.zig:31-40)
//         qs  plane  [R][nb][32]   = int8 quants
//         d   plane  [R][nb]       = f16 scales
//   Q6_K  (210 B / 256 elements, dequant.zig:219-235)
//         ql plane [R][nsb][128], qh plane [R][nsb][64],
//         sc plane [R][nsb][16] (int8), d plane [R][nsb] (f16)
//   F32   [R][cols]
//
// R = n_experts * rows (expert e owns rows [e*rows, (e+1)*rows)).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stddef.h>

namespace lt {

constexpr int kWave = 64;

struct DevTensor {
    uint32_t type;      // GgmlType id
    size_t rows;        // rows per expert
    size_t cols;        // GGUF row length (elements)
    size_t n_experts;   // 1 for 2-D tensors
    size_t total_rows;  // n_experts * rows
    size_t bytes;       // == GGUF byte count
    uint8_t *base;      // device allocation (256-byte aligned)
    // plane pointers (into base)
    const uint8_t *p0;  // Q4_K hdr | Q8_0 qs | Q6_K ql | F32 data
    const uint8_t *p1;  // Q4_K qs  | Q8_0 d  | Q6_K qh
    const uint8_t *p2;  // Q6_K sc
    const uint8_t *p3;  // Q6_K d
    size_t blocks_per_row;  // nsb (K-quants) or nb (Q8_0)
};

// ---------------------------------------------------------------- helpers
// Exact IEEE binary16 -> binary32 (v_cvt_f32_f16 keeps f16 subnormals), the
// behaviour of quant/dequant.zig:302-305.
__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
    return __half2float(__ushort_as_half((unsigned short)(bits16 & 0xffffu)));
}

// Q4_K packed 6-bit scale/min of sub-block j (get_scale_min_k4,
// quant/dequant.zig:291-300); s0 = scales[0..3], s1 = [4..7], s2 = [8..11]
// as little-endian dwords.
__device__ __forceinline__ void q4k_scale_min(int j, uint32_t s0, uint32_t s1, uint32_t s2, float &sc,
                                              float &mn) {
    if (j < 4) {
        sc = (float)((s0 >> (8 * j)) & 63u);
        mn = (float)((s1 >> (8 * j)) & 63u);
    } else {
        int i = j - 4;
        uint32_t b8 = (s2 >> (8 * i)) & 0xffu;      // scales[j+4]
        uint32_t blo = (s0 >> (8 * i)) & 0xffu;     // scales[j-4]
        uint32_t bhi = (s1 >> (8 * i)) & 0xffu;     // scales[j]
        sc = (float)((b8 & 15u) | ((blo >> 6) << 4));
        mn = (float)((b8 >> 4) | ((bhi >> 6) << 4));
    }
}

// Sum over groups of G lanes (G a power of two <= 64), result in every lane
// of the group.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ float act_silu(float g) { return g / (1.0f + __expf(-g)); }

__device__ __forceinline__ float act_gelu_tanh(float g) {
    const float c = 0.7978845608028654f;
    float inner = c * (g + 0.044715f * g * g * g);
    return 0.5f * g * (1.0f + tanhf(inner));
}

__device__ __forceinline__ float act_apply(uint32_t act, float g) {
    return act == 1u ? act_gelu_tanh(g) : act_silu(g);
}

__device__ __forceinline__ uint4 ldg16(const uint8_t *p) { return *reinterpret_cast<const uint4 *>(p); }
__device__ __forceinline__ float4 ldg16f(const float *p) { return *reinterpret_cast<const float4 *>(p); }

}  // namespace lt

// --------------------------------------------------------------- launchers
// Each returns hipSuccess or the launch error.  All shapes are validated by
// the caller (lt_api.cpp) before these are called.
namespace lt {
hipError_t launch_matvec_q4k(const DevTensor &W, size_t row0, size_t nrows, const float *x, float *y,
                             hipStream_t s);
hipError_t launch_matvec_q8_0(const DevTensor &W, const float *x, float *y, hipStream_t s);
hipError_t launch_matvec_q6k(const DevTensor &W, const float *x, float *y, hipStream_t s);
hipError_t launch_matvec_f32(const DevTensor &W, const float *x, float *y, hipStream_t s);
hipError_t launch_gate_up_q8_0(const DevTensor &Wg, const DevTensor &Wu, const float *x, uint32_t act,
                               float *h, hipStream_t s);
hipError_t launch_router_f32(const DevTensor &R, const float *x, const float *bias, float *logits,
                             hipStream_t s);
hipError_t launch_router_q8_0(const DevTensor &R, const float *x, const float *bias, float *logits,
                              hipStream_t s);
hipError_t launch_topk_softmax(const float *logits, uint32_t n, uint32_t k, uint32_t norm, uint32_t *ids,
                               float *w, float *scores, hipStream_t s);
hipError_t launch_expert_gate_up_q4k(const DevTensor &GU, const float *x, const uint32_t *ids, uint32_t k,
                                     uint32_t d_expert, uint32_t down_cols, uint32_t act, float *h,
                                     hipStream_t s);
hipError_t launch_expert_down_q4k(const DevTensor &D, const float *h, const uint32_t *ids, const float *w,
                                  uint32_t k, const float *base, int accumulate, float *out, hipStream_t s);
}  // namespace lt
