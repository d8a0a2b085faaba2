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
//   Q5_0  qs [R][nb][16], qh [R][nb][4], d [R][nb]        (22 B / 32)
//   Q5_1  qs [R][nb][16], qh [R][nb][4], d|m [R][nb][2]   (24 B / 32)
//   IQ4_NL qs [R][nb][16], d [R][nb]                      (18 B / 32)
//   Q3_K  qs [R][nsb][64], hmask [R][nsb][32], scales [R][nsb][12],
//         d [R][nsb]                                      (110 B / 256)
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

// Hides the known-zero bits of a value from the optimiser, so that byte
// extractions of a masked word stay single v_cvt_f32_ubyte{0..3} ops
// instead of being rewritten into v_bfe + v_cvt_f32_ubyte0.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

// Cross-lane moves.  DPP controls (gfx9 encoding): quad_perm [1,0,3,2] =
// 0xB1, [2,3,0,1] = 0x4E, row_ror:n = 0x120 + n, row_half_mirror = 0x141.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
// lane i <- lane i ^ 16 (within each 32-lane half)
__device__ __forceinline__ float xor16(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401f));
}
// v_permlane32_swap exchanges the two 32-lane halves between its operands;
// with both operands equal, one of its two results holds the value of lane
// i ^ 32 in every lane.  p32_first(lane) tells which one (computed once).
__device__ __forceinline__ bool p32_first(int lane) {
    auto pr = __builtin_amdgcn_permlane32_swap((unsigned)lane, (unsigned)lane, false, false);
    return (int)pr[0] != lane;
}
__device__ __forceinline__ float xor32(float v, bool first) {
    auto pr = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(first ? pr[0] : pr[1]);
}

// Workgroups of 256 threads that the persistent streaming kernels launch at
// most: 256 CUs x 4 workgroups (their occupancy at ~120 VGPRs).
constexpr int kStreamBlocks = 1024;

// Sum over each aligned group of G consecutive lanes (G = 4, 8, 16, 32 or
// 64), total in every lane of the group, with DPP row operations (and
// ds_swizzle / v_permlane32_swap across rows): no LDS round trips.
template <int G>
__device__ __forceinline__ float group_sum_dpp(float t, bool first) {
    static_assert(G == 4 || G == 8 || G == 16 || G == 32 || G == 64, "G");
    if (G >= 64) t += xor32(t, first);
    if (G >= 32) t += xor16(t);
    if (G >= 16) t += dpp<0x128>(t);  // row_ror:8 (lane i ^ 8 within a row)
    if (G >= 8) t += dpp<0x141>(t);   // row_half_mirror
    t += dpp<0x4E>(t);                // quad_perm [2,3,0,1]
    t += dpp<0xB1>(t);                // quad_perm [1,0,3,2]
    return t;
}

// Sums V values (V = 1, 2, 4 or 8) over the 64 lanes of a wavefront with
// log2(V) exchange steps (each halves the values a lane carries) followed by
// a plain reduction over the remaining lane bits.  Returns, in every lane,
// the total of value index lane >> (6 - log2 V).
template <int V>
__device__ __forceinline__ float wave_sum_transposed(float (&v)[V], int lane, bool first) {
    static_assert(V == 1 || V == 2 || V == 4 || V == 8, "V");
    float a[V];
#pragma unroll
    for (int i = 0; i < V; i++) a[i] = v[i];
    int n = V;
    if (n > 1) {  // lane bit 5
        const bool hi = lane & 32;
#pragma unroll
        for (int i = 0; i < V / 2; i++) {
            const float send = hi ? a[i] : a[i + V / 2], keep = hi ? a[i + V / 2] : a[i];
            a[i] = keep + xor32(send, first);
        }
        n = V / 2;
    }
    if (n > 1) {  // lane bit 4
        const bool hi = lane & 16;
#pragma unroll
        for (int i = 0; i < V / 4; i++) {
            const float send = hi ? a[i] : a[i + V / 4], keep = hi ? a[i + V / 4] : a[i];
            a[i] = keep + xor16(send);
        }
        n = V / 4;
    }
    if (n > 1) {  // lane bit 3 (row_ror:8 pairs i with i ^ 8 inside a 16-lane row)
        const bool hi = lane & 8;
        const float send = hi ? a[0] : a[1], keep = hi ? a[1] : a[0];
        a[0] = keep + dpp<0x128>(send);
    }
    float t = a[0];
    if (V == 8) {  // lane bits 0..2
        t += dpp<0xB1>(t);
        t += dpp<0x4E>(t);
        t += dpp<0x141>(t);
    } else {  // lane bits 0..3, then 4 and 5 as needed
        t += dpp<0x128>(t);
        t += dpp<0x124>(t);
        t += dpp<0x122>(t);
        t += dpp<0x121>(t);
        if (V <= 2) t += xor16(t);
        if (V == 1) t += xor32(t, first);
    }
    return t;
}

// Sums V values (V = 1, 2, 4 or 8) over each aligned group of 8 lanes.
// Returns, in lane g*8 + j, the group's total of value index j * V / 8
// (for V = 8: value j).
template <int V>
__device__ __forceinline__ float group8_sum_transposed(float (&v)[V], int lane) {
    static_assert(V == 1 || V == 2 || V == 4 || V == 8, "V");
    float a[V];
#pragma unroll
    for (int i = 0; i < V; i++) a[i] = v[i];
    int n = V;
    if (n > 1) {  // lane bit 2: row_half_mirror pairs i with 7 - i
        const bool hi = lane & 4;
#pragma unroll
        for (int i = 0; i < V / 2; i++) {
            const float send = hi ? a[i] : a[i + V / 2], keep = hi ? a[i + V / 2] : a[i];
            a[i] = keep + dpp<0x141>(send);
        }
        n = V / 2;
    } else {
        a[0] += dpp<0x141>(a[0]);
    }
    if (n > 1) {  // lane bit 1
        const bool hi = lane & 2;
#pragma unroll
        for (int i = 0; i < V / 4; i++) {
            const float send = hi ? a[i] : a[i + V / 4], keep = hi ? a[i + V / 4] : a[i];
            a[i] = keep + dpp<0x4E>(send);
        }
        n = V / 4;
    } else {
        a[0] += dpp<0x4E>(a[0]);
    }
    if (n > 1) {  // lane bit 0
        const bool hi = lane & 1;
        const float send = hi ? a[0] : a[1], keep = hi ? a[1] : a[0];
        a[0] = keep + dpp<0xB1>(send);
    } else {
        a[0] += dpp<0xB1>(a[0]);
    }
    return a[0];
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

// The prefill's f16 copy of X (X rows scaled into f16's range, K in the
// order the f16 dequantisation produces): a row with max |x| = m > 0 is
// divided by 2^e = 2^ilogb(m), so that its largest element lies in [1, 2)
// (exact: a power of two), whether m is large or small; e is kept in
// [-100, 127] (2^-e stays finite for every fp32 row); rows of zeros and
// rows holding inf or NaN pass unscaled (e = 0).  The activations between
// the two GEMMs are kept divided by 2^(2e) (see k_prefill_gate_up), which
// holds them inside f16's range whatever the row's magnitude.
__device__ __forceinline__ int prefill_x_exp(float m) {
    int e = 0;
    if (m > 0.0f && m <= 3.4e38f) e = min(max(ilogbf(m), -100), 127);
    return e;
}

// Elements i..i+7 of a row (i % 8 == 0) times inv as f16 at dst + i, each
// aligned 4 in the order (0, 2, 1, 3).
__device__ __forceinline__ void prefill_x_store8(const float *xr, float inv, _Float16 *hr, int i) {
    typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 h8;
    const float4 a = ldg16f(xr + i), b = ldg16f(xr + i + 4);
    h8 o;
    o[0] = (_Float16)(a.x * inv); o[1] = (_Float16)(a.z * inv); o[2] = (_Float16)(a.y * inv); o[3] = (_Float16)(a.w * inv);
    o[4] = (_Float16)(b.x * inv); o[5] = (_Float16)(b.z * inv); o[6] = (_Float16)(b.y * inv); o[7] = (_Float16)(b.w * inv);
    *reinterpret_cast<h8 *>(hr + i) = o;
}
// 16-byte load with the non-temporal hint (global_load_dwordx4 ... nt), for
// weight streams that a launch reads once (the Q6_K stream: 23.6 -> 22.7 us
// on 128 MB).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ldg16_nt(const uint8_t *p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// ---------------------------------------------------------------- hand-over words
// The single-launch kernels (lt_moe_fused.hip, lt_ffn_fused.hip) pass
// results between workgroups as 64-bit words, a 32-bit payload beside the
// 32-bit launch epoch, written and read with relaxed atomics: a reader waits
// until every word it needs carries the current epoch, so the memory never
// needs clearing between launches.
__device__ __forceinline__ void hand_put(uint64_t *p, uint32_t v, uint32_t ep) {
    __hip_atomic_store(p, (uint64_t)v | ((uint64_t)ep << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A word read only by blocks of the writer's own group.  With local set
// (blocks with equal bid % 8 share an XCD: checked once per context by
// probe_xcd_groups), a workgroup-scope store leaves it dirty in that XCD's
// L2, where the readers' agent-scope loads find it: about 0.2 us instead
// of the 0.6 us a round trip through memory takes.  Otherwise agent scope.
__device__ __forceinline__ void hand_put_group(uint64_t *p, uint32_t v, uint32_t ep, int local) {
    const uint64_t w = (uint64_t)v | ((uint64_t)ep << 32);
    if (local)
        __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    else
        __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t hand_get(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool tag_is(uint64_t w, uint32_t ep) { return (uint32_t)(w >> 32) == ep; }

// The context's host-mapped error words (16): [0] code bits (the fused
// kernels' timed-out waits below 0x100), [2..6] the first wait's details,
// [8] the prefill's count of saturated f16 activations (code bit 0x100);
// 0x400: a prefill down block's wait for its chunk's activations.
constexpr uint32_t kErrCodePrefillSat = 0x100u;
constexpr int kErrPrefillSat = 8;
constexpr uint32_t kErrCodePrefillWait = 0x400u;
__device__ __forceinline__ void report_timeout(uint32_t *err, uint32_t code) {
    __hip_atomic_fetch_or(err, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
// The first timed-out wait of a call also leaves what it saw in err[2..6]:
// block + 1, site code, the word index, the word's epoch tag (or count)
// seen, and the epoch expected.
__device__ __forceinline__ void report_detail(uint32_t *err, int bid, uint32_t code, uint32_t index, uint32_t seen,
                                              uint32_t ep) {
    uint32_t zero = 0;
    if (__hip_atomic_compare_exchange_strong(err + 2, &zero, (uint32_t)bid + 1u, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_SYSTEM)) {
        __hip_atomic_store(err + 3, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(err + 4, index, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(err + 5, seen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(err + 6, ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// The launch counter of block bid: epoch_peek reads it (issued early, its
// value used late), epoch_commit stores the incremented value; the new value
// is the launch epoch.
__device__ __forceinline__ uint32_t epoch_peek(const uint32_t *counters, int bid) {
    return __hip_atomic_load(counters + bid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t epoch_commit(uint32_t *counters, int bid, uint32_t c) {
    __hip_atomic_store(counters + bid, c + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return c + 1u;
}

}  // namespace lt

namespace lt {
// ------------------------------------------- host <-> device tensor copies
// (lt_upload.hip) Raw GGUF blocks cross PCIe in kUpChunk pieces staged in
// pinned host memory, up to kUpWorkers pieces in flight on their own
// streams; a device kernel splits each piece into the planes.
constexpr int kUpWorkers = 8;
constexpr int kUpSlots = 2 * kUpWorkers;  // two staging slots per worker
constexpr size_t kUpChunk = 4u << 20;     // bytes per staging slot
struct UploadStaging {
    int workers = 0;  // workers whose stream and slots exist
    hipStream_t st[kUpWorkers] = {};
    uint8_t *pinned[kUpSlots] = {};
    uint8_t *dev[kUpSlots] = {};
    hipEvent_t ev[kUpSlots] = {};
};
// t.base must hold t.bytes; src holds the tensor's GGUF blocks.  Returns
// after every copy has finished.
hipError_t upload_planar(UploadStaging &S, int device, const DevTensor &t, const uint8_t *src);
// The inverse: the tensor's GGUF blocks into dst (t.bytes bytes).
hipError_t download_planar(UploadStaging &S, const DevTensor &t, uint8_t *dst);
void free_staging(UploadStaging &S);

// ------------------------------------------------------ norms (lt_norm.hip)
constexpr int kMaxNormCols = 16384;  // row staged in LDS (64 KiB)
// op 0: out = rmsnorm(a, w) (w null: no weight); 1: out = rmsnorm(a + b, w);
// 2: out = weighted, out2 = raw-scaled (w2 = raw_scale, scale = global);
// 3: MoE tail, out = x in place, a = moe, b = dense, w2 = post_ffw_norm_2,
// w = post_ffw_norm, scale = layer_output_scale.  One workgroup per row.
hipError_t launch_norm(int op, const float *a, const float *b, const float *w, const float *w2, float *out,
                       float *out2, int rows, int n, float eps, float scale, int precise, int one_plus_w,
                       hipStream_t s);

// --------------------------------------------------------------- launchers
// Each returns hipSuccess or the launch error.  All shapes are validated by
// the caller (lt_api.cpp) before these are called.
hipError_t launch_matvec_q4k(const DevTensor &W, size_t row0, size_t nrows, const float *x, float *y,
                             hipStream_t s);
hipError_t launch_matvec_q8_0(const DevTensor &W, const float *x, float *y, hipStream_t s);
hipError_t launch_matvec_q6k(const DevTensor &W, const float *x, float *y, hipStream_t s);
hipError_t launch_matvec_f32(const DevTensor &W, const float *x, float *y, hipStream_t s);
// Q5_0, Q5_1, IQ4_NL, Q3_K (lt_formats.hip)
hipError_t launch_matvec_fmt(const DevTensor &W, const float *x, float *y, hipStream_t s);
// Expert-indexed gate/up and down over those formats (lt_formats.hip); the
// down staging needs k * down_cols * 4 <= 64 KiB, x rows <= 16384 floats.
hipError_t launch_expert_gate_up_fmt(const DevTensor &GU, const float *x, const uint32_t *ids, uint32_t k,
                                     uint32_t d_expert, uint32_t down_cols, uint32_t act, float *h, hipStream_t s);
// The same, routing for itself: every block runs softmax + top-k over the
// router logits (n_experts <= 256) and block (0, 0) writes the selection to
// ids_out / w_out for the down kernel.
hipError_t launch_expert_gate_up_fmt_routed(const DevTensor &GU, const float *x, const float *logits, uint32_t k,
                                            uint32_t norm, uint32_t d_expert, uint32_t down_cols, uint32_t act,
                                            float *h, uint32_t *ids_out, float *w_out, hipStream_t s);
hipError_t launch_expert_down_fmt(const DevTensor &D, const float *h, const uint32_t *ids, const float *w,
                                  uint32_t k, const float *base, int accumulate, const float *dscale, float *out,
                                  hipStream_t s);
hipError_t launch_gate_up_q8_0(const DevTensor &Wg, const DevTensor &Wu, const float *x, uint32_t act,
                               float *h, hipStream_t s);
// Router logits (F32 or Q8_0 router, exact reference order) plus softmax /
// top-k in the same launch.  ticket: a zero-initialised counter owned by the
// caller, left at zero after every launch.  k = 0 computes logits only.
// Gemma4 router-input prep fused into the Q8_0 router (null raw_scale: off).
struct RouterPrep {
    const float *raw_scale;   // router_scale [cols]
    const float *weight;      // pre_ffw_norm_2 [cols]
    float *moe_in;            // [cols], written: (x * rms_inv) * weight
    float raw_global_scale;   // 1 / sqrt(cols)
    float eps;
};
hipError_t launch_router(const DevTensor &R, const float *x, const float *bias, float *logits, unsigned *ticket,
                         uint32_t k, uint32_t norm, uint32_t *ids, float *w, float *scores, hipStream_t s,
                         const RouterPrep *prep = nullptr);
// Router logits for T tokens (X [T][cols] -> logits [T][rows]) and per-token
// softmax + top-k (ids, w: [T][k]).
// Batched router logits and top-k of T tokens (prefill).  With the F32 tile
// kernel (cols % 256 == 0, at least 32 router rows) the router launch also
// writes the prefill's f16 X (Xh, row scales rs); *x_done reports whether
// it did.
hipError_t launch_router_batched(const DevTensor &R, const float *X, int T, const float *bias, float *logits,
                                 uint32_t k, uint32_t norm, uint32_t *ids, float *w, _Float16 *Xh, float *rs,
                                 bool *x_done, hipStream_t s);
// Batched prefill MoE (Q4_K experts), see lt_prefill.hip.  ws: workspace of
// prefill_workspace_bytes(T, k, E, F, D) bytes.
size_t prefill_workspace_bytes(int T, int k, int E, int F, int D);
// xcd_local (blocks with equal index % 8 share an XCD): both GEMMs in one
// launch, H handed over in the XCD's L2; else one launch each.
hipError_t launch_moe_prefill(const DevTensor &R, const DevTensor &GU, const DevTensor &Dn, const float *X, int T,
                              const float *bias, int k, int F, uint32_t act, uint32_t norm, void *ws, float *out,
                              uint32_t *out_ids, float *out_w, uint32_t *err, int xcd_local, hipStream_t s);
hipError_t launch_expert_gate_up_q4k(const DevTensor &GU, const float *x, const uint32_t *ids, uint32_t k,
                                     uint32_t d_expert, uint32_t down_cols, uint32_t act, float *h,
                                     hipStream_t s);
// Gate/up that routes for itself: every block runs softmax + top-k over the
// router logits (n_experts <= 256) and block (0, 0) writes the selection to
// ids_out / w_out for the down kernel.
hipError_t launch_expert_gate_up_q4k_routed(const DevTensor &GU, const float *x, const float *logits, uint32_t k,
                                            uint32_t norm, uint32_t d_expert, uint32_t down_cols, uint32_t act,
                                            float *h, uint32_t *ids_out, float *w_out, hipStream_t s);
hipError_t launch_expert_down_q4k(const DevTensor &D, const float *h, const uint32_t *ids, const float *w,
                                  uint32_t k, const float *base, int accumulate, float *out, hipStream_t s,
                                  const float *dscale = nullptr);

// The whole decode MoE layer in one launch (lt_moe_fused.hip): F32 or Q8_0
// router, Q4_K gate_up and down, optionally a Q8_0 shared dense FFN -- or a
// Q8_0 dense FFN alone.  The grid is always kFusedBlocks workgroups, which
// keeps the per-block launch counters equal.
constexpr int kFusedBlocks = 1024;
constexpr int kFusedMaxRouterBlocks = 64;  // E <= 256, 4 logits per block
constexpr int kLgCopy = kFusedMaxRouterBlocks * 16;  // words per copy of the logits (8 copies)
struct FusedPlan {
    bool ok;     // the shape fits the fused kernel
    int per;     // logits per lane in the top-k wavefront (2 or 4)
    int wide;    // expert gate/up rows of 9-16 super-blocks (two positions per lane)
    int qrouter; // Q8_0 router (dotQ8_0 order), else F32
    int NRg;     // router blocks per XCD group
    int rb;      // logit rows per router block (2, or 4 when the grid is full)
    int SPG;     // slots per XCD group (ceil(k / 8))
    int G;       // h groups of 16 per slot (down K / 16)
    int NDg;     // down blocks per slot
    int NCg;     // combining blocks per XCD group (deterministic combine only)
    int Ewait;   // logit rows published and waited for (>= E: placeholders cover start-value blocks)
    int shared;  // a shared FFN in the launch (blocks of its own)
    int gemma;   // the Gemma4 block around the layer (GemmaBlock; one tail block in XCD group 0)
    int fmt;     // APEX expert formats (Q3_K gate/up, IQ4_NL / Q5_0 / Q5_1 down): the format instance
    int NSg;     // shared gate/up blocks per XCD group (the shared down rows are in the down blocks)
    int sg_rows; // shared h rows per shared gate/up block (<= 32)
    size_t lds;  // dynamic LDS bytes per block
};
// The Gemma4 MoE block around the layer (gemma4/forward.zig:403-497) in the
// same launch: router input (x * (rms_inv / sqrt(n))) * raw_scale and
// expert input (x * rms_inv) * pre_ffw_norm_2 from one RMS of x (math.zig:
// 51-82, the tree order of the Q8_0 router's prep), down_exps_scale per
// expert, and the tail x = (x + rmsnorm(dense + rmsnorm(moe, w2), w)) *
// layer_output_scale (the tree order of the tail kernel).
struct GemmaBlock {
    const float *raw_scale, *pre_ffw_norm_2, *down_exps_scale, *dense, *post_ffw_norm_2, *post_ffw_norm;
    float *x;  // read as the layer's input, written by the tail
    float raw_global_scale, eps, layer_output_scale;
};
// A layer for the fused kernel.  MoE: R, GU, Dn set (E experts, k > 0),
// optionally a shared FFN SG, SU, SD (Q8_0, S rows) added to the experts'
// combine, or the Gemma4 block around it (gb: Q8_0 router, no shared FFN,
// atomic combine).  Dense FFN alone: R, GU, Dn null, k = 0, SG, SU, SD set.
struct FusedLayer {
    const DevTensor *R, *GU, *Dn;
    const DevTensor *SG, *SU, *SD;
    int E, D, F, Kd, k, S;
    int det;  // slot-order combine (combining blocks; no shared FFN)
    const GemmaBlock *gb = nullptr;
};
// Device memory the fused kernel hands results over through; zeroed once
// when allocated and never cleared again (words carry launch epochs).
struct FusedScratch {
    uint32_t *counters;  // [kFusedBlocks]
    uint64_t *lg;        // [8][kLgCopy] logit words, one copy per XCD group
    uint64_t *hl;        // [kFusedBlocks][16] h record lines
    uint64_t *pl;        // [4 * kFusedBlocks][16] partial-output lines
    uint32_t *err;       // host-mapped error word (device address)
    int xcd_local;       // blocks with equal index % 8 share an XCD (probe_xcd_groups)
    uint64_t *stamps = nullptr;  // LT_PROFILE=timeline: [kFusedBlocks][kStamps] phase stamps, else null
    uint64_t *shh = nullptr;     // shared FFN h words [kFusedMaxShared]
};
// Phase stamps of one launch (LT_PROFILE=timeline): thread 0 of block b
// writes stamps[b * kStamps + i], wall-clock ticks (100 MHz) at the end of
// phase i of its role, and stamps[b * kStamps + kStamps - 1] = role | slot
// << 8 | XCD << 16 | HW_ID << 32 (role 0 none, 1 router, 2 gate/up, 3 down,
// 4 combine, 5 shared-FFN gate/up, 6 shared-FFN down, 7 Gemma4 tail; HW_ID
// the hardware register naming the CU, shader array and engine the block
// ran on).
constexpr int kStamps = 8;
enum : int { kStampStart = 0 };
// router: 1 first row chunk in, 2 logit published, 3 all row terms in (Q8_0
// router); gate/up: 1 logits seen, 2 expert known, 3 dot products done, 4 h
// record published; down: 1 logits seen, 2 weight loads issued, 3 h records
// read, 4 adds issued, with a shared FFN 5 its h slice read, 6 its rows
// added; combine: 1 rows written; shared gate/up: 1 h rows out; shared
// down only (a group without a slot): 5 h slice read, 6 rows added; Gemma4
// tail: 1 down blocks done, 2 x written
// Byte layout of that hand-over memory (a context's own allocation, or the
// library's static scratch in lt_noalloc.hip): launch counters, 8 logit
// copies, h record lines, partial-output lines, the XCD probe's ids, and
// the routing outputs (ids, weights) of the allocation-free entry point.
constexpr size_t kFusedCntOff = 0;
constexpr size_t kFusedLgOff = kFusedCntOff + (size_t)kFusedBlocks * 4;
constexpr size_t kFusedHlOff = kFusedLgOff + (size_t)8 * kLgCopy * 8;
constexpr size_t kFusedPlOff = kFusedHlOff + (size_t)kFusedBlocks * 16 * 8;
constexpr size_t kFusedXccOff = kFusedPlOff + (size_t)kFusedBlocks * 4 * 16 * 8;
constexpr size_t kFusedIdsOff = kFusedXccOff + (size_t)kFusedBlocks * 4;
constexpr size_t kFusedWOff = kFusedIdsOff + 256;
// The shared FFN's h values ([S] hand-over words, S <= kFusedMaxShared)
// follow.
constexpr int kFusedMaxShared = 4096;
constexpr size_t kFusedShOff = kFusedWOff + 256;
constexpr size_t kFusedScratchBytes = kFusedShOff + (size_t)kFusedMaxShared * 8;  // 762,368 B
// counters, lg, hl, pl at base; err and xcd_local are the caller's
inline FusedScratch fused_scratch_at(uint8_t *base, uint32_t *err, int xcd_local) {
    FusedScratch s;
    s.counters = reinterpret_cast<uint32_t *>(base + kFusedCntOff);
    s.lg = reinterpret_cast<uint64_t *>(base + kFusedLgOff);
    s.hl = reinterpret_cast<uint64_t *>(base + kFusedHlOff);
    s.pl = reinterpret_cast<uint64_t *>(base + kFusedPlOff);
    s.err = err;
    s.xcd_local = xcd_local;
    s.shh = reinterpret_cast<uint64_t *>(base + kFusedShOff);
    return s;
}
// Device address of this GPU's copy of the static scratch of lt_noalloc.hip
// (kFusedScratchBytes, zero when the library loads); `device` must be the
// current device.  The address is looked up once per device and kept.
hipError_t noalloc_scratch(int device, uint8_t **base);
// Launches kFusedBlocks one-wave blocks that record their XCD in dev_ids
// [kFusedBlocks], waits, and sets *local when every block b ran on the XCD
// of block b % 8 (the round-robin placement the fused kernel's same-XCD
// hand-overs rely on for speed).
hipError_t probe_xcd_groups(uint32_t *dev_ids, hipStream_t s, int *local);
FusedPlan plan_moe_fused(const FusedLayer &L);
// A Q8_0 dense FFN (gate, up [S][D], down [D][S]) in one launch
// (lt_ffn_fused.hip): D <= 2048, S <= kFfnMaxS, both multiples of 32.
constexpr int kFfnMaxS = 8192;
constexpr int kFfnFlags = 128;
struct FfnPlan {
    bool ok;
    int P, Q;    // gate/up passes (4 h rows each), down steps (16 rows each) per block
    int NG, ND;  // gate/up and down blocks per XCD group
    int cu;      // 64-unit spans of a gate/up row per lane
    size_t lds;
};
// Hand-over memory of that kernel: launch counters [kFusedBlocks], h words
// [kFfnMaxS], start-value flags [kFfnFlags]; zeroed once when allocated.
struct FfnScratch {
    uint32_t *counters;
    uint64_t *hw;
    uint64_t *flags;
    uint32_t *err;  // the context's host-mapped error word (device address)
    int xcd_local;
};
constexpr size_t kFfnScratchBytes = (size_t)kFusedBlocks * 4 + (size_t)kFfnMaxS * 8 + (size_t)kFfnFlags * 8;
inline FfnScratch ffn_scratch_at(uint8_t *base, uint32_t *err, int xcd_local) {
    FfnScratch s;
    s.counters = reinterpret_cast<uint32_t *>(base);
    s.hw = reinterpret_cast<uint64_t *>(base + (size_t)kFusedBlocks * 4);
    s.flags = s.hw + kFfnMaxS;
    s.err = err;
    s.xcd_local = xcd_local;
    return s;
}
FfnPlan plan_ffn_fused(int D, int S);
// Reads nbytes (a multiple of 16) at buf once (lt_probe.hip).
hipError_t launch_stream_read(const void *buf, size_t nbytes, uint32_t *sink, hipStream_t s);
hipError_t launch_ffn_fused(const FfnPlan &pl, const DevTensor &G, const DevTensor &U, const DevTensor &Dn,
                            const float *x, uint32_t act, float *out, const FfnScratch &sc, hipStream_t s);
hipError_t launch_moe_fused(const FusedPlan &pl, const FusedLayer &L, const float *bias, const float *x,
                            uint32_t act, uint32_t norm, const float *base, int accumulate, int deterministic,
                            float *out, uint32_t *ids_out, float *w_out, const FusedScratch &sc, hipStream_t s);
}  // namespace lt
