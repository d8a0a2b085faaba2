// lt_formats.hip -- matvec over the Gemma4 APEX expert formats: Q5_0, Q5_1,
// IQ4_NL (32-element blocks) and Q3_K (256-element super-blocks), on the
// planar layout lt_tensor_upload makes:
//
//   Q5_0    qs [R][nb][16], qh [R][nb][4] (u32 LE), d [R][nb] (f16)
//           value = d * ((nibble | high bit << 4) - 16)       dequant.zig:189-217
//   Q5_1    qs [R][nb][16], qh [R][nb][4], dm [R][nb][2] (f16 d, f16 m)
//           value = d * (nibble | high bit << 4) + m          dequant.zig:456-486
//   IQ4_NL  qs [R][nb][16], d [R][nb]
//           value = d * table[nibble]                         dequant.zig:607-640
//   Q3_K    qs [R][nsb][64], hmask [R][nsb][32], scales [R][nsb][12], d [R][nsb]
//           element 128h + 32j + 16g + l: value = d * (sc[8h + 2j + g] - 32)
//           * (((qs[32h + 16g + l] >> 2j) & 3) - 4 * !(hmask[16g + l] >> (j + 4h) & 1))
//                                                             dequant.zig:366-454
//
// Work unit: one 32-element block (Q5_0/Q5_1/IQ4_NL) or one 32-element
// group of a Q3_K super-block (one scale pair).  A wavefront takes 1-8 rows
// at a time (lanes striding over each row's units) and the workgroups walk
// all rows, so x is staged in LDS once per workgroup.  fp32 accumulation in an
// order of our own: parity with the reference's quantMatvec is to tolerance
// (its GPU matvec fuzz bound, 1e-4 of max |y|), not bit-exact.
#include "llmtoy_hip.h"
#include "lt_internal.h"

namespace lt {

namespace {

constexpr int kFmtWaves = 4;  // rows per workgroup

// Length of the x runs whose sums are staged beside x: one Q3_K scale's 16
// elements, or one 32-element block.
template <int T>
constexpr int kSumLen = T == LT_TYPE_Q3_K ? 16 : 32;

template <int T>
size_t lds_floats(size_t n) { return n + n / kSumLen<T>; }

__device__ __forceinline__ float f16_at(const uint8_t *p) {
    return f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(p));
}

// Unsigned 5-bit codes of a Q5 block as bytes: word i of the result holds
// elements 4i..4i+3 (low nibbles of qs word i + high bit 4i..4i+3 of qh) and
// word 4 + i elements 16+4i..16+4i+3 (high nibbles + bits 16+4i..).  The
// four high bits of an element group spread into bits 4, 12, 20, 28 with one
// 24-bit multiply: (v * 0x204081) & 0x01010101 puts bit j of v at bit 8j,
// and no two partial products meet.
__device__ __forceinline__ uint32_t spread4(uint32_t v4) { return (__umul24(v4, 0x204081u) & 0x01010101u) << 4; }

// Byte i of v as a float (one v_cvt_f32_ubyte<i>).
__device__ __forceinline__ float ubyte_f(uint32_t v, int i) { return (float)((v >> (8 * i)) & 0xffu); }

// sum over the block of (code) * x: codes 0..31 as unsigned bytes,
// converted with v_cvt_f32_ubyte0..3.
__device__ __forceinline__ float q5u_block_dot(uint4 qv, uint32_t qh, const float *x) {
    const uint32_t w[4] = {qv.x, qv.y, qv.z, qv.w};
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 lo = *reinterpret_cast<const float4 *>(x + 4 * i);
        const float4 hi = *reinterpret_cast<const float4 *>(x + 16 + 4 * i);
        const uint32_t cl = (w[i] & 0x0f0f0f0fu) | spread4((qh >> (4 * i)) & 15u);
        const uint32_t ch = ((w[i] >> 4) & 0x0f0f0f0fu) | spread4((qh >> (16 + 4 * i)) & 15u);
        acc += ubyte_f(cl, 0) * lo.x;
        acc += ubyte_f(cl, 1) * lo.y;
        acc += ubyte_f(cl, 2) * lo.z;
        acc += ubyte_f(cl, 3) * lo.w;
        acc += ubyte_f(ch, 0) * hi.x;
        acc += ubyte_f(ch, 1) * hi.y;
        acc += ubyte_f(ch, 2) * hi.z;
        acc += ubyte_f(ch, 3) * hi.w;
    }
    return acc;
}

// IQ4_NL table + 128 as unsigned bytes (1..241): entries 0-3, 4-7, 8-11, 12-15.
constexpr uint32_t kIq4T0 = 0x3f2d1801u, kIq4T1 = 0x766a5d4fu, kIq4T2 = 0xa6998d81u, kIq4T3 = 0xf1d9c5b5u;

// table[n] + 128 for the four nibbles in the bytes of n4 (each 0..15):
// v_perm_b32 picks bytes by 3-bit index from the low and high half tables,
// bit 3 chooses between them (v_bfi_b32 on a byte mask).
__device__ __forceinline__ uint32_t iq4_lookup4(uint32_t n4) {
    const uint32_t sel = n4 & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(kIq4T1, kIq4T0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(kIq4T3, kIq4T2, sel);
    const uint32_t b3 = (n4 >> 3) & 0x01010101u;
    const uint32_t m = (b3 << 8) - b3;  // 0x00 or 0xff per byte
    return (hi & m) | (lo & ~m);
}

__device__ __forceinline__ float iq4u_block_dot(uint4 qv, const float *x) {
    const uint32_t w[4] = {qv.x, qv.y, qv.z, qv.w};
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 lo = *reinterpret_cast<const float4 *>(x + 4 * i);
        const float4 hi = *reinterpret_cast<const float4 *>(x + 16 + 4 * i);
        const uint32_t tl = iq4_lookup4(w[i] & 0x0f0f0f0fu), th = iq4_lookup4((w[i] >> 4) & 0x0f0f0f0fu);
        acc += ubyte_f(tl, 0) * lo.x;
        acc += ubyte_f(tl, 1) * lo.y;
        acc += ubyte_f(tl, 2) * lo.z;
        acc += ubyte_f(tl, 3) * lo.w;
        acc += ubyte_f(th, 0) * hi.x;
        acc += ubyte_f(th, 1) * hi.y;
        acc += ubyte_f(th, 2) * hi.z;
        acc += ubyte_f(th, 3) * hi.w;
    }
    return acc;
}

// Q3_K scale i (0..15) from the 12 packed bytes s[0..2] (little-endian
// dwords): low 4 bits from byte i (i < 8) or the high nibble of byte i - 8,
// high 2 bits from bits 2 (i / 4) of byte 8 + i % 4.
__device__ __forceinline__ int q3k_scale(const uint32_t s[3], int i) {
    const uint32_t lo = i < 8 ? (s[i >> 2] >> (8 * (i & 3))) & 15u : (s[(i - 8) >> 2] >> (8 * ((i - 8) & 3) + 4)) & 15u;
    const uint32_t hi = (s[2] >> (8 * (i & 3) + 2 * (i >> 2))) & 3u;
    return (int)(lo | (hi << 4));
}

// Group u = 4 h + j of a Q3_K super-block: elements 128 h + 32 j + [0, 32)
// (16 from qs[32 h ..] and hmask[0 ..], 16 from qs[32 h + 16 ..] and
// hmask[16 ..]) against x.  Each element's 3-bit unsigned code
// c = q2 | hbit << 2 (value c - 4) is built four to a dword and converted
// with v_cvt_f32_ubyte<i>; the -4 folds into x16 = the sums of the group's
// two 16-element halves of x.
__device__ __forceinline__ float q3k_group_dot(const uint8_t *qs64, const uint8_t *hm32, const uint32_t sc[3],
                                               float d, int u, const float *x, const float *x16) {
    const int h = u >> 2, j = u & 3;
    const uint4 q0 = *reinterpret_cast<const uint4 *>(qs64 + 32 * h);
    const uint4 q1 = *reinterpret_cast<const uint4 *>(qs64 + 32 * h + 16);
    const uint4 m0 = *reinterpret_cast<const uint4 *>(hm32);
    const uint4 m1 = *reinterpret_cast<const uint4 *>(hm32 + 16);
    const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    const uint32_t mw[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
    const int qsh = 2 * j, msh = j + 4 * h;
    float total = 0.f;
#pragma unroll
    for (int g = 0; g < 2; g++) {
        float acc = 0.f;
#pragma unroll
        for (int w4 = 0; w4 < 4; w4++) {
            const float4 xv = *reinterpret_cast<const float4 *>(x + 16 * g + 4 * w4);
            const uint32_t c = ((qw[4 * g + w4] >> qsh) & 0x03030303u) | (((mw[4 * g + w4] >> msh) & 0x01010101u) << 2);
            acc += ubyte_f(c, 0) * xv.x;
            acc += ubyte_f(c, 1) * xv.y;
            acc += ubyte_f(c, 2) * xv.z;
            acc += ubyte_f(c, 3) * xv.w;
        }
        total += (d * (float)(q3k_scale(sc, 8 * h + 2 * j + g) - 32)) * (acc - 4.f * x16[g]);
    }
    return total;
}

// Contribution of unit u of a row (block u, or Q3_K group u) against the
// row's x (xs = element 0 of the row's columns, in LDS; xsum = sums of x over
// kSumLen<T> elements, for the offsets the unsigned codes leave out).
template <int T>
__device__ __forceinline__ float unit_dot(const DevTensor &W, size_t row, int u, const float *xs, const float *xsum) {
    const int nb = (int)W.blocks_per_row;
    if (T == LT_TYPE_Q3_K) {
        const size_t sb = row * nb + (u >> 3);
        const uint32_t *s3 = reinterpret_cast<const uint32_t *>(W.p2 + sb * 12);
        const uint32_t sc[3] = {s3[0], s3[1], s3[2]};
        return q3k_group_dot(W.p0 + sb * 64, W.p1 + sb * 32, sc, f16_at(W.p3 + sb * 2), u & 7,
                             xs + 256 * (u >> 3) + 32 * (u & 7), xsum + 2 * u);
    }
    const size_t b = row * nb + u;
    const uint4 qv = *reinterpret_cast<const uint4 *>(W.p0 + b * 16);
    const float *xb = xs + 32 * u;
    if (T == LT_TYPE_IQ4_NL)  // d * (sum (table + 128) x - 128 sum x)
        return f16_at(W.p1 + b * 2) * (iq4u_block_dot(qv, xb) - 128.f * xsum[u]);
    const uint32_t qh = *reinterpret_cast<const uint32_t *>(W.p1 + b * 4);
    const float dot = q5u_block_dot(qv, qh, xb);
    if (T == LT_TYPE_Q5_0) return f16_at(W.p2 + b * 2) * (dot - 16.f * xsum[u]);  // codes - 16
    return f16_at(W.p2 + b * 4) * dot + f16_at(W.p2 + b * 4 + 2) * xsum[u];        // Q5_1: d q + m
}

template <int T>
__device__ __forceinline__ int units_per_row(const DevTensor &W) {
    return T == LT_TYPE_Q3_K ? 8 * (int)W.blocks_per_row : (int)W.blocks_per_row;
}

template <int LPR>
__device__ __forceinline__ float seg_sum(float v) {
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Stage n floats into LDS and their sums over kSumLen<T> elements
// (sums[j] = sum of dst[L j .. L j + L)) right after them.
template <int T>
__device__ __forceinline__ void stage(float *dst, const float *src, int n) {
    constexpr int L = kSumLen<T>;
    for (int i = threadIdx.x; i < n; i += blockDim.x) dst[i] = src[i];
    __syncthreads();
    for (int j = threadIdx.x; j < n / L; j += blockDim.x) {
        float t = 0.f;
#pragma unroll 8
        for (int e = 0; e < L; e++) t += dst[L * j + e];
        dst[n + j] = t;
    }
    __syncthreads();
}

// Workgroup = kFmtWaves waves; a wave takes RPW rows at a time (64 / RPW
// lanes per row, striding over the row's units) and walks the rows with a
// grid-wide stride, so x is staged in LDS once per workgroup.
template <int T, int RPW>
__global__ __launch_bounds__(64 * kFmtWaves) void k_matvec_fmt(DevTensor W, const float *__restrict__ x,
                                                               float *__restrict__ y) {
    extern __shared__ __attribute__((aligned(16))) float xs[];  // cols floats + their run sums
    constexpr int LPR = kWave / RPW;
    stage<T>(xs, x, (int)W.cols);
    const float *xsum = xs + W.cols;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int r = lane / LPR, sub = lane % LPR;
    const int U = units_per_row<T>(W);
    const size_t stride = (size_t)gridDim.x * kFmtWaves * RPW;
    for (size_t row0 = ((size_t)blockIdx.x * kFmtWaves + wave) * RPW; row0 < W.total_rows; row0 += stride) {
        const size_t row = row0 + r;
        const bool live = row < W.total_rows;
        float acc = 0.f;
        if (live)
            for (int u = sub; u < U; u += LPR) acc += unit_dot<T>(W, row, u, xs, xsum);
        acc = seg_sum<LPR>(acc);
        if (live && sub == 0) y[row] = acc;
    }
}

// Expert-indexed gate/up (ops/moe.zig:55-73): slot s = blockIdx.y, expert
// e = ids[s]; row pair j = (gate row e 2F + j, up row e 2F + F + j);
// h[s][j] = act(gate . x) * (up . x), h[s][F, down_cols) = 0.  Waves walk
// the row pairs of their slot with a stride of gridDim.x * kFmtWaves * RPW.
template <int T, int RPW>
__global__ __launch_bounds__(64 * kFmtWaves) void k_expert_gu_fmt(DevTensor W, const float *__restrict__ x,
                                                                  const uint32_t *__restrict__ ids, int F,
                                                                  int down_cols, uint32_t act, float *__restrict__ h) {
    extern __shared__ __attribute__((aligned(16))) float xs[];  // cols floats + their run sums
    constexpr int LPR = kWave / RPW;
    stage<T>(xs, x, (int)W.cols);
    const float *xsum = xs + W.cols;
    const int s = blockIdx.y;
    const uint32_t e = __builtin_amdgcn_readfirstlane(ids[s]);
    float *hs = h + (size_t)s * down_cols;
    if (blockIdx.x == 0)
        for (int j = F + threadIdx.x; j < down_cols; j += blockDim.x) hs[j] = 0.f;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int r = lane / LPR, sub = lane % LPR;
    const int U = units_per_row<T>(W);
    const bool valid = e < (uint32_t)W.n_experts;
    const int stride = gridDim.x * kFmtWaves * RPW;
    for (int j0 = (blockIdx.x * kFmtWaves + wave) * RPW; j0 < F; j0 += stride) {
        const int j = j0 + r;
        const bool live = j < F;
        float ag = 0.f, au = 0.f;
        if (live && valid) {
            const size_t g = (size_t)e * 2 * F + j, up = g + F;
            for (int u = sub; u < U; u += LPR) {
                ag += unit_dot<T>(W, g, u, xs, xsum);
                au += unit_dot<T>(W, up, u, xs, xsum);
            }
        }
        ag = seg_sum<LPR>(ag);
        au = seg_sum<LPR>(au);
        if (live && sub == 0) hs[j] = valid ? act_apply(act, ag) * au : 0.f;  // invalid id: the slot adds zeros
    }
}

// Expert-indexed down with the weighted combine (ops/moe.zig:67-76):
//   out[i] = base[i] + (accumulate ? out[i] : 0) + sum_s w'[s] (D_{ids[s]} row i) . h[s]
// with w'[s] = dscale[ids[s]] * w[s] when a per-expert down scale is given
// (gemma4/forward.zig:477).  h [k][down_cols] is staged in LDS once per
// workgroup; waves walk the output rows.
template <int T, int RPW>
__global__ __launch_bounds__(64 * kFmtWaves) void k_expert_down_fmt(DevTensor W, const float *__restrict__ h,
                                                                    const uint32_t *__restrict__ ids,
                                                                    const float *__restrict__ wts, int k,
                                                                    const float *base, int accumulate,
                                                                    const float *dscale, float *out) {
    extern __shared__ __attribute__((aligned(16))) float hsm[];  // k * down_cols floats + their block sums
    __shared__ uint32_t s_e[16];
    __shared__ float s_w[16];
    constexpr int LPR = kWave / RPW;
    const int Kd = (int)W.cols;
    if ((int)threadIdx.x < k) {  // the slots' experts and combine weights, once per workgroup
        const uint32_t e = ids[threadIdx.x];
        s_e[threadIdx.x] = e;
        s_w[threadIdx.x] = e < (uint32_t)W.n_experts ? (dscale ? dscale[e] * wts[threadIdx.x] : wts[threadIdx.x]) : 0.f;
    }
    stage<T>(hsm, h, k * Kd);
    const float *hsum = hsm + k * Kd;  // run sums: slot s's at hsum + s * (Kd / kSumLen<T>)
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int r = lane / LPR, sub = lane % LPR;
    const int U = units_per_row<T>(W);
    const int D = (int)W.rows;
    const int stride = gridDim.x * kFmtWaves * RPW;
    for (int i0 = (blockIdx.x * kFmtWaves + wave) * RPW; i0 < D; i0 += stride) {
        const int i = i0 + r;
        const bool live = i < D;
        float acc = 0.f;
        if (live) {
            for (int s = 0; s < k; s++) {
                const uint32_t e = s_e[s];
                if (e >= (uint32_t)W.n_experts) continue;
                float t = 0.f;
                for (int u = sub; u < U; u += LPR)
                    t += unit_dot<T>(W, (size_t)e * D + i, u, hsm + s * Kd, hsum + s * (Kd / kSumLen<T>));
                acc += s_w[s] * t;
            }
        }
        acc = seg_sum<LPR>(acc);
        if (live && sub == 0) {
            float v = accumulate ? out[i] + acc : acc;
            out[i] = base ? base[i] + v : v;
        }
    }
}

int pick_rpw(size_t units) { return units >= 48 ? 1 : units >= 24 ? 2 : units >= 12 ? 4 : 8; }

// Allow the largest staging (16384 floats and their 16-element run sums:
// 68 KiB of dynamic LDS), once per kernel and device.
hipError_t allow_lds(const void *fn, bool *set) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    if (set[dev]) return hipSuccess;
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (16384 + 16384 / 16) * 4);
    if (e == hipSuccess) set[dev] = true;
    return e;
}

template <int T, int RPW>
hipError_t launch_mv(const DevTensor &W, const float *x, float *y, hipStream_t s) {
    static bool set[64] = {};
    hipError_t e = allow_lds((const void *)k_matvec_fmt<T, RPW>, set);
    if (e != hipSuccess) return e;
    // up to 8 workgroups per CU, each walking many rows
    const size_t need = (W.total_rows + kFmtWaves * RPW - 1) / (kFmtWaves * RPW);
    const dim3 grid((unsigned)(need < 2048 ? need : 2048));
    hipLaunchKernelGGL((k_matvec_fmt<T, RPW>), grid, dim3(64 * kFmtWaves), lds_floats<T>(W.cols) * sizeof(float), s,
                       W, x, y);
    return hipGetLastError();
}

template <int T, int RPW>
hipError_t launch_gu(const DevTensor &W, const float *x, const uint32_t *ids, int k, int F, int down_cols,
                     uint32_t act, float *h, hipStream_t s) {
    static bool set[64] = {};
    hipError_t e = allow_lds((const void *)k_expert_gu_fmt<T, RPW>, set);
    if (e != hipSuccess) return e;
    const int need = (F + kFmtWaves * RPW - 1) / (kFmtWaves * RPW);
    const dim3 grid((unsigned)(need < 128 ? need : 128), (unsigned)k);  // up to 128 x k workgroups walk the rows
    hipLaunchKernelGGL((k_expert_gu_fmt<T, RPW>), grid, dim3(64 * kFmtWaves), lds_floats<T>(W.cols) * sizeof(float),
                       s, W, x, ids,
                       F, down_cols, act, h);
    return hipGetLastError();
}

template <int T, int RPW>
hipError_t launch_dn(const DevTensor &W, const float *h, const uint32_t *ids, const float *w, int k,
                     const float *base, int accumulate, const float *dscale, float *out, hipStream_t s) {
    static bool set[64] = {};
    hipError_t e = allow_lds((const void *)k_expert_down_fmt<T, RPW>, set);
    if (e != hipSuccess) return e;
    const int D = (int)W.rows;
    const int need = (D + kFmtWaves * RPW - 1) / (kFmtWaves * RPW);
    const dim3 grid((unsigned)(need < 1024 ? need : 1024));
    hipLaunchKernelGGL((k_expert_down_fmt<T, RPW>), grid, dim3(64 * kFmtWaves),
                       lds_floats<T>((size_t)k * W.cols) * sizeof(float), s, W, h, ids, w, k, base,
                       accumulate, dscale, out);
    return hipGetLastError();
}

template <int T>
hipError_t launch_t(const DevTensor &W, const float *x, float *y, hipStream_t s) {
    switch (pick_rpw(T == LT_TYPE_Q3_K ? 8 * W.blocks_per_row : W.blocks_per_row)) {
    case 1: return launch_mv<T, 1>(W, x, y, s);
    case 2: return launch_mv<T, 2>(W, x, y, s);
    case 4: return launch_mv<T, 4>(W, x, y, s);
    default: return launch_mv<T, 8>(W, x, y, s);
    }
}

template <int T>
hipError_t launch_gu_t(const DevTensor &W, const float *x, const uint32_t *ids, int k, int F, int down_cols,
                       uint32_t act, float *h, hipStream_t s) {
    switch (pick_rpw(T == LT_TYPE_Q3_K ? 8 * W.blocks_per_row : W.blocks_per_row)) {
    case 1: return launch_gu<T, 1>(W, x, ids, k, F, down_cols, act, h, s);
    case 2: return launch_gu<T, 2>(W, x, ids, k, F, down_cols, act, h, s);
    case 4: return launch_gu<T, 4>(W, x, ids, k, F, down_cols, act, h, s);
    default: return launch_gu<T, 8>(W, x, ids, k, F, down_cols, act, h, s);
    }
}

template <int T>
hipError_t launch_dn_t(const DevTensor &W, const float *h, const uint32_t *ids, const float *w, int k,
                       const float *base, int accumulate, const float *dscale, float *out, hipStream_t s) {
    switch (pick_rpw(T == LT_TYPE_Q3_K ? 8 * W.blocks_per_row : W.blocks_per_row)) {
    case 1: return launch_dn<T, 1>(W, h, ids, w, k, base, accumulate, dscale, out, s);
    case 2: return launch_dn<T, 2>(W, h, ids, w, k, base, accumulate, dscale, out, s);
    case 4: return launch_dn<T, 4>(W, h, ids, w, k, base, accumulate, dscale, out, s);
    default: return launch_dn<T, 8>(W, h, ids, w, k, base, accumulate, dscale, out, s);
    }
}

}  // namespace

hipError_t launch_matvec_fmt(const DevTensor &W, const float *x, float *y, hipStream_t s) {
    switch (W.type) {
    case LT_TYPE_Q5_0: return launch_t<LT_TYPE_Q5_0>(W, x, y, s);
    case LT_TYPE_Q5_1: return launch_t<LT_TYPE_Q5_1>(W, x, y, s);
    case LT_TYPE_IQ4_NL: return launch_t<LT_TYPE_IQ4_NL>(W, x, y, s);
    case LT_TYPE_Q3_K: return launch_t<LT_TYPE_Q3_K>(W, x, y, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_expert_gate_up_fmt(const DevTensor &GU, const float *x, const uint32_t *ids, uint32_t k,
                                     uint32_t d_expert, uint32_t down_cols, uint32_t act, float *h, hipStream_t s) {
    const int K = (int)k, F = (int)d_expert, Kd = (int)down_cols;
    switch (GU.type) {
    case LT_TYPE_Q5_0: return launch_gu_t<LT_TYPE_Q5_0>(GU, x, ids, K, F, Kd, act, h, s);
    case LT_TYPE_Q5_1: return launch_gu_t<LT_TYPE_Q5_1>(GU, x, ids, K, F, Kd, act, h, s);
    case LT_TYPE_IQ4_NL: return launch_gu_t<LT_TYPE_IQ4_NL>(GU, x, ids, K, F, Kd, act, h, s);
    case LT_TYPE_Q3_K: return launch_gu_t<LT_TYPE_Q3_K>(GU, x, ids, K, F, Kd, act, h, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_expert_down_fmt(const DevTensor &D, const float *h, const uint32_t *ids, const float *w,
                                  uint32_t k, const float *base, int accumulate, const float *dscale, float *out,
                                  hipStream_t s) {
    const int K = (int)k;
    switch (D.type) {
    case LT_TYPE_Q5_0: return launch_dn_t<LT_TYPE_Q5_0>(D, h, ids, w, K, base, accumulate, dscale, out, s);
    case LT_TYPE_Q5_1: return launch_dn_t<LT_TYPE_Q5_1>(D, h, ids, w, K, base, accumulate, dscale, out, s);
    case LT_TYPE_IQ4_NL: return launch_dn_t<LT_TYPE_IQ4_NL>(D, h, ids, w, K, base, accumulate, dscale, out, s);
    case LT_TYPE_Q3_K: return launch_dn_t<LT_TYPE_Q3_K>(D, h, ids, w, K, base, accumulate, dscale, out, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace lt
