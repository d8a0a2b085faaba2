// lt_q6k.hip -- Q6_K decode matvec for gfx950 (wave64).
//
// Q6_K super-block (quant/dequant.zig:219-287): ql[128], qh[64], int8 sc[16],
// f16 d; for half hf (128 elements) and l < 32:
//   q1 = ql[64hf+l]    & 15 | (qh[32hf+l]      & 3) << 4  -> element 128hf+l
//   q2 = ql[64hf+l+32] & 15 | (qh[32hf+l] >> 2 & 3) << 4  -> +32
//   q3 = ql[64hf+l]    >> 4 | (qh[32hf+l] >> 4 & 3) << 4  -> +64
//   q4 = ql[64hf+l+32] >> 4 | (qh[32hf+l] >> 6)     << 4  -> +96
// value = (d * sc[8hf + l/16 + 2g]) * (q - 32), g = 0..3.
// Device layout: ql [R][nsb][128], qh [R][nsb][64], sc [R][nsb][16], d [R][nsb].
// Work unit of one lane: (super-block, half hf, l0 in {0,16}) = 64 elements
// from two 16-byte ql vectors and one 16-byte qh vector; 4 units per
// super-block.
#include "lt_internal.h"

namespace lt {

namespace {

struct Q6Unit {
    uint4 qa, qb, qh;
    uint2 sc;
    uint16_t d;
};

__device__ __forceinline__ float q6_unit_dot(const Q6Unit &U, int is, const float *xv /*64*/) {
    const float d = f16_bits_to_f32(U.d);
    const uint32_t sa[4] = {U.qa.x, U.qa.y, U.qa.z, U.qa.w};
    const uint32_t sb[4] = {U.qb.x, U.qb.y, U.qb.z, U.qb.w};
    const uint32_t sh[4] = {U.qh.x, U.qh.y, U.qh.z, U.qh.w};
    float dot[4] = {0.f, 0.f, 0.f, 0.f}, xsum[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; t++) {
        uint32_t g[4];
        g[0] = (sa[t] & 0x0f0f0f0fu) | ((sh[t] & 0x03030303u) << 4);
        g[1] = (sb[t] & 0x0f0f0f0fu) | (((sh[t] >> 2) & 0x03030303u) << 4);
        g[2] = ((sa[t] >> 4) & 0x0f0f0f0fu) | (((sh[t] >> 4) & 0x03030303u) << 4);
        g[3] = ((sb[t] >> 4) & 0x0f0f0f0fu) | (((sh[t] >> 6) & 0x03030303u) << 4);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float *xg = xv + 16 * q + 4 * t;
            dot[q] += (float)(g[q] & 0xffu) * xg[0];
            dot[q] += (float)((g[q] >> 8) & 0xffu) * xg[1];
            dot[q] += (float)((g[q] >> 16) & 0xffu) * xg[2];
            dot[q] += (float)(g[q] >> 24) * xg[3];
            xsum[q] += (xg[0] + xg[1]) + (xg[2] + xg[3]);
        }
    }
    // scale bytes: sc[8hf + is + 2q] = byte (is + 2q) of the 8-byte half-row
    const uint32_t s_lo = U.sc.x, s_hi = U.sc.y;
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int bi = is + 2 * q;
        const uint32_t word = bi < 4 ? s_lo : s_hi;
        const float scale = (float)(int8_t)((word >> (8 * (bi & 3))) & 0xffu);
        acc += (d * scale) * (dot[q] - 32.0f * xsum[q]);
    }
    return acc;
}

}  // namespace

// G lanes per row, CPL units per lane, R rows per lane group; 256 threads.
template <int G, int CPL, int R>
__global__ void __launch_bounds__(256) k_matvec_q6k(const uint8_t *__restrict__ ql, const uint8_t *__restrict__ qh,
                                                    const uint8_t *__restrict__ sc, const uint16_t *__restrict__ dp,
                                                    const float *__restrict__ x, float *__restrict__ y, int nrows,
                                                    int nsb) {
    extern __shared__ float xs[];
    for (int i = threadIdx.x * 4; i < nsb * 256; i += blockDim.x * 4)
        *reinterpret_cast<float4 *>(xs + i) = *reinterpret_cast<const float4 *>(x + i);
    __syncthreads();
    const int groups = 256 / G;
    const int g = threadIdx.x / G, lane = threadIdx.x % G;
    const int rbase = (blockIdx.x * groups + g) * R;
    const int nu = nsb * 4;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; i++) {
        const int u = lane + G * i;
        if (u < nu) {
            const int sbi = u >> 2, hf = (u >> 1) & 1, l0 = (u & 1) * 16;
            Q6Unit U[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int row = rbase + r;
                if (row < nrows) {
                    const size_t blk = (size_t)row * nsb + sbi;
                    U[r].qa = ldg16(ql + blk * 128 + 64 * hf + l0);
                    U[r].qb = ldg16(ql + blk * 128 + 64 * hf + 32 + l0);
                    U[r].qh = ldg16(qh + blk * 64 + 32 * hf + l0);
                    U[r].sc = *reinterpret_cast<const uint2 *>(sc + blk * 16 + 8 * hf);
                    U[r].d = dp[blk];
                }
            }
            float xv[64];
            const float *px = xs + sbi * 256 + 128 * hf + l0;
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int t = 0; t < 16; t += 4) {
                    float4 a = *reinterpret_cast<const float4 *>(px + 32 * q + t);
                    xv[16 * q + t] = a.x; xv[16 * q + t + 1] = a.y;
                    xv[16 * q + t + 2] = a.z; xv[16 * q + t + 3] = a.w;
                }
#pragma unroll
            for (int r = 0; r < R; r++)
                if (rbase + r < nrows) acc[r] += q6_unit_dot(U[r], l0 >> 4, xv);
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float v = group_sum<G>(acc[r]);
        if (lane == 0 && rbase + r < nrows) y[rbase + r] = v;
    }
}

// ------------------------------------------------------------------------
// Streaming matvec for rows of NSB = 1, 2, 4, 8 or 16 super-blocks (the
// config-2b output projection, 151936 x 1024, is NSB = 4).  Persistent
// waves: lane L takes unit u = L % LPR (LPR = 4 NSB lanes per row) of rows
// RPS = 64 / LPR apart, so its 64 x values are loop-invariant and live in
// registers (no LDS, no barrier); each wave walks row slabs `stride` apart
// and loads slab i + 1 while it computes slab i (two static buffers: a
// register copy between them would make the compiler wait for the loads in
// flight).  Row sums are DPP reductions over the row's LPR lanes.
struct Q6Regs {
    uint4 qa, qb, qh;
    uint2 sc;
    uint32_t d;
};

__device__ __forceinline__ void q6_load(Q6Regs &w, const uint8_t *ql, const uint8_t *qh, const uint8_t *sc,
                                        const uint16_t *dp, size_t blk, int hf, int l0) {
    w.qa = ldg16(ql + blk * 128 + 64 * hf + l0);
    w.qb = ldg16(ql + blk * 128 + 64 * hf + 32 + l0);
    w.qh = ldg16(qh + blk * 64 + 32 * hf + l0);
    w.sc = *reinterpret_cast<const uint2 *>(sc + blk * 16 + 8 * hf);
    w.d = dp[blk];
}

// sum over the unit's 64 elements of (d * sc) * (q - 32) * x, with x in
// registers (xv[16 q + i] partners q-group q) and xs[q] = sum of group q's x
__device__ __forceinline__ float q6_unit_dot_regs(const Q6Regs &w, int is, const float (&xv)[64],
                                                  const float (&xs)[4]) {
    const uint32_t sa[4] = {w.qa.x, w.qa.y, w.qa.z, w.qa.w};
    const uint32_t sb[4] = {w.qb.x, w.qb.y, w.qb.z, w.qb.w};
    const uint32_t sh[4] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w};
    float dot[4][2] = {{0.f, 0.f}, {0.f, 0.f}, {0.f, 0.f}, {0.f, 0.f}};
#pragma unroll
    for (int t = 0; t < 4; t++) {
        uint32_t g[4];
        g[0] = opaque((sa[t] & 0x0f0f0f0fu) | ((sh[t] << 4) & 0x30303030u));
        g[1] = opaque((sb[t] & 0x0f0f0f0fu) | ((sh[t] << 2) & 0x30303030u));
        g[2] = opaque(((sa[t] >> 4) & 0x0f0f0f0fu) | (sh[t] & 0x30303030u));
        g[3] = opaque(((sb[t] >> 4) & 0x0f0f0f0fu) | ((sh[t] >> 2) & 0x30303030u));
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float *xg = xv + 16 * q + 4 * t;
            dot[q][0] = fmaf((float)(g[q] & 0xffu), xg[0], dot[q][0]);
            dot[q][1] = fmaf((float)((g[q] >> 8) & 0xffu), xg[1], dot[q][1]);
            dot[q][0] = fmaf((float)((g[q] >> 16) & 0xffu), xg[2], dot[q][0]);
            dot[q][1] = fmaf((float)(g[q] >> 24), xg[3], dot[q][1]);
        }
    }
    const float d = f16_bits_to_f32(w.d);
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int bi = is + 2 * q;  // sc[8 hf + is + 2 q]: byte bi of the half's 8 scale bytes
        const uint32_t word = bi < 4 ? w.sc.x : w.sc.y;
        const float scale = (float)(int8_t)((word >> (8 * (bi & 3))) & 0xffu);
        acc = fmaf(d * scale, fmaf(-32.0f, xs[q], dot[q][0] + dot[q][1]), acc);
    }
    return acc;
}

template <int NSB>
__global__ void __launch_bounds__(256) k_matvec_q6k_stream(const uint8_t *__restrict__ ql,
                                                           const uint8_t *__restrict__ qh,
                                                           const uint8_t *__restrict__ sc,
                                                           const uint16_t *__restrict__ dp,
                                                           const float *__restrict__ x, float *__restrict__ y,
                                                           int nrows) {
    constexpr int LPR = 4 * NSB, RPS = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int u = lane % LPR, rs = lane / LPR;
    const int sbi = u >> 2, hf = (u >> 1) & 1, l0 = (u & 1) * 16;
    const int stride = gridDim.x * 4 * RPS;
    int base = (blockIdx.x * 4 + (threadIdx.x >> 6)) * RPS;
    const bool first = p32_first(lane);
    auto ld = [&](Q6Regs &w, int rb) {
        int row = rb + rs;
        row = row < nrows ? row : nrows - 1;  // every load unconditional (see the wait counts above)
        q6_load(w, ql, qh, sc, dp, (size_t)row * NSB + sbi, hf, l0);
    };
    Q6Regs a, b;
    ld(a, base);
    float xv[64], xs[4];
    {
        const float *px = x + sbi * 256 + 128 * hf + l0;
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int t = 0; t < 16; t += 4) {
                const float4 v = *reinterpret_cast<const float4 *>(px + 32 * q + t);
                xv[16 * q + t] = v.x;
                xv[16 * q + t + 1] = v.y;
                xv[16 * q + t + 2] = v.z;
                xv[16 * q + t + 3] = v.w;
            }
#pragma unroll
        for (int q = 0; q < 4; q++) {
            float s0 = 0.f;
#pragma unroll
            for (int t = 0; t < 16; t += 4)
                s0 += (xv[16 * q + t] + xv[16 * q + t + 1]) + (xv[16 * q + t + 2] + xv[16 * q + t + 3]);
            xs[q] = s0;
        }
    }
    auto step = [&](const Q6Regs &w, int rb) {
        const float v = group_sum_dpp<LPR>(q6_unit_dot_regs(w, l0 >> 4, xv, xs), first);
        const int row = rb + rs;
        if (u == 0 && row < nrows) y[row] = v;
    };
    // loads stay unconditional (clamped rows); the math of a slab past the
    // last row is skipped (wave-uniform branch)
    for (; base < nrows; base += 2 * stride) {
        ld(b, base + stride);
        step(a, base);
        ld(a, base + 2 * stride);
        if (base + stride < nrows) step(b, base + stride);
    }
}

template <int NSB>
static hipError_t launch_q6_stream(const DevTensor &W, const float *x, float *y, hipStream_t s) {
    constexpr int RPS = 16 / NSB;  // 64 / (4 NSB)
    const int nrows = (int)W.total_rows;
    // at least two row slabs per wave (x loaded once for both; see lt_q4k.hip)
    const int slabs = (nrows + RPS - 1) / RPS;
    int nblk = (slabs + 7) / 8;
    if (nblk > kStreamBlocks) nblk = kStreamBlocks;
    hipLaunchKernelGGL((k_matvec_q6k_stream<NSB>), dim3(nblk), dim3(256), 0, s, W.p0, W.p1, W.p2,
                       (const uint16_t *)W.p3, x, y, nrows);
    return hipGetLastError();
}

template <int G, int CPL>
static hipError_t launch_q6_t(const DevTensor &W, const float *x, float *y, hipStream_t s) {
    constexpr int R = 2;
    const int nrows = (int)W.total_rows, nsb = (int)W.blocks_per_row;
    const int groups = 256 / G;
    const int nblk = (nrows + groups * R - 1) / (groups * R);
    hipLaunchKernelGGL((k_matvec_q6k<G, CPL, R>), dim3(nblk), dim3(256), (size_t)nsb * 256 * sizeof(float), s,
                       W.p0, W.p1, W.p2, (const uint16_t *)W.p3, x, y, nrows, nsb);
    return hipGetLastError();
}

hipError_t launch_matvec_q6k(const DevTensor &W, const float *x, float *y, hipStream_t s) {
    switch (W.blocks_per_row) {
    case 1: return launch_q6_stream<1>(W, x, y, s);
    case 2: return launch_q6_stream<2>(W, x, y, s);
    case 4: return launch_q6_stream<4>(W, x, y, s);
    case 8: return launch_q6_stream<8>(W, x, y, s);
    case 16: return launch_q6_stream<16>(W, x, y, s);
    default: break;
    }
    const int nu = (int)W.blocks_per_row * 4;
    if (nu <= 4) return launch_q6_t<4, 1>(W, x, y, s);
    if (nu <= 8) return launch_q6_t<8, 1>(W, x, y, s);
    if (nu <= 16) return launch_q6_t<16, 1>(W, x, y, s);
    if (nu <= 32) return launch_q6_t<32, 1>(W, x, y, s);
    switch ((nu + 63) / 64) {
    case 1: return launch_q6_t<64, 1>(W, x, y, s);
    case 2: return launch_q6_t<64, 2>(W, x, y, s);
    case 3: return launch_q6_t<64, 3>(W, x, y, s);
    case 4: return launch_q6_t<64, 4>(W, x, y, s);
    default: return hipErrorInvalidValue;  // K > 16384: rejected by the API layer
    }
}

}  // namespace lt
