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
#include "lt_limbs.h"

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
// registers as int8 limbs (lt_limbs.h: the block converts x once through
// LDS; the 6-bit codes meet the limbs in v_dot4).  Each wave walks row
// slabs `stride` apart with ND slabs in flight: ND static buffers, loaded
// between the load and the conversion of x, each reloaded ND slabs ahead
// as soon as it has been used (a register copy between buffers would make the compiler wait
// for the loads in flight).  Row sums are DPP reductions over the row's
// LPR lanes.
struct Q6Regs {
    uint4 qa, qb, qh;
    uint2 sc;
    uint32_t d;
};

__device__ __forceinline__ void q6_load(Q6Regs &w, const uint8_t *ql, const uint8_t *qh, const uint8_t *sc,
                                        const uint16_t *dp, size_t blk, int hf, int l0) {
    w.qa = ldg16_nt(ql + blk * 128 + 64 * hf + l0);
    w.qb = ldg16_nt(ql + blk * 128 + 64 * hf + 32 + l0);
    w.qh = ldg16_nt(qh + blk * 64 + 32 * hf + l0);
    w.sc = *reinterpret_cast<const uint2 *>(sc + blk * 16 + 8 * hf);
    w.d = dp[blk];
}

// The unit's 64 activations as int8 limbs (lt_limbs.h): group q (16
// elements, partners of the q-th 6-bit code of each byte position) in
// a[q] / b[q], its limb scale sp[q] and fp32 sum xs[q].
struct Q6Limbs {
    uint32_t a[4][4], b[4][4];
    float sp[4], xs[4];
};

// sum over the unit's 64 elements of (d * sc) * (q - 32) * x: each group's
// sum q * x from v_dot4 over its four code words and both limbs, minus
// 32 * (sum of x), times d * sc in fp32
__device__ __forceinline__ float q6_unit_dot_limbs(const Q6Regs &w, int is, const Q6Limbs &xl) {
    const uint32_t sa[4] = {w.qa.x, w.qa.y, w.qa.z, w.qa.w};
    const uint32_t sb[4] = {w.qb.x, w.qb.y, w.qb.z, w.qb.w};
    const uint32_t sh[4] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w};
    int A[4], B[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        uint32_t g[4];
        g[0] = (sa[t] & 0x0f0f0f0fu) | ((sh[t] << 4) & 0x30303030u);
        g[1] = (sb[t] & 0x0f0f0f0fu) | ((sh[t] << 2) & 0x30303030u);
        g[2] = ((sa[t] >> 4) & 0x0f0f0f0fu) | (sh[t] & 0x30303030u);
        g[3] = ((sb[t] >> 4) & 0x0f0f0f0fu) | ((sh[t] >> 2) & 0x30303030u);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            if (t == 0) {
                A[q] = sdot4_first((int)g[q], (int)xl.a[q][0]);
                B[q] = sdot4_first((int)g[q], (int)xl.b[q][0]);
            } else {
                A[q] = __builtin_amdgcn_sdot4((int)g[q], (int)xl.a[q][t], A[q], false);
                B[q] = __builtin_amdgcn_sdot4((int)g[q], (int)xl.b[q][t], B[q], false);
            }
        }
    }
    const float d = f16_bits_to_f32(w.d);
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int bi = is + 2 * q;  // sc[8 hf + is + 2 q]: byte bi of the half's 8 scale bytes
        const uint32_t word = bi < 4 ? w.sc.x : w.sc.y;
        const float scale = (float)(int8_t)((word >> (8 * (bi & 3))) & 0xffu);
        const float c = (float)((A[q] << 8) + B[q]);
        acc = fmaf(d * scale, fmaf(xl.sp[q], c, -32.0f * xl.xs[q]), acc);
    }
    return acc;
}

// Waves per SIMD the streaming kernel is compiled for (VGPR budget 128 at
// 4, 168 at 3) and hence its workgroups per CU.
constexpr int q6k_stream_waves(int nd) { return nd <= 3 ? 4 : 3; }

template <int NSB, int ND>
__global__ void __launch_bounds__(256, q6k_stream_waves(ND)) k_matvec_q6k_stream(const uint8_t *ql, const uint8_t *qh, const uint8_t *sc,
                                                              const uint16_t *dp, const float *x, float *y,
                                                              int nrows) {
    constexpr int LPR = 4 * NSB, RPS = 64 / LPR;
    __shared__ __attribute__((aligned(16))) uint32_t la[64 * NSB], lb[64 * NSB];
    __shared__ __attribute__((aligned(16))) float lsp[16 * NSB], lxs[16 * NSB];
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
    float xv[16];
    stage_x_load(x, 256 * NSB, xv);  // x first: its wait does not include the weights
    asm volatile("" ::: "memory");  // keep the x loads ahead of the weight loads
    Q6Regs w[ND];
#pragma unroll
    for (int i = 0; i < ND; i++) ld(w[i], base + i * stride);
    __builtin_amdgcn_sched_barrier(0);  // the weight loads issued before the conversion
    stage_limbs_store(xv, 256 * NSB, la, lb, lsp, lxs);
    Q6Limbs xl;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        // group q of the unit: elements 256 sbi + 128 hf + l0 + 32 q + [0, 16)
        const int g = 16 * sbi + 8 * hf + (l0 >> 4) + 2 * q;
        read_group_limbs(la, lb, g, xl.a[q], xl.b[q]);
        xl.sp[q] = lsp[g];
        xl.xs[q] = lxs[g];
    }
    auto step = [&](const Q6Regs &r, int rb) {
        const float v = group_sum_dpp<LPR>(q6_unit_dot_limbs(r, l0 >> 4, xl), first);
        const int row = rb + rs;
        if (u == 0 && row < nrows) y[row] = v;
    };
    // loads stay unconditional (clamped rows); the math of a slab past the
    // last row is skipped (wave-uniform branch)
    for (; base < nrows; base += ND * stride) {
#pragma unroll
        for (int i = 0; i < ND; i++) {
            if (i == 0 || base + i * stride < nrows) step(w[i], base + i * stride);
            ld(w[i], base + (i + ND) * stride);
        }
    }
}

constexpr int kQ6StreamND = 3;

template <int NSB>
static hipError_t launch_q6_stream(const DevTensor &W, const float *x, float *y, hipStream_t s) {
    constexpr int RPS = 16 / NSB;  // 64 / (4 NSB)
    const int nrows = (int)W.total_rows;
    const int slabs = (nrows + RPS - 1) / RPS;
    // Small matrices: at least two row slabs per wave, both in flight from
    // the start (see lt_q4k.hip); large ones: every workgroup resident with
    // kQ6StreamND slabs in flight per wave (four would spill at the
    // 128-VGPR budget of four waves per SIMD).
    constexpr int nblk_big = 256 * q6k_stream_waves(kQ6StreamND);
    if (slabs >= nblk_big * 4 * 2 * kQ6StreamND) {
        hipLaunchKernelGGL((k_matvec_q6k_stream<NSB, kQ6StreamND>), dim3(nblk_big), dim3(256), 0, s, W.p0, W.p1,
                           W.p2, (const uint16_t *)W.p3, x, y, nrows);
    } else {
        int nblk = (slabs + 7) / 8;
        if (nblk > kStreamBlocks) nblk = kStreamBlocks;
        hipLaunchKernelGGL((k_matvec_q6k_stream<NSB, 2>), dim3(nblk), dim3(256), 0, s, W.p0, W.p1, W.p2,
                           (const uint16_t *)W.p3, x, y, nrows);
    }
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
