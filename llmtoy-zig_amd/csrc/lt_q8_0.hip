// lt_q8_0.hip -- Q8_0 decode kernels for gfx950 (wave64).
//
// Q8_0 block (quant/dequant.zig:31-78): f16 d + int8 q[32]; value = d*q.
// Device layout: qs plane [R][nb][32], d plane [R][nb] (f16).
// Work unit of one lane: a 16-byte half block (16 int8 quants); the units of
// a row are consecutive 16-byte vectors of the qs plane.  The lane computes
// d * sum(q*x) over its 16 elements (the reference applies d after the
// in-block sum too, dequant.zig:75).
#include "lt_internal.h"

namespace lt {

namespace {

__device__ __forceinline__ float q8_half_dot(uint4 q, float d, const float *xv) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        acc += (float)(int8_t)(w[t] & 0xffu) * xv[4 * t + 0];
        acc += (float)(int8_t)((w[t] >> 8) & 0xffu) * xv[4 * t + 1];
        acc += (float)(int8_t)((w[t] >> 16) & 0xffu) * xv[4 * t + 2];
        acc += (float)(int8_t)(w[t] >> 24) * xv[4 * t + 3];
    }
    return d * acc;
}

__device__ __forceinline__ void stage_x8(float *xs, const float *x, int n) {
    for (int i = threadIdx.x * 4; i < n; i += blockDim.x * 4)
        *reinterpret_cast<float4 *>(xs + i) = *reinterpret_cast<const float4 *>(x + i);
    __syncthreads();
}

__device__ __forceinline__ void load_x16(const float *xs, int u, float *xv) {
    const float *p = xs + u * 16;
#pragma unroll
    for (int t = 0; t < 16; t += 4) {
        float4 a = *reinterpret_cast<const float4 *>(p + t);
        xv[t] = a.x; xv[t + 1] = a.y; xv[t + 2] = a.z; xv[t + 3] = a.w;
    }
}

}  // namespace

// y[r] = W[r] . x  (single) or h[r] = act(Wg[r] . x) * (Wu[r] . x)  (DUAL).
// G lanes per row, CPL units per lane, R rows per lane group; 256 threads.
template <int G, int CPL, int R, bool DUAL>
__global__ void __launch_bounds__(256) k_matvec_q8_0(const uint8_t *__restrict__ qa, const uint16_t *__restrict__ da,
                                                     const uint8_t *__restrict__ qb, const uint16_t *__restrict__ db,
                                                     const float *__restrict__ x, float *__restrict__ y, int nrows,
                                                     int nb, uint32_t act) {
    extern __shared__ float xs[];
    stage_x8(xs, x, nb * 32);
    const int groups = 256 / G;
    const int g = threadIdx.x / G, lane = threadIdx.x % G;
    const int rbase = (blockIdx.x * groups + g) * R;
    const int nu = nb * 2;
    float aa[R], ab[R];
#pragma unroll
    for (int r = 0; r < R; r++) aa[r] = ab[r] = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; i++) {
        const int u = lane + G * i;
        if (u < nu) {
            const int b = u >> 1;
            uint4 qva[R], qvb[R];
            uint16_t dva[R], dvb[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int row = rbase + r;
                if (row < nrows) {
                    const size_t blk = (size_t)row * nb + b;
                    qva[r] = ldg16(qa + blk * 32 + (u & 1) * 16);
                    dva[r] = da[blk];
                    if (DUAL) {
                        qvb[r] = ldg16(qb + blk * 32 + (u & 1) * 16);
                        dvb[r] = db[blk];
                    }
                }
            }
            float xv[16];
            load_x16(xs, u, xv);
#pragma unroll
            for (int r = 0; r < R; r++)
                if (rbase + r < nrows) {
                    aa[r] += q8_half_dot(qva[r], f16_bits_to_f32(dva[r]), xv);
                    if (DUAL) ab[r] += q8_half_dot(qvb[r], f16_bits_to_f32(dvb[r]), xv);
                }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float va = group_sum<G>(aa[r]);
        float vb = 0.f;
        if (DUAL) vb = group_sum<G>(ab[r]);
        if (lane == 0 && rbase + r < nrows) y[rbase + r] = DUAL ? act_apply(act, va) * vb : va;
    }
}

template <int G, int CPL, bool DUAL>
static hipError_t launch_q8_t(const DevTensor &A, const DevTensor *B, const float *x, float *y, uint32_t act,
                              hipStream_t s) {
    const int nrows = (int)A.total_rows, nb = (int)A.blocks_per_row;
    const int groups = 256 / G;
    // fewer rows per group when the matrix is short, so the grid still covers the chip
    const int R = (nrows >= groups * 4 * 512) ? 4 : (nrows >= groups * 2 * 512 ? 2 : 1);
    const int nblk = (nrows + groups * R - 1) / (groups * R);
    const uint8_t *qb = DUAL ? B->p0 : nullptr;
    const uint16_t *db = DUAL ? (const uint16_t *)B->p1 : nullptr;
    const size_t lds = (size_t)nb * 32 * sizeof(float);
    if (R == 4)
        hipLaunchKernelGGL((k_matvec_q8_0<G, CPL, 4, DUAL>), dim3(nblk), dim3(256), lds, s, A.p0,
                           (const uint16_t *)A.p1, qb, db, x, y, nrows, nb, act);
    else if (R == 2)
        hipLaunchKernelGGL((k_matvec_q8_0<G, CPL, 2, DUAL>), dim3(nblk), dim3(256), lds, s, A.p0,
                           (const uint16_t *)A.p1, qb, db, x, y, nrows, nb, act);
    else
        hipLaunchKernelGGL((k_matvec_q8_0<G, CPL, 1, DUAL>), dim3(nblk), dim3(256), lds, s, A.p0,
                           (const uint16_t *)A.p1, qb, db, x, y, nrows, nb, act);
    return hipGetLastError();
}

template <bool DUAL>
static hipError_t launch_q8_any(const DevTensor &A, const DevTensor *B, const float *x, float *y, uint32_t act,
                                hipStream_t s) {
    const int nu = (int)A.blocks_per_row * 2;
    if (nu <= 8) return launch_q8_t<8, 1, DUAL>(A, B, x, y, act, s);
    if (nu <= 16) return launch_q8_t<16, 1, DUAL>(A, B, x, y, act, s);
    if (nu <= 32) return launch_q8_t<32, 1, DUAL>(A, B, x, y, act, s);
    switch ((nu + 63) / 64) {
    case 1: return launch_q8_t<64, 1, DUAL>(A, B, x, y, act, s);
    case 2: return launch_q8_t<64, 2, DUAL>(A, B, x, y, act, s);
    case 3: return launch_q8_t<64, 3, DUAL>(A, B, x, y, act, s);
    case 4: return launch_q8_t<64, 4, DUAL>(A, B, x, y, act, s);
    case 5: return launch_q8_t<64, 5, DUAL>(A, B, x, y, act, s);
    case 6: return launch_q8_t<64, 6, DUAL>(A, B, x, y, act, s);
    case 7: return launch_q8_t<64, 7, DUAL>(A, B, x, y, act, s);
    case 8: return launch_q8_t<64, 8, DUAL>(A, B, x, y, act, s);
    case 9: return launch_q8_t<64, 9, DUAL>(A, B, x, y, act, s);
    case 10: return launch_q8_t<64, 10, DUAL>(A, B, x, y, act, s);
    case 11: return launch_q8_t<64, 11, DUAL>(A, B, x, y, act, s);
    case 12: return launch_q8_t<64, 12, DUAL>(A, B, x, y, act, s);
    case 13: return launch_q8_t<64, 13, DUAL>(A, B, x, y, act, s);
    case 14: return launch_q8_t<64, 14, DUAL>(A, B, x, y, act, s);
    case 15: return launch_q8_t<64, 15, DUAL>(A, B, x, y, act, s);
    case 16: return launch_q8_t<64, 16, DUAL>(A, B, x, y, act, s);
    default: return hipErrorInvalidValue;  // K > 16384: rejected by the API layer
    }
}

hipError_t launch_matvec_q8_0(const DevTensor &W, const float *x, float *y, hipStream_t s) {
    return launch_q8_any<false>(W, nullptr, x, y, 0, s);
}

hipError_t launch_gate_up_q8_0(const DevTensor &Wg, const DevTensor &Wu, const float *x, uint32_t act, float *h,
                               hipStream_t s) {
    return launch_q8_any<true>(Wg, &Wu, x, h, act, s);
}

}  // namespace lt
