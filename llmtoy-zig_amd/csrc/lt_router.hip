// lt_router.hip -- MoE router: logits with the reference's exact fp32
// operation order, then softmax + top-k in one wavefront.
//
// Routing must match the CPU path bit for bit.  Selection depends only on the
// order of the logits, so the logits are computed with exactly the rounded
// multiplies and adds of the reference's dot products (no FMA contraction):
//   F32 router:  dotf32 (ops/math.zig:96-116): 32 independent chains
//                acc_{c/8}[c%8] over i = c, c+32, ...; acc = (acc0+acc1) +
//                (acc2+acc3) per lane l; 8-wide tail; ordered lane reduce;
//                scalar tail.
//   Q8_0 router: dotQ8_0 (quant/dequant.zig:59-78): per block, 8 lane
//                accumulators over 4 groups, ordered reduce, times d, added
//                to a running total in block order.
#include "lt_internal.h"

#include <math.h>

namespace lt {

// One thread per (row, chain); 8 rows x 32 chains per 256-thread block.
__global__ void __launch_bounds__(256) k_router_f32(const float *__restrict__ W, const float *__restrict__ x,
                                                    const float *__restrict__ bias, float *__restrict__ logits,
                                                    int rows, int cols) {
#pragma clang fp contract(off)
    __shared__ float chain[8][32];
    const int rl = threadIdx.x >> 5, c = threadIdx.x & 31;
    const int row = blockIdx.x * 8 + rl;
    const int n32 = cols & ~31;
    const float *w = W + (size_t)(row < rows ? row : 0) * cols;
    float a = 0.0f;
    if (row < rows) {
#pragma unroll 16
        for (int i = 0; i < n32; i += 32) {
            float p = w[i + c] * x[i + c];
            a = a + p;
        }
    }
    chain[rl][c] = a;
    __syncthreads();
    if (c == 0 && row < rows) {
        float acc[8];
#pragma unroll
        for (int l = 0; l < 8; l++) {
            float s01 = chain[rl][l] + chain[rl][8 + l];
            float s23 = chain[rl][16 + l] + chain[rl][24 + l];
            acc[l] = s01 + s23;
        }
        int i = n32;
        for (; i + 8 <= cols; i += 8)
#pragma unroll
            for (int l = 0; l < 8; l++) {
                float p = w[i + l] * x[i + l];
                acc[l] = acc[l] + p;
            }
        float sum = acc[0];
#pragma unroll
        for (int l = 1; l < 8; l++) sum = sum + acc[l];
        for (; i < cols; i++) {
            float p = w[i] * x[i];
            sum = sum + p;
        }
        if (bias) sum = sum + bias[row];
        logits[row] = sum;
    }
}

hipError_t launch_router_f32(const DevTensor &R, const float *x, const float *bias, float *logits,
                             hipStream_t s) {
    const int rows = (int)R.total_rows, cols = (int)R.cols;
    hipLaunchKernelGGL(k_router_f32, dim3((rows + 7) / 8), dim3(256), 0, s, (const float *)R.p0, x, bias, logits,
                       rows, cols);
    return hipGetLastError();
}

hipError_t launch_matvec_f32(const DevTensor &W, const float *x, float *y, hipStream_t s) {
    return launch_router_f32(W, x, nullptr, y, s);
}

// One block per row: thread b computes block b's term reduce(acc)*d exactly,
// then thread 0 adds the terms in block order.
__global__ void __launch_bounds__(256) k_router_q8_0(const int8_t *__restrict__ qs, const uint16_t *__restrict__ dp,
                                                     const float *__restrict__ x, const float *__restrict__ bias,
                                                     float *__restrict__ logits, int nb) {
#pragma clang fp contract(off)
    extern __shared__ float term[];
    const int row = blockIdx.x;
    for (int b = threadIdx.x; b < nb; b += blockDim.x) {
        const int8_t *q = qs + ((size_t)row * nb + b) * 32;
        const float *v = x + b * 32;
        const float d = f16_bits_to_f32(dp[(size_t)row * nb + b]);
        float acc[8];
#pragma unroll
        for (int l = 0; l < 8; l++) acc[l] = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int l = 0; l < 8; l++) {
                float p = (float)q[8 * j + l] * v[8 * j + l];
                acc[l] = acc[l] + p;
            }
        float r = acc[0];
#pragma unroll
        for (int l = 1; l < 8; l++) r = r + acc[l];
        term[b] = r * d;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float total = 0.0f;
        for (int b = 0; b < nb; b++) total = total + term[b];
        if (bias) total = total + bias[row];
        logits[row] = total;
    }
}

hipError_t launch_router_q8_0(const DevTensor &R, const float *x, const float *bias, float *logits,
                              hipStream_t s) {
    const int rows = (int)R.total_rows, nb = (int)R.blocks_per_row;
    hipLaunchKernelGGL(k_router_q8_0, dim3(rows), dim3(128), nb * sizeof(float), s, (const int8_t *)R.p0,
                       (const uint16_t *)R.p1, x, bias, logits, nb);
    return hipGetLastError();
}

// ------------------------------------------------------------------------
// Softmax + top-k in a single wavefront (n <= 1024, k <= 16).
// Selection is on the logits, descending, the lowest index winning ties --
// the rule of every top-k in the reference (strict '>': ops/moe.zig:87,
// gemma4/forward.zig:612-625).  NaN logits never win over a number.
// w[i] = exp(l_i - max) / sum_j exp(l_j - max); with norm, w[i] is divided by
// the sum of the selected weights taken in selection order.
__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) {
    // true if (va, ia) ranks before (vb, ib)
    return va > vb || (!(va < vb) && ia < ib);
}

__global__ void __launch_bounds__(64) k_topk_softmax(const float *__restrict__ logits, int n, int k, int norm,
                                                     uint32_t *__restrict__ ids, float *__restrict__ w,
                                                     float *__restrict__ scores) {
    const int lane = threadIdx.x;
    constexpr int PER = 16;
    float v[PER];
    bool taken[PER];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int idx = lane + 64 * j;
        float t = idx < n ? logits[idx] : -INFINITY;
        if (t != t) t = -INFINITY;  // NaN ranks last
        v[j] = t;
        taken[j] = idx >= n;
        m = fmaxf(m, t);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    float se = 0.0f;
#pragma unroll
    for (int j = 0; j < PER; j++)
        if (lane + 64 * j < n) se += expf(v[j] - m);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) se += __shfl_xor(se, off, 64);

    float selv[16];
    int seli[16];
    for (int r = 0; r < k; r++) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int idx = lane + 64 * j;
            if (!taken[j] && better(v[j], idx, bv, bi)) {
                bv = v[j];
                bi = idx;
            }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            float ov = __shfl_xor(bv, off, 64);
            int oi = __shfl_xor(bi, off, 64);
            if (better(ov, oi, bv, bi)) {
                bv = ov;
                bi = oi;
            }
        }
#pragma unroll
        for (int j = 0; j < PER; j++)
            if (lane + 64 * j == bi) taken[j] = true;
        selv[r] = bv;
        seli[r] = bi;
    }
    // bv/bi, hence selv/seli, m and se, are identical in every lane here.
    float p[16];
    float ps = 0.0f;
    for (int r = 0; r < k; r++) {
        p[r] = expf(selv[r] - m) / se;
        ps = ps + p[r];
    }
    if (lane == 0)
        for (int r = 0; r < k; r++) {
            ids[r] = (uint32_t)seli[r];
            w[r] = norm ? p[r] / ps : p[r];
        }
    if (scores) {
        // routerTopKSoftmax's buffer: probabilities at the selected experts,
        // logits elsewhere.  Each lane writes only its own entries.
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int idx = lane + 64 * j;
            if (idx < n) {
                float val = logits[idx];
                for (int r = 0; r < k; r++)
                    if (seli[r] == idx) val = p[r];
                scores[idx] = val;
            }
        }
    }
}

hipError_t launch_topk_softmax(const float *logits, uint32_t n, uint32_t k, uint32_t norm, uint32_t *ids,
                               float *w, float *scores, hipStream_t s) {
    hipLaunchKernelGGL(k_topk_softmax, dim3(1), dim3(64), 0, s, logits, (int)n, (int)k, (int)norm, ids, w, scores);
    return hipGetLastError();
}

}  // namespace lt
