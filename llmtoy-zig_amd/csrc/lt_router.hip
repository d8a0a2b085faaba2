// lt_router.hip -- MoE router: logits with the reference's exact fp32
// operation order, then softmax + top-k in the last block to finish.
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
// The block that finishes last (atomic ticket) runs softmax + top-k over all
// logits in one wavefront, so routing costs one launch.
#include "lt_internal.h"
#include "lt_topk.h"

#include <math.h>

namespace lt {

namespace {

struct TopkArgs {
    unsigned *ticket;  // zero-initialised; wraps back to 0 after each launch
    int k;             // 0: logits only
    int norm;
    uint32_t *ids;
    float *w;
    float *scores;
};

// After this block's logits are stored: the last block to arrive runs the
// top-k.  Must be called by every thread of the block.
__device__ __forceinline__ void last_block_topk(const float *logits, int n, const TopkArgs &a) {
    if (a.k == 0) return;
    __shared__ int is_last;
    __threadfence();  // release this block's logits
    __syncthreads();
    if (threadIdx.x == 0) is_last = atomicInc(a.ticket, gridDim.x - 1) == gridDim.x - 1;
    __syncthreads();
    if (is_last && threadIdx.x < 64) {
        __threadfence();  // acquire the other blocks' logits
        const int lane = threadIdx.x;
        if (n <= 64)
            topk_softmax_wave<1>(logits, n, a.k, a.norm, a.ids, a.w, a.scores, lane);
        else if (n <= 128)
            topk_softmax_wave<2>(logits, n, a.k, a.norm, a.ids, a.w, a.scores, lane);
        else if (n <= 256)
            topk_softmax_wave<4>(logits, n, a.k, a.norm, a.ids, a.w, a.scores, lane);
        else
            topk_softmax_wave<16>(logits, n, a.k, a.norm, a.ids, a.w, a.scores, lane);
    }
}

}  // namespace

// One wavefront per two rows; lane = (row of the pair, chain c).  All
// MAXIT loads of a chain are issued before its first add.
template <int MAXIT>
__global__ void __launch_bounds__(64) k_router_f32(const float *__restrict__ W, const float *__restrict__ x,
                                                   const float *__restrict__ bias, float *__restrict__ logits,
                                                   int rows, int cols, TopkArgs ta) {
#pragma clang fp contract(off)
    __shared__ float chain[2][32];
    x += (size_t)blockIdx.y * cols;  // token blockIdx.y of a batch (decode: 0)
    logits += (size_t)blockIdx.y * rows;
    const int rl = threadIdx.x >> 5, c = threadIdx.x & 31;
    const int row = blockIdx.x * 2 + rl;
    const int nit = cols >> 5, n32 = nit << 5;
    const float *wr = W + (size_t)(row < rows ? row : 0) * cols;
    float a = 0.0f;
    if (row < rows) {
        for (int it0 = 0; it0 < nit; it0 += MAXIT) {
            float wv[MAXIT], xv[MAXIT];
#pragma unroll
            for (int t = 0; t < MAXIT; t++)
                if (it0 + t < nit) {
                    wv[t] = wr[(it0 + t) * 32 + c];
                    xv[t] = x[(it0 + t) * 32 + c];
                }
#pragma unroll
            for (int t = 0; t < MAXIT; t++)
                if (it0 + t < nit) {
                    float p = wv[t] * xv[t];
                    a = a + p;
                }
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
                float p = wr[i + l] * x[i + l];
                acc[l] = acc[l] + p;
            }
        float sum = acc[0];
#pragma unroll
        for (int l = 1; l < 8; l++) sum = sum + acc[l];
        for (; i < cols; i++) {
            float p = wr[i] * x[i];
            sum = sum + p;
        }
        if (bias) sum = sum + bias[row];
        logits[row] = sum;
    }
    last_block_topk(logits, rows, ta);
}

// One block (2 waves) per row: thread b computes block b's term
// reduce(acc)*d exactly, then thread 0 adds the terms in block order.
// With pa.raw_scale set (decode, one token), the router input is the
// Gemma4 prep of x (math.zig:51-82): every block takes the RMS of x in one
// fixed tree order (same bits in every block), uses
// (x * (rms_inv * raw_global_scale)) * raw_scale as its input, and writes its
// share of moe_in = (x * rms_inv) * weight for the expert kernels.
__global__ void __launch_bounds__(128) k_router_q8_0(const int8_t *__restrict__ qs, const uint16_t *__restrict__ dp,
                                                     const float *__restrict__ x, const float *__restrict__ bias,
                                                     float *__restrict__ logits, int nb, int rows, TopkArgs ta,
                                                     RouterPrep pa) {
#pragma clang fp contract(off)
    extern __shared__ float term[];
    x += (size_t)blockIdx.y * nb * 32;  // token blockIdx.y of a batch (decode: 0)
    logits += (size_t)blockIdx.y * rows;
    const int row = blockIdx.x;
    const int n = nb * 32;
    float raw_base = 0.0f;
    // Decode with the prep and one block per thread: the block's operands
    // (32 quants, d, x, raw_scale) are loaded before the RMS below, so their
    // latency overlaps it; the products and sums are the same as in the loop.
    const bool pre = pa.raw_scale && nb <= (int)blockDim.x;
    const int b0 = threadIdx.x;
    uint4 q4[2];
    float xv[32], sv[32];
    uint16_t d0 = 0;
    if (pre && b0 < nb) {
        const uint4 *qp = reinterpret_cast<const uint4 *>(qs + ((size_t)row * nb + b0) * 32);
        q4[0] = qp[0];
        q4[1] = qp[1];
        d0 = dp[(size_t)row * nb + b0];
        const float4 *xp = reinterpret_cast<const float4 *>(x + b0 * 32);
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const float4 v4 = xp[t];
            xv[4 * t] = v4.x;
            xv[4 * t + 1] = v4.y;
            xv[4 * t + 2] = v4.z;
            xv[4 * t + 3] = v4.w;
        }
#pragma unroll
        for (int e = 0; e < 32; e++) sv[e] = pa.raw_scale[b0 * 32 + e];
    }
    if (pa.raw_scale) {
        __shared__ float red[3];
        // float4 loads, 8 in flight per thread (n is a multiple of 32)
        float ss = 0.0f;
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
#pragma unroll 8
        for (int i = threadIdx.x; i < n / 4; i += blockDim.x) {
            const float4 v4 = x4[i];
            ss = ss + v4.x * v4.x;
            ss = ss + v4.y * v4.y;
            ss = ss + v4.z * v4.z;
            ss = ss + v4.w * v4.w;
        }
#pragma unroll
        for (int off = kWave / 2; off > 0; off >>= 1) ss = ss + __shfl_xor(ss, off, kWave);
        if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = ss;
        __syncthreads();
        const float r = 1.0f / sqrtf((red[0] + red[1]) / (float)n + pa.eps);
        raw_base = r * pa.raw_global_scale;
        const int per = (n + gridDim.x - 1) / gridDim.x;
        for (int i = row * per + threadIdx.x; i < n && i < (row + 1) * per; i += blockDim.x)
            pa.moe_in[i] = (x[i] * r) * pa.weight[i];
    }
    if (pre && b0 < nb) {
        const uint32_t qw[8] = {q4[0].x, q4[0].y, q4[0].z, q4[0].w, q4[1].x, q4[1].y, q4[1].z, q4[1].w};
        float acc[8];
#pragma unroll
        for (int l = 0; l < 8; l++) acc[l] = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int l = 0; l < 8; l++) {
                const int e = 8 * j + l;
                const int qe = (int)(int8_t)(qw[e >> 2] >> (8 * (e & 3)));
                const float vin = (xv[e] * raw_base) * sv[e];
                float p = (float)qe * vin;
                acc[l] = acc[l] + p;
            }
        float r = acc[0];
#pragma unroll
        for (int l = 1; l < 8; l++) r = r + acc[l];
        term[b0] = r * f16_bits_to_f32(d0);
    }
    for (int b = pre ? nb : threadIdx.x; b < nb; b += blockDim.x) {
        const int8_t *q = qs + ((size_t)row * nb + b) * 32;
        const float *v = x + b * 32;
        const float d = f16_bits_to_f32(dp[(size_t)row * nb + b]);
        float acc[8];
#pragma unroll
        for (int l = 0; l < 8; l++) acc[l] = 0.0f;
        if (pa.raw_scale) {
            const float *rs = pa.raw_scale + b * 32;
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int l = 0; l < 8; l++) {
                    const float vin = (v[8 * j + l] * raw_base) * rs[8 * j + l];
                    float p = (float)q[8 * j + l] * vin;
                    acc[l] = acc[l] + p;
                }
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int l = 0; l < 8; l++) {
                    float p = (float)q[8 * j + l] * v[8 * j + l];
                    acc[l] = acc[l] + p;
                }
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
    last_block_topk(logits, rows, ta);
}

hipError_t launch_router(const DevTensor &R, const float *x, const float *bias, float *logits, unsigned *ticket,
                         uint32_t k, uint32_t norm, uint32_t *ids, float *w, float *scores, hipStream_t s,
                         const RouterPrep *prep) {
    const RouterPrep pa = prep ? *prep : RouterPrep{};
    if (pa.raw_scale && R.type == 0) return hipErrorInvalidValue;  // the prep is fused into the Q8_0 router only
    const TopkArgs ta{ticket, (int)k, (int)norm, ids, w, scores};
    const int rows = (int)R.total_rows;
    if (R.type == 0) {  // F32
        const int cols = (int)R.cols;
        hipLaunchKernelGGL(k_router_f32<64>, dim3((rows + 1) / 2), dim3(64), 0, s, (const float *)R.p0, x, bias,
                           logits, rows, cols, ta);
    } else {  // Q8_0
        const int nb = (int)R.blocks_per_row;
        hipLaunchKernelGGL(k_router_q8_0, dim3(rows), dim3(128), nb * sizeof(float), s, (const int8_t *)R.p0,
                           (const uint16_t *)R.p1, x, bias, logits, nb, rows, ta, pa);
    }
    return hipGetLastError();
}

// Batched F32 router (prefill): block = RB router rows x TB tokens.  Thread
// (c = tid % 32, g = tid / 32) runs dotf32 chain c (elements 32 it + c) of
// 4 rows x 4 tokens side by side -- the same rounded products and adds in
// the same order per chain as k_router_f32, so the logits are identical --
// with K staged through LDS 256 at a time (double-buffered) and each loaded
// value used by 4 chains.  The 32 chain totals of a (row, token) then meet
// in LDS for the (acc0+acc1)+(acc2+acc3) and ordered lane reduce.
// Requires cols % 256 == 0.
// With Xh set, the same launch writes the prefill's f16 X (Xh, row scales
// rs; prefill_x_exp / prefill_x_store8): token t0 + j of the tile is
// converted by wavefront w of the row block with j = blockIdx.x + gridDim.x
// * w (gridDim.x >= TB / 4), its max |x| taken from the X chunks as they
// pass through LDS.  (Running the top-k in the last row block of each token
// tile as well, behind an arrival ticket, made the launch 70 us instead of
// 15: the release fences of 512 blocks write back the L2s the f16 rows have
// filled.)
constexpr int RT_RB = 8, RT_TB = 16, RT_KC = 256;

__global__ void __launch_bounds__(256) k_router_f32_tile(const float *__restrict__ W, const float *__restrict__ X,
                                                         const float *__restrict__ bias, float *__restrict__ logits,
                                                         int rows, int cols, int T, _Float16 *__restrict__ Xh,
                                                         float *__restrict__ rs) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) float ws[2][RT_RB][RT_KC];
    __shared__ __attribute__((aligned(16))) float xs[2][RT_TB][RT_KC];
    __shared__ float ch[RT_RB][RT_TB][33];
    const int tid = threadIdx.x, c = tid & 31, g = tid >> 5;
    const int wave = tid >> 6, lane = tid & 63;
    const int rg = g & 1, tg = g >> 1;  // rows 4 rg + [0, 4), tokens 4 tg + [0, 4)
    const int r0 = blockIdx.x * RT_RB, t0 = blockIdx.y * RT_TB;
    // this wavefront's token for the f16 X (uniform over the wavefront)
    const int xj = blockIdx.x + gridDim.x * wave;
    const bool xconv = Xh && xj < RT_TB && t0 + xj < T;
    float xmax = 0.0f;
    // stage loads: W tile 8 x 256 = 512 float4 (2 per thread), X tile
    // 16 x 256 = 1024 float4 (4 per thread); rows / tokens past the end
    // re-read the last valid one (never used)
    const float *wsrc[2], *xsrc[4];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int f = tid + 256 * u, r = f >> 6;
        wsrc[u] = W + (size_t)min(r0 + r, rows - 1) * cols + (f & 63) * 4;
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int f = tid + 256 * u, t = f >> 6;
        xsrc[u] = X + (size_t)min(t0 + t, T - 1) * cols + (f & 63) * 4;
    }
    float4 wr[2], xr[4];
#pragma unroll
    for (int u = 0; u < 2; u++) wr[u] = ldg16f(wsrc[u]);
#pragma unroll
    for (int u = 0; u < 4; u++) xr[u] = ldg16f(xsrc[u]);
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = 0.0f;
    const int nkc = cols / RT_KC;
    for (int kc = 0; kc < nkc; kc++) {
        const int b = kc & 1;
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int f = tid + 256 * u;
            *reinterpret_cast<float4 *>(&ws[b][f >> 6][(f & 63) * 4]) = wr[u];
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int f = tid + 256 * u;
            *reinterpret_cast<float4 *>(&xs[b][f >> 6][(f & 63) * 4]) = xr[u];
        }
        __syncthreads();
        if (kc + 1 < nkc) {  // next chunk's loads in flight during this one
#pragma unroll
            for (int u = 0; u < 2; u++) wr[u] = ldg16f(wsrc[u] + (kc + 1) * RT_KC);
#pragma unroll
            for (int u = 0; u < 4; u++) xr[u] = ldg16f(xsrc[u] + (kc + 1) * RT_KC);
        }
        if (xconv) {
            const float4 v = *reinterpret_cast<const float4 *>(&xs[b][xj][4 * lane]);
            xmax = fmaxf(xmax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
#pragma unroll
        for (int it = 0; it < RT_KC / 32; it++) {
            float wv[4], xv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) wv[i] = ws[b][4 * rg + i][it * 32 + c];
#pragma unroll
            for (int j = 0; j < 4; j++) xv[j] = xs[b][4 * tg + j][it * 32 + c];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float p = wv[i] * xv[j];
                    acc[i][j] = acc[i][j] + p;
                }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) ch[4 * rg + i][4 * tg + j][c] = acc[i][j];
    __syncthreads();
    if (tid < RT_RB * RT_TB) {
        const int r = tid / RT_TB, t = tid % RT_TB, row = r0 + r, tok = t0 + t;
        if (row < rows && tok < T) {
            const float *cv = ch[r][t];
            float a8[8];
#pragma unroll
            for (int l = 0; l < 8; l++) {
                const float s01 = cv[l] + cv[8 + l];
                const float s23 = cv[16 + l] + cv[24 + l];
                a8[l] = s01 + s23;
            }
            float sum = a8[0];
#pragma unroll
            for (int l = 1; l < 8; l++) sum = sum + a8[l];
            if (bias) sum = sum + bias[row];
            logits[(size_t)tok * rows + row] = sum;
        }
    }
    if (xconv) {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) xmax = fmaxf(xmax, __shfl_xor(xmax, off, 64));
        const int e = prefill_x_exp(xmax);
        const int tok = t0 + xj;
        if (lane == 0) rs[tok] = ldexpf(1.0f, e);
        const float inv = ldexpf(1.0f, -e);
        const float *xrow = X + (size_t)tok * cols;
        _Float16 *hrow = Xh + (size_t)tok * cols;
        for (int i = 8 * lane; i < cols; i += 8 * 64) prefill_x_store8(xrow, inv, hrow, i);
    }
}

// Softmax + top-k of token blockIdx.x of a batch of logits rows.
template <int PER>
__global__ void __launch_bounds__(64) k_topk_rows(const float *__restrict__ logits, int n, int k, int norm,
                                                  uint32_t *__restrict__ ids, float *__restrict__ w) {
    const size_t t = blockIdx.x;
    topk_softmax_wave<PER>(logits + t * n, n, k, norm, ids + t * k, w + t * k, nullptr, threadIdx.x);
}

hipError_t launch_router_batched(const DevTensor &R, const float *X, int T, const float *bias, float *logits,
                                 uint32_t k, uint32_t norm, uint32_t *ids, float *w, _Float16 *Xh, float *rs,
                                 bool *x_done, hipStream_t s) {
    const TopkArgs none{nullptr, 0, 0, nullptr, nullptr, nullptr};
    const int rows = (int)R.total_rows;
    *x_done = false;
    if (R.type == 0 && R.cols % RT_KC == 0) {
        const int gx = (rows + RT_RB - 1) / RT_RB;
        *x_done = Xh && 4 * gx >= RT_TB;  // every token of a tile has a wavefront to convert it
        hipLaunchKernelGGL(k_router_f32_tile, dim3(gx, (T + RT_TB - 1) / RT_TB), dim3(256), 0, s,
                           (const float *)R.p0, X, bias, logits, rows, (int)R.cols, T, *x_done ? Xh : nullptr, rs);
    } else if (R.type == 0)
        hipLaunchKernelGGL(k_router_f32<64>, dim3((rows + 1) / 2, T), dim3(64), 0, s, (const float *)R.p0, X, bias,
                           logits, rows, (int)R.cols, none);
    else
        hipLaunchKernelGGL(k_router_q8_0, dim3(rows, T), dim3(128), R.blocks_per_row * sizeof(float), s,
                           (const int8_t *)R.p0, (const uint16_t *)R.p1, X, bias, logits, (int)R.blocks_per_row,
                           rows, none, RouterPrep{});
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (rows <= 64)
        hipLaunchKernelGGL(k_topk_rows<1>, dim3(T), dim3(64), 0, s, logits, rows, (int)k, (int)norm, ids, w);
    else if (rows <= 128)
        hipLaunchKernelGGL(k_topk_rows<2>, dim3(T), dim3(64), 0, s, logits, rows, (int)k, (int)norm, ids, w);
    else if (rows <= 256)
        hipLaunchKernelGGL(k_topk_rows<4>, dim3(T), dim3(64), 0, s, logits, rows, (int)k, (int)norm, ids, w);
    else
        hipLaunchKernelGGL(k_topk_rows<16>, dim3(T), dim3(64), 0, s, logits, rows, (int)k, (int)norm, ids, w);
    return hipGetLastError();
}

hipError_t launch_matvec_f32(const DevTensor &W, const float *x, float *y, hipStream_t s) {
    return launch_router(W, x, nullptr, y, nullptr, 0, 0, nullptr, nullptr, nullptr, s);
}

}  // namespace lt
