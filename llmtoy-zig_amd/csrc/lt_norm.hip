// lt_norm.hip -- RMS normalisation and the Gemma4 MoE tail on the device.
//
//   k_norm<OP>, OP = kRms        out = x * rms_inv * w          math.zig:19-25
//                                (w null: rmsnormRaw, math.zig:42-48;
//                                 (1 + w) with LT_NORM_ONE_PLUS_W, rmsnorm.glsl)
//                    kAddRms     out = rmsnorm(a + b, w)        add_rmsnorm.glsl
//                    kWrs        weighted and raw-scaled outputs math.zig:51-82
//                    kTail       x = (x + rmsnorm(dense + rmsnorm(moe, w2), w)) * s
//                                                               gemma4/forward.zig:482-497
//
// One workgroup per row (rows of n <= kMaxNormCols floats).  The row is
// staged in LDS once; the sum of squares is either a fixed-shape tree
// (per-lane strided partials, wavefront butterfly, then the wavefront
// totals in order: same bits on every run) or, with LT_NORM_PRECISE, the
// reference's sequential index-order sum taken by one lane (bit-exact with
// the CPU code; n dependent adds).  Every product and sum is a separately
// rounded operation (FMA contraction is off for this file), and rms_inv =
// 1 / sqrt(ss / n + eps) uses HIP's correctly rounded fp32 division and
// sqrtf (the default -fhip-fp32-correctly-rounded-divide-sqrt), as the
// reference's f32 arithmetic does.  (HIP's __fadd_rn / __fmul_rn are plain
// operators that may still be contracted, and __fsqrt_rn is the native
// approximation, so neither is used.)
#include "llmtoy_hip.h"
#include "lt_internal.h"

#pragma clang fp contract(off)

namespace lt {

namespace {

enum NormOp { kRms = 0, kAddRms = 1, kWrs = 2, kTail = 3 };

constexpr int kNormThreads = 1024;

struct NormArgs {
    const float *a, *b;   // kRms/kWrs: a = x; kAddRms: a + b; kTail: a = moe, b = dense
    const float *w, *w2;  // kWrs: w2 = raw_scale; kTail: w2 = post_ffw_norm_2, w = post_ffw_norm
    float *out, *out2;    // kWrs: out2 = raw-scaled output; kTail: out = x (read and written)
    int n;
    float eps, scale;     // kWrs: raw_global_scale; kTail: layer_output_scale
    int precise, one_plus_w;
};

// Sum of v[i]^2 over the LDS row, returned to every thread.  red holds
// kNormThreads / kWave + 1 floats; the last one carries the result.
__device__ float row_sum_sq(const float *v, int n, int precise, float *red) {
    constexpr int kOut = kNormThreads / kWave;
    const int tid = threadIdx.x, nw = blockDim.x / kWave;
    if (precise) {
        if (tid == 0) {
            float ss = 0.0f;
            for (int i = 0; i < n; i++) ss = ss + v[i] * v[i];
            red[kOut] = ss;
        }
    } else {
        float s = 0.0f;
        for (int i = tid; i < n; i += blockDim.x) s = s + v[i] * v[i];
#pragma unroll
        for (int off = kWave / 2; off > 0; off >>= 1) s = s + __shfl_xor(s, off, kWave);
        if (tid % kWave == 0) red[tid / kWave] = s;
        __syncthreads();
        if (tid == 0) {
            float t = red[0];
            for (int i = 1; i < nw; i++) t = t + red[i];
            red[kOut] = t;
        }
    }
    __syncthreads();
    const float ss = red[kOut];
    __syncthreads();  // red may be reused by the next reduction
    return ss;
}

__device__ __forceinline__ float rms_inv_of(float ss, int n, float eps) {
    return 1.0f / sqrtf(ss / (float)n + eps);
}

template <int OP>
__global__ __launch_bounds__(kNormThreads) void k_norm(NormArgs p) {
    extern __shared__ float v[];  // n floats
    __shared__ float red[kNormThreads / kWave + 1];
    const int n = p.n, tid = threadIdx.x;
    const size_t row = (size_t)blockIdx.x * n;
    const float *a = p.a + row;
    const float *b = p.b ? p.b + row : nullptr;
    // kTail over rows of up to kPre * blockDim.x floats: the operands of the
    // two later passes (dense, the two norm weights, x) are loaded now, so
    // their latency overlaps the staging and the first reduction.
    constexpr int kPre = 4;
    const bool pre = OP == kTail && n <= kPre * (int)blockDim.x;
    float tb[kPre], tw2[kPre], tx[kPre], tw[kPre];
    if (pre) {
#pragma unroll
        for (int k = 0; k < kPre; k++) {
            const int i = tid + k * (int)blockDim.x;
            if (i < n) {
                tb[k] = b[i];
                tw2[k] = p.w2[i];
                tx[k] = p.out[row + i];
                tw[k] = p.w[i];
            }
        }
    }
    for (int i = tid; i < n; i += blockDim.x) v[i] = OP == kAddRms ? a[i] + b[i] : a[i];
    __syncthreads();
    float r = rms_inv_of(row_sum_sq(v, n, p.precise, red), n, p.eps);
    const float bias = p.one_plus_w ? 1.0f : 0.0f;
    if (OP == kRms || OP == kAddRms) {
        float *out = p.out + row;
        for (int i = tid; i < n; i += blockDim.x) {
            const float t = v[i] * r;
            out[i] = p.w ? t * (bias + p.w[i]) : t;
        }
    } else if (OP == kWrs) {
        const float raw_base = r * p.scale;
        for (int i = tid; i < n; i += blockDim.x) {
            p.out[row + i] = (v[i] * r) * p.w[i];
            p.out2[row + i] = (v[i] * raw_base) * p.w2[i];
        }
    } else {  // kTail: v = moe
        if (pre) {
#pragma unroll
            for (int k = 0; k < kPre; k++) {
                const int i = tid + k * (int)blockDim.x;
                if (i < n) v[i] = tb[k] + (v[i] * r) * tw2[k];  // dense + rmsnorm(moe, w2)
            }
        } else {
            for (int i = tid; i < n; i += blockDim.x) v[i] = b[i] + (v[i] * r) * p.w2[i];
        }
        __syncthreads();
        r = rms_inv_of(row_sum_sq(v, n, p.precise, red), n, p.eps);
        float *x = p.out + row;
        if (pre) {
#pragma unroll
            for (int k = 0; k < kPre; k++) {
                const int i = tid + k * (int)blockDim.x;
                if (i < n) {
                    float y = tx[k] + (v[i] * r) * tw[k];
                    if (p.scale != 1.0f) y = y * p.scale;
                    x[i] = y;
                }
            }
        } else {
            for (int i = tid; i < n; i += blockDim.x) {
                float y = x[i] + (v[i] * r) * p.w[i];
                if (p.scale != 1.0f) y = y * p.scale;
                x[i] = y;
            }
        }
    }
}

}  // namespace

hipError_t launch_norm(int op, const float *a, const float *b, const float *w, const float *w2, float *out,
                       float *out2, int rows, int n, float eps, float scale, int precise, int one_plus_w,
                       hipStream_t s) {
    if (n < 1 || n > kMaxNormCols || rows < 1) return hipErrorInvalidValue;
    const NormArgs p{a, b, w, w2, out, out2, n, eps, scale, precise, one_plus_w};
    const size_t lds = (size_t)n * sizeof(float);
    const dim3 grid(rows), block(kNormThreads);
    const void *fn = op == kRms      ? (const void *)k_norm<kRms>
                     : op == kAddRms ? (const void *)k_norm<kAddRms>
                     : op == kWrs    ? (const void *)k_norm<kWrs>
                     : op == kTail   ? (const void *)k_norm<kTail>
                                     : nullptr;
    if (!fn) return hipErrorInvalidValue;
    // rows of more than 16 K - 17 floats take more than 64 KiB of LDS with the
    // static part: allow the full row, once per kernel and device
    static bool lds_set[4][64] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    if (!lds_set[op][dev]) {
        e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)(kMaxNormCols * 4));
        if (e != hipSuccess) return e;
        lds_set[op][dev] = true;
    }
    switch (op) {
    case kRms: hipLaunchKernelGGL(k_norm<kRms>, grid, block, lds, s, p); break;
    case kAddRms: hipLaunchKernelGGL(k_norm<kAddRms>, grid, block, lds, s, p); break;
    case kWrs: hipLaunchKernelGGL(k_norm<kWrs>, grid, block, lds, s, p); break;
    default: hipLaunchKernelGGL(k_norm<kTail>, grid, block, lds, s, p); break;
    }
    return hipGetLastError();
}

}  // namespace lt
