// lt_prefill.hip -- batched prefill of one MoE layer (Q4_K experts) on MFMA.
//
// The reference prefills one token at a time through the decode path
// (main.zig:1916-1922).  Here T tokens go through the layer together:
//   1. router logits for all tokens with the reference's exact dotf32 order
//      and per-token softmax / top-k (lt_router.hip);
//   2. dispatch: one block counts tokens per expert, lays out per-expert
//      row ranges and a list of 32-row tiles, and scatters (token, slot)
//      assignments into them;
//   3. grouped gate/up GEMM: per (tile, 64 output columns) block, X rows
//      are converted to bf16 and the expert's Q4_K gate and up rows are
//      dequantised to bf16 in LDS, half a super-block (128 K) at a time;
//      v_mfma_f32_32x32x16_bf16 accumulates in fp32; the epilogue applies
//      act(gate) * up and stores H (bf16);
//   4. grouped down GEMM: H tiles (bf16, read straight into MFMA operand
//      registers) times the expert's dequantised down rows -> Y (fp32);
//   5. combine: out[t] = sum over slots in slot order of w[t][s] * Y[pos].
// A row's result does not depend on which tile position it lands in, so the
// atomically assigned positions leave the output bit-identical run to run.
#include "lt_internal.h"

namespace lt {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float floatx16;

namespace {

constexpr int BM = 32;        // tokens (rows of X / H) per tile
constexpr int KS = 128;       // K per LDS stage: half a Q4_K super-block
constexpr int LDK = KS + 8;   // padded LDS row (bf16 elements)
constexpr int BN1 = 64;       // gate/up output columns per block (x2 for gate and up)
constexpr int BN2 = 128;      // down output columns per block

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

struct Ws {
    float *logits;
    uint32_t *ids;
    float *w;
    int *offsets;   // [E+1]
    int *tiles;     // [max_tiles][2] = (expert, first row)
    int *n_tiles;   // [1]
    int *perm;      // [T*k] token of each sorted row
    int *pos;       // [T*k] sorted row of assignment t*k + s
    __bf16 *H;      // [T*k][Kd]
    float *Y;       // [T*k][D]
};

int max_tiles(int TK, int E) { return (TK + BM - 1) / BM + E; }

Ws carve(void *base, int T, int k, int E, int Kd, int D) {
    uint8_t *p = (uint8_t *)base;
    const size_t TK = (size_t)T * k;
    Ws w;
    w.logits = (float *)p; p += align256((size_t)T * E * 4);
    w.ids = (uint32_t *)p; p += align256(TK * 4);
    w.w = (float *)p; p += align256(TK * 4);
    w.offsets = (int *)p; p += align256((size_t)(E + 1) * 4);
    w.tiles = (int *)p; p += align256((size_t)max_tiles((int)TK, E) * 8);
    w.n_tiles = (int *)p; p += 256;
    w.perm = (int *)p; p += align256(TK * 4);
    w.pos = (int *)p; p += align256(TK * 4);
    w.H = (__bf16 *)p; p += align256(TK * Kd * 2);
    w.Y = (float *)p; p += align256(TK * D * 4);
    return w;
}

// Q4_K chunk cc (0..7) of a super-block dequantised to fp32 -> bf16:
// out_lo[t] = element 64p + 16(cc&1) + t, out_hi[t] = that + 32 (p = cc/2).
__device__ __forceinline__ void q4k_chunk_to_bf16(uint4 hdr, uint4 q, int cc, __bf16 *out_lo, __bf16 *out_hi) {
    const float d = f16_bits_to_f32(hdr.x), dmin = f16_bits_to_f32(hdr.x >> 16);
    const int p = cc >> 1;
    const int sh = (p & 1) * 16;
    const uint32_t ys = hdr.y >> sh, zs = hdr.z >> sh, ws = hdr.w >> sh;
    const uint32_t scp = opaque(p < 2 ? (ys & 0x3f3fu) : ((ws & 0x0f0fu) | ((ys >> 2) & 0x3030u)));
    const uint32_t mnp = opaque(p < 2 ? (zs & 0x3f3fu) : (((ws >> 4) & 0x0f0fu) | ((zs >> 2) & 0x3030u)));
    const float d1 = d * (float)(scp & 0xffu), m1 = dmin * (float)(mnp & 0xffu);
    const float d2 = d * (float)((scp >> 8) & 0xffu), m2 = dmin * (float)((mnp >> 8) & 0xffu);
    const uint32_t wv[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint32_t lo = opaque(wv[t] & 0x0f0f0f0fu), hi = opaque((wv[t] >> 4) & 0x0f0f0f0fu);
        out_lo[4 * t + 0] = (__bf16)(d1 * (float)(lo & 0xffu) - m1);
        out_lo[4 * t + 1] = (__bf16)(d1 * (float)((lo >> 8) & 0xffu) - m1);
        out_lo[4 * t + 2] = (__bf16)(d1 * (float)((lo >> 16) & 0xffu) - m1);
        out_lo[4 * t + 3] = (__bf16)(d1 * (float)(lo >> 24) - m1);
        out_hi[4 * t + 0] = (__bf16)(d2 * (float)(hi & 0xffu) - m2);
        out_hi[4 * t + 1] = (__bf16)(d2 * (float)((hi >> 8) & 0xffu) - m2);
        out_hi[4 * t + 2] = (__bf16)(d2 * (float)((hi >> 16) & 0xffu) - m2);
        out_hi[4 * t + 3] = (__bf16)(d2 * (float)(hi >> 24) - m2);
    }
}

// Dequantise rows [row0 + r] (r < NR) for K stage ks (half super-block) into
// Bs[r][0..KS).  Stage ks covers chunks 4*(ks&1) .. +3 of super-block ks/2;
// chunk cc's elements land at local K 64*(p - 2*(ks&1)) + 16*(cc&1) + t and
// +32.
template <int NR>
__device__ __forceinline__ void stage_weights(__bf16 (*Bs)[LDK], const uint8_t *hdr, const uint8_t *qs, int nsb,
                                              int ks, const size_t *wrow) {
    const int sb = ks >> 1, half = ks & 1;
    for (int u = threadIdx.x; u < NR * 4; u += blockDim.x) {
        const int r = u >> 2, c = u & 3, cc = half * 4 + c;
        const size_t blk = wrow[r] * nsb + sb;
        const uint4 h16 = ldg16(hdr + blk * 16), q16 = ldg16(qs + blk * 128 + cc * 16);
        const int local = 64 * ((cc >> 1) - 2 * half) + 16 * (cc & 1);
        q4k_chunk_to_bf16(h16, q16, cc, &Bs[r][local], &Bs[r][local + 32]);
    }
}

}  // namespace

// ---------------------------------------------------------------- dispatch
__global__ void __launch_bounds__(1024) k_prefill_dispatch(const uint32_t *__restrict__ ids, int TK, int k, int E,
                                                           int *__restrict__ offsets, int *__restrict__ tiles,
                                                           int *__restrict__ n_tiles, int *__restrict__ perm,
                                                           int *__restrict__ pos) {
    __shared__ int cnt[1024], cur[1024], toff[1024];
    for (int e = threadIdx.x; e < E; e += blockDim.x) cnt[e] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < TK; i += blockDim.x) {
        const uint32_t e = ids[i];
        if (e < (uint32_t)E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int off = 0, to = 0;
        for (int e = 0; e < E; e++) {
            offsets[e] = off;
            cur[e] = off;
            toff[e] = to;
            off += cnt[e];
            to += (cnt[e] + BM - 1) / BM;
        }
        offsets[E] = off;
        *n_tiles = to;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x)
        for (int j = 0; j * BM < cnt[e]; j++) {
            tiles[2 * (toff[e] + j)] = e;
            tiles[2 * (toff[e] + j) + 1] = j * BM;
        }
    for (int i = threadIdx.x; i < TK; i += blockDim.x) {
        const uint32_t e = ids[i];
        if (e < (uint32_t)E) {
            const int p = atomicAdd(&cur[e], 1);
            perm[p] = i / k;
            pos[i] = p;
        } else {
            pos[i] = -1;
        }
    }
}

// ---------------------------------------------------------------- gate/up
// Block: tile (expert e, rows m0..m0+31 of its range) x output columns
// [n0, n0+64) of both gate and up.  Waves 0,1 hold gate columns n0+32w..,
// waves 2,3 the matching up columns.
__global__ void __launch_bounds__(256) k_prefill_gate_up(const uint8_t *__restrict__ hdr,
                                                         const uint8_t *__restrict__ qs, int nsb, int F,
                                                         const float *__restrict__ X, int D,
                                                         const int *__restrict__ tiles,
                                                         const int *__restrict__ n_tiles,
                                                         const int *__restrict__ offsets,
                                                         const int *__restrict__ perm, uint32_t act,
                                                         __bf16 *__restrict__ H, int Kd) {
    if ((int)blockIdx.x >= *n_tiles) return;
    const int e = tiles[2 * blockIdx.x], m0 = tiles[2 * blockIdx.x + 1];
    const int base = offsets[e], cnt = offsets[e + 1] - base;
    const int n0 = blockIdx.y * BN1;
    __shared__ __attribute__((aligned(16))) __bf16 As[BM][LDK];
    __shared__ __attribute__((aligned(16))) __bf16 Bs[2 * BN1][LDK];
    __shared__ int tok[BM];
    __shared__ size_t wrow[2 * BN1];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    if (tid < BM) tok[tid] = (m0 + tid < cnt) ? perm[base + m0 + tid] : -1;
    if (tid < 2 * BN1)
        wrow[tid] = (size_t)e * 2 * F + (tid < BN1 ? n0 + tid : F + n0 + (tid - BN1));
    floatx16 acc = {};
    for (int ks = 0; ks < 2 * nsb; ks++) {
        __syncthreads();  // previous stage consumed; tok / wrow visible
        for (int i = tid; i < BM * KS / 4; i += 256) {
            const int m = i / (KS / 4), c4 = i % (KS / 4);
            const int t = tok[m];
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (t >= 0) v = ldg16f(X + (size_t)t * D + ks * KS + c4 * 4);
            As[m][c4 * 4 + 0] = (__bf16)v.x;
            As[m][c4 * 4 + 1] = (__bf16)v.y;
            As[m][c4 * 4 + 2] = (__bf16)v.z;
            As[m][c4 * 4 + 3] = (__bf16)v.w;
        }
        stage_weights<2 * BN1>(Bs, hdr, qs, nsb, ks, wrow);
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < KS / 16; kk++) {
            const bf16x8 a = *reinterpret_cast<const bf16x8 *>(&As[lane & 31][kk * 16 + (lane >> 5) * 8]);
            const bf16x8 b = *reinterpret_cast<const bf16x8 *>(&Bs[32 * wave + (lane & 31)][kk * 16 + (lane >> 5) * 8]);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
        }
    }
    // epilogue: acc[i] is C[(i/4)*8 + (lane/32)*4 + i%4][lane%32]
    __syncthreads();
    float *xch = reinterpret_cast<float *>(&Bs[0][0]);  // 2 x 16 x 64 floats
    if (wave >= 2)
#pragma unroll
        for (int i = 0; i < 16; i++) xch[(wave - 2) * 1024 + i * 64 + lane] = acc[i];
    __syncthreads();
    if (wave < 2) {
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int m = (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
            const int col = n0 + 32 * wave + (lane & 31);
            const float u = xch[wave * 1024 + i * 64 + lane];
            if (m0 + m < cnt) H[(size_t)(base + m0 + m) * Kd + col] = (__bf16)(act_apply(act, acc[i]) * u);
        }
    }
    if (blockIdx.y == 0 && Kd > F)  // zero K padding of the down product
        for (int i = tid; i < BM * (Kd - F); i += 256) {
            const int m = i / (Kd - F), col = F + i % (Kd - F);
            if (m0 + m < cnt) H[(size_t)(base + m0 + m) * Kd + col] = (__bf16)0.f;
        }
}

// ---------------------------------------------------------------- down
// Block: tile (expert e, rows m0..m0+31) x output columns [n0, n0+128);
// wave w holds columns n0 + 32w ...  H rows are read straight from global
// into MFMA A-operand registers (8 consecutive bf16 per lane).
__global__ void __launch_bounds__(256) k_prefill_down(const uint8_t *__restrict__ hdr, const uint8_t *__restrict__ qs,
                                                      int nsb, int D, const __bf16 *__restrict__ H, int Kd,
                                                      const int *__restrict__ tiles, const int *__restrict__ n_tiles,
                                                      const int *__restrict__ offsets, float *__restrict__ Y) {
    if ((int)blockIdx.x >= *n_tiles) return;
    const int e = tiles[2 * blockIdx.x], m0 = tiles[2 * blockIdx.x + 1];
    const int base = offsets[e], cnt = offsets[e + 1] - base;
    const int n0 = blockIdx.y * BN2;
    __shared__ __attribute__((aligned(16))) __bf16 Bs[BN2][LDK];
    __shared__ size_t wrow[BN2];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    if (tid < BN2) wrow[tid] = (size_t)e * D + n0 + tid;
    const int m = lane & 31;
    const bool row_ok = m0 + m < cnt;
    const __bf16 *hrow = H + (size_t)(base + m0 + (row_ok ? m : 0)) * Kd;
    floatx16 acc = {};
    for (int ks = 0; ks < 2 * nsb; ks++) {
        __syncthreads();
        stage_weights<BN2>(Bs, hdr, qs, nsb, ks, wrow);
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < KS / 16; kk++) {
            bf16x8 a = {};
            if (row_ok) a = *reinterpret_cast<const bf16x8 *>(hrow + ks * KS + kk * 16 + (lane >> 5) * 8);
            const bf16x8 b = *reinterpret_cast<const bf16x8 *>(&Bs[32 * wave + (lane & 31)][kk * 16 + (lane >> 5) * 8]);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
        }
    }
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int mm = (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
        if (m0 + mm < cnt) Y[(size_t)(base + m0 + mm) * D + n0 + 32 * wave + (lane & 31)] = acc[i];
    }
}

// ---------------------------------------------------------------- combine
__global__ void __launch_bounds__(256) k_prefill_combine(const float *__restrict__ Y, const int *__restrict__ pos,
                                                         const float *__restrict__ w, int k, int D,
                                                         float *__restrict__ out) {
    const int t = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    if (i >= D) return;
    float acc = 0.f;
    for (int s = 0; s < k; s++) {
        const int p = pos[t * k + s];
        if (p >= 0) acc += w[t * k + s] * Y[(size_t)p * D + i];
    }
    out[(size_t)t * D + i] = acc;
}

size_t prefill_workspace_bytes(int T, int k, int E, int Kd, int D) {
    const size_t TK = (size_t)T * k;
    return align256((size_t)T * E * 4) + 2 * align256(TK * 4) + align256((size_t)(E + 1) * 4) +
           align256((size_t)max_tiles((int)TK, E) * 8) + 256 + 2 * align256(TK * 4) + align256(TK * Kd * 2) +
           align256(TK * D * 4);
}

hipError_t launch_moe_prefill(const DevTensor &R, const DevTensor &GU, const DevTensor &Dn, const float *X, int T,
                              const float *bias, int k, int F, uint32_t act, uint32_t norm, void *ws, float *out,
                              uint32_t *out_ids, float *out_w, hipStream_t s) {
    const int E = (int)GU.n_experts, D = (int)GU.cols, Kd = (int)Dn.cols;
    const int TK = T * k;
    Ws w = carve(ws, T, k, E, Kd, D);
    hipError_t e = launch_router_batched(R, X, T, bias, w.logits, k, norm, w.ids, w.w, s);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_prefill_dispatch, dim3(1), dim3(1024), 0, s, w.ids, TK, k, E, w.offsets, w.tiles,
                       w.n_tiles, w.perm, w.pos);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const int mt = max_tiles(TK, E);
    hipLaunchKernelGGL(k_prefill_gate_up, dim3(mt, F / BN1), dim3(256), 0, s, GU.p0, GU.p1, (int)GU.blocks_per_row,
                       F, X, D, w.tiles, w.n_tiles, w.offsets, w.perm, act, w.H, Kd);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(k_prefill_down, dim3(mt, D / BN2), dim3(256), 0, s, Dn.p0, Dn.p1, (int)Dn.blocks_per_row, D,
                       w.H, Kd, w.tiles, w.n_tiles, w.offsets, w.Y);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(k_prefill_combine, dim3((D + 255) / 256, T), dim3(256), 0, s, w.Y, w.pos, w.w, k, D, out);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (out_ids) {
        if ((e = hipMemcpyAsync(out_ids, w.ids, (size_t)TK * 4, hipMemcpyDefault, s)) != hipSuccess) return e;
    }
    if (out_w) {
        if ((e = hipMemcpyAsync(out_w, w.w, (size_t)TK * 4, hipMemcpyDefault, s)) != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace lt
