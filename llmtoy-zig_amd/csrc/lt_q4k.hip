// lt_q4k.hip -- Q4_K decode kernels for gfx950 (wave64).
//
// Q4_K super-block (quant/dequant.zig:136-187): 256 elements, d, dmin (f16),
// 12 bytes of packed 6-bit (scale, min) for 8 sub-blocks of 32, and 128 bytes
// of nibbles: qs[32p + i] holds element 64p + i (low nibble, sub-block 2p)
// and 64p + 32 + i (high nibble, sub-block 2p + 1).
//
// Work unit of one lane: a 16-byte "chunk" cc (0..7) of a super-block's qs
// plane, i.e. 32 elements: bytes qs[32p + h + t] (p = cc/2, h = 16*(cc%2),
// t < 16) give elements 64p + h + t (low nibbles) and 64p + 32 + h + t (high
// nibbles).  With the planar layout the 8 chunks of a super-block, and the
// super-blocks of a row, are consecutive 16-byte vectors, so a wavefront's
// qs loads are one contiguous stream.  Each lane also loads its super-block's
// 16-byte header (d, dmin, scales); the 8 lanes of a super-block load the
// same header in the same instruction.
//
// The element value is (d*sc)*q - (dmin*mn); the kernels use
// (d*sc)*sum(q*x) - (dmin*mn)*sum(x) per 16-element half, which is the same
// sum reassociated (fp32 accumulation, checked to 1e-3 rel-L2 against the
// oracle's element-wise dequant then dotf32).
#include "lt_internal.h"
#include "lt_topk.h"
#include "lt_limbs.h"

namespace lt {

namespace {

// x values of chunk cc of super-block sb: 16 low-nibble partners and 16
// high-nibble partners.
struct XChunk {
    float lo[16];
    float hi[16];
    float slo, shi;  // sums, for the min term
};

__device__ __forceinline__ void load_xchunk(const float *xs, int sb, int cc, XChunk &xc) {
    const float *p = xs + sb * 256 + 64 * (cc >> 1) + 16 * (cc & 1);
#pragma unroll
    for (int t = 0; t < 16; t += 4) {
        float4 a = *reinterpret_cast<const float4 *>(p + t);
        float4 b = *reinterpret_cast<const float4 *>(p + 32 + t);
        xc.lo[t] = a.x; xc.lo[t + 1] = a.y; xc.lo[t + 2] = a.z; xc.lo[t + 3] = a.w;
        xc.hi[t] = b.x; xc.hi[t + 1] = b.y; xc.hi[t + 2] = b.z; xc.hi[t + 3] = b.w;
    }
}

// The x sums used by the min term; kept apart from load_xchunk so that the
// adds can be placed after the weight loads are issued.
__device__ __forceinline__ void sum_xchunk(XChunk &xc) {
    float slo = 0.f, shi = 0.f;
#pragma unroll
    for (int t = 0; t < 16; t += 4) {
        slo += (xc.lo[t] + xc.lo[t + 1]) + (xc.lo[t + 2] + xc.lo[t + 3]);
        shi += (xc.hi[t] + xc.hi[t + 1]) + (xc.hi[t + 2] + xc.hi[t + 3]);
    }
    xc.slo = slo;
    xc.shi = shi;
}

// Dot of one 16-byte qs chunk with its x values.
__device__ __forceinline__ float q4k_chunk_dot(uint4 hdr, uint4 q, int cc, const XChunk &xc) {
    const float d = f16_bits_to_f32(hdr.x);
    const float dmin = f16_bits_to_f32(hdr.x >> 16);
    // get_scale_min_k4 for the sub-block pair (2p, 2p+1) of this chunk, both
    // fields at once: the pair's bytes sit at byte offset 2*(p&1) of the
    // scale words (hdr.y = scales[0..3], hdr.z = [4..7], hdr.w = [8..11]).
    const int p = cc >> 1;
    const int sh = (p & 1) * 16;
    const uint32_t ys = hdr.y >> sh, zs = hdr.z >> sh, ws = hdr.w >> sh;
    const uint32_t scp = opaque(p < 2 ? (ys & 0x3f3fu) : ((ws & 0x0f0fu) | ((ys >> 2) & 0x3030u)));
    const uint32_t mnp = opaque(p < 2 ? (zs & 0x3f3fu) : (((ws >> 4) & 0x0f0fu) | ((zs >> 2) & 0x3030u)));
    const float sc0 = (float)(scp & 0xffu), sc1 = (float)((scp >> 8) & 0xffu);
    const float mn0 = (float)(mnp & 0xffu), mn1 = (float)((mnp >> 8) & 0xffu);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    float dl0 = 0.f, dl1 = 0.f, dh0 = 0.f, dh1 = 0.f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint32_t lo = opaque(w[t] & 0x0f0f0f0fu);
        const uint32_t hi = opaque((w[t] >> 4) & 0x0f0f0f0fu);
        dl0 = fmaf((float)(lo & 0xffu), xc.lo[4 * t + 0], dl0);
        dl1 = fmaf((float)((lo >> 8) & 0xffu), xc.lo[4 * t + 1], dl1);
        dl0 = fmaf((float)((lo >> 16) & 0xffu), xc.lo[4 * t + 2], dl0);
        dl1 = fmaf((float)(lo >> 24), xc.lo[4 * t + 3], dl1);
        dh0 = fmaf((float)(hi & 0xffu), xc.hi[4 * t + 0], dh0);
        dh1 = fmaf((float)((hi >> 8) & 0xffu), xc.hi[4 * t + 1], dh1);
        dh0 = fmaf((float)((hi >> 16) & 0xffu), xc.hi[4 * t + 2], dh0);
        dh1 = fmaf((float)(hi >> 24), xc.hi[4 * t + 3], dh1);
    }
    const float dl = dl0 + dl1, dh = dh0 + dh1;
    return ((d * sc0) * dl - (dmin * mn0) * xc.slo) + ((d * sc1) * dh - (dmin * mn1) * xc.shi);
}

// The limbs of one chunk's activations (lt_limbs.h): group 0 = the 16
// low-nibble partners, group 1 = the 16 high-nibble partners.
struct ChunkLimbs {
    uint32_t a[2][4], b[2][4];
    float sp[2], xs[2];
};

// q4k_chunk_dot against int8-limb activations: the nibbles meet both limbs
// in v_dot4 (exact int32 sums per 16-element group), then the group scales.
__device__ __forceinline__ float q4k_chunk_dot_limbs(uint4 hdr, uint4 q, int cc, const ChunkLimbs &x) {
    const float d = f16_bits_to_f32(hdr.x);
    const float dmin = f16_bits_to_f32(hdr.x >> 16);
    const int p = cc >> 1;
    const int sh = (p & 1) * 16;
    const uint32_t ys = hdr.y >> sh, zs = hdr.z >> sh, ws = hdr.w >> sh;
    const uint32_t scp = opaque(p < 2 ? (ys & 0x3f3fu) : ((ws & 0x0f0fu) | ((ys >> 2) & 0x3030u)));
    const uint32_t mnp = opaque(p < 2 ? (zs & 0x3f3fu) : (((ws >> 4) & 0x0f0fu) | ((zs >> 2) & 0x3030u)));
    const float sc0 = (float)(scp & 0xffu), sc1 = (float)((scp >> 8) & 0xffu);
    const float mn0 = (float)(mnp & 0xffu), mn1 = (float)((mnp >> 8) & 0xffu);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    int A0 = 0, B0 = 0, A1 = 0, B1 = 0;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int lo = (int)(w[t] & 0x0f0f0f0fu), hi = (int)((w[t] >> 4) & 0x0f0f0f0fu);
        if (t == 0) {
            A0 = sdot4_first(lo, (int)x.a[0][0]);
            B0 = sdot4_first(lo, (int)x.b[0][0]);
            A1 = sdot4_first(hi, (int)x.a[1][0]);
            B1 = sdot4_first(hi, (int)x.b[1][0]);
        } else {
            A0 = __builtin_amdgcn_sdot4(lo, (int)x.a[0][t], A0, false);
            B0 = __builtin_amdgcn_sdot4(lo, (int)x.b[0][t], B0, false);
            A1 = __builtin_amdgcn_sdot4(hi, (int)x.a[1][t], A1, false);
            B1 = __builtin_amdgcn_sdot4(hi, (int)x.b[1][t], B1, false);
        }
    }
    const float dl = x.sp[0] * (float)((A0 << 8) + B0), dh = x.sp[1] * (float)((A1 << 8) + B1);
    return ((d * sc0) * dl - (dmin * mn0) * x.xs[0]) + ((d * sc1) * dh - (dmin * mn1) * x.xs[1]);
}

// Stage x[0..n) into LDS with 16-byte loads (n % 4 == 0).
__device__ __forceinline__ void stage_x(float *xs, const float *x, int n) {
    for (int i = threadIdx.x * 4; i < n; i += blockDim.x * 4)
        *reinterpret_cast<float4 *>(xs + i) = *reinterpret_cast<const float4 *>(x + i);
    __syncthreads();
}

}  // namespace

// ------------------------------------------------------------------------
// Generic matvec y[r] = W[row0 + r] . x for r < nrows.
// G lanes per row (power of two), CPL chunks per lane, R rows per lane group.
// Block: 256 threads = 256/G groups.  Grid: ceil(nrows / (groups * R)).
template <int G, int CPL, int R>
__global__ void __launch_bounds__(256) k_matvec_q4k(const uint8_t *__restrict__ hdr,
                                                    const uint8_t *__restrict__ qs,
                                                    const float *__restrict__ x, float *__restrict__ y,
                                                    int row0, int nrows, int nsb) {
    extern __shared__ float xs[];
    stage_x(xs, x, nsb * 256);
    const int groups = 256 / G;
    const int g = threadIdx.x / G, lane = threadIdx.x % G;
    const int rbase = (blockIdx.x * groups + g) * R;
    const int nch = nsb * 8;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; i++) {
        const int c = lane + G * i;
        if (c < nch) {
            const int sb = c >> 3, cc = c & 7;
            uint4 hv[R], qv[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                int row = rbase + r;
                if (row < nrows) {
                    size_t blk = (size_t)(row0 + row) * nsb + sb;
                    hv[r] = ldg16(hdr + blk * 16);
                    qv[r] = ldg16(qs + blk * 128 + cc * 16);
                }
            }
            XChunk xc;
            load_xchunk(xs, sb, cc, xc);
            sum_xchunk(xc);
#pragma unroll
            for (int r = 0; r < R; r++)
                if (rbase + r < nrows) acc[r] += q4k_chunk_dot(hv[r], qv[r], cc, xc);
        }
    }
    if constexpr (G == 64) {
        // row r's total lands in lanes [r*64/R, (r+1)*64/R)
        const float t = wave_sum_transposed<R>(acc, lane, p32_first(lane));
        constexpr int SH = R == 8 ? 3 : (R == 4 ? 4 : (R == 2 ? 5 : 6));
        const int r = lane >> SH;
        if ((lane & ((1 << SH) - 1)) == 0 && rbase + r < nrows) y[rbase + r] = t;
    } else {
#pragma unroll
        for (int r = 0; r < R; r++) {
            float v = group_sum<G>(acc[r]);
            if (lane == 0 && rbase + r < nrows) y[rbase + r] = v;
        }
    }
}

// ------------------------------------------------------------------------
// Streaming matvec for rows of NSB = 1, 2, 4, 8 or 16 super-blocks (config 2
// is NSB = 16).  Work unit of a lane: one sub-block pair (p = 0..3) of a
// super-block, 64 weights: qs bytes 32p..32p+31 (two 16-byte loads) and
// header word p, the quad of lanes holding pairs 0..3 of one super-block
// sharing the header through DPP.  Lane L takes pairs u = L % LPR + LPR j
// (j < UPL) of rows RPS apart (LPR = min(64, 4 NSB) lanes per row, UPL =
// 4 NSB / LPR), so its 64 UPL activations are loop-invariant registers,
// held as int8 limbs (lt_limbs.h; the block converts x once through LDS):
// a pair costs 24 bit operations, 32 v_dot4 and one scale decode instead
// of 64 conversions and 64 fma.  Persistent waves, each with ND row slabs
// in flight: the ND buffers are loaded between the load and the
// conversion of x, and each is reloaded ND slabs ahead as soon as it has
// been used; DPP row sums (at NSB = 16, where a row is one slab, the ND
// slabs' sums in one transposed reduction).  NSB <= 16: x fits one group
// per thread.
template <int UPL>
struct Q4Regs {
    uint4 q0[UPL], q1[UPL];
    uint32_t h[UPL];
};

// Waves per SIMD the streaming kernel is compiled for (its VGPR budget: 128
// at 4, 168 at 3) and hence its workgroups per CU.
constexpr int q4k_stream_waves(int nd) { return nd <= 4 ? 4 : 3; }

// Row slabs in flight per wave on large matrices.
constexpr int kQ4StreamND = 4;

template <int NSB, int ND>
__global__ void __launch_bounds__(256, q4k_stream_waves(ND)) k_matvec_q4k_stream(const uint8_t *hdr, const uint8_t *qs,
                                                                                 const float *x, float *y, int row0,
                                                                                 int nrows) {
    constexpr int PPR = 4 * NSB, LPR = PPR < 64 ? PPR : 64, UPL = PPR / LPR, RPS = 64 / LPR;
    __shared__ __attribute__((aligned(16))) uint32_t la[64 * NSB], lb[64 * NSB];
    __shared__ __attribute__((aligned(16))) float lsp[16 * NSB], lxs[16 * NSB];
    const int lane = threadIdx.x & 63;
    const int l = lane % LPR, rs = lane / LPR;
    const int p = l & 3;  // the same pair index for every j (LPR % 4 == 0)
    const int stride = gridDim.x * 4 * RPS;
    int base = (blockIdx.x * 4 + (threadIdx.x >> 6)) * RPS;
    const bool first = p32_first(lane);
    auto ld = [&](Q4Regs<UPL> &w, int rb) {
        int row = rb + rs;
        row = row < nrows ? row : nrows - 1;  // every load unconditional
        const size_t b0 = (size_t)(row0 + row) * NSB;
#pragma unroll
        for (int j = 0; j < UPL; j++) {
            const size_t blk = b0 + ((l + LPR * j) >> 2);
            w.q0[j] = ldg16(qs + blk * 128 + 32 * p);
            w.q1[j] = ldg16(qs + blk * 128 + 32 * p + 16);
            w.h[j] = *reinterpret_cast<const uint32_t *>(hdr + blk * 16 + 4 * p);
        }
    };
    float xv[16];
    stage_x_load(x, 256 * NSB, xv);  // x first: its wait does not include the weights
    asm volatile("" ::: "memory");  // keep the x loads ahead of the weight loads
    Q4Regs<UPL> w[ND];
#pragma unroll
    for (int i = 0; i < ND; i++) ld(w[i], base + i * stride);
    __builtin_amdgcn_sched_barrier(0);  // the weight loads issued before the conversion
    stage_limbs_store(xv, 256 * NSB, la, lb, lsp, lxs);
    Limbs xl[UPL];
#pragma unroll
    for (int j = 0; j < UPL; j++) read_pair_limbs(la, lb, lsp, lxs, 4 * (l + LPR * j), xl[j]);
    auto lane_dot = [&](const Q4Regs<UPL> &r) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < UPL; j++) {
            uint32_t h0, h1, h2, h3;
            quad_header(r.h[j], h0, h1, h2, h3);
            const PairScale ps = pair_scale(h0, h1, h2, h3, p);
            const uint32_t w8[8] = {r.q0[j].x, r.q0[j].y, r.q0[j].z, r.q0[j].w,
                                    r.q1[j].x, r.q1[j].y, r.q1[j].z, r.q1[j].w};
            acc += q4k_pair_dot(w8, ps, xl[j]);
        }
        return acc;
    };
    // a slab past the last row is neither reloaded nor computed (wave-uniform
    // branches; a wave's last reloads would only delay its end)
    if constexpr (LPR == 64) {
        // one row per slab: the ND slabs' row sums in one transposed
        // reduction, lane 64 i / ND storing slab i's row
        constexpr int SH = ND == 2 ? 5 : ND == 4 ? 4 : 3;
        for (; base < nrows; base += ND * stride) {
            float acc[ND];
#pragma unroll
            for (int i = 0; i < ND; i++) {
                acc[i] = (i == 0 || base + i * stride < nrows) ? lane_dot(w[i]) : 0.f;
                if (base + (i + ND) * stride < nrows) ld(w[i], base + (i + ND) * stride);
            }
            const float t = wave_sum_transposed<ND>(acc, lane, first);
            const int row = base + (lane >> SH) * stride;
            if ((lane & ((1 << SH) - 1)) == 0 && row < nrows) y[row] = t;
        }
    } else {
        for (; base < nrows; base += ND * stride) {
#pragma unroll
            for (int i = 0; i < ND; i++) {
                if (i == 0 || base + i * stride < nrows) {
                    const float v = group_sum_dpp<LPR>(lane_dot(w[i]), first);
                    const int row = base + i * stride + rs;
                    if (l == 0 && row < nrows) y[row] = v;
                }
                if (base + (i + ND) * stride < nrows) ld(w[i], base + (i + ND) * stride);
            }
        }
    }
}

template <int NSB>
static hipError_t launch_q4k_stream(const DevTensor &W, size_t row0, size_t nrows, const float *x, float *y,
                                    hipStream_t s) {
    constexpr int LPR = 4 * NSB < 64 ? 4 * NSB : 64, RPS = 64 / LPR;
    const size_t slabs = (nrows + RPS - 1) / RPS;
    // Small matrices: four slabs per wave, all in flight from the start
    // (config 2, 4096 rows: 4.49 us per launch; two slabs per wave on twice
    // the workgroups 4.59, one slab per wave 7.3 with an older kernel).
    // Large ones: every workgroup resident (256 CUs x its waves per SIMD)
    // with kQ4StreamND slabs in flight per wave.
    constexpr size_t nblk_big = (size_t)256 * q4k_stream_waves(kQ4StreamND);
    if (slabs >= nblk_big * 4 * 2 * kQ4StreamND) {
        hipLaunchKernelGGL((k_matvec_q4k_stream<NSB, kQ4StreamND>), dim3((unsigned)nblk_big), dim3(256), 0, s, W.p0,
                           W.p1, x, y, (int)row0, (int)nrows);
    } else {
        constexpr size_t cap = (size_t)256 * q4k_stream_waves(4);
        size_t nblk = (slabs + 15) / 16;
        if (nblk > cap) nblk = cap;
        hipLaunchKernelGGL((k_matvec_q4k_stream<NSB, 4>), dim3((unsigned)nblk), dim3(256), 0, s, W.p0, W.p1, x, y,
                           (int)row0, (int)nrows);
    }
    return hipGetLastError();
}

template <int G, int CPL>
static hipError_t launch_mv_q4k_t(const DevTensor &W, size_t row0, size_t nrows, const float *x, float *y,
                                  hipStream_t s) {
    constexpr int R = 4;
    const int groups = 256 / G;
    const int nblk = (int)((nrows + (size_t)groups * R - 1) / ((size_t)groups * R));
    const int nsb = (int)W.blocks_per_row;
    hipLaunchKernelGGL((k_matvec_q4k<G, CPL, R>), dim3(nblk), dim3(256), nsb * 256 * sizeof(float), s, W.p0, W.p1,
                       x, y, (int)row0, (int)nrows, nsb);
    return hipGetLastError();
}

hipError_t launch_matvec_q4k(const DevTensor &W, size_t row0, size_t nrows, const float *x, float *y,
                             hipStream_t s) {
    if ((row0 + nrows) * W.blocks_per_row < (size_t)1 << 31) {  // int row indices in the streaming kernel
        switch (W.blocks_per_row) {
        case 1: return launch_q4k_stream<1>(W, row0, nrows, x, y, s);
        case 2: return launch_q4k_stream<2>(W, row0, nrows, x, y, s);
        case 4: return launch_q4k_stream<4>(W, row0, nrows, x, y, s);
        case 8: return launch_q4k_stream<8>(W, row0, nrows, x, y, s);
        case 16: return launch_q4k_stream<16>(W, row0, nrows, x, y, s);
        default: break;
        }
    }
    const int nch = (int)W.blocks_per_row * 8;
    if (nch <= 8) return launch_mv_q4k_t<8, 1>(W, row0, nrows, x, y, s);
    if (nch <= 16) return launch_mv_q4k_t<16, 1>(W, row0, nrows, x, y, s);
    if (nch <= 32) return launch_mv_q4k_t<32, 1>(W, row0, nrows, x, y, s);
    switch ((nch + 63) / 64) {
    case 1: return launch_mv_q4k_t<64, 1>(W, row0, nrows, x, y, s);
    case 2: return launch_mv_q4k_t<64, 2>(W, row0, nrows, x, y, s);
    case 3: return launch_mv_q4k_t<64, 3>(W, row0, nrows, x, y, s);
    case 4: return launch_mv_q4k_t<64, 4>(W, row0, nrows, x, y, s);
    case 5: return launch_mv_q4k_t<64, 5>(W, row0, nrows, x, y, s);
    case 6: return launch_mv_q4k_t<64, 6>(W, row0, nrows, x, y, s);
    case 7: return launch_mv_q4k_t<64, 7>(W, row0, nrows, x, y, s);
    case 8: return launch_mv_q4k_t<64, 8>(W, row0, nrows, x, y, s);
    default: return hipErrorInvalidValue;  // K > 16384: rejected by the API layer
    }
}

// ------------------------------------------------------------------------
// Expert-indexed gate/up with the activation fused.
// Slot s = blockIdx.y selects expert e = ids[s]; its gate rows are
// [e*2F, e*2F+F) and its up rows [e*2F+F, e*2F+2F) of the flattened tensor
// (ops/moe.zig:55-73).  h[s][j] = act(gate_j . x) * (up_j . x) for j < F;
// h[s][F..down_cols) = 0 (zero K padding of the down product).
// One wavefront (64 lanes) per row pair, CPL chunks per lane, R row pairs per
// wave, WPB waves per block.  Every weight load of the wave is issued before
// any arithmetic; x comes from L2 straight into registers first.
// ROUTE = 0: ids come from the caller.  ROUTE = PER > 0: each block routes
// for itself -- wave 0 runs softmax + top-k over the router logits
// (PER logits per lane) while the other waves load x; block (0, 0) also
// publishes the selection (ids, weights) for the down kernel.
struct RouteArgs {
    const float *logits;  // [n_experts]
    int k;
    int norm;
    uint32_t *ids_out;    // [k]
    float *w_out;         // [k]
};

template <int CPL, int R, int WPB, int ROUTE>
__global__ void __launch_bounds__(256) k_expert_gate_up_q4k(const uint8_t *__restrict__ hdr,
                                                            const uint8_t *__restrict__ qs,
                                                            const float *__restrict__ x,
                                                            const uint32_t *__restrict__ ids, int n_experts,
                                                            int nsb, int F, int down_cols, uint32_t act,
                                                            float *__restrict__ h, RouteArgs ra) {
    const int s = blockIdx.y;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int jbase = (blockIdx.x * WPB + wave) * R;
    const int nch = nsb * 8;
    const int ng = nsb * 16;  // 16-element groups of x
    // x first (L2-resident), so its latency overlaps the routing below:
    // thread t holds groups t and t + 256 (nsb <= 32), converted to int8
    // limbs in LDS once the weight loads are out
    __shared__ __attribute__((aligned(16))) uint32_t la[32 * 64], lb[32 * 64];
    __shared__ __attribute__((aligned(16))) float lsp[32 * 16], lxs[32 * 16];
    float xv[2][16];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int gi = min((int)threadIdx.x + 256 * u, ng - 1);
#pragma unroll
        for (int t = 0; t < 16; t += 4) {
            const float4 f = ldg16f(x + 16 * gi + t);
            xv[u][t] = f.x; xv[u][t + 1] = f.y; xv[u][t + 2] = f.z; xv[u][t + 3] = f.w;
        }
    }
    uint32_t e;
    if constexpr (ROUTE > 0) {
        __shared__ uint32_t s_ids[16];
        __shared__ float s_w[16];
        if (wave == 0) topk_softmax_wave<ROUTE>(ra.logits, n_experts, ra.k, ra.norm, s_ids, s_w, nullptr, lane);
        __syncthreads();
        if (blockIdx.x == 0 && blockIdx.y == 0 && (int)threadIdx.x < ra.k) {
            ra.ids_out[threadIdx.x] = s_ids[threadIdx.x];
            ra.w_out[threadIdx.x] = s_w[threadIdx.x];
        }
        e = __builtin_amdgcn_readfirstlane(s_ids[s]);
    } else {
        e = __builtin_amdgcn_readfirstlane(ids[s]);
    }
    float *hs = h + (size_t)s * down_cols;
    if (blockIdx.x == 0)
        for (int j = F + threadIdx.x; j < down_cols; j += blockDim.x) hs[j] = 0.f;
    if (e >= (uint32_t)n_experts) {  // invalid id from the caller: the slot contributes zeros
        if (lane < R && jbase + lane < F) hs[jbase + lane] = 0.f;
        return;
    }
    const size_t gate0 = (size_t)e * 2 * F, up0 = gate0 + F;
    // weights row by row, so that rows can be consumed as their loads land
    // (vmcnt retires in issue order)
    uint4 hg[R][CPL], qg[R][CPL], hu[R][CPL], qu[R][CPL];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int j = jbase + r;
#pragma unroll
        for (int i = 0; i < CPL; i++) {
            const int c = lane + kWave * i;
            const int sb = c >> 3, cc = c & 7;
            if (c < nch && j < F) {
                const size_t bg = (gate0 + j) * nsb + sb, bu = (up0 + j) * nsb + sb;
                hg[r][i] = ldg16(hdr + bg * 16);
                qg[r][i] = ldg16(qs + bg * 128 + cc * 16);
                hu[r][i] = ldg16(hdr + bu * 16);
                qu[r][i] = ldg16(qs + bu * 128 + cc * 16);
            }
        }
    }
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int gi = (int)threadIdx.x + 256 * u;
        if (gi < ng) {
            uint32_t a4[4], b4[4];
            float sp, xs;
            limbs16(xv[u], a4, b4, sp, xs);
            *reinterpret_cast<uint4 *>(la + 4 * gi) = make_uint4(a4[0], a4[1], a4[2], a4[3]);
            *reinterpret_cast<uint4 *>(lb + 4 * gi) = make_uint4(b4[0], b4[1], b4[2], b4[3]);
            lsp[gi] = sp;
            lxs[gi] = xs;
        }
    }
    __syncthreads();
    // chunk c = 8 sb + cc: low nibbles meet group 16 sb + 4 (cc / 2) + cc % 2,
    // high nibbles that group + 2
    ChunkLimbs xc[CPL];
#pragma unroll
    for (int i = 0; i < CPL; i++) {
        const int c = min(lane + kWave * i, nch - 1);
        const int g0 = 16 * (c >> 3) + 4 * ((c & 7) >> 1) + (c & 1);
#pragma unroll
        for (int h2 = 0; h2 < 2; h2++) {
            read_group_limbs(la, lb, g0 + 2 * h2, xc[i].a[h2], xc[i].b[h2]);
            xc[i].sp[h2] = lsp[g0 + 2 * h2];
            xc[i].xs[h2] = lxs[g0 + 2 * h2];
        }
    }
    float ag[R], au[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        ag[r] = au[r] = 0.f;
#pragma unroll
        for (int i = 0; i < CPL; i++) {
            const int c = lane + kWave * i;
            if (c < nch && jbase + r < F) {
                ag[r] += q4k_chunk_dot_limbs(hg[r][i], qg[r][i], c & 7, xc[i]);
                au[r] += q4k_chunk_dot_limbs(hu[r][i], qu[r][i], c & 7, xc[i]);
            }
        }
    }
    // 2R partial sums per lane -> one total per 64/(2R) lanes: gate row r in
    // lanes [r*S, (r+1)*S), up row r in the same lanes + 32 (S = 64/(2R)).
    float v[2 * R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        v[r] = ag[r];
        v[R + r] = au[r];
    }
    const bool first = p32_first(lane);
    const float t = wave_sum_transposed<2 * R>(v, lane, first);
    const float u = xor32(t, first);
    constexpr int SH = (2 * R == 8) ? 3 : (2 * R == 4 ? 4 : 5);
    const int r = lane >> SH;
    if (lane < 32 && (lane & ((1 << SH) - 1)) == 0 && jbase + r < F) hs[jbase + r] = act_apply(act, t) * u;
}

template <int CPL, int R, int ROUTE>
static hipError_t launch_gu_t(const DevTensor &GU, const float *x, const uint32_t *ids, uint32_t k, uint32_t F,
                              uint32_t down_cols, uint32_t act, float *h, const RouteArgs &ra, hipStream_t s) {
    constexpr int WPB = 4;
    dim3 grid((F + WPB * R - 1) / (WPB * R), k);
    hipLaunchKernelGGL((k_expert_gate_up_q4k<CPL, R, WPB, ROUTE>), grid, dim3(64 * WPB), 0, s, GU.p0, GU.p1, x, ids,
                       (int)GU.n_experts, (int)GU.blocks_per_row, (int)F, (int)down_cols, act, h, ra);
    return hipGetLastError();
}

// At most 4 chunk dots per lane (CPL x R row pairs): more, shorter waves
// keep more loads in flight per CU than fewer, longer ones (config 3:
// R = 2 takes 5.8 us against 7.0 us for R = 4).  Rows of 9-16 super-blocks
// (CPL = 2) also take 2 row pairs per wave: the Gemma4 block (11) runs
// 35.1 us/token against 38.4 with one.
template <int ROUTE>
static hipError_t launch_gu_route(const DevTensor &GU, const float *x, const uint32_t *ids, uint32_t k,
                                  uint32_t d_expert, uint32_t down_cols, uint32_t act, float *h, const RouteArgs &ra,
                                  hipStream_t s) {
    const int nch = (int)GU.blocks_per_row * 8;
    switch ((nch + 63) / 64) {
    case 1: return launch_gu_t<1, 2, ROUTE>(GU, x, ids, k, d_expert, down_cols, act, h, ra, s);
    case 2: return launch_gu_t<2, 2, ROUTE>(GU, x, ids, k, d_expert, down_cols, act, h, ra, s);
    case 3: return launch_gu_t<3, 1, ROUTE>(GU, x, ids, k, d_expert, down_cols, act, h, ra, s);
    case 4: return launch_gu_t<4, 1, ROUTE>(GU, x, ids, k, d_expert, down_cols, act, h, ra, s);
    default: return hipErrorInvalidValue;  // d_model > 8192: rejected by the API layer
    }
}

hipError_t launch_expert_gate_up_q4k(const DevTensor &GU, const float *x, const uint32_t *ids, uint32_t k,
                                     uint32_t d_expert, uint32_t down_cols, uint32_t act, float *h,
                                     hipStream_t s) {
    const RouteArgs none{nullptr, 0, 0, nullptr, nullptr};
    return launch_gu_route<0>(GU, x, ids, k, d_expert, down_cols, act, h, none, s);
}

hipError_t launch_expert_gate_up_q4k_routed(const DevTensor &GU, const float *x, const float *logits, uint32_t k,
                                            uint32_t norm, uint32_t d_expert, uint32_t down_cols, uint32_t act,
                                            float *h, uint32_t *ids_out, float *w_out, hipStream_t s) {
    const RouteArgs ra{logits, (int)k, (int)norm, ids_out, w_out};
    const int E = (int)GU.n_experts;
    if (E <= 64) return launch_gu_route<1>(GU, x, nullptr, k, d_expert, down_cols, act, h, ra, s);
    if (E <= 128) return launch_gu_route<2>(GU, x, nullptr, k, d_expert, down_cols, act, h, ra, s);
    if (E <= 256) return launch_gu_route<4>(GU, x, nullptr, k, d_expert, down_cols, act, h, ra, s);
    return hipErrorInvalidValue;  // more experts: the caller uses the router's top-k
}

// ------------------------------------------------------------------------
// Expert-indexed down with the weighted combine fused:
//   out[i] = base[i] + sum_{s in slot order} w[s] * (D_{ids[s]} row i) . h[s]
// (w[s] times dscale[ids[s]] when a per-expert down scale is given)
// (base = previous out with accumulate, the shared-FFN output, or 0).
// Block: NW = min(nsb, 4) waves x RD output rows.  Wave w handles
// super-blocks w, w+NW, ... of the K = down_cols dimension; lane = (slot
// within an 8-slot pass, chunk cc), so one load instruction covers the same
// super-block of 8 experts (8 contiguous 128-byte runs).  Per-(row, slot,
// super-block) partial sums go through LDS and are combined in a fixed
// order, so the result does not depend on scheduling.
template <int RD>
__global__ void __launch_bounds__(256) k_expert_down_q4k(const uint8_t *__restrict__ hdr,
                                                         const uint8_t *__restrict__ qs,
                                                         const float *__restrict__ h,
                                                         const uint32_t *__restrict__ ids,
                                                         const float *__restrict__ wts, int k, int n_experts,
                                                         int rows_per_expert, int nsb, const float *base,
                                                         int accumulate, const float *dscale, float *out) {
    __shared__ float part[RD][16][16];  // [row][slot][super-block]
    const int NW = blockDim.x / kWave;
    const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int sl = lane >> 3, cc = lane & 7;
    const int row0 = blockIdx.x * RD;
    const int K = nsb * 256;
    for (int pass = 0; pass * 8 < k; pass++) {
        const int s = pass * 8 + sl;
        const bool active = s < k;
        const uint32_t e = active ? ids[s] : 0u;
        const bool valid = active && e < (uint32_t)n_experts;
        const float *hs = h + (size_t)(valid ? s : 0) * K;
        for (int sb = w; sb < nsb; sb += NW) {
            XChunk xc;
            load_xchunk(hs, sb, cc, xc);
            uint4 hv[RD], qv[RD];
#pragma unroll
            for (int r = 0; r < RD; r++) {
                const int row = row0 + r;
                if (valid && row < rows_per_expert) {
                    const size_t blk = ((size_t)e * rows_per_expert + row) * nsb + sb;
                    hv[r] = ldg16(hdr + blk * 16);
                    qv[r] = ldg16(qs + blk * 128 + cc * 16);
                }
            }
            sum_xchunk(xc);
            float v[RD];
#pragma unroll
            for (int r = 0; r < RD; r++)
                v[r] = (valid && row0 + r < rows_per_expert) ? q4k_chunk_dot(hv[r], qv[r], cc, xc) : 0.f;
            // lane (slot, cc) receives the 8-lane total of row cc * RD / 8
            const float t = group8_sum_transposed<RD>(v, lane);
            constexpr int SPLIT = 8 / RD;  // lanes per row after the reduction
            if (active && cc % SPLIT == 0) part[cc / SPLIT][s][sb] = t;
        }
    }
    __syncthreads();
    if (threadIdx.x < RD) {
        const int r = threadIdx.x, row = row0 + r;
        if (row < rows_per_expert) {
            float acc = accumulate ? out[row] : 0.f;
            for (int s = 0; s < k; s++) {
                float t = part[r][s][0];
                for (int b = 1; b < nsb; b++) t += part[r][s][b];
                const uint32_t e = ids[s];
                if (e < (uint32_t)n_experts) {
                    // expert_scale = down_exps_scale[e] * w (gemma4/forward.zig:477)
                    const float ws = dscale ? dscale[e] * wts[s] : wts[s];
                    acc += ws * t;
                }
            }
            if (base) acc = base[row] + acc;
            out[row] = acc;
        }
    }
}

hipError_t launch_expert_down_q4k(const DevTensor &D, const float *h, const uint32_t *ids, const float *w,
                                  uint32_t k, const float *base, int accumulate, float *out, hipStream_t s,
                                  const float *dscale) {
    constexpr int RD = 2;  // 2 rows per block: 7.5 -> 6.5 us against 8 rows (config 3)
    const int nsb = (int)D.blocks_per_row;  // <= 16, k <= 16: checked by the API layer
    const int nw = nsb < 4 ? nsb : 4;
    const int rows = (int)D.rows;
    dim3 grid((rows + RD - 1) / RD);
    hipLaunchKernelGGL((k_expert_down_q4k<RD>), grid, dim3(64 * nw), 0, s, D.p0, D.p1, h, ids, w, (int)k,
                       (int)D.n_experts, rows, nsb, base, accumulate, dscale, out);
    return hipGetLastError();
}

}  // namespace lt
