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
// all rows, so x is staged in LDS once per workgroup, as two int8 limbs per
// 16-element group (lt_limbs.h: x ~= sp (256 a + b), error <= max |x| /
// 65024 of the group) with the group's fp32 sum: the codes (unsigned 5-bit
// for Q5_0 / Q5_1, the signed IQ4_NL table values, unsigned 3-bit for Q3_K)
// meet both limbs in v_dot4_i32_i8, exact int32 sums per group, and the
// formats' offsets (-16, m, -4) come back through the group sums.  fp32
// accumulation in an order of our own: parity with the reference's
// quantMatvec is to tolerance (its GPU matvec fuzz bound, 1e-4 of max |y|),
// not bit-exact.
#include "llmtoy_hip.h"
#include "lt_fmt.h"
#include "lt_limbs.h"
#include "lt_topk.h"

namespace lt {

namespace {

constexpr int kFmtWaves = 4;  // rows per workgroup

// Staged activations: n elements (n % 16 == 0) as limb words la [n / 4],
// lb [n / 4] (word i: elements 4i..4i+3), then per 16-element group its
// scale lsp [n / 16] and fp32 sum lxs [n / 16].
size_t lds_bytes(size_t n) { return n * 2 + n / 4 * 2; }

// Block-wide: src[0..n) into limbs at base, one 16-element group per thread
// and pass, then a barrier.
__device__ __forceinline__ void stage_limbs(uint32_t *base, const float *src, int n) {
    uint32_t *la = base, *lb = base + n / 4;
    float *lsp = reinterpret_cast<float *>(base + n / 2), *lxs = lsp + n / 16;
    for (int g = threadIdx.x; g < n / 16; g += blockDim.x) {
        float v[16];
#pragma unroll
        for (int t = 0; t < 16; t += 4) {
            const float4 f = ldg16f(src + 16 * g + t);
            v[t] = f.x; v[t + 1] = f.y; v[t + 2] = f.z; v[t + 3] = f.w;
        }
        uint32_t a[4], b[4];
        float sp, xs;
        limbs16(v, a, b, sp, xs);
        *reinterpret_cast<uint4 *>(la + 4 * g) = make_uint4(a[0], a[1], a[2], a[3]);
        *reinterpret_cast<uint4 *>(lb + 4 * g) = make_uint4(b[0], b[1], b[2], b[3]);
        lsp[g] = sp;
        lxs[g] = xs;
    }
    __syncthreads();
}

template <int LPR>
__device__ __forceinline__ float seg_sum(float v) {
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Workgroup = kFmtWaves waves; a wave takes RPW groups of R rows at a time
// (64 / RPW lanes per group, striding over the rows' units; each lane loads
// a unit's x once and applies it to the R rows) and walks the rows with a
// grid-wide stride, so x is staged in LDS once per workgroup.
template <int T, int RPW, int R>
__global__ __launch_bounds__(64 * kFmtWaves) void k_matvec_fmt(DevTensor W, const float *__restrict__ x,
                                                               float *__restrict__ y) {
    extern __shared__ __attribute__((aligned(16))) uint32_t xl[];  // x as limbs (lds_bytes(cols))
    constexpr int LPR = kWave / RPW;
    stage_limbs(xl, x, (int)W.cols);
    const LimbView xv = limb_view(xl, (int)W.cols);
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int grp = lane / LPR, sub = lane % LPR;
    const int U = units_per_row<T>(W);
    const size_t n = W.total_rows;
    const size_t stride = (size_t)gridDim.x * kFmtWaves * RPW * R;
    for (size_t base = ((size_t)blockIdx.x * kFmtWaves + wave) * RPW * R; base < n; base += stride) {
        const size_t row0 = base + (size_t)grp * R;
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.f;
        if (row0 < n) {
            for (int u = sub; u < U; u += LPR) {
                UnitW<T> w[R];
#pragma unroll
                for (int r = 0; r < R; r++) w[r] = load_unit<T>(W, row0 + r < n ? row0 + r : n - 1, u);
                const UnitX ux = load_ux(xv, u);
#pragma unroll
                for (int r = 0; r < R; r++) acc[r] += dot_unit<T>(w[r], u, ux);
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float v = seg_sum<LPR>(acc[r]);
            if (sub == 0 && row0 + r < n) y[row0 + r] = v;
        }
    }
}

// Routing done by the gate/up blocks themselves (ROUTE = PER > 0): wave 0 of
// every block runs softmax + top-k over the router logits (PER per lane)
// while the block stages x, and block (0, 0) publishes the selection for
// the down kernel -- instead of the router's last block doing it behind an
// arrival ticket and two fences.
struct FmtRoute {
    const float *logits;  // [n_experts]
    int k;
    int norm;
    uint32_t *ids_out;    // [k]
    float *w_out;         // [k]
};

// Expert-indexed gate/up (ops/moe.zig:55-73): slot s = blockIdx.y, expert
// e = ids[s] (or the block's own selection); row pair j = (gate row e 2F +
// j, up row e 2F + F + j); h[s][j] = act(gate . x) * (up . x), h[s][F,
// down_cols) = 0.  A lane group takes R row pairs at a time (one x load per
// unit for 2 R rows); waves walk the row pairs of their slot with a stride
// of gridDim.x * kFmtWaves * RPW * R.
template <int T, int RPW, int R, int ROUTE>
__global__ __launch_bounds__(64 * kFmtWaves) void k_expert_gu_fmt(DevTensor W, const float *__restrict__ x,
                                                                  const uint32_t *__restrict__ ids, int F,
                                                                  int down_cols, uint32_t act, float *__restrict__ h,
                                                                  FmtRoute ra) {
    extern __shared__ __attribute__((aligned(16))) uint32_t xl[];  // x as limbs (lds_bytes(cols))
    constexpr int LPR = kWave / RPW;
    const int s = blockIdx.y;
    uint32_t e;
    if constexpr (ROUTE > 0) {
        __shared__ uint32_t s_ids[16];
        __shared__ float s_w[16];
        if (threadIdx.x < kWave)
            topk_softmax_wave<ROUTE>(ra.logits, (int)W.n_experts, ra.k, ra.norm, s_ids, s_w, nullptr, threadIdx.x);
        stage_limbs(xl, x, (int)W.cols);  // (its barrier also publishes s_ids / s_w)
        if (blockIdx.x == 0 && blockIdx.y == 0 && (int)threadIdx.x < ra.k) {
            ra.ids_out[threadIdx.x] = s_ids[threadIdx.x];
            ra.w_out[threadIdx.x] = s_w[threadIdx.x];
        }
        e = __builtin_amdgcn_readfirstlane(s_ids[s]);
    } else {
        stage_limbs(xl, x, (int)W.cols);
        e = __builtin_amdgcn_readfirstlane(ids[s]);
    }
    const LimbView xv = limb_view(xl, (int)W.cols);
    float *hs = h + (size_t)s * down_cols;
    if (blockIdx.x == 0)
        for (int j = F + threadIdx.x; j < down_cols; j += blockDim.x) hs[j] = 0.f;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int grp = lane / LPR, sub = lane % LPR;
    const int U = units_per_row<T>(W);
    const bool valid = e < (uint32_t)W.n_experts;
    const int stride = gridDim.x * kFmtWaves * RPW * R;
    for (int base = (blockIdx.x * kFmtWaves + wave) * RPW * R; base < F; base += stride) {
        const int j0 = base + grp * R;
        float ag[R], au[R];
#pragma unroll
        for (int r = 0; r < R; r++) ag[r] = au[r] = 0.f;
        if (j0 < F && valid) {
            const size_t g0 = (size_t)e * 2 * F;
            for (int u = sub; u < U; u += LPR) {
                UnitW<T> wg[R], wu[R];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const size_t j = (size_t)(j0 + r < F ? j0 + r : F - 1);
                    wg[r] = load_unit<T>(W, g0 + j, u);
                    wu[r] = load_unit<T>(W, g0 + F + j, u);
                }
                const UnitX ux = load_ux(xv, u);
#pragma unroll
                for (int r = 0; r < R; r++) {
                    ag[r] += dot_unit<T>(wg[r], u, ux);
                    au[r] += dot_unit<T>(wu[r], u, ux);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float g = seg_sum<LPR>(ag[r]), up = seg_sum<LPR>(au[r]);
            if (sub == 0 && j0 + r < F) hs[j0 + r] = valid ? act_apply(act, g) * up : 0.f;  // invalid id: zeros
        }
    }
}

// Expert-indexed down with the weighted combine (ops/moe.zig:67-76):
//   out[i] = base[i] + (accumulate ? out[i] : 0) + sum_s w'[s] (D_{ids[s]} row i) . h[s]
// with w'[s] = dscale[ids[s]] * w[s] when a per-expert down scale is given
// (gemma4/forward.zig:477).  h [k][down_cols] is staged in LDS once per
// workgroup; waves walk the output rows, and a row's lanes stride over its
// k * units (slot, unit) pairs, so the slots' loads are in flight together.
template <int T, int RPW>
__global__ __launch_bounds__(64 * kFmtWaves) void k_expert_down_fmt(DevTensor W, const float *__restrict__ h,
                                                                    const uint32_t *__restrict__ ids,
                                                                    const float *__restrict__ wts, int k,
                                                                    const float *base, int accumulate,
                                                                    const float *dscale, float *out) {
    extern __shared__ __attribute__((aligned(16))) uint32_t hl[];  // h [k][down_cols] as limbs
    __shared__ uint32_t s_e[16];
    __shared__ float s_w[16];
    constexpr int LPR = kWave / RPW;
    const int Kd = (int)W.cols;
    if ((int)threadIdx.x < k) {  // the slots' experts and combine weights, once per workgroup
        const uint32_t e = ids[threadIdx.x];
        s_e[threadIdx.x] = e;
        s_w[threadIdx.x] = e < (uint32_t)W.n_experts ? (dscale ? dscale[e] * wts[threadIdx.x] : wts[threadIdx.x]) : 0.f;
    }
    stage_limbs(hl, h, k * Kd);
    const LimbView hv = limb_view(hl, k * Kd);
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int r = lane / LPR, sub = lane % LPR;
    const int U = units_per_row<T>(W);
    const int D = (int)W.rows;
    const int stride = gridDim.x * kFmtWaves * RPW;
    for (int i0 = (blockIdx.x * kFmtWaves + wave) * RPW; i0 < D; i0 += stride) {
        const int i = i0 + r;
        float acc = 0.f;
        if (i < D) {
            int s = sub / U, u = sub % U;
            while (s < k) {
                const uint32_t e = s_e[s];
                if (e < (uint32_t)W.n_experts) {
                    const UnitW<T> w = load_unit<T>(W, (size_t)e * D + i, u);
                    const UnitX ux = load_ux(hv, s * U + u);  // U = Kd / 32 units per slot
                    acc += s_w[s] * dot_unit<T>(w, u, ux);
                }
                u += LPR;
                while (u >= U) {
                    u -= U;
                    s++;
                }
            }
        }
        acc = seg_sum<LPR>(acc);
        if (i < D && sub == 0) {
            float v = accumulate ? out[i] + acc : acc;
            out[i] = base ? base[i] + v : v;
        }
    }
}

// Row groups per wave for rows of `units` work units.  A full-wave group
// whose last pass leaves most lanes idle (88 units: 128 lane slots, 69%
// busy) takes two 32-lane groups instead (96 slots, 92%).
int pick_rpw(size_t units) {
    if (units >= 48) {
        const size_t slots64 = (units + 63) / 64 * 64, slots32 = (units + 31) / 32 * 32;
        return units * 100 < slots64 * 85 && units * 100 >= slots32 * 85 ? 2 : 1;
    }
    return units >= 24 ? 2 : units >= 12 ? 4 : 8;
}

// Allow the largest staging (16384 activations as limbs: 40 KiB of dynamic
// LDS), once per kernel and device.
hipError_t allow_lds(const void *fn, bool *set) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    if (set[dev]) return hipSuccess;
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes(16384));
    if (e == hipSuccess) set[dev] = true;
    return e;
}

// Rows per lane group: x reuse against the weight registers a lane holds
// (a Q3_K unit is 20 dwords, a block unit 6).
template <int T>
constexpr int kMvRows = T == LT_TYPE_Q3_K ? 2 : 4;
template <int T>
constexpr int kGuPairs = T == LT_TYPE_Q3_K ? 1 : 2;

template <int T, int RPW>
hipError_t launch_mv(const DevTensor &W, const float *x, float *y, hipStream_t s) {
    constexpr int R = kMvRows<T>;
    static bool set[64] = {};
    hipError_t e = allow_lds((const void *)k_matvec_fmt<T, RPW, R>, set);
    if (e != hipSuccess) return e;
    // up to 8 workgroups per CU, each walking many rows
    const size_t per = (size_t)kFmtWaves * RPW * R;
    const size_t need = (W.total_rows + per - 1) / per;
    const dim3 grid((unsigned)(need < 2048 ? need : 2048));
    hipLaunchKernelGGL((k_matvec_fmt<T, RPW, R>), grid, dim3(64 * kFmtWaves), lds_bytes(W.cols), s, W, x, y);
    return hipGetLastError();
}

template <int T, int RPW, int ROUTE>
hipError_t launch_gu(const DevTensor &W, const float *x, const uint32_t *ids, int k, int F, int down_cols,
                     uint32_t act, float *h, const FmtRoute &ra, hipStream_t s) {
    constexpr int R = kGuPairs<T>;
    static bool set[64] = {};
    hipError_t e = allow_lds((const void *)k_expert_gu_fmt<T, RPW, R, ROUTE>, set);
    if (e != hipSuccess) return e;
    const int per = kFmtWaves * RPW * R;
    const int need = (F + per - 1) / per;
    const dim3 grid((unsigned)(need < 128 ? need : 128), (unsigned)k);  // up to 128 x k workgroups walk the rows
    hipLaunchKernelGGL((k_expert_gu_fmt<T, RPW, R, ROUTE>), grid, dim3(64 * kFmtWaves),
                       lds_bytes(W.cols), s, W, x, ids, F, down_cols, act, h, ra);
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
                       lds_bytes((size_t)k * W.cols), s, W, h, ids, w, k, base,
                       accumulate, dscale, out);
    return hipGetLastError();
}

// Streaming Q3_K matvec for rows of NSB = 1, 2, 4, 8 or 16 super-blocks.  A
// lane owns quant chunk j (qs bytes 16 j .. 16 j + 15: half h = j / 2,
// 16-element run g = j % 2, all four bit pairs) of one super-block and the
// hmask bytes 16 g .. 16 g + 15 those elements need; lanes 0-2 of the
// aligned quad load scale dwords 0-2 and lane 3 the f16 d, shared over DPP.
// Per 64 weights that is two 16-byte loads and one small one, where the
// unit kernel above loads 20 dwords per 32 weights.  The lane's four limb
// groups (16 sb + 8 h + 2 jp + g, jp = bit pair) stay in registers; each
// wave keeps ND row slabs in flight (as k_matvec_q4k_stream).
template <int NSB, int ND>
__global__ void __launch_bounds__(256, 4) k_matvec_q3k_stream(DevTensor W, const float *x, float *y) {
    constexpr int LPR = 4 * NSB, RPS = 64 / LPR;
    __shared__ __attribute__((aligned(16))) uint32_t la[64 * NSB], lb[64 * NSB];
    __shared__ __attribute__((aligned(16))) float lsp[16 * NSB], lxs[16 * NSB];
    const int nrows = (int)W.total_rows;
    const int lane = threadIdx.x & 63;
    const int l = lane % LPR, rs = lane / LPR;
    const int sb = l >> 2, j = l & 3, h = j >> 1, g = j & 1;
    const int stride = gridDim.x * 4 * RPS;
    int base = (blockIdx.x * 4 + (threadIdx.x >> 6)) * RPS;
    const bool first = p32_first(lane);
    struct Regs {
        uint4 q, m;
        uint32_t hd;
    };
    auto ld = [&](Regs &w, int rb) {
        int row = rb + rs;
        row = row < nrows ? row : nrows - 1;
        const size_t blk = (size_t)row * NSB + sb;
        w.q = ldg16(W.p0 + blk * 64 + 16 * j);
        w.m = ldg16(W.p1 + blk * 32 + 16 * g);
        w.hd = j < 3 ? *reinterpret_cast<const uint32_t *>(W.p2 + blk * 12 + 4 * j)
                     : (uint32_t)*reinterpret_cast<const uint16_t *>(W.p3 + blk * 2);
    };
    float xv[16];
    stage_x_load(x, 256 * NSB, xv);  // x first: its wait does not include the weights
    asm volatile("" ::: "memory");  // keep the x loads ahead of the weight loads
    Regs w[ND];
#pragma unroll
    for (int i = 0; i < ND; i++) ld(w[i], base + i * stride);
    __builtin_amdgcn_sched_barrier(0);  // the weight loads issued before the conversion
    stage_limbs_store(xv, 256 * NSB, la, lb, lsp, lxs);
    uint32_t xa[4][4], xb[4][4];
    float xsp[4], xsum[4];
#pragma unroll
    for (int jp = 0; jp < 4; jp++) {
        const int gi = 16 * sb + 8 * h + 2 * jp + g;
        read_group_limbs(la, lb, gi, xa[jp], xb[jp]);
        xsp[jp] = lsp[gi];
        xsum[jp] = lxs[gi];
    }
    auto lane_dot = [&](const Regs &r) {
        const uint32_t s0 = quad_bcast<0x00>(r.hd), s1 = quad_bcast<0x55>(r.hd), s2 = quad_bcast<0xAA>(r.hd);
        const float d = f16_bits_to_f32(quad_bcast<0xFF>(r.hd) & 0xffffu);
        const uint32_t qw[4] = {r.q.x, r.q.y, r.q.z, r.q.w}, mw[4] = {r.m.x, r.m.y, r.m.z, r.m.w};
        float acc = 0.f;
#pragma unroll
        for (int jp = 0; jp < 4; jp++) {
            uint32_t c[4];
#pragma unroll
            for (int m = 0; m < 4; m++)
                c[m] = ((qw[m] >> (2 * jp)) & 0x03030303u) | (((mw[m] >> (jp + 4 * h)) & 0x01010101u) << 2);
            int A = sdot4_first((int)c[0], (int)xa[jp][0]);
            int B = sdot4_first((int)c[0], (int)xb[jp][0]);
#pragma unroll
            for (int m = 1; m < 4; m++) {
                A = __builtin_amdgcn_sdot4((int)c[m], (int)xa[jp][m], A, false);
                B = __builtin_amdgcn_sdot4((int)c[m], (int)xb[jp][m], B, false);
            }
            const float dot = xsp[jp] * (float)((A << 8) + B);
            const int sc = q3k_scale(s0, s1, s2, 8 * h + 2 * jp + g);
            acc += (d * (float)(sc - 32)) * (dot - 4.f * xsum[jp]);
        }
        return acc;
    };
    // a slab past the last row is neither reloaded nor computed
    if constexpr (LPR == 64) {
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
hipError_t launch_q3k_stream(const DevTensor &W, const float *x, float *y, hipStream_t s) {
    constexpr int RPS = 64 / (4 * NSB);
    const size_t slabs = (W.total_rows + RPS - 1) / RPS;
    size_t nblk = (slabs + 15) / 16;  // four slabs per wave
    if (nblk > (size_t)kStreamBlocks) nblk = kStreamBlocks;
    hipLaunchKernelGGL((k_matvec_q3k_stream<NSB, 4>), dim3((unsigned)nblk), dim3(256), 0, s, W, x, y);
    return hipGetLastError();
}

template <int T>
hipError_t launch_t(const DevTensor &W, const float *x, float *y, hipStream_t s) {
    if constexpr (T == LT_TYPE_Q3_K) {
        switch (W.cols == 256 * W.blocks_per_row ? W.blocks_per_row : 0) {
        case 1: return launch_q3k_stream<1>(W, x, y, s);
        case 2: return launch_q3k_stream<2>(W, x, y, s);
        case 4: return launch_q3k_stream<4>(W, x, y, s);
        case 8: return launch_q3k_stream<8>(W, x, y, s);
        case 16: return launch_q3k_stream<16>(W, x, y, s);
        default: break;
        }
    }
    switch (pick_rpw(T == LT_TYPE_Q3_K ? 8 * W.blocks_per_row : W.blocks_per_row)) {
    case 1: return launch_mv<T, 1>(W, x, y, s);
    case 2: return launch_mv<T, 2>(W, x, y, s);
    case 4: return launch_mv<T, 4>(W, x, y, s);
    default: return launch_mv<T, 8>(W, x, y, s);
    }
}

template <int T, int ROUTE>
hipError_t launch_gu_r(const DevTensor &W, const float *x, const uint32_t *ids, int k, int F, int down_cols,
                       uint32_t act, float *h, const FmtRoute &ra, hipStream_t s) {
    switch (pick_rpw(T == LT_TYPE_Q3_K ? 8 * W.blocks_per_row : W.blocks_per_row)) {
    case 1: return launch_gu<T, 1, ROUTE>(W, x, ids, k, F, down_cols, act, h, ra, s);
    case 2: return launch_gu<T, 2, ROUTE>(W, x, ids, k, F, down_cols, act, h, ra, s);
    case 4: return launch_gu<T, 4, ROUTE>(W, x, ids, k, F, down_cols, act, h, ra, s);
    default: return launch_gu<T, 8, ROUTE>(W, x, ids, k, F, down_cols, act, h, ra, s);
    }
}

template <int T>
hipError_t launch_gu_t(const DevTensor &W, const float *x, const uint32_t *ids, int k, int F, int down_cols,
                       uint32_t act, float *h, const FmtRoute &ra, hipStream_t s) {
    if (!ra.logits) return launch_gu_r<T, 0>(W, x, ids, k, F, down_cols, act, h, ra, s);
    const int E = (int)W.n_experts;
    if (E <= 64) return launch_gu_r<T, 1>(W, x, ids, k, F, down_cols, act, h, ra, s);
    if (E <= 128) return launch_gu_r<T, 2>(W, x, ids, k, F, down_cols, act, h, ra, s);
    if (E <= 256) return launch_gu_r<T, 4>(W, x, ids, k, F, down_cols, act, h, ra, s);
    return hipErrorInvalidValue;  // more experts: the caller uses the router's top-k
}

hipError_t launch_gu_any(const DevTensor &GU, const float *x, const uint32_t *ids, uint32_t k, uint32_t d_expert,
                         uint32_t down_cols, uint32_t act, float *h, const FmtRoute &ra, hipStream_t s) {
    const int K = (int)k, F = (int)d_expert, Kd = (int)down_cols;
    switch (GU.type) {
    case LT_TYPE_Q5_0: return launch_gu_t<LT_TYPE_Q5_0>(GU, x, ids, K, F, Kd, act, h, ra, s);
    case LT_TYPE_Q5_1: return launch_gu_t<LT_TYPE_Q5_1>(GU, x, ids, K, F, Kd, act, h, ra, s);
    case LT_TYPE_IQ4_NL: return launch_gu_t<LT_TYPE_IQ4_NL>(GU, x, ids, K, F, Kd, act, h, ra, s);
    case LT_TYPE_Q3_K: return launch_gu_t<LT_TYPE_Q3_K>(GU, x, ids, K, F, Kd, act, h, ra, s);
    default: return hipErrorInvalidValue;
    }
}

template <int T>
hipError_t launch_dn_t(const DevTensor &W, const float *h, const uint32_t *ids, const float *w, int k,
                       const float *base, int accumulate, const float *dscale, float *out, hipStream_t s) {
    // a row's lanes share its k * units (slot, unit) pairs
    switch (pick_rpw((size_t)k * (T == LT_TYPE_Q3_K ? 8 * W.blocks_per_row : W.blocks_per_row))) {
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
    const FmtRoute none{nullptr, 0, 0, nullptr, nullptr};
    return launch_gu_any(GU, x, ids, k, d_expert, down_cols, act, h, none, s);
}

hipError_t launch_expert_gate_up_fmt_routed(const DevTensor &GU, const float *x, const float *logits, uint32_t k,
                                            uint32_t norm, uint32_t d_expert, uint32_t down_cols, uint32_t act,
                                            float *h, uint32_t *ids_out, float *w_out, hipStream_t s) {
    const FmtRoute ra{logits, (int)k, (int)norm, ids_out, w_out};
    return launch_gu_any(GU, x, nullptr, k, d_expert, down_cols, act, h, ra, s);
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
