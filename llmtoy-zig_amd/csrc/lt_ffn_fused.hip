// lt_ffn_fused.hip -- a Q8_0 dense FFN at batch 1 in one launch:
// out = W_down . (act(W_gate . x) * (W_up . x)), the dense FFN of
// model/forward.zig:304-307 (the three quantMatvec calls of ops/math.zig:
// 127-171 with the gated activation between them).  Two launches pay two
// launch latencies and leave HBM idle while the second one fills; here the
// gate/up and the down weights stream at the same time.
//
// Placement.  Workgroups are dealt to the 8 XCDs round robin (group x = bid
// % 8, in-group index i = bid / 8; the same placement the MoE kernel probes
// for).  Group x owns the h rows [32 kb0, 32 kb1) (the S / 32 down-K blocks
// split in 8): its first NG blocks compute them -- one row per wavefront and
// pass, P passes -- and hand them over inside the group (workgroup-scope
// stores in the XCD's L2 when the placement holds); its next ND blocks
// compute, for output rows 16 Q j + [0, 16 Q), the partial dot over the
// group's K slice and add it into out with float atomics.  The 8 groups'
// partial rows meet in out: group 0's down block j first stores those rows'
// start value (0) with coherent stores and, once they are acknowledged,
// publishes a flag that the other groups' block j waits for before adding.
//
// Blocks only wait for blocks with smaller indices (down waits for its
// group's gate/up blocks and for group 0's down block of the same rows), so
// the waits end even when the grid does not fit on the GPU at once; every
// wait is bounded by a wall-clock limit (error word, NaN rows).  The last
// bits of out depend on the order of the 8 atomic adds per row.
//
// Arithmetic: Q8_0 blocks (quant/dequant.zig:31-78) times fp32 x, 16
// products per lane and unit in two fma chains, the block scale applied to
// the unit's sum; fp32 throughout.
#include "lt_internal.h"

#include <algorithm>

namespace lt {

namespace {

constexpr int kThreads = 256;
constexpr uint64_t kWaitTicks = 20000000;  // 200 ms of the 100 MHz wall clock
constexpr int kPMax = 4;                    // gate/up passes per block (template P)
constexpr int kQMax = 2;                    // down steps (16 rows each) per block
constexpr int kMV = 4;                      // down units per lane (K slice <= 64 units: S <= 8192)

struct FfnArgs {
    const uint8_t *gq, *uq, *dq;   // quant planes: gate, up [S][D/32][32], down [D][S/32][32]
    const uint16_t *gd, *ud, *dd;  // f16 scale planes
    const float *x;
    float *out;
    uint32_t *counters;  // [kFusedBlocks] launch counters
    uint64_t *hw;        // [S] h words
    uint64_t *flags;     // [kFfnFlags] start-value flags of group 0's down blocks
    uint32_t *err;
    int D, S, nbD, nbS, act, local;
    int P, Q, NG, ND;
};

// the slice of down-K blocks of group x
__device__ __forceinline__ void k_slice(int nbS, int x, int &kb0, int &kb1) {
    kb0 = (x * nbS) >> 3;
    kb1 = ((x + 1) * nbS) >> 3;
}

// sum over 16 quants of q * x
__device__ __forceinline__ float q8_unit(uint4 q, const float *xv) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        a0 = fmaf((float)(int8_t)(w[t] & 0xffu), xv[4 * t], a0);
        a1 = fmaf((float)(int8_t)((w[t] >> 8) & 0xffu), xv[4 * t + 1], a1);
        a0 = fmaf((float)(int8_t)((w[t] >> 16) & 0xffu), xv[4 * t + 2], a0);
        a1 = fmaf((float)(int8_t)(w[t] >> 24), xv[4 * t + 3], a1);
    }
    return a0 + a1;
}

__device__ __forceinline__ void lds16(const float *p, float (&xv)[16]) {
#pragma unroll
    for (int t = 0; t < 16; t += 4) {
        const float4 v = *reinterpret_cast<const float4 *>(p + t);
        xv[t] = v.x;
        xv[t + 1] = v.y;
        xv[t + 2] = v.z;
        xv[t + 3] = v.w;
    }
}

// Gate/up block i of group x: h rows 32 kb0 + 4 (p NG + i) + w (p < P) of
// the slice, wavefront w -- pass p of the NG blocks covers 4 NG consecutive
// rows, so the rows past the slice fall to the last pass of the last
// blocks, and with NG a multiple of 32 (blocks i and i + 32 share a CU)
// every CU carries the same share of the stream up to one pass; lane l
// takes units l + 64 c (c < CU) of the row (16 quants each).  x goes to LDS
// once; every load is issued before the first product, unconditionally (a
// row past the slice reloads the block's pass-0 row), so that each pass
// waits only for its own data.
template <int CU, int P>
__device__ __forceinline__ void role_gate_up(const FfnArgs &a, float *xs, uint32_t *s_ep, int x, int i, int bid,
                                             int tid, int wave, int lane) {
    const int nu = 2 * a.nbD;
    int kb0, kb1;
    k_slice(a.nbS, x, kb0, kb1);
    const int j_end = 32 * kb1;
    const int jb = 32 * kb0 + 4 * i + wave;  // pass 0's row
    // x: thread t loads float4 t and t + 256 (D <= 2048)
    const float4 x0 = *reinterpret_cast<const float4 *>(a.x + min(4 * tid, a.D - 4));
    const float4 x1 = *reinterpret_cast<const float4 *>(a.x + min(4 * (tid + kThreads), a.D - 4));
    __builtin_amdgcn_sched_barrier(0);  // keeps the x loads ahead of the weight loads
    uint4 qg[P][CU], qu[P][CU];
    uint32_t dg[P][CU], du[P][CU];
#pragma unroll
    for (int p = 0; p < P; p++) {
        const int jp = jb + 4 * a.NG * p;
        const int j = jp < j_end ? jp : min(jb, j_end - 1);
#pragma unroll
        for (int c = 0; c < CU; c++) {
            const int u = min(lane + 64 * c, nu - 1);
            const size_t blk = (size_t)j * a.nbD + (u >> 1);
            qg[p][c] = ldg16_nt(a.gq + blk * 32 + (u & 1) * 16);  // (non-temporal: read once)
            qu[p][c] = ldg16_nt(a.uq + blk * 32 + (u & 1) * 16);
            dg[p][c] = a.gd[blk];
            du[p][c] = a.ud[blk];
        }
    }
    if (4 * tid < a.D) *reinterpret_cast<float4 *>(xs + 4 * tid) = x0;
    if (4 * (tid + kThreads) < a.D) *reinterpret_cast<float4 *>(xs + 4 * (tid + kThreads)) = x1;
    if (tid == 0) *s_ep = epoch_commit(a.counters, bid, epoch_peek(a.counters, bid));
    __syncthreads();  // xs, s_ep
    const uint32_t ep = *s_ep;
    const bool first = p32_first(lane);
#pragma unroll
    for (int p = 0; p < P; p++) {
        const int j = jb + 4 * a.NG * p;
        float g = 0.0f, up = 0.0f;
#pragma unroll
        for (int c = 0; c < CU; c++) {
            const int u = lane + 64 * c;
            if (u < nu) {
                float xv[16];
                lds16(xs + 16 * u, xv);
                g = fmaf(f16_bits_to_f32(dg[p][c]), q8_unit(qg[p][c], xv), g);
                up = fmaf(f16_bits_to_f32(du[p][c]), q8_unit(qu[p][c], xv), up);
            }
        }
        g = group_sum_dpp<64>(g, first);
        up = group_sum_dpp<64>(up, first);
        if (lane == 0 && j < j_end) hand_put_group(a.hw + j, __float_as_uint(act_apply((uint32_t)a.act, g) * up), ep,
                                                   a.local);
    }
}

// Down block j of group x: output rows r0 = 16 Q j + 16 q + 4 w + (lane >>
// 4) (q < Q), 16 lanes per row, lane l16 taking units l16 + 16 m (m < kMV)
// of the group's K slice.  Group 0 stores the rows' start values first;
// the weights are loaded while the slice's h words are awaited.
__device__ __forceinline__ void role_down(const FfnArgs &a, float *hs, uint32_t *s_ep, int *s_fail, int x, int jd,
                                          int bid, int tid, int wave, int lane) {
    int kb0, kb1;
    k_slice(a.nbS, x, kb0, kb1);
    const int nk = kb1 - kb0, nv = 2 * nk;
    const int r0 = jd * 16 * a.Q;
    const int l16 = lane & 15;
    if (tid == 0) {
        *s_ep = epoch_commit(a.counters, bid, epoch_peek(a.counters, bid));
        *s_fail = 0;
    }
    __syncthreads();
    const uint32_t ep = *s_ep;
    if (x == 0) {  // start values, acknowledged before the flag goes out
        if (tid < 16 * a.Q && r0 + tid < a.D)
            __hip_atomic_store(a.out + r0 + tid, 0.0f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) hand_put(a.flags + jd, 1u, ep);
    }
    uint4 qw[kQMax][kMV];
    uint32_t dw[kQMax][kMV];
#pragma unroll
    for (int q = 0; q < kQMax; q++) {
        // (a step past Q reloads step Q - 1's rows: every load
        // unconditional, so that each wait counts only later loads)
        const int r = min(r0 + 16 * min(q, a.Q - 1) + 4 * wave + (lane >> 4), a.D - 1);
#pragma unroll
        for (int m = 0; m < kMV; m++) {
            const int v = min(l16 + 16 * m, nv - 1);
            const size_t blk = (size_t)r * a.nbS + kb0 + (v >> 1);
            qw[q][m] = ldg16(a.dq + blk * 32 + (v & 1) * 16);
            dw[q][m] = a.dd[blk];
        }
    }
    // the slice's h: thread 0 waits for its last word (and, outside group
    // 0, for the start-value flag), then every word is read with its epoch
    // checked
    if (tid == 0) {
        const uint64_t t0 = wall_clock64();
        bool ok = true;
        auto wait = [&](const uint64_t *w, uint32_t code, uint32_t index) {
            while (ok && !tag_is(hand_get(w), ep)) {
                if (wall_clock64() - t0 > kWaitTicks) {
                    ok = false;
                    report_detail(a.err, bid, code, index, (uint32_t)(hand_get(w) >> 32), ep);
                }
                __builtin_amdgcn_s_sleep(2);
            }
        };
        wait(a.hw + 32 * kb1 - 1, 0x40u, (uint32_t)(32 * kb1 - 1));
        if (x != 0) wait(a.flags + jd, 0x80u, (uint32_t)jd);
        if (!ok) *s_fail = 1;
    }
    __syncthreads();
    {
        const uint64_t t0 = wall_clock64();
        bool ok = *s_fail == 0;
        for (int t = tid; t < 32 * nk && ok; t += kThreads) {
            uint64_t w = hand_get(a.hw + 32 * kb0 + t);
            while (!tag_is(w, ep)) {
                if (wall_clock64() - t0 > kWaitTicks) {
                    ok = false;
                    report_detail(a.err, bid, 0x40u, (uint32_t)(32 * kb0 + t), (uint32_t)(w >> 32), ep);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
                w = hand_get(a.hw + 32 * kb0 + t);
            }
            hs[t] = __uint_as_float((uint32_t)w);
        }
        if (!ok) atomicOr(s_fail, 1);
    }
    __syncthreads();
    const bool fail = *s_fail != 0;
#pragma unroll
    for (int q = 0; q < kQMax; q++) {
        if (q >= a.Q) break;
        float acc = 0.0f;
#pragma unroll
        for (int m = 0; m < kMV; m++) {
            const int v = l16 + 16 * m;
            if (v < nv) {
                float hv[16];
                lds16(hs + 16 * v, hv);
                acc = fmaf(f16_bits_to_f32(dw[q][m]), q8_unit(qw[q][m], hv), acc);
            }
        }
        acc = group_sum_dpp<16>(acc, false);
        const int row = r0 + 16 * q + 4 * wave + (lane >> 4);
        if (l16 == 0 && row < a.D)
            (void)__hip_atomic_fetch_add(a.out + row, fail ? __int_as_float(0x7fc00000) : acc, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    }
    if (tid == 0 && fail) report_timeout(a.err, 0x40u);
}

template <int CU, int P>
__global__ void __launch_bounds__(kThreads) k_ffn_fused(FfnArgs a) {
    extern __shared__ __align__(16) float smem[];
    __shared__ uint32_t s_ep;
    __shared__ int s_fail;
    const int bid = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int x = bid & 7, i = bid >> 3;
    if (i < a.NG) {
        role_gate_up<CU, P>(a, smem, &s_ep, x, i, bid, tid, wave, lane);
    } else if (i < a.NG + a.ND) {
        role_down(a, smem, &s_ep, &s_fail, x, i - a.NG, bid, tid, wave, lane);
    } else if (tid == 0) {  // no role: keep the launch counter in step
        (void)epoch_commit(a.counters, bid, epoch_peek(a.counters, bid));
    }
}

}  // namespace

FfnPlan plan_ffn_fused(int D, int S) {
    FfnPlan pl{};
    pl.ok = false;
    if (D < 64 || D > 2048 || D % 32 != 0 || S < 256 || S > kFfnMaxS || S % 32 != 0) return pl;
    const int nbS = S / 32;
    const int rows_max = 32 * ((nbS + 7) / 8);  // the largest group slice
    if (2 * ((nbS + 7) / 8) > 16 * kMV) return pl;
    pl.cu = (2 * (D / 32) + 63) / 64;
    // fewest down steps first, then fewest gate/up passes (measured on
    // config 1: 3 passes / 1 step 7.3 us, 2 / 2 7.4, 4 / 1 8.4; a 2048-block
    // grid with 1 / 1 7.6); the gate/up blocks rounded up to a multiple of
    // 32 where the grid has room (every CU the same share)
    for (int Q = 1; Q <= kQMax && !pl.ok; Q++)
        for (int P = 1; P <= kPMax && !pl.ok; P++) {
            const int ND = (D + 16 * Q - 1) / (16 * Q);
            int NG = (rows_max + 4 * P - 1) / (4 * P);
            if ((NG + 31) / 32 * 32 + ND <= kFusedBlocks / 8) NG = (NG + 31) / 32 * 32;
            if (NG + ND <= kFusedBlocks / 8 && ND <= kFfnFlags) {
                pl.P = P;
                pl.Q = Q;
                pl.NG = NG;
                pl.ND = ND;
                pl.ok = true;
            }
        }
    pl.lds = (size_t)std::max(D, 32 * ((nbS + 7) / 8)) * 4;
    return pl;
}

hipError_t launch_ffn_fused(const FfnPlan &pl, const DevTensor &G, const DevTensor &U, const DevTensor &Dn,
                            const float *x, uint32_t act, float *out, const FfnScratch &sc, hipStream_t s) {
    FfnArgs a{};
    a.gq = G.p0;
    a.gd = reinterpret_cast<const uint16_t *>(G.p1);
    a.uq = U.p0;
    a.ud = reinterpret_cast<const uint16_t *>(U.p1);
    a.dq = Dn.p0;
    a.dd = reinterpret_cast<const uint16_t *>(Dn.p1);
    a.x = x;
    a.out = out;
    a.counters = sc.counters;
    a.hw = sc.hw;
    a.flags = sc.flags;
    a.err = sc.err;
    a.D = (int)G.cols;
    a.S = (int)G.total_rows;
    a.nbD = a.D / 32;
    a.nbS = a.S / 32;
    a.act = (int)act;
    a.local = sc.xcd_local;
    a.P = pl.P;
    a.Q = pl.Q;
    a.NG = pl.NG;
    a.ND = pl.ND;
#define LT_FFN_CASE(C, PP)                                                                      \
    if (pl.cu == C && pl.P == PP) {                                                             \
        hipLaunchKernelGGL((k_ffn_fused<C, PP>), dim3(kFusedBlocks), dim3(kThreads), pl.lds, s, a); \
        return hipGetLastError();                                                               \
    }
    LT_FFN_CASE(1, 1) LT_FFN_CASE(1, 2) LT_FFN_CASE(1, 3) LT_FFN_CASE(1, 4)
    LT_FFN_CASE(2, 1) LT_FFN_CASE(2, 2) LT_FFN_CASE(2, 3) LT_FFN_CASE(2, 4)
#undef LT_FFN_CASE
    return hipErrorInvalidValue;
}

}  // namespace lt
