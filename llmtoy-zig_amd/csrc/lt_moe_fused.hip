// lt_moe_fused.hip -- one decode MoE layer (batch 1) in a single launch.
//
// The layer is three dependent steps: router logits + softmax/top-k
// (ops/moe.zig:44-52, gemma4/forward.zig:645-668), the selected experts'
// gate/up products with the gated activation (moe.zig:55-66), and their down
// products with the weighted combine (moe.zig:67-76).  Three launches cost
// three launch latencies plus three HBM round trips in series; here one grid
// of kFusedBlocks workgroups runs all of it.
//
// Placement.  Workgroups are dealt to the 8 XCDs round robin, so the blocks
// with equal bid % 8 ("group" x) share one XCD and its L2.  Slot s (the s-th
// selected expert) is computed entirely inside group s % 8: its gate/up
// blocks publish h and its down blocks read that h.  Within group x the
// in-group index i = bid / 8 picks the role:
//
//   i < NRg                 router: logit rows 2*bid + [0, 2), dotf32 order
//                           (4*bid + [0, 4) when the grid has no room), or
//                           dotQ8_0 order for a Q8_0 router
//   next NSg                shared FFN gate/up: sg_rows h rows of the
//                           group's K slice of the shared down product
//   next SPG*G              gate/up: slot x + 8u, h group jg (16 values)
//   next SPG*NDg            down: slot x + 8u, rows 64j + [0, 64); the first
//                           NDg also add the shared FFN's rows 64j + [0, 64)
//                           over the group's K slice
//   next NCg                combine: rows 8c + [0, 8), c = 8(i - ...) + x
//   the rest                no role
//
// (SPG = slots per group = ceil(k / 8), G = Kd / 16, NDg = ceil(D / 64),
// NCg = NDg with the deterministic combine, else 0, NSg = 0 without a
// shared FFN; NRg also covers one router block per 256 output rows,
// store_starts).  Every hand-over is
// coherent across XCDs except the h records (and the shared FFN's h) when
// local is set: those are workgroup-scope stores that only the writer's L2
// holds, correct only while the round-robin placement holds (probed once per
// context by probe_xcd_groups).  Were it to change, the down blocks' bounded
// waits would time out (NaN outputs, the error word set); the host then
// reports LT_ERR_DEVICE at the next synchronising call and clears local.
//
// Combine.  By default the down blocks add their slot's weighted rows
// straight into out with float atomics (agent scope): the router blocks
// set out to its starting value (0, the shared FFN output, or out + that
// when accumulating) with coherent stores after their logits and flag them
// once acknowledged; every block waits for its rows' flag before adding,
// so each add lands after the start value.  The order of the k adds to a row
// varies, so the result's last bits may differ run to run.  With det set,
// the down blocks publish per-slot partial rows instead and the combining
// blocks add them in slot order (moeForward's order, ops/moe.zig:67-76):
// bit-identical results at the cost of one more hand-over.
//
// Hand-over.  Results move as 64-bit words (32-bit payload, 32-bit launch
// epoch) written and read with relaxed atomics: agent-scope loads (sc1:
// coherent across the XCDs' L2s without cache flushes) and agent-scope
// stores, or workgroup-scope stores for the h records, which only blocks on
// the writer's XCD read (see hand_put_group).  Each word has one writing
// wavefront.  A reader waits until every word it needs carries the current
// epoch.  The epoch of a launch is the launch count: block b keeps its own
// counter counters[b] (no contended atomic), and since every launch runs the
// same kFusedBlocks blocks, all counters stay equal.
//
// Blocks only wait for blocks with smaller indices (combine -> down ->
// gate/up -> router), and workgroups are dispatched in index order, so the
// waits always end even when the grid does not fit on the GPU at once.
// Every wait is also bounded by a wall-clock limit; on expiry the block sets
// the host-visible error word and its outputs become NaN.
//
// Arithmetic.  Router logits reproduce dotf32 (ops/math.zig:96-116) bit for
// bit (exact routing).  The expert products multiply 4-bit weights by fp32
// activations split into two int8 limbs per element over groups of 16:
// x ~= sp * (256*a + b), a in [-127, 127], b in [-128, 127], sp = max|x| /
// (127*256); |x - sp*(256a+b)| <= max|x| / 65024.  Weight nibbles and limbs
// meet in v_dot4 (4 products per instruction, exact int32 sums); the Q4_K
// scale and min terms are applied per sub-block in fp32
// (quant/dequant.zig:157-187 reassociated).  Gate/up blocks publish h
// already in this limb form.
#include "lt_internal.h"
#include "lt_topk.h"
#include "lt_limbs.h"
#include "lt_fmt.h"

#include <math.h>

#include <algorithm>

namespace lt {

namespace {

constexpr int kThreads = 256;
constexpr int kFusedMaxD = 4096;            // d_model of the single-launch kernel
constexpr int kDownRows = 64;               // output rows per down block (16 lane groups x 4)
constexpr int kCombRows = 8;                // output rows per combining block
constexpr uint64_t kWaitTicks = 20000000;   // 200 ms of the 100 MHz wall clock
constexpr int kRecWords = 10;               // h record: a[4] b[4] sp xs

struct FusedArgs {
    const float *router;  // [E][D] fp32
    const float *bias;    // [E] or null
    const uint8_t *gu_hdr, *gu_qs;  // gate_up planes, E*2F rows of nsb super-blocks
    const uint8_t *dn_hdr, *dn_qs;  // down planes, E*D rows of nsbd super-blocks
    const float *x;
    const float *base;  // added to the result (shared FFN output) or null
    float *out;
    uint32_t *ids_out;
    float *w_out;
    uint32_t *counters;  // [kFusedBlocks]
    uint64_t *lg;        // logits, 8 copies of kLgCopy words (logit r = word r)
    uint64_t *hl;        // h record lines [k*G][16]
    uint64_t *pl;        // partial-output lines [k*NDg*4][16]
    uint32_t *err;       // host-mapped error word (bit mask of the waits that timed out)
    uint64_t *stamps;    // phase stamps (LT_PROFILE=timeline) or null
    int E, D, nsb, F, nsbd, k, norm, act, accumulate, det, local;
    int dn_delay;  // wall-clock ticks from seeing the logits to the down weight loads
    int rb;        // logit rows per router block: 2 or 4
    int NRg, SPG, G, NDg, NCg;
    int Ewait;  // logit rows published and waited for (E)
    // the Gemma-style instances (SH 1 and 2) only
    const uint8_t *rq;   // Q8_0 router: quant plane [E][nb][32] (qrouter)
    const uint16_t *rd;  //   and f16 scale plane [E][nb]
    const uint8_t *sgq, *suq, *sdq;   // shared FFN (Q8_0) quant planes: gate, up [S][D/32], down [D][S/32]
    const uint16_t *sgd, *sud, *sdd;  //   and their scale planes
    uint64_t *shh;       // shared FFN h [S], hand-over words
    int qrouter, S;      // S = 0: no shared FFN
    int NSg;             // shared gate/up blocks per XCD group
    int sg_rows;         // shared h rows per shared gate/up block
    // the Gemma4 block (gemma; the SH 2 instance): out is the experts' sum
    // (moe), x the block's input, overwritten by the tail block
    const float *g_raw_scale, *g_pre, *g_dscale, *g_dense, *g_w2, *g_w;
    float *g_x;
    float g_raw_global, g_eps, g_out_scale;
    int gemma;
    uint64_t *done;      // [k * NDg] down blocks' completion words, awaited by the tail block
    // the format instance (SH 3): the expert tensors' types and their other
    // planes (Q3_K gate/up: qs gu_hdr, hmask gu_qs, scales gu_p2, d gu_p3;
    // IQ4_NL / Q5_0 / Q5_1 down: qs dn_hdr, then dn_qs, dn_p2)
    int gu_type, dn_type;
    const uint8_t *gu_p2, *gu_p3, *dn_p2;
};

// Phase stamps (LT_PROFILE=timeline), thread 0's: held in registers and
// written at the block's end, or (wt, the Gemma-style instance, which needs
// those registers) written straight to the block's row, cleared at its
// start.  wt is a constant of each kernel instance.
struct Stamps {
    bool wt;
    bool on;
    uint64_t *row;  // stamps + bid * kStamps, or null
    uint64_t t[kStamps];
    __device__ __forceinline__ void mark(int i, int tid) {
        if (wt) {
            if (row && tid == 0) row[i] = wall_clock64();
        } else if (on && tid == 0) {
            t[i] = wall_clock64();
        }
    }
};

__device__ __forceinline__ uint4 ld16(const uint8_t *p) { return *reinterpret_cast<const uint4 *>(p); }

// Single-lane wait for one hand-over word (the probe), with a short sleep
// between reads, so that waiting blocks put little load on the memory
// system; the caller then reads everything it needs once.  False on timeout.
__device__ __forceinline__ bool probe_wait(const uint64_t *w, uint32_t ep, uint64_t t0) {
    while (!tag_is(hand_get(w), ep)) {
        if (wall_clock64() - t0 > kWaitTicks) return false;
        __builtin_amdgcn_s_sleep(2);
    }
    return true;
}

// One wavefront waits for the E logits and returns them in v[j] = logit
// lane + 64j.  The router publishes 8 copies (logit r = word r of each) and
// a block reads copy bid % 8: with one copy, the 640 reading wavefronts
// queued on the same few lines at the memory side.  Lane 0 first waits for
// one line (chosen by block index, spreading the probes over the lines),
// then the wavefront reads all of them.  False on timeout.
template <int PER>
__device__ bool poll_logits(const FusedArgs &a, uint32_t ep, float (&v)[PER], int lane) {
    const uint64_t t0 = wall_clock64();
    bool ok = true;
    const uint64_t *lg = a.lg + (size_t)(blockIdx.x & 7) * kLgCopy;  // this group's copy
    if (lane == 0) ok = probe_wait(lg + (size_t)((blockIdx.x >> 3) % ((a.E + 15) >> 4)) * 16, ep, t0);
    if (!__all(ok)) return false;
    while (true) {
        uint64_t wv[PER];
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int r = lane + 64 * j;
            wv[j] = r < a.Ewait ? hand_get(lg + r) : ((uint64_t)ep << 32);
        }
        bool good = true;
#pragma unroll
        for (int j = 0; j < PER; j++) {
            good = good && tag_is(wv[j], ep);
            v[j] = __uint_as_float((uint32_t)wv[j]);
        }
        if (__all(good)) return true;
        if (wall_clock64() - t0 > kWaitTicks) return false;
        __builtin_amdgcn_s_sleep(1);
    }
}

// Sum of 4 values per lane over each 32-lane half, transposed: returns in
// every lane the half's total of value index (lane >> 3) & 3.
__device__ __forceinline__ float half_sum4(const float (&v)[4], int lane) {
    float a0, a1;
    {
        const bool hi = lane & 16;  // lane bit 4: keep values {0,1} or {2,3}
        const float s0 = hi ? v[0] : v[2], k0 = hi ? v[2] : v[0];
        const float s1 = hi ? v[1] : v[3], k1 = hi ? v[3] : v[1];
        a0 = k0 + xor16(s0);
        a1 = k1 + xor16(s1);
    }
    float t;
    {
        const bool hi = lane & 8;  // lane bit 3 (row_ror:8 pairs i with i ^ 8 in a 16-lane row)
        const float send = hi ? a0 : a1, keep = hi ? a1 : a0;
        t = keep + dpp<0x128>(send);
    }
    t += dpp<0xB1>(t);   // lane bit 0
    t += dpp<0x4E>(t);   // lane bit 1
    t += dpp<0x141>(t);  // lane bit 2 (row_half_mirror)
    return t;
}


// ---------------------------------------------------------------- router
// Wavefront w computes logit row bid*4 + w with dotf32's rounded operations
// (ops/math.zig:96-116; the same sequence as k_router_f32 in lt_router.hip):
// one rounding per product, 32 sequential chains over the 32-element
// strides, (acc0+acc1)+(acc2+acc3) per lane l < 8, the ordered 8-lane
// reduce, then + bias.  D % 256 == 0 and D <= 2048 (checked by the host).
// The row arrives as nsb chunks of 256 elements, one float4 per lane each,
// all loads in flight at once.  As each chunk lands its products pass
// through the wavefront's LDS area to the chain lanes (lane l < 32 owns
// chain l, elements l + 32 it), which add its 8 strides: the chains run
// while later chunks are still in flight.  The final reduce stays in
// registers and every wavefront publishes its own logit, so the block never
// synchronises.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Atomic combine: the start values of out (0, the base, or out + base).
// Router block c stores rows 256 c + [0, 256) with coherent stores (the
// plan gives the grid at least ceil(D / 256) router blocks) after its
// logits, and flags them once acknowledged (flag_starts).
__device__ __forceinline__ void store_starts(const FusedArgs &a, int bid, int tid) {
    const int orow = bid * kThreads + tid;
    if (!a.det && orow < a.D && !(a.accumulate && !a.base)) {
        const float start = a.accumulate ? a.out[orow] + a.base[orow] : (a.base ? a.base[orow] : 0.0f);
        __hip_atomic_store(a.out + orow, start, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Router block b < ceil(D / 256) stores the start values of out rows 256 b
// + [0, 256) after publishing its logits, and once the stores are
// acknowledged sets word kStartFlagOff + b of every logit copy; every block
// adding into out waits for the flag of its rows first.  (Stores count in
// vmcnt with the loads, in order: stored before the router's loads, or
// acknowledged before its logits, they delayed the logits by the time an
// acknowledgement takes while the weight streams fill the memory system,
// up to 3 us.)
constexpr int kStartFlagOff = kLgCopy - 16;
__device__ __forceinline__ bool starts_stored_by_router(const FusedArgs &a) {
    return !a.det && !(a.accumulate && !a.base);
}
__device__ __forceinline__ void flag_starts(const FusedArgs &a, int bid, int tid, uint32_t ep) {
    if (!starts_stored_by_router(a) || bid * kThreads >= a.D) return;  // (uniform over the block)
    store_starts(a, bid, tid);
    __builtin_amdgcn_s_waitcnt(0);  // this thread's start store acknowledged
    __syncthreads();
    if (tid < 8) hand_put(a.lg + (size_t)tid * kLgCopy + kStartFlagOff + bid, 1u, ep);
}
__device__ __forceinline__ const uint64_t *start_flag(const FusedArgs &a, int x, int row) {
    return a.lg + (size_t)x * kLgCopy + kStartFlagOff + (row >> 8);
}

__device__ __forceinline__ void role_router(const FusedArgs &a, uint8_t *smem, int bid, int tid, int wave,
                                            int lane, Stamps &S) {
#pragma clang fp contract(off)
    float *prod = reinterpret_cast<float *>(smem) + wave * 512;  // two chunk buffers
    const int row = bid * 4 + wave;
    const bool valid = row < a.E;
    const float *wr = a.router + (size_t)(valid ? row : 0) * a.D;
    // every load unconditional (chunk indices clamped), so that the waits
    // for chunk i count only the loads issued after it
    float4 wv[8], xv[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int ci = i < a.nsb ? i : a.nsb - 1;
        wv[i] = *reinterpret_cast<const float4 *>(wr + ci * 256 + 4 * lane);
        xv[i] = *reinterpret_cast<const float4 *>(a.x + ci * 256 + 4 * lane);
    }
    const float bias = *(a.bias ? a.bias + (valid ? row : 0) : a.x);
    const uint32_t c0 = epoch_peek(a.counters, bid);
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        if (i < a.nsb) {
            float4 pr;
            pr.x = wv[i].x * xv[i].x;
            pr.y = wv[i].y * xv[i].y;
            pr.z = wv[i].z * xv[i].z;
            pr.w = wv[i].w * xv[i].w;
            float *buf = prod + (i & 1) * 256;
            *reinterpret_cast<float4 *>(buf + 4 * lane) = pr;
            if (i == 0) S.mark(1, tid);
            wave_lds_sync();
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = buf[u * 32 + (lane & 31)];
#pragma unroll
            for (int u = 0; u < 8; u++) acc = acc + v[u];
        }
    }
    // lanes l < 8: (c[l] + c[l+8]) + (c[l+16] + c[l+24]); then the ordered
    // sum over l
    const float s2 = acc + dpp<0x128>(acc);
    const float a8 = s2 + xor16(s2);
    float sum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a8), 0));
#pragma unroll
    for (int l = 1; l < 8; l++) sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a8), l));
    if (a.bias) sum = sum + bias;
    __syncthreads();
    if (lane < 8 && row < a.Ewait) hand_put(a.lg + (size_t)lane * kLgCopy + row, __float_as_uint(sum), c0 + 1u);  // copy lane
    S.mark(2, tid);
    flag_starts(a, bid, tid, c0 + 1u);
    if (tid == 0) (void)epoch_commit(a.counters, bid, c0);
}

// Router, two logit rows per block (rows 2 bid + (w >> 1)): wavefront w owns
// chains 16 (w & 1) + [0, 16) of its row, so a CU moves 16 KB of router
// rows (4 rows: 32 KB) and the rows arrive sooner, while each chain still
// adds its strides as they land: load q, lane L take the float4 of stride
// it = 16q + L/4, chains 16 (w & 1) + 4 (L & 3) + [0, 4); the products pass
// through the wavefront's LDS to chain lanes c < 16.  Then (acc0+acc1) is
// formed in each wavefront (lanes l and l + 8), (acc2+acc3) crosses to the
// row's first wavefront through LDS, and it finishes the ordered 8-lane sum
// and the bias: the operations of role_router in the same order.
__device__ __forceinline__ void role_router_pair(const FusedArgs &a, uint8_t *smem, int bid, int tid, int wave,
                                                 int lane, Stamps &S) {
#pragma clang fp contract(off)
    const int nit = a.D >> 5;                                       // strides per chain
    float *prod = reinterpret_cast<float *>(smem) + wave * 512;    // two [16][16] chunk buffers
    float *xch = reinterpret_cast<float *>(smem) + 4 * 512;        // [2][8]
    const int h = wave & 1, rl = wave >> 1;
    const int row = 2 * bid + rl;
    const bool valid = row < a.E;
    const float *wr = a.router + (size_t)(valid ? row : 0) * a.D;
    // loads in batches of 4 (64 strides: D <= 2048 in one batch, 4096 in
    // two); every load unconditional (stride clamped), so that the wait for
    // load q counts only the loads issued after it.  The first batch goes
    // out before the bias and counter loads.
    float4 wv[4], xv[4];
    auto load_batch = [&](int qb) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            int it = 16 * (qb + q) + (lane >> 2);
            it = it < nit ? it : nit - 1;
            const int e = 32 * it + 16 * h + 4 * (lane & 3);
            wv[q] = *reinterpret_cast<const float4 *>(wr + e);
            xv[q] = *reinterpret_cast<const float4 *>(a.x + e);
        }
    };
    load_batch(0);
    const float bias = *(a.bias ? a.bias + (valid ? row : 0) : a.x);
    const uint32_t c0 = epoch_peek(a.counters, bid);
    float acc = 0.0f;
    for (int qb = 0; 16 * qb < nit; qb += 4) {
        if (qb > 0) load_batch(qb);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            if (16 * (qb + q) < nit) {
                float4 pr;
                pr.x = wv[q].x * xv[q].x;
                pr.y = wv[q].y * xv[q].y;
                pr.z = wv[q].z * xv[q].z;
                pr.w = wv[q].w * xv[q].w;
                float *buf = prod + (q & 1) * 256;
                *reinterpret_cast<float4 *>(buf + 4 * lane) = pr;
                if (q == 0) S.mark(1, tid);
                wave_lds_sync();
                // n = 8 or 16 strides in this load; reads past n stay inside the
                // buffer and are not added
                const int n = nit - 16 * (qb + q) < 16 ? nit - 16 * (qb + q) : 16;
                float v[16];
#pragma unroll
                for (int u = 0; u < 16; u++) v[u] = buf[u * 16 + (lane & 15)];
#pragma unroll
                for (int u0 = 0; u0 < 16; u0 += 8)
                    if (u0 < n)
#pragma unroll
                        for (int u = 0; u < 8; u++) acc = acc + v[u0 + u];
            }
        }
    }
    // lanes l < 8: chains 16h + l and 16h + l + 8
    const float s2 = acc + dpp<0x128>(acc);
    if (h == 1 && lane < 8) xch[rl * 8 + lane] = s2;
    __syncthreads();
    if (h == 0) {
        const float a8 = s2 + xch[rl * 8 + (lane & 7)];
        float sum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a8), 0));
#pragma unroll
        for (int l = 1; l < 8; l++) sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a8), l));
        if (a.bias) sum = sum + bias;
        if (lane < 8 && row < a.Ewait) hand_put(a.lg + (size_t)lane * kLgCopy + row, __float_as_uint(sum), c0 + 1u);  // copy lane
        S.mark(2, tid);
    }
    flag_starts(a, bid, tid, c0 + 1u);
    if (tid == 0) (void)epoch_commit(a.counters, bid, c0);
}

// The same for rows of at most 2048 (one batch of loads).
__device__ __forceinline__ void role_router_pair_one(const FusedArgs &a, uint8_t *smem, int bid, int tid, int wave,
                                                     int lane, Stamps &S) {
#pragma clang fp contract(off)
    const int nit = a.D >> 5;                                       // strides per chain
    float *prod = reinterpret_cast<float *>(smem) + wave * 512;    // two [16][16] chunk buffers
    float *xch = reinterpret_cast<float *>(smem) + 4 * 512;        // [2][8]
    const int h = wave & 1, rl = wave >> 1;
    const int row = 2 * bid + rl;
    const bool valid = row < a.E;
    const float *wr = a.router + (size_t)(valid ? row : 0) * a.D;
    // every load unconditional (stride clamped), so that the wait for load
    // q counts only the loads issued after it
    float4 wv[4], xv[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        int it = 16 * q + (lane >> 2);
        it = it < nit ? it : nit - 1;
        const int e = 32 * it + 16 * h + 4 * (lane & 3);
        wv[q] = *reinterpret_cast<const float4 *>(wr + e);
        xv[q] = *reinterpret_cast<const float4 *>(a.x + e);
    }
    const float bias = *(a.bias ? a.bias + (valid ? row : 0) : a.x);
    const uint32_t c0 = epoch_peek(a.counters, bid);
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        if (16 * q < nit) {
            float4 pr;
            pr.x = wv[q].x * xv[q].x;
            pr.y = wv[q].y * xv[q].y;
            pr.z = wv[q].z * xv[q].z;
            pr.w = wv[q].w * xv[q].w;
            float *buf = prod + (q & 1) * 256;
            *reinterpret_cast<float4 *>(buf + 4 * lane) = pr;
            if (q == 0) S.mark(1, tid);
            wave_lds_sync();
            // n = 8 or 16 strides in this load; reads past n stay inside the
            // buffer and are not added
            const int n = nit - 16 * q < 16 ? nit - 16 * q : 16;
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; u++) v[u] = buf[u * 16 + (lane & 15)];
#pragma unroll
            for (int u0 = 0; u0 < 16; u0 += 8)
                if (u0 < n)
#pragma unroll
                    for (int u = 0; u < 8; u++) acc = acc + v[u0 + u];
        }
    }
    // lanes l < 8: chains 16h + l and 16h + l + 8
    const float s2 = acc + dpp<0x128>(acc);
    if (h == 1 && lane < 8) xch[rl * 8 + lane] = s2;
    __syncthreads();
    if (h == 0) {
        const float a8 = s2 + xch[rl * 8 + (lane & 7)];
        float sum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a8), 0));
#pragma unroll
        for (int l = 1; l < 8; l++) sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a8), l));
        if (a.bias) sum = sum + bias;
        if (lane < 8 && row < a.Ewait) hand_put(a.lg + (size_t)lane * kLgCopy + row, __float_as_uint(sum), c0 + 1u);  // copy lane
        S.mark(2, tid);
    }
    flag_starts(a, bid, tid, c0 + 1u);
    if (tid == 0) (void)epoch_commit(a.counters, bid, c0);
}

// ---------------------------------------------------------------- Gemma4 block
// s + shfl_xor(s, 32), then 16, 8, 4, 2, 1 (the butterfly of the Q8_0
// router's prep and of the norm kernels), bit for bit, over DPP and lane
// swaps instead of LDS permutes: after the steps over lane bits 5..3 every
// lane's value depends only on lane % 8, so row_ror:4 reads a lane holding
// the value of lane ^ 4.
__device__ __forceinline__ float butterfly_sum64(float s, bool first) {
#pragma clang fp contract(off)
    s = s + xor32(s, first);
    s = s + xor16(s);
    s = s + dpp<0x128>(s);  // row_ror:8 = lane ^ 8
    s = s + dpp<0x124>(s);  // row_ror:4
    s = s + dpp<0x4E>(s);   // quad_perm [2,3,0,1] = lane ^ 2
    s = s + dpp<0xB1>(s);   // quad_perm [1,0,3,2] = lane ^ 1
    return s;
}

// rms_inv of x (the Gemma4 block's input, D floats) in the order of the Q8_0
// router kernel's prep (k_router_q8_0, 128 threads): thread t < 128 sums
// x^2 over float4 chunks t, t + 128, ... in order, the 64-lane xor
// butterfly, then wavefront 0's total plus wavefront 1's; 1 / sqrt(ss / n +
// eps) with correctly rounded division and square root.  gemma_rms_load
// issues the (at most 8) chunks of a thread at once (indices clamped: only
// those in range are added, in the loop's order); gemma_rms_inv, called by
// every thread of the block (a barrier inside), returns the same bits to
// all.
struct RmsLoads {
    float4 v[8];
};
__device__ __forceinline__ void gemma_rms_load(const FusedArgs &a, int tid, RmsLoads &r) {
    if (tid >= 128) return;
    const float4 *x4 = reinterpret_cast<const float4 *>(a.x);
    const int n4 = a.D / 4;  // <= 1024
#pragma unroll
    for (int m = 0; m < 8; m++) r.v[m] = x4[min(tid + 128 * m, n4 - 1)];
}
__device__ __forceinline__ float gemma_rms_inv(const FusedArgs &a, int tid, const RmsLoads &r) {
#pragma clang fp contract(off)
    __shared__ float red[2];
    if (tid < 128) {
        const int n4 = a.D / 4;
        float ss = 0.0f;
#pragma unroll
        for (int m = 0; m < 8; m++) {
            if (tid + 128 * m < n4) {
                ss = ss + r.v[m].x * r.v[m].x;
                ss = ss + r.v[m].y * r.v[m].y;
                ss = ss + r.v[m].z * r.v[m].z;
                ss = ss + r.v[m].w * r.v[m].w;
            }
        }
        ss = butterfly_sum64(ss, p32_first(tid & 63));
        if ((tid & 63) == 0) red[tid >> 6] = ss;
    }
    __syncthreads();
    return 1.0f / sqrtf((red[0] + red[1]) / (float)a.D + a.g_eps);
}
__device__ __forceinline__ float gemma_rms_inv(const FusedArgs &a, int tid) {
    RmsLoads r;
    gemma_rms_load(a, tid, r);
    return gemma_rms_inv(a, tid, r);
}

// ---------------------------------------------------------------- Q8_0 router
// Rows 2 bid + [0, 2) of a Q8_0 router: thread t of half h = t >> 7 takes
// block b = t & 127 (b < nb = D / 32 <= 128) of row 2 bid + h and computes
// dotQ8_0's block term (quant/dequant.zig:59-78: 8 lane accumulators over 4
// groups of 8 products, the ordered 8-lane sum, times d) into LDS; the first
// wavefront of each half adds the nb terms in block order (the reference's
// running total) and the bias, and lanes 0-7 publish the logit's 8 copies.
template <int GEM>
__device__ __forceinline__ void role_router_q8(const FusedArgs &a, uint8_t *smem, int bid, int tid, int lane,
                                               Stamps &S) {
#pragma clang fp contract(off)
    float *terms = reinterpret_cast<float *>(smem);  // [2][128]
    const int h = tid >> 7, b = tid & 127;
    const int nb = a.D >> 5;
    const int row = 2 * bid + h;
    const bool valid = row < a.E;
    float xv[32];
    const int bc = b < nb ? b : nb - 1;
    uint4 q0, q1;
    uint32_t d16;
    float bias;
    uint32_t c0;
    if (GEM && a.gemma) {
        // The Gemma4 block: the router input (x * (rms_inv * raw_global)) *
        // raw_scale, as the Q8_0 router kernel's prep forms it, once per block:
        // x and raw_scale float4 c = tid + 256 m go to LDS (x first, for the
        // RMS), then the prepared row replaces x there and each thread reads
        // its block's 32 values (both rows' threads share them).
        float4 *xs4 = reinterpret_cast<float4 *>(smem + 2 * 128 * 4);  // [D / 4], after terms
        const float4 *x4 = reinterpret_cast<const float4 *>(a.x);
        const float4 *s4 = reinterpret_cast<const float4 *>(a.g_raw_scale);
        const int n4 = a.D / 4;  // <= 1024
        float4 xr[4], sr[4];
#pragma unroll
        for (int m = 0; m < 4; m++) xr[m] = x4[min(tid + kThreads * m, n4 - 1)];
        // every load unconditional (clamped row and block)
        const size_t blk = (size_t)(valid ? row : 0) * nb + bc;
        q0 = ld16(a.rq + blk * 32);
        q1 = ld16(a.rq + blk * 32 + 16);
        d16 = a.rd[blk];
#pragma unroll
        for (int m = 0; m < 4; m++) sr[m] = s4[min(tid + kThreads * m, n4 - 1)];
        bias = *(a.bias ? a.bias + (valid ? row : 0) : a.x);
        c0 = epoch_peek(a.counters, bid);
#pragma unroll
        for (int m = 0; m < 4; m++)
            if (tid + kThreads * m < n4) xs4[tid + kThreads * m] = xr[m];
        __syncthreads();
        RmsLoads rms;  // k_router_q8_0's order: thread t < 128 takes chunks t + 128 m
        if (tid < 128)
#pragma unroll
            for (int m = 0; m < 8; m++) rms.v[m] = xs4[min(tid + 128 * m, n4 - 1)];
        const float raw_base = gemma_rms_inv(a, tid, rms) * a.g_raw_global;  // (a barrier inside)
#pragma unroll
        for (int m = 0; m < 4; m++)
            if (tid + kThreads * m < n4) {
                float4 v = xr[m];
                v.x = (v.x * raw_base) * sr[m].x;
                v.y = (v.y * raw_base) * sr[m].y;
                v.z = (v.z * raw_base) * sr[m].z;
                v.w = (v.w * raw_base) * sr[m].w;
                xs4[tid + kThreads * m] = v;
            }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const float4 v4 = xs4[bc * 8 + t];
            xv[4 * t] = v4.x;
            xv[4 * t + 1] = v4.y;
            xv[4 * t + 2] = v4.z;
            xv[4 * t + 3] = v4.w;
        }
    } else {
        // every load unconditional (clamped row and block)
        const size_t blk = (size_t)(valid ? row : 0) * nb + bc;
        q0 = ld16(a.rq + blk * 32);
        q1 = ld16(a.rq + blk * 32 + 16);
        d16 = a.rd[blk];
        const float4 *xp = reinterpret_cast<const float4 *>(a.x + bc * 32);
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const float4 v4 = xp[t];
            xv[4 * t] = v4.x;
            xv[4 * t + 1] = v4.y;
            xv[4 * t + 2] = v4.z;
            xv[4 * t + 3] = v4.w;
        }
        bias = *(a.bias ? a.bias + (valid ? row : 0) : a.x);
        c0 = epoch_peek(a.counters, bid);
    }
    const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    float acc[8];
#pragma unroll
    for (int l = 0; l < 8; l++) acc[l] = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int l = 0; l < 8; l++) {
            const int e = 8 * j + l;
            const float p = (float)(int)(int8_t)(qw[e >> 2] >> (8 * (e & 3))) * xv[e];
            acc[l] = acc[l] + p;
        }
    float r = acc[0];
#pragma unroll
    for (int l = 1; l < 8; l++) r = r + acc[l];
    // past the row's nb blocks the term is -0, which leaves any sum as it is
    // (x + -0 = x, also for x = +0 and -0): the ordered sum below runs over
    // whole chunks of 16 without a branch per term
    terms[h * 128 + b] = b < nb ? r * f16_bits_to_f32(d16) : -0.0f;
    S.mark(1, tid);
    __syncthreads();
    S.mark(3, tid);
    if (b < 64) {  // wavefronts 0 and 2: one row each
        // the ordered sum over the block terms (every lane the same, LDS
        // broadcast reads of 16 terms at a time)
        const float *tr = terms + h * 128;
        float total = 0.0f;
        for (int c = 0; c < nb; c += 16) {
            float t16[16];
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                const float4 v4 = *reinterpret_cast<const float4 *>(tr + c + i);
                t16[i] = v4.x; t16[i + 1] = v4.y; t16[i + 2] = v4.z; t16[i + 3] = v4.w;
            }
#pragma unroll
            for (int i = 0; i < 16; i++) total = total + t16[i];
        }
        if (a.bias) total = total + bias;
        if (lane < 8 && row < a.Ewait) hand_put(a.lg + (size_t)lane * kLgCopy + row, __float_as_uint(total), c0 + 1u);
        S.mark(2, tid);
    }
    flag_starts(a, bid, tid, c0 + 1u);
    if (tid == 0) (void)epoch_commit(a.counters, bid, c0);
}

// ---------------------------------------------------------------- shared FFN
// A Q8_0 dense FFN (the shared expert, gemma4/forward.zig:392-397, or the
// dense FFN alone, model/forward.zig:304-307) inside the same launch.
// sum over 16 quants of q * x (the half block's share of a Q8_0 block)
__device__ __forceinline__ float q8_half_sum(uint4 q, const float *xv) {
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

__device__ __forceinline__ void lds_x16(const float *p, float (&xv)[16]) {
#pragma unroll
    for (int t = 0; t < 16; t += 4) {
        const float4 v = *reinterpret_cast<const float4 *>(p + t);
        xv[t] = v.x;
        xv[t + 1] = v.y;
        xv[t + 2] = v.z;
        xv[t + 3] = v.w;
    }
}

// The shared FFN has two roles of its own in each XCD group, placed after
// the router blocks and before the experts' blocks, so that the experts'
// gate/up blocks poll the logits with no weight stream of their own in
// flight (a wavefront's loads complete in issue order, so a probe issued
// behind a stream waits for the stream).  The down product is split along K
// by XCD group: group x owns the Q8_0 blocks [x nb / 8, (x + 1) nb / 8) of
// each down row (nb = S / 32), i.e. h rows 32 x nb / 8 ... of the same slice.
// Its shared gate/up blocks compute exactly those h rows and its shared down
// blocks read only them, so h never crosses an XCD (handed over like the
// experts' h records), and the 8 groups' partial rows meet in out through
// float atomics.  Every wait of these roles is for a block of a smaller
// index: shared down waits for shared gate/up and for the router's start
// values.  d_model <= kShMaxD (three 64-lane spans of half blocks per row).
constexpr int kShMaxD = 3072;
__device__ __forceinline__ void sh_slice(const FusedArgs &a, int x, int &kb0, int &kb1) {
    const int nb = a.S >> 5;
    kb0 = (x * nb) >> 3;
    kb1 = ((x + 1) * nb) >> 3;
}

// Shared gate/up block q (< NSg) of group x: h rows [j0, j1) = the slice's
// rows q R + [0, R), R = sg_rows <= 32; wavefront w takes rows j0 + w + 4p,
// its next row's weights in flight while this row's dots run (two register
// sets).  Lane l takes the half blocks v = l + 64 m of a row (m < 3: D <=
// kShMaxD), x comes from LDS.  x is loaded first and the block's launch epoch
// read before any weight load, so that neither waits behind the stream.
// The row's act(gate . x) * (up . x) goes out as a hand-over word.
__device__ __forceinline__ void role_shared_gate_up(const FusedArgs &a, uint8_t *smem, int x, int q, int bid,
                                                    int tid, int wave, int lane, Stamps &S) {
    float *xs = reinterpret_cast<float *>(smem);
    const int nb = a.D >> 5, nu = 2 * nb;
    int kb0, kb1;
    sh_slice(a, x, kb0, kb1);
    const int j0 = 32 * kb0 + q * a.sg_rows, j1 = min(32 * kb1, j0 + a.sg_rows);
    if (j1 <= j0) return;  // no rows left for this block (the whole block)
    // three named values, not an array (an array held across the barrier
    // below ends up in scratch memory); every load unconditional (clamped)
    auto xat = [&](int t) { return *reinterpret_cast<const float4 *>(a.x + min((tid + kThreads * t) * 4, a.D - 4)); };
    const float4 x0 = xat(0), x1 = xat(1), x2 = xat(2);
    const uint32_t ep = epoch_peek(a.counters, bid) + 1u;
    __builtin_amdgcn_sched_barrier(0);  // x and the counter ahead of the weight loads
    const int nr = j1 - j0 > wave ? (j1 - j0 - wave + 3) >> 2 : 0;  // rows of this wavefront
    const int jlast = j1 - 1;
    uint4 qg0[3], qu0[3], qg1[3], qu1[3];
    uint32_t dg0[3], du0[3], dg1[3], du1[3];
    // every weight load unconditional (row and half block clamped): the
    // compiler's wait before a row's dots then counts exactly the loads of
    // the row after it
    auto load = [&](uint4 (&qg)[3], uint4 (&qu)[3], uint32_t (&dg)[3], uint32_t (&du)[3], int p) {
        const int jl = min(j0 + wave + 4 * p, jlast);
#pragma unroll
        for (int m = 0; m < 3; m++) {
            const int v = min(lane + 64 * m, nu - 1);
            const size_t blk = (size_t)jl * nb + (v >> 1);
            qg[m] = ld16(a.sgq + blk * 32 + (v & 1) * 16);
            qu[m] = ld16(a.suq + blk * 32 + (v & 1) * 16);
            dg[m] = a.sgd[blk];
            du[m] = a.sud[blk];
        }
    };
    const bool first = p32_first(lane);
    auto row = [&](const uint4 (&qg)[3], const uint4 (&qu)[3], const uint32_t (&dg)[3], const uint32_t (&du)[3],
                   int p) {
        if (p >= nr) return;  // (uniform over the wavefront)
        float g = 0.0f, up = 0.0f;
#pragma unroll
        for (int m = 0; m < 3; m++) {
            const int v = lane + 64 * m;
            if (v < nu) {
                float xv[16];
                lds_x16(xs + v * 16, xv);
                g = fmaf(f16_bits_to_f32(dg[m]), q8_half_sum(qg[m], xv), g);
                up = fmaf(f16_bits_to_f32(du[m]), q8_half_sum(qu[m], xv), up);
            }
        }
        g = group_sum_dpp<64>(g, first);
        up = group_sum_dpp<64>(up, first);
        if (lane == 0)
            hand_put_group(a.shh + j0 + wave + 4 * p, __float_as_uint(act_apply((uint32_t)a.act, g) * up), ep,
                           a.local);
    };
    load(qg0, qu0, dg0, du0, 0);
    {
        const int i = tid * 4;
        if (i < a.D) *reinterpret_cast<float4 *>(xs + i) = x0;
        if (i + 4 * kThreads < a.D) *reinterpret_cast<float4 *>(xs + i + 4 * kThreads) = x1;
        if (i + 8 * kThreads < a.D) *reinterpret_cast<float4 *>(xs + i + 8 * kThreads) = x2;
    }
    __syncthreads();  // x in LDS
    // (the loads past the wavefront's last row reload that row: clamped,
    // and unconditional so that each wait counts only the loads after it)
    for (int p = 0; p < nr; p += 2) {
        load(qg1, qu1, dg1, du1, p + 1);
        row(qg0, qu0, dg0, du0, p);
        load(qg0, qu0, dg0, du0, p + 2);
        row(qg1, qu1, dg1, du1, p + 1);
    }
    S.mark(1, tid);
}

// Shared down rows of down-position block u (< NDg) of group x: output rows
// [64 u, 64 u + 64) over the group's K slice (nk = kb1 - kb0 <= 16 blocks:
// S <= 4096, nv = 2 nk half blocks).  When the block starts, wavefronts 1-3
// load the rows' weights and store them in LDS (sh_stage_*): all 6.3 MB
// of config 4's shared down weights are then read in the routing phase, and
// none of them competes with the experts' weight streams later.  The rows
// are added after the block's own rows (sh_down_add): a CU returns loads
// in issue order across its wavefronts, so a wait for the shared h issued
// while the gate/up blocks on the same CU stream their experts' weights
// lasts until those streams end, and placed before the block's own weight
// loads or its h records it held them back by 3 us (config 4).  By the time
// the block's own rows are out the streams are over; the slice of h is read
// once the block's own weight loads are issued, and its rows are summed into
// LDS while the block waits for its own h records.  LDS from kShOff:
// quants [64][nv] x 16 B, f16 scales [64][nk], the slice of h (fp32), its
// limbs [nv][2] x 16 B, group scales [nv], row sums [64].
constexpr int kShOff = 2560;  // past the down role's h records (G <= 64: 40 G bytes)
__host__ __device__ inline size_t sh_down_lds(int S) {
    const int nk = (S / 32 + 7) / 8;  // blocks of the largest slice
    return (size_t)kShOff + (size_t)kDownRows * 2 * nk * 16 + (size_t)kDownRows * nk * 2 + (size_t)32 * nk * 4 +
           (size_t)2 * nk * 36 + (size_t)kDownRows * 4;  // + limbs and scales of its 2 nk groups, row sums
}
// Wavefronts 1-3 issue the loads when the block starts (sh_stage_load) and
// store the data in LDS while wavefront 0 polls the logits (sh_stage_store):
// quants chunk c = row * nv + v, 11 per thread at most (64 rows x 32 half
// blocks over 192 threads), scales 6 per thread; rows past r1 clamped
// (loaded, never used).
struct ShStage {
    uint4 q[11];
    uint32_t d[6];
};
__device__ __forceinline__ void sh_stage_load(const FusedArgs &a, ShStage &w, int x, int u, int tid) {
    if (tid < 64) return;  // (wavefront 0 polls the logits)
    const int nb = a.S >> 5;
    int kb0, kb1;
    sh_slice(a, x, kb0, kb1);
    const int nk = kb1 - kb0, nv = 2 * nk;
    const int r0 = u * kDownRows, r1 = min(a.D, r0 + kDownRows);
    const int t = tid - 64;
#pragma unroll
    for (int m = 0; m < 11; m++) {
        const int c = min(t + 192 * m, kDownRows * nv - 1);
        const int row = min(r0 + c / nv, r1 - 1), v = c % nv;
        w.q[m] = ld16(a.sdq + ((size_t)row * nb + kb0 + (v >> 1)) * 32 + (v & 1) * 16);
    }
#pragma unroll
    for (int m = 0; m < 6; m++) {
        const int c = min(t + 192 * m, kDownRows * nk - 1);
        const int row = min(r0 + c / nk, r1 - 1);
        w.d[m] = a.sdd[(size_t)row * nb + kb0 + c % nk];
    }
}
__device__ __forceinline__ void sh_stage_store(const FusedArgs &a, uint8_t *smem, const ShStage &w, int x, int tid) {
    if (tid < 64) return;
    int kb0, kb1;
    sh_slice(a, x, kb0, kb1);
    const int nk = kb1 - kb0, nv = 2 * nk;
    uint4 *lq = reinterpret_cast<uint4 *>(smem + kShOff);
    uint16_t *ld = reinterpret_cast<uint16_t *>(lq + kDownRows * nv);
    const int t = tid - 64;
#pragma unroll
    for (int m = 0; m < 11; m++)
        if (t + 192 * m < kDownRows * nv) lq[t + 192 * m] = w.q[m];
#pragma unroll
    for (int m = 0; m < 6; m++)
        if (t + 192 * m < kDownRows * nk) ld[t + 192 * m] = (uint16_t)w.d[m];
}
// The group's slice of the shared h into LDS after the staged weights (every
// word's epoch checked; the words come from shared gate/up blocks, of smaller
// index).  The down role reads it in the same pass as its own h records,
// which it waits for long after the slice was written.  False on timeout
// (error word 0x20).
__device__ __forceinline__ float *sh_h_lds(uint8_t *smem, int nk) {
    return reinterpret_cast<float *>(smem + kShOff + (size_t)kDownRows * 2 * nk * 16 + (size_t)kDownRows * nk * 2);
}
__device__ __forceinline__ bool sh_read_h(const FusedArgs &a, uint8_t *smem, uint32_t ep, int x, int bid, int tid) {
    int kb0, kb1;
    sh_slice(a, x, kb0, kb1);
    float *hs = sh_h_lds(smem, kb1 - kb0);
    const uint64_t t0 = wall_clock64();
    for (int i = tid; i < 32 * (kb1 - kb0); i += kThreads) {
        uint64_t hw = hand_get(a.shh + 32 * kb0 + i);
        while (!tag_is(hw, ep)) {
            if (wall_clock64() - t0 > kWaitTicks) {
                report_detail(a.err, bid, 0x20u, (uint32_t)(32 * kb0 + i), (uint32_t)(hw >> 32), ep);
                return false;
            }
            __builtin_amdgcn_s_sleep(1);
            hw = hand_get(a.shh + 32 * kb0 + i);
        }
        hs[i] = __uint_as_float((uint32_t)hw);
    }
    return true;
}
// The shared down rows [64 u, 64 u + 64) from the staged weights and the
// slice of h in LDS (sh_down_rows: sums into LDS; sh_down_add: added into
// out with float atomics).  Each half block's 16 h values become two int8
// limbs (as the experts' h records: h ~= sp (256 a + b), error <= max|h| /
// 65024 per element; thread g converts group g), so a Q8_0 half block meets
// them in 8 v_dot4 instead of 16 conversions and 16 fma.  16 lanes per row
// (lane l16 takes half blocks l16 and l16 + 16), four rows per wavefront
// and step, four steps.
__device__ __forceinline__ float *sh_row_sums(uint8_t *smem, int nk) {
    return sh_h_lds(smem, nk) + 16 * 2 * nk + 2 * 2 * nk * 4 + 2 * nk;  // after h, limbs and group scales
}
__device__ __forceinline__ void sh_down_rows(const FusedArgs &a, uint8_t *smem, int x, int u, int tid, int wave,
                                             int lane) {
    int kb0, kb1;
    sh_slice(a, x, kb0, kb1);
    const int nk = kb1 - kb0, nv = 2 * nk;
    const uint4 *lq = reinterpret_cast<const uint4 *>(smem + kShOff);
    const uint16_t *ld = reinterpret_cast<const uint16_t *>(lq + kDownRows * nv);
    const float *hs = sh_h_lds(smem, nk);
    uint4 *la = reinterpret_cast<uint4 *>(const_cast<float *>(hs) + 16 * nv);  // [nv][2]: limbs a, b
    float *lsp = reinterpret_cast<float *>(la + 2 * nv);                       // [nv]
    float *ps = sh_row_sums(smem, nk);                                         // [64]
    if (tid < nv) {  // (limbs16: NaN / inf groups give sp = NaN, tiny groups are scaled first)
        float v[16];
        lds_x16(hs + tid * 16, v);
        uint32_t pa[4], pb[4];
        float sp, xs;
        limbs16(v, pa, pb, sp, xs);
        la[2 * tid] = make_uint4(pa[0], pa[1], pa[2], pa[3]);
        la[2 * tid + 1] = make_uint4(pb[0], pb[1], pb[2], pb[3]);
        lsp[tid] = sp;
    }
    __syncthreads();
    const int l16 = lane & 15;
#pragma unroll
    for (int st = 0; st < 4; st++) {
        const int rr = 16 * st + 4 * wave + (lane >> 4);  // row within the block
        float acc = 0.0f;
#pragma unroll
        for (int m = 0; m < 2; m++) {
            const int v = l16 + 16 * m;
            if (v < nv) {
                const uint4 q = lq[rr * nv + v], ga = la[2 * v], gb = la[2 * v + 1];
                int ia = sdot4_first((int)q.x, (int)ga.x);
                ia = __builtin_amdgcn_sdot4((int)q.y, (int)ga.y, ia, false);
                ia = __builtin_amdgcn_sdot4((int)q.z, (int)ga.z, ia, false);
                ia = __builtin_amdgcn_sdot4((int)q.w, (int)ga.w, ia, false);
                int ib = sdot4_first((int)q.x, (int)gb.x);
                ib = __builtin_amdgcn_sdot4((int)q.y, (int)gb.y, ib, false);
                ib = __builtin_amdgcn_sdot4((int)q.z, (int)gb.z, ib, false);
                ib = __builtin_amdgcn_sdot4((int)q.w, (int)gb.w, ib, false);
                acc = fmaf(f16_bits_to_f32(ld[rr * nk + (v >> 1)]) * lsp[v], (float)(256 * ia + ib), acc);
            }
        }
        acc = group_sum_dpp<16>(acc, false);
        if (l16 == 0) ps[rr] = acc;
    }
}
// (after a barrier that follows sh_down_rows) fail: NaN rows (error word 0x20)
__device__ __forceinline__ void sh_down_add(const FusedArgs &a, uint8_t *smem, int x, int u, bool fail, int tid,
                                            Stamps &S) {
    int kb0, kb1;
    sh_slice(a, x, kb0, kb1);
    const float *ps = sh_row_sums(smem, kb1 - kb0);
    const int r0 = u * kDownRows, r1 = min(a.D, r0 + kDownRows);
    if (tid < kDownRows && r0 + tid < r1)
        (void)__hip_atomic_fetch_add(a.out + r0 + tid, fail ? __int_as_float(0x7fc00000) : ps[tid], __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
    if (tid == 0 && fail) report_timeout(a.err, 0x20u);
    S.mark(6, tid);
}

// ---------------------------------------------------------------- gate/up
// The block's 16 h values (s_h, written by every wavefront before the call)
// as one limb record line g: a-words, b-words, scale, sum (kRecWords words,
// group-local hand-over words); a routing timeout publishes a NaN record.
__device__ __forceinline__ void publish_h_record(const FusedArgs &a, const float *s_h, const int *s_fail, int g,
                                                 uint32_t ep, int tid, int wave, int lane, Stamps &S) {
    __syncthreads();
    if (wave == 0) {
        // the 16 h values as one limb record: lanes 0..15 own one value each
        const float hv = lane < 16 ? s_h[lane] : 0.0f;
        float m = fabsf(hv);
        m = fmaxf(m, dpp<0x128>(m));
        m = fmaxf(m, dpp<0x124>(m));
        m = fmaxf(m, dpp<0x122>(m));
        m = fmaxf(m, dpp<0x121>(m));
        float xs = hv;
        xs += dpp<0x128>(xs);
        xs += dpp<0x124>(xs);
        xs += dpp<0x122>(xs);
        xs += dpp<0x121>(xs);
        xs = __shfl(xs, 0, 64);
        m = __shfl(m, 0, 64);
        const float inv = m > 0.0f ? 127.0f / m : 0.0f;
        float sp = m * (1.0f / 32512.0f);
        if (!(fabsf(xs) <= 3.0e38f) || !(m <= 3.0e38f)) sp = __int_as_float(0x7fc00000);
        const float tt = hv * inv;
        const float fa = rintf(tt);
        const float fb = fminf(rintf((tt - fa) * 256.0f), 127.0f);
        uint32_t pa = ((uint32_t)(int)fa & 0xffu) << (8 * (lane & 3));
        uint32_t pb = ((uint32_t)(int)fb & 0xffu) << (8 * (lane & 3));
        pa |= dppw<0xB1>(pa);
        pa |= dppw<0x4E>(pa);
        pb |= dppw<0xB1>(pb);
        pb |= dppw<0x4E>(pb);
        // record word i: a-words from lanes 0,4,8,12; b-words; sp; xs
        const int src = lane < 4 ? 4 * lane : (lane < 8 ? 4 * (lane - 4) : 0);
        const uint32_t ga = (uint32_t)__shfl((int)pa, src, 64);
        const uint32_t gb = (uint32_t)__shfl((int)pb, src, 64);
        uint32_t word = lane < 4 ? ga : (lane < 8 ? gb : (lane == 8 ? __float_as_uint(sp) : __float_as_uint(xs)));
        if (*s_fail) word = lane < 8 ? 0u : 0x7fc00000u;  // routing timed out: NaN record
        if (lane < kRecWords) hand_put_group(a.hl + (size_t)g * 16 + lane, word, ep, a.local);
        S.mark(4, tid);
    }
}

// The block's activations as limb groups in LDS (la, lb [D / 4] words, lsp,
// lxs [D / 16]): thread t converts elements 8t + [0, 8) (half of group
// t / 2).  GEM: with a.gemma, the Gemma4 block's expert input (x * rms_inv)
// * pre_ffw_norm_2 (math.zig:51-82) is formed first.
template <int GEM>
__device__ __forceinline__ void stage_x_limbs(const FusedArgs &a, uint32_t *la, uint32_t *lb, float *lsp, float *lxs,
                                              int tid) {
    const bool gem = GEM && a.gemma;
    const float grms = gem ? gemma_rms_inv(a, tid) : 0.0f;  // (a.gemma is uniform: every thread or none)
    for (int t8 = tid; t8 < a.D / 8; t8 += kThreads) {  // one pass for D <= 2048
        const float *xsrc = a.x;
        const float4 f0 = *reinterpret_cast<const float4 *>(xsrc + 8 * t8);
        const float4 f1 = *reinterpret_cast<const float4 *>(xsrc + 8 * t8 + 4);
        float v[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
        if (gem) {
#pragma clang fp contract(off)
            const float4 w0 = *reinterpret_cast<const float4 *>(a.g_pre + 8 * t8);
            const float4 w1 = *reinterpret_cast<const float4 *>(a.g_pre + 8 * t8 + 4);
            const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = (v[i] * grms) * wv[i];
        }
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) m = fmaxf(m, fabsf(v[i]));
        m = fmaxf(m, dpp<0xB1>(m));  // the other half of the group (lane ^ 1)
        const float h8 = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
        const float xs = h8 + dpp<0xB1>(h8);
        const float inv = m > 0.0f ? 127.0f / m : 0.0f;
        float sp = m * (1.0f / 32512.0f);
        if (!(fabsf(xs) <= 3.0e38f) || !(m <= 3.0e38f)) sp = __int_as_float(0x7fc00000);
        uint32_t pa[2] = {0u, 0u}, pb[2] = {0u, 0u};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float t = v[i] * inv;
            const float fa = rintf(t);
            const float fb = fminf(rintf((t - fa) * 256.0f), 127.0f);
            pa[i >> 2] |= ((uint32_t)(int)fa & 0xffu) << (8 * (i & 3));
            pb[i >> 2] |= ((uint32_t)(int)fb & 0xffu) << (8 * (i & 3));
        }
        *reinterpret_cast<uint2 *>(la + 2 * t8) = make_uint2(pa[0], pa[1]);
        *reinterpret_cast<uint2 *>(lb + 2 * t8) = make_uint2(pb[0], pb[1]);
        if ((t8 & 1) == 0) {
            lsp[t8 >> 1] = sp;
            lxs[t8 >> 1] = xs;
        }
    }
}


// Block: slot s, h indices j0 = 16 jg + [0, 16), jg < G = Kd/16 (indices
// >= F are the zero padding of the down K); its record is line s*G + jg.
// Wavefront w: pairs j0 + 4w + [0, 4).  Lanes 0-31 take the gate row, lanes
// 32-63 the up row; lane & 31 = (super-block, sub-block pair) position, so
// a lane reads 32 bytes of quants per row and one header word (the quad's
// four words are shared over DPP).
// WIDE (rows of 9-16 super-blocks): lane position pos covers pos and pos
// + 32; the second position's weights are loaded as the first's products
// finish, its x limbs are read from LDS after them.
// GEM (the SH 2 instance): with a.gemma the activations are the Gemma4
// block's expert input (x * rms_inv) * pre_ffw_norm_2 (math.zig:51-82).
template <int PER, int WIDE, int GEM>
__device__ __forceinline__ void role_gate_up(const FusedArgs &a, uint8_t *smem, uint32_t *s_ids, uint32_t *s_ep,
                                             int *s_fail, int bid, int s, int jg, int tid, int wave, int lane,
                                             Stamps &S) {
    const int G = a.G;  // records per slot (down K / 16)
    const int g = s * G + jg;  // record line
    const int j0 = jg * 16;
    const int half = lane >> 5, pos = lane & 31, sb = pos >> 2, p = pos & 3;
    const bool lane_on = pos < 4 * a.nsb;
    const bool first = p32_first(lane);
    const uint32_t c0 = epoch_peek(a.counters, bid);
    // activation limbs, once per block: thread t converts elements 8t + [0, 8)
    // (half of group t / 2) into LDS; each lane then reads its window's 4
    // groups.  LDS: limb-a words [D/4], limb-b words [D/4], sp [D/16], xs [D/16].
    uint32_t *la = reinterpret_cast<uint32_t *>(smem + 64);
    uint32_t *lb = la + a.D / 4;
    float *lsp = reinterpret_cast<float *>(lb + a.D / 4);
    float *lxs = lsp + a.D / 16;
    stage_x_limbs<GEM>(a, la, lb, lsp, lxs, tid);
    if (tid == 0) *s_ep = epoch_commit(a.counters, bid, c0);
    __syncthreads();  // limbs (and s_ep)
    auto read_limbs = [&](Limbs &xl, int gi) {  // gi: first of the window's 4 groups
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const uint4 va = *reinterpret_cast<const uint4 *>(la + (gi + g) * 4);
            const uint4 vb = *reinterpret_cast<const uint4 *>(lb + (gi + g) * 4);
            xl.a[g][0] = va.x; xl.a[g][1] = va.y; xl.a[g][2] = va.z; xl.a[g][3] = va.w;
            xl.b[g][0] = vb.x; xl.b[g][1] = vb.y; xl.b[g][2] = vb.z; xl.b[g][3] = vb.w;
        }
        const float4 sp4 = *reinterpret_cast<const float4 *>(lsp + gi);
        const float4 xs4 = *reinterpret_cast<const float4 *>(lxs + gi);
        xl.sp[0] = sp4.x; xl.sp[1] = sp4.y; xl.sp[2] = sp4.z; xl.sp[3] = sp4.w;
        xl.xs_lo = xs4.x + xs4.y;
        xl.xs_hi = xs4.z + xs4.w;
    };
    Limbs xl;
    read_limbs(xl, lane_on ? sb * 16 + 4 * p : 0);
    const uint32_t ep = *s_ep;
    if (wave == 0) {  // only this slot's expert: s + 1 selection rounds, no softmax
        float lv[PER];
        const bool ok = poll_logits<PER>(a, ep, lv, lane);
        S.mark(1, tid);
        const int idx = topk_index_at<PER>(lv, a.E, s, lane);
        S.mark(2, tid);
        if (lane == 0) {
            s_ids[0] = (uint32_t)idx;
            if (!ok) *s_fail = 1;
        }
    }
    __syncthreads();  // s_ids[0], s_fail
    uint32_t e = s_ids[0];
    if (e >= (uint32_t)a.E) e = 0;
    const int jb = j0 + wave * 4;
    uint4 q0[4], q1[4];
    uint32_t hw[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        q0[r] = q1[r] = make_uint4(0u, 0u, 0u, 0u);
        hw[r] = 0u;
        if (lane_on && jb + r < a.F) {
            const size_t row = (size_t)e * 2 * a.F + (size_t)half * a.F + (jb + r);
            const size_t blk = row * a.nsb + sb;
            q0[r] = ld16(a.gu_qs + blk * 128 + 32 * p);
            q1[r] = ld16(a.gu_qs + blk * 128 + 32 * p + 16);
            hw[r] = *reinterpret_cast<const uint32_t *>(a.gu_hdr + blk * 16 + 4 * (lane & 3));
        }
    }
    // second position (WIDE): super-block sb + 8 (clamped to the first
    // when the row has none there: the products are then not added); its
    // loads reuse row r's registers once row r's first products are done
    const bool lane_on2 = WIDE && pos + 32 < 4 * a.nsb;
    const int sb2 = lane_on2 ? sb + 8 : sb;
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        uint32_t h0, h1, h2, h3;
        quad_header(hw[r], h0, h1, h2, h3);
        const PairScale ps = pair_scale(h0, h1, h2, h3, p);
        const uint32_t w8[8] = {q0[r].x, q0[r].y, q0[r].z, q0[r].w, q1[r].x, q1[r].y, q1[r].z, q1[r].w};
        v[r] = (lane_on && jb + r < a.F) ? q4k_pair_dot(w8, ps, xl) : 0.0f;
        if (WIDE) {
            const int jr = jb + r < a.F ? jb + r : a.F - 1;
            const size_t row = (size_t)e * 2 * a.F + (size_t)half * a.F + jr;
            const size_t blk = row * a.nsb + sb2;
            q0[r] = ld16(a.gu_qs + blk * 128 + 32 * p);
            q1[r] = ld16(a.gu_qs + blk * 128 + 32 * p + 16);
            hw[r] = *reinterpret_cast<const uint32_t *>(a.gu_hdr + blk * 16 + 4 * (lane & 3));
        }
    }
    if (WIDE) {
        read_limbs(xl, sb2 * 16 + 4 * p);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            uint32_t h0, h1, h2, h3;
            quad_header(hw[r], h0, h1, h2, h3);
            const PairScale ps = pair_scale(h0, h1, h2, h3, p);
            const uint32_t w8[8] = {q0[r].x, q0[r].y, q0[r].z, q0[r].w, q1[r].x, q1[r].y, q1[r].z, q1[r].w};
            const float d2 = q4k_pair_dot(w8, ps, xl);
            if (lane_on2 && jb + r < a.F) v[r] += d2;
        }
    }
    S.mark(3, tid);
    const float t = half_sum4(v, lane);
    const float u = xor32(t, first);  // the up total of the same pair
    float *s_h = reinterpret_cast<float *>(smem);
    if (lane < 32 && (lane & 7) == 0) {
        const int r = lane >> 3;
        s_h[wave * 4 + r] = (jb + r < a.F) ? act_apply((uint32_t)a.act, t) * u : 0.0f;
    }
    publish_h_record(a, reinterpret_cast<const float *>(smem), s_fail, g, ep, tid, wave, lane, S);
}

// Q3_K gate/up rows (the format instance): the block's 16 h rows j0 + r of
// slot s as 32 D / 128 tasks (row r, gate or up, super-block half hu: the
// 128 weights of qs[32 h ..] with all of hmask, the scales and d); a thread
// loads up to 4 tasks of one half up front (D <= 4096), then adds each
// task's four 32-element groups in order against the limbs (lt_fmt.h
// q3k_group_dot; the groups' limbs read once for its tasks) into part[task];
// thread 2r + gu sums row r's halves in order, and h = act(gate) * up goes
// out as the record (publish_h_record).  Rows past F give h = 0.
template <int PER, int GEM>
__device__ __forceinline__ void role_gate_up_q3k(const FusedArgs &a, uint8_t *smem, uint32_t *s_ids, uint32_t *s_ep,
                                                 int *s_fail, int bid, int s, int jg, int tid, int wave, int lane,
                                                 Stamps &S) {
    const int g = s * a.G + jg;  // record line
    const int j0 = jg * 16;
    const uint32_t c0 = epoch_peek(a.counters, bid);
    uint32_t *la = reinterpret_cast<uint32_t *>(smem + 64);
    uint32_t *lb = la + a.D / 4;
    float *lsp = reinterpret_cast<float *>(lb + a.D / 4);
    float *lxs = lsp + a.D / 16;
    float *part = lxs + a.D / 16;  // [32 D / 128]
    stage_x_limbs<GEM>(a, la, lb, lsp, lxs, tid);
    if (tid == 0) *s_ep = epoch_commit(a.counters, bid, c0);
    __syncthreads();  // limbs (and s_ep)
    const uint32_t ep = *s_ep;
    if (wave == 0) {  // only this slot's expert: s + 1 selection rounds, no softmax
        float lv[PER];
        const bool ok = poll_logits<PER>(a, ep, lv, lane);
        S.mark(1, tid);
        const int idx = topk_index_at<PER>(lv, a.E, s, lane);
        S.mark(2, tid);
        if (lane == 0) {
            s_ids[0] = (uint32_t)idx;
            if (!ok) *s_fail = 1;
        }
    }
    __syncthreads();  // s_ids[0], s_fail
    uint32_t e = s_ids[0];
    if (e >= (uint32_t)a.E) e = 0;
    // thread tid takes super-block half hu = tid % nh of the rows and
    // (row, gate / up) combinations cb = tid / nh + tph i (cb < 32): the
    // half's four limb groups are read from LDS once for all of them
    const int nh = a.D / 128, tph = kThreads / nh;
    const int hu = tid % nh, kb = tid / nh;
    DevTensor W{};
    W.p0 = a.gu_hdr;
    W.p1 = a.gu_qs;
    W.p2 = a.gu_p2;
    W.p3 = a.gu_p3;
    W.blocks_per_row = (size_t)a.nsb;
    // up to three tasks loaded at once (d_model <= 2816: every task); a
    // fourth (d_model >= 3072) after them
    auto task_w = [&](int cb) {
        cb = min(cb, 31);  // (clamped: every load unconditional)
        const int row = min(j0 + (cb >> 1), a.F - 1);
        return load_unit<LT_TYPE_Q3_K>(W, (size_t)e * 2 * a.F + (size_t)(cb & 1) * a.F + row, 4 * hu);
    };
    UnitW<LT_TYPE_Q3_K> w[3];
#pragma unroll
    for (int i = 0; i < 3; i++) w[i] = task_w(kb + tph * i);
    const LimbView xv{la, lb, lsp, lxs};
    if (kb < tph) {  // (threads past nh tph have no half)
        float acc[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const UnitX ux = load_ux(xv, 4 * hu + j);
#pragma unroll
            for (int i = 0; i < 3; i++)
                if (kb + tph * i < 32) acc[i] += dot_unit<LT_TYPE_Q3_K>(w[i], 4 * hu + j, ux);
        }
#pragma unroll
        for (int i = 0; i < 3; i++) {
            const int cb = kb + tph * i;
            if (cb < 32) part[(cb >> 1) * 2 * nh + (cb & 1) * nh + hu] = acc[i];
        }
        const int cb = kb + tph * 3;
        if (cb < 32) {
            const UnitW<LT_TYPE_Q3_K> w3 = task_w(cb);
            float a3 = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; j++) a3 += dot_unit<LT_TYPE_Q3_K>(w3, 4 * hu + j, load_ux(xv, 4 * hu + j));
            part[(cb >> 1) * 2 * nh + (cb & 1) * nh + hu] = a3;
        }
    }
    S.mark(3, tid);
    __syncthreads();  // part
    float *s_h = reinterpret_cast<float *>(smem);
    if (tid < 32) {
        const int r = tid >> 1;
        const float *pr = part + tid * nh;  // row r, gate (tid even) or up
        float sum = 0.0f;
        for (int hu = 0; hu < nh; hu++) sum += pr[hu];
        const float other = __shfl_xor(sum, 1, 64);
        if ((tid & 1) == 0) s_h[r] = (j0 + r < a.F) ? act_apply((uint32_t)a.act, sum) * other : 0.0f;
    }
    publish_h_record(a, s_h, s_fail, g, ep, tid, wave, lane, S);
}

// ---------------------------------------------------------------- Gemma4 tail
// One block (XCD group 0, after the down blocks) waits for every down
// block's completion word, then x = (x + rmsnorm(dense + rmsnorm(moe, w2),
// w)) * layer_output_scale (gemma4/forward.zig:482-497) over the D
// elements, with the tail kernel's tree order for both sums of squares
// (lt_norm.hip k_norm<kTail>, 1024 threads: thread t of the 1024 sums
// v[i]^2 for i = t, t + 1024, ... in order, a 64-lane xor butterfly per
// wavefront, then the 16 wavefront totals in order).  Thread t here plays
// threads t + 256 m of those (m < 4; their wavefronts are w + 4 m) and holds
// element t + 256 m' in register m' (m' < 16), so the element sums and the
// four butterflies run from registers; every thread then adds the 16 totals
// itself (one barrier per sum, red distinct per sum).  moe is read with
// agent-scope loads (the down blocks added into it with device atomics).  A
// wait that times out makes x NaN (error word 0x200).  (The last down block
// to finish running the tail instead, found with a counter of finished
// blocks, measured 1.7 us slower per block: the increments of one word
// queue, and the operands below are not loaded ahead.)
constexpr int kTailT = kFusedMaxD / kThreads;  // elements per thread
__device__ __forceinline__ float tail_sum_sq(const float (&v)[kTailT], int n, int tid, int wave, int lane,
                                             float *red) {
#pragma clang fp contract(off)
    float s[4];
#pragma unroll
    for (int m = 0; m < 4; m++) {
        s[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < kTailT / 4; j++)
            if (tid + kThreads * (m + 4 * j) < n) s[m] = s[m] + v[m + 4 * j] * v[m + 4 * j];
    }
    const bool first = p32_first(lane);
#pragma unroll
    for (int m = 0; m < 4; m++) s[m] = butterfly_sum64(s[m], first);
    if (lane == 0) {
#pragma unroll
        for (int m = 0; m < 4; m++) red[wave + 4 * m] = s[m];
    }
    __syncthreads();
    float t = red[0];
#pragma unroll
    for (int i = 1; i < 16; i++) t = t + red[i];
    return t;
}
__device__ __forceinline__ void role_gemma_tail(const FusedArgs &a, int bid, int tid, int wave, int lane,
                                                Stamps &S) {
#pragma clang fp contract(off)
    constexpr int kT = kTailT;
    __shared__ float red[32];
    __shared__ int t_fail;
    // the arguments in registers: the compiler would otherwise read them
    // again from the kernel arguments (a scalar load and its wait) after the
    // barriers and inside the branches below
    typedef __attribute__((address_space(1))) float gfloat;
    const int n = a.D, nd = a.k * a.NDg;
    float eps = a.g_eps, osc = a.g_out_scale;
    typedef __attribute__((address_space(1))) uint64_t gword;
    const gfloat *out = (const gfloat *)a.out;
    const gword *done = (const gword *)a.done;
    float *gx = a.g_x;
    asm volatile("" : "+s"(eps), "+s"(osc), "+s"(out), "+s"(done));  // (kept in registers)
    const uint32_t ep = epoch_peek(a.counters, bid) + 1u;
    // the operands that do not depend on the experts, loaded while the down
    // blocks work (indices clamped: every load unconditional)
    float dv[kT], w2v[kT], wv[kT], xv[kT];
#pragma unroll
    for (int m = 0; m < kT; m++) {
        const int i = min(tid + kThreads * m, n - 1);
        dv[m] = a.g_dense[i];
        w2v[m] = a.g_w2[i];
        wv[m] = a.g_w[i];
        xv[m] = gx[i];
    }
    if (tid == 0) t_fail = 0;
    __syncthreads();
    {
        const uint64_t t0 = wall_clock64();
        bool ok = true;
        for (int i = tid; i < nd && ok; i += kThreads) {
            while (!tag_is(__hip_atomic_load(done + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), ep)) {
                if (wall_clock64() - t0 > kWaitTicks) {
                    ok = false;
                    report_detail(a.err, bid, 0x200u, (uint32_t)i, 0, ep);
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
        }
        if (!ok) t_fail = 1;
    }
    __syncthreads();
    S.mark(1, tid);
    float v[kT];
#pragma unroll
    for (int m = 0; m < kT; m++)
        v[m] = __hip_atomic_load(out + min(tid + kThreads * m, n - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    float r = 1.0f / sqrtf(tail_sum_sq(v, n, tid, wave, lane, red) / (float)n + eps);
#pragma unroll
    for (int m = 0; m < kT; m++) v[m] = dv[m] + (v[m] * r) * w2v[m];  // dense + rmsnorm(moe, w2)
    r = 1.0f / sqrtf(tail_sum_sq(v, n, tid, wave, lane, red + 16) / (float)n + eps);
    const bool fail = t_fail != 0;
#pragma unroll
    for (int m = 0; m < kT; m++) {
        float y = xv[m] + (v[m] * r) * wv[m];
        if (osc != 1.0f) y = y * osc;
        v[m] = fail ? __int_as_float(0x7fc00000) : y;
        asm volatile("" : "+v"(v[m]));  // (computed here, not inside each store's branch)
    }
    // Agent-scope stores: written through, not left dirty in the L2 for the
    // end of the kernel to write back (0.3 us per block).  The lane's global
    // address is an opaque register value, which the compiler cannot re-derive
    // from the kernel arguments (a scalar load and a wait) before each store.
    gfloat *px = (gfloat *)(gx + tid);
    asm volatile("" : "+v"(px));
#pragma unroll
    for (int m = 0; m < kT; m++)
        if (tid + kThreads * m < n) __hip_atomic_store(px + kThreads * m, v[m], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid == 0 && fail) report_timeout(a.err, 0x200u);
    S.mark(2, tid);
}

// ---------------------------------------------------------------- down
// Sums V values per lane over each aligned group of 16 lanes, transposed:
// returns the group's total of value index (lane & 15) >> log2(16 / V).
template <int V>
__device__ __forceinline__ float group16_sum_transposed(const float (&v)[V], int lane) {
    float a[V];
#pragma unroll
    for (int i = 0; i < V; i++) a[i] = v[i];
    if (V >= 2) {  // lane bit 3: row_ror:8 pairs i with i ^ 8
        const bool hi = lane & 8;
#pragma unroll
        for (int i = 0; i < V / 2; i++) {
            const float send = hi ? a[i] : a[i + V / 2], keep = hi ? a[i + V / 2] : a[i];
            a[i] = keep + dpp<0x128>(send);
        }
    }
    if (V >= 4) {  // lane bit 2: row_half_mirror pairs i with 7 - i
        const bool hi = lane & 4;
#pragma unroll
        for (int i = 0; i < V / 4; i++) {
            const float send = hi ? a[i] : a[i + V / 4], keep = hi ? a[i + V / 4] : a[i];
            a[i] = keep + dpp<0x141>(send);
        }
    }
    if (V >= 8) {  // lane bit 1: quad_perm [2,3,0,1]
        const bool hi = lane & 2;
        const float send = hi ? a[0] : a[1], keep = hi ? a[1] : a[0];
        a[0] = keep + dpp<0x4E>(send);
    }
    float t = a[0];
    if (V < 8) t += dpp<0x4E>(t);
    if (V < 4) t += dpp<0x141>(t);
    if (V < 2) t += dpp<0x128>(t);
    t += dpp<0xB1>(t);
    return t;
}

// Block: output rows row0 + [0, kDownRows) for all k slots.  Threads form
// groups of 16: group q = tid >> 4 takes slot q % k and rows (q / k) * RPT +
// [0, RPT) (groups with q / k >= 8 / RPT idle); lane (tid & 15) = (super-
// block, sub-block pair) position.  Down weights are loaded and their
// scales decoded while the gate/up blocks run; once every gate/up block has
// counted itself done, the h records are read into LDS, each group sums its
// row partials over DPP, and the rows are combined over slots in slot order.
// Block: slot s, output rows row0 = 16 RPG j + [0, 16 RPG).  Thread groups
// of 16: group rg = tid >> 4 takes rows row0 + RPG rg + [0, RPG); lane l16 =
// tid & 15 = (super-block, sub-block pair) position.  Its down weights are
// loaded and their scales decoded while the gate/up blocks run; then the
// block reads the slot's G h records (same XCD), each group sums its row
// partials over DPP, and the rows, times the slot weight, are added into out
// (float atomics) or, with det (RPG = 4), wavefront w writes rows 16w +
// [0, 16) as one line of partial-output words.
// FILL: the block also adds the shared FFN's down rows 64 j + [0, 64) over
// its group's K slice: sh_stage_load when it starts, sh_stage_store during
// its logit poll, sh_read_h with its h records, sh_down_add after its own
// rows.
// DT: the down tensor's type (Q4_K, or IQ4_NL / Q5_0 / Q5_1: then lane l16
// of a row group takes 32-element blocks l16 and l16 + 16 of its rows, K <=
// 1024, each block's activations the two h records it spans).
template <int PER, int RPG, int FILL, int DT = LT_TYPE_Q4_K>
__device__ __forceinline__ void role_down(const FusedArgs &a, uint8_t *smem, uint32_t *s_ids, float *s_w,
                                          uint32_t *s_ep, int *s_fail, int bid, int s, int j, int tid, int wave,
                                          int lane, Stamps &S) {
    const int G = a.G;
    const int row0 = j * 16 * RPG;
    const int rg = tid >> 4, l16 = tid & 15;
    const int sb = l16 >> 2, p = l16 & 3;
    constexpr bool kQ4 = DT == LT_TYPE_Q4_K;
    const bool t_on = kQ4 ? sb < a.nsbd : true;
    uint32_t *rec_a = reinterpret_cast<uint32_t *>(smem);
    uint32_t *rec_b = rec_a + G * 4;
    float *rec_sp = reinterpret_cast<float *>(rec_b + G * 4);
    float *rec_xs = rec_sp + G;
    const bool fill = FILL == 1 && a.S > 0 && s < 8;
    __shared__ int sh_fail;
    ShStage sst;
    if (fill) sh_stage_load(a, sst, bid & 7, j, tid);
    if (fill && tid == 0) sh_fail = 0;
    if (tid == 0) *s_ep = epoch_commit(a.counters, bid, epoch_peek(a.counters, bid));
    __syncthreads();
    const uint32_t ep = *s_ep;
    // The gate/up weights are needed first: the down weight loads wait until
    // dn_delay ticks after the logits are seen, when most of the gate/up
    // stream has arrived, so that its tail is not shared with them (the
    // down weights then land shortly before the h records).
    __shared__ uint64_t s_seen;
    if (wave == 0) {
        float lv[PER];
        const bool ok = poll_logits<PER>(a, ep, lv, lane);
        if (lane == 0) s_seen = wall_clock64();
        S.mark(1, tid);
        uint32_t key[PER];
        int my_i;
        float my_p;
        topk_softmax_regs<PER>(lv, a.E, a.k, a.norm, s_ids, s_w, key, my_i, my_p, lane);
        if (!ok && lane == 0) *s_fail = 1;
    } else if (fill) {
        sh_stage_store(a, smem, sst, bid & 7, tid);
    }
    __syncthreads();
    uint32_t e = s_ids[s];
    if (e >= (uint32_t)a.E) e = 0;
    {
        const uint64_t t_go = s_seen + (uint64_t)a.dn_delay;
        while (wall_clock64() < t_go) __builtin_amdgcn_s_sleep(4);
    }
    S.mark(2, tid);
    uint4 q0[RPG], q1[RPG];
    uint32_t hw[RPG];
    UnitW<DT> fw[kQ4 ? 1 : RPG][2];  // (block formats: blocks l16, l16 + 16 of each row)
    DevTensor fW{};
    fW.p0 = a.dn_hdr;
    fW.p1 = a.dn_qs;
    fW.p2 = a.dn_p2;
    fW.blocks_per_row = (size_t)a.nsbd;
#pragma unroll
    for (int i = 0; i < RPG; i++) {
        const int row = row0 + rg * RPG + i;
        if constexpr (kQ4) {
            q0[i] = q1[i] = make_uint4(0u, 0u, 0u, 0u);
            hw[i] = 0u;
            if (t_on && row < a.D) {
                const size_t blk = ((size_t)e * a.D + row) * a.nsbd + sb;
                q0[i] = ld16(a.dn_qs + blk * 128 + 32 * p);
                q1[i] = ld16(a.dn_qs + blk * 128 + 32 * p + 16);
                hw[i] = *reinterpret_cast<const uint32_t *>(a.dn_hdr + blk * 16 + 4 * p);
            }
        } else {
#pragma unroll
            for (int m = 0; m < 2; m++) {
                const int u = l16 + 16 * m;
                // (clamped: every load unconditional; a block past the row's
                // end or a row past D is loaded but not added)
                fw[i][m] = load_unit<DT>(fW, (size_t)e * a.D + min(row, a.D - 1), min(u, a.nsbd - 1));
            }
        }
    }
    // the shared FFN's rows while these weights are in flight: its slice of
    // h (written long before; the reads return once this CU's earlier loads
    // have), summed into LDS
    if (fill) {
        if (!sh_read_h(a, smem, ep, bid & 7, bid, tid)) sh_fail = 1;
        __syncthreads();
        sh_down_rows(a, smem, bid & 7, j, tid, wave, lane);
        S.mark(5, tid);
    }
    // scales decoded, and the nibbles of rows 0-1 unpacked, while the h
    // records are awaited (the dots after their arrival are VALU-bound; all
    // four rows unpacked would exceed 128 VGPRs); the empty asm keeps the
    // compiler from sinking the unpacking to its use
    // (block formats: each block's codes formed now, the table lookups or
    // high bits off the path after the records)
    BlockCodes bc[kQ4 ? 1 : RPG][2];
    if constexpr (!kQ4) {
#pragma unroll
        for (int i = 0; i < RPG; i++)
#pragma unroll
            for (int m = 0; m < 2; m++) {
                bc[i][m] = block_codes<DT>(fw[i][m]);
#pragma unroll
                for (int q = 0; q < 8; q++) asm volatile("" : "+v"(bc[i][m].c[q]));
            }
    }
    PairScale ps[RPG];
    uint32_t nlo[2][8], nhi[2][8];
#pragma unroll
    for (int i = 0; i < (kQ4 ? RPG : 0); i++) {
        uint32_t h0, h1, h2, h3;
        quad_header(hw[i], h0, h1, h2, h3);
        ps[i] = pair_scale(h0, h1, h2, h3, p);
        if (i >= 2) continue;
        const uint32_t w8[8] = {q0[i].x, q0[i].y, q0[i].z, q0[i].w, q1[i].x, q1[i].y, q1[i].z, q1[i].w};
#pragma unroll
        for (int m = 0; m < 8; m++) {
            nlo[i][m] = w8[m] & 0x0f0f0f0fu;
            nhi[i][m] = (w8[m] >> 4) & 0x0f0f0f0fu;
            asm volatile("" : "+v"(nlo[i][m]), "+v"(nhi[i][m]));
        }
    }
    // the slot's h records: thread 0 waits for one record line, then thread
    // q*10 + wl (q < 25) reads word wl of lines q + 25 m, all loads of a
    // pass in flight at once
    if (tid == 0 && !a.det && starts_stored_by_router(a) && !probe_wait(start_flag(a, bid & 7, row0), ep, wall_clock64()))
        *s_fail = 1;  // (reported as the logit wait: the start values come with the routing)
    if (tid == 0 && !probe_wait(a.hl + ((size_t)s * G + (size_t)(j % G)) * 16, ep, wall_clock64())) *s_fail = 2;
    __syncthreads();
    bool ok = true;
    {
        const int qq = tid / kRecWords, wl = tid - qq * kRecWords;
        const bool on = tid < 25 * kRecWords;
        const uint64_t *src = a.hl + (size_t)s * G * 16;
        const uint64_t t0 = wall_clock64();
        for (int L0 = qq; L0 < G; L0 += 25 * 4) {
            while (true) {
                uint64_t w[4];
#pragma unroll
                for (int m = 0; m < 4; m++) {
                    const int L = L0 + 25 * m;
                    w[m] = (on && L < G) ? hand_get(src + (size_t)L * 16 + wl) : ((uint64_t)ep << 32);
                }
                bool good = true;
#pragma unroll
                for (int m = 0; m < 4; m++) good = good && tag_is(w[m], ep);
                if (__all(good)) {
#pragma unroll
                    for (int m = 0; m < 4; m++) {
                        const int L = L0 + 25 * m;
                        if (on && L < G) {
                            const uint32_t val = (uint32_t)w[m];
                            if (wl < 4) rec_a[L * 4 + wl] = val;
                            else if (wl < 8) rec_b[L * 4 + wl - 4] = val;
                            else if (wl == 8) rec_sp[L] = __uint_as_float(val);
                            else rec_xs[L] = __uint_as_float(val);
                        }
                    }
                    break;
                }
                if (wall_clock64() - t0 > kWaitTicks) {
                    ok = false;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            if (!ok) break;
        }
    }
    if (!ok) atomicOr(s_fail, 2);
    __syncthreads();  // records, s_ids / s_w
    S.mark(3, tid);
    if (s == 0 && j == 0 && tid < a.k) {  // the routing, for the caller
        a.ids_out[tid] = s_ids[tid];
        a.w_out[tid] = s_w[tid];
    }
    const float ws = FILL == 2 && a.gemma && a.g_dscale ? a.g_dscale[e] * s_w[s] : s_w[s];  // (down_exps_scale[e] * p_e, gemma4/forward.zig:477)
    float v[RPG];
#pragma unroll
    for (int i = 0; i < RPG; i++) v[i] = 0.0f;
    if constexpr (!kQ4) {
#pragma unroll
        for (int m = 0; m < 2; m++) {
            const int u = l16 + 16 * m;
            if (u < a.nsbd) {
                // block u's activations: records 2u (elements 0-15) and 2u + 1
                UnitX ux;
                const uint4 *pa = reinterpret_cast<const uint4 *>(rec_a + 8 * u);
                const uint4 *pb = reinterpret_cast<const uint4 *>(rec_b + 8 * u);
#pragma unroll
                for (int g = 0; g < 2; g++) {
                    const uint4 qa = pa[g], qb = pb[g];
                    ux.a[4 * g] = qa.x; ux.a[4 * g + 1] = qa.y; ux.a[4 * g + 2] = qa.z; ux.a[4 * g + 3] = qa.w;
                    ux.b[4 * g] = qb.x; ux.b[4 * g + 1] = qb.y; ux.b[4 * g + 2] = qb.z; ux.b[4 * g + 3] = qb.w;
                }
                ux.sp[0] = rec_sp[2 * u];
                ux.sp[1] = rec_sp[2 * u + 1];
                ux.xs[0] = rec_xs[2 * u];
                ux.xs[1] = rec_xs[2 * u + 1];
#pragma unroll
                for (int i = 0; i < RPG; i++) v[i] += block_codes_dot<DT>(bc[i][m], ux);
            }
        }
    }
    if (kQ4 && t_on) {
        const int gi = sb * 16 + 4 * p;  // first of the window's 4 groups
        Limbs xl;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const uint4 va = *reinterpret_cast<const uint4 *>(rec_a + (gi + g) * 4);
            const uint4 vb = *reinterpret_cast<const uint4 *>(rec_b + (gi + g) * 4);
            xl.a[g][0] = va.x; xl.a[g][1] = va.y; xl.a[g][2] = va.z; xl.a[g][3] = va.w;
            xl.b[g][0] = vb.x; xl.b[g][1] = vb.y; xl.b[g][2] = vb.z; xl.b[g][3] = vb.w;
        }
        const float4 sp4 = *reinterpret_cast<const float4 *>(rec_sp + gi);
        const float4 xs4 = *reinterpret_cast<const float4 *>(rec_xs + gi);
        xl.sp[0] = sp4.x; xl.sp[1] = sp4.y; xl.sp[2] = sp4.z; xl.sp[3] = sp4.w;
        xl.xs_lo = xs4.x + xs4.y;
        xl.xs_hi = xs4.z + xs4.w;
#pragma unroll
        for (int i = 0; i < (kQ4 ? RPG : 0); i++) {
            if (i < 2) {
                v[i] = q4k_pair_dot_nib(nlo[i], nhi[i], ps[i], xl);
            } else {
                const uint32_t w8[8] = {q0[i].x, q0[i].y, q0[i].z, q0[i].w, q1[i].x, q1[i].y, q1[i].z, q1[i].w};
                v[i] = q4k_pair_dot(w8, ps[i], xl);
            }
        }
    }
    // row rg*RPG + l16 / (16 / RPG) in lanes l16 = 0, 16 / RPG, ... of each
    // group; with RPG = 4 the wave's 4 groups cover rows 16 wave + [0, 16) =
    // one partial line
    const float t = group16_sum_transposed<RPG>(v, lane);
    if ((l16 & (16 / RPG - 1)) == 0) {
        const int rr = rg * RPG + l16 / (16 / RPG);  // row within the block
        const float val = *s_fail ? __int_as_float(0x7fc00000) : ws * t;
        if (a.det)
            hand_put(a.pl + ((size_t)(s * a.NDg + j) * 4 + (rr >> 4)) * 16 + (rr & 15), __float_as_uint(val), ep);
        else if (row0 + rr < a.D)
            (void)__hip_atomic_fetch_add(a.out + row0 + rr, val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    S.mark(4, tid);
    // (the start values of these rows were awaited with the h records; the
    // row sums are behind the barrier after the records)
    if (fill) sh_down_add(a, smem, bid & 7, j, sh_fail != 0 || *s_fail != 0, tid, S);
    if (FILL == 2 && a.gemma) {  // the Gemma4 block's tail waits for every down block's adds
        __builtin_amdgcn_s_waitcnt(0);  // this thread's adds acknowledged
        __syncthreads();
        if (tid == 0) hand_put(a.done + (size_t)s * a.NDg + j, 1u, ep);
    }
}

// ---------------------------------------------------------------- combine
// Rows 8c + [0, 8): out = base + (prev + sum over slots in slot order of the
// weighted slot rows), the combine of moeForward (ops/moe.zig:67-76).  Lane
// r < 8 reads row 8c + r of every slot (one word of a partial line each).
__device__ __forceinline__ void role_combine(const FusedArgs &a, uint32_t *s_ep, int bid, int c, int tid,
                                             Stamps &S) {
    if (tid == 0) *s_ep = epoch_commit(a.counters, bid, epoch_peek(a.counters, bid));
    if (!a.det) return;  // the down blocks added into out themselves
    __syncthreads();
    if (tid >= kCombRows) return;
    const uint32_t ep = *s_ep;
    const int row = c * kCombRows + tid;
    if (row >= a.D) return;
    const int j = row / kDownRows, rr = row % kDownRows;
    float v[16];
    bool ok = false;
    const uint64_t t0 = wall_clock64();
    if (tid == 0) (void)probe_wait(a.pl + ((size_t)j * 4 + (rr >> 4)) * 16 + (rr & 15), ep, t0);
    while (true) {
        uint64_t w[16];
#pragma unroll
        for (int s = 0; s < 16; s++)
            w[s] = s < a.k ? hand_get(a.pl + ((size_t)(s * a.NDg + j) * 4 + (rr >> 4)) * 16 + (rr & 15))
                           : ((uint64_t)ep << 32);
        bool good = true;
#pragma unroll
        for (int s = 0; s < 16; s++) {
            good = good && tag_is(w[s], ep);
            v[s] = __uint_as_float((uint32_t)w[s]);
        }
        if (good) {
            ok = true;
            break;
        }
        if (wall_clock64() - t0 > kWaitTicks) break;
        __builtin_amdgcn_s_sleep(1);
    }
    float acc = a.accumulate ? a.out[row] : 0.0f;
#pragma unroll
    for (int s = 0; s < 16; s++)
        if (s < a.k) acc = acc + v[s];
    if (a.base) acc = a.base[row] + acc;
    if (!ok) {
        acc = __int_as_float(0x7fc00000);
        report_timeout(a.err, 8u);
    }
    a.out[row] = acc;
    S.mark(1, tid);
}

// SH 1: the Gemma-style instance (Q8_0 router role, shared-FFN roles); SH
// 2: the Gemma4 block (Q8_0 router with the block's input norms, expert
// input norm and scales, the tail role; no shared FFN); SH 3: SH 2's roles
// plus the APEX expert formats (Q3_K gate/up, IQ4_NL / Q5_0 / Q5_1 down),
// with or without the Gemma4 block; SH 0 holds only the
// F32 router roles and the experts' roles, and WIDE (rows over 2048) only
// the router variants those rows use: less code per instance (the roles of
// a CU's four workgroups share its instruction cache; the Gemma4 code in the
// SH 1 instance made config 4 0.7 us slower).
template <int PER, int WIDE, int SH>
// (SH 1, 2: at most 128 VGPRs, four blocks per SIMD, for the whole grid to be
// resident; the others fit without the bound, which costs config 3 0.07 us)
__global__ void __launch_bounds__(kThreads, SH ? 4 : 1) k_moe_fused(FusedArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ uint32_t s_ep;
    __shared__ uint32_t s_ids[16];
    __shared__ float s_w[16];
    __shared__ int s_fail;
    const int bid = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int x = bid & 7, i = bid >> 3;
    Stamps S;
    S.wt = SH;
    S.on = a.stamps != nullptr;
    S.row = a.stamps ? a.stamps + (size_t)bid * kStamps : nullptr;
    if (SH) {
        if (S.row && tid == 0)
            for (int q = 1; q < kStamps; q++) S.row[q] = 0;
    } else {
#pragma unroll
        for (int q = 0; q < kStamps; q++) S.t[q] = 0;
    }
    S.mark(kStampStart, tid);
    uint32_t role = 0;
    if (tid == 0) s_fail = 0;
    // in-group order: router, shared gate/up, gate/up, down, combine --
    // every role waits only for earlier ones.  (Computing a role code first
    // and dispatching on it, or reading it from a table in the kernel
    // arguments, made config 3 0.07-0.45 us slower.)
    int u = i;
    if (u < a.NRg) {
        if (SH && a.qrouter)
            role_router_q8<SH >= 2>(a, smem, bid, tid, lane, S);
        else if (!WIDE && a.rb == 2)
            role_router_pair_one(a, smem, bid, tid, wave, lane, S);
        else if (WIDE)
            role_router_pair(a, smem, bid, tid, wave, lane, S);
        else
            role_router(a, smem, bid, tid, wave, lane, S);
        role = 1;
    } else if ((u -= a.NRg) < a.NSg) {
        if (SH == 1) role_shared_gate_up(a, smem, x, u, bid, tid, wave, lane, S);
        role = 5;
    } else if ((u -= a.NSg) < a.SPG * a.G) {
        const int s = x + 8 * (u / a.G);
        if (s < a.k) {
            if (SH == 3 && a.gu_type == LT_TYPE_Q3_K)
                role_gate_up_q3k<PER, 1>(a, smem, s_ids, &s_ep, &s_fail, bid, s, u % a.G, tid, wave, lane, S);
            else
                role_gate_up<PER, WIDE, SH >= 2>(a, smem, s_ids, &s_ep, &s_fail, bid, s, u % a.G, tid, wave, lane, S);
            if (tid == 0 && s_fail) report_timeout(a.err, 1u);  // logits
            role = 2u | (uint32_t)s << 8;
        }
    } else if ((u -= a.SPG * a.G) < a.SPG * a.NDg) {
        const int s = x + 8 * (u / a.NDg);
        if (s < a.k) {
            if (SH == 3 && a.dn_type == LT_TYPE_IQ4_NL)
                role_down<PER, 4, 2, LT_TYPE_IQ4_NL>(a, smem, s_ids, s_w, &s_ep, &s_fail, bid, s, u % a.NDg, tid, wave,
                                                      lane, S);
            else if (SH == 3 && a.dn_type == LT_TYPE_Q5_0)
                role_down<PER, 4, 2, LT_TYPE_Q5_0>(a, smem, s_ids, s_w, &s_ep, &s_fail, bid, s, u % a.NDg, tid, wave,
                                                    lane, S);
            else if (SH == 3 && a.dn_type == LT_TYPE_Q5_1)
                role_down<PER, 4, 2, LT_TYPE_Q5_1>(a, smem, s_ids, s_w, &s_ep, &s_fail, bid, s, u % a.NDg, tid, wave,
                                                    lane, S);
            else
                role_down<PER, 4, SH == 3 ? 2 : SH>(a, smem, s_ids, s_w, &s_ep, &s_fail, bid, s, u % a.NDg, tid, wave,
                                                    lane, S);
            if (tid == 0 && s_fail) report_timeout(a.err, (uint32_t)s_fail << 1);  // 2 logits, 4 h records
            role = 3u | (uint32_t)s << 8;
        } else if (SH == 1 && a.S > 0 && u < a.NDg) {  // a group without a slot still adds its shared rows
            const uint32_t ep = epoch_peek(a.counters, bid) + 1u;
            ShStage sst;
            sh_stage_load(a, sst, x, u, tid);
            sh_stage_store(a, smem, sst, x, tid);
            if (tid == 0 && starts_stored_by_router(a) && !probe_wait(start_flag(a, x, u * kDownRows), ep, wall_clock64()))
                s_fail = 1;
            if (!sh_read_h(a, smem, ep, x, bid, tid)) s_fail = 1;
            __syncthreads();
            sh_down_rows(a, smem, x, u, tid, wave, lane);
            __syncthreads();
            sh_down_add(a, smem, x, u, s_fail != 0, tid, S);
            role = 6;
        }
    } else if ((u -= a.SPG * a.NDg) < a.NCg) {
        role_combine(a, &s_ep, bid, 8 * u + x, tid, S);
        role = 4;
    } else if (SH >= 2 && a.gemma && x == 0 && u == a.NCg) {  // the Gemma4 block's tail
        role_gemma_tail(a, bid, tid, wave, lane, S);
        role = 7;
    }
    // no role in this configuration, or a shared-FFN role: keep the counter in step
    // (roles 5-7 carry no slot bits; 2 and 3 do, and commit in their role)
    if ((role == 0 || (role >= 5 && role <= 7)) && tid == 0)
        (void)epoch_commit(a.counters, bid, epoch_peek(a.counters, bid));
    if (S.row && tid == 0) {
        uint32_t xcc, hw;  // the XCD and the CU this block ran on
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
        const uint64_t w = role | (uint64_t)(xcc & 0xfu) << 16 | (uint64_t)hw << 32;
        if (SH) {
            S.row[kStamps - 1] = w;
        } else {
            S.t[kStamps - 1] = w;
#pragma unroll
            for (int q = 0; q < kStamps; q++) S.row[q] = S.t[q];
        }
    }
}

// Block b records the XCD it runs on (hardware register XCC_ID).
__global__ void k_xcc_probe(uint32_t *ids) {
    if (threadIdx.x != 0) return;
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    ids[blockIdx.x] = v & 0xfu;
}

}  // namespace

hipError_t probe_xcd_groups(uint32_t *dev_ids, hipStream_t s, int *local) {
    *local = 0;
    hipLaunchKernelGGL(k_xcc_probe, dim3(kFusedBlocks), dim3(64), 0, s, dev_ids);
    hipError_t e = hipGetLastError();
    uint32_t ids[kFusedBlocks];
    if (e == hipSuccess) e = hipMemcpyAsync(ids, dev_ids, sizeof(ids), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return e;
    int same = 1;
    for (int b = 8; b < kFusedBlocks; b++) same &= ids[b] == ids[b & 7];
    *local = same;
    return hipSuccess;
}

FusedPlan plan_moe_fused(const FusedLayer &L) {
    FusedPlan pl{};
    pl.ok = false;
    const bool moe = L.k > 0, sh = L.SG != nullptr;
    const int D = L.D;
    if (!moe && !sh) return pl;
    if (D < 256 || D > 4096 || D % (moe ? 256 : 32) != 0) return pl;
    int used = 0;
    if (moe) {
        const int E = L.E, k = L.k, Kd = L.Kd;
        if (!L.R || !L.GU || !L.Dn) return pl;
        const uint32_t gt = L.GU->type, dt = L.Dn->type;
        const bool dq4 = dt == LT_TYPE_Q4_K;
        if (gt != LT_TYPE_Q4_K && gt != LT_TYPE_Q3_K) return pl;
        if (!dq4 && dt != LT_TYPE_IQ4_NL && dt != LT_TYPE_Q5_0 && dt != LT_TYPE_Q5_1) return pl;
        pl.fmt = gt != LT_TYPE_Q4_K || !dq4;
        if (pl.fmt && (sh || L.det)) return pl;  // (the format instance: no shared FFN, atomic combine)
        // 16 lanes per down row: 4 super-blocks x 4 pairs (Q4_K), or 2 x 16
        // blocks of 32 (the block formats)
        if (Kd % (dq4 ? 256 : 32) != 0 || Kd < L.F || Kd > 1024) return pl;
        if (E < 1 || E > 256 || k > 16 || k > E) return pl;
        pl.per = E <= 128 ? 2 : 4;
        pl.wide = D > 2048;
        pl.qrouter = L.R->type == 8u;  // GGML Q8_0 (else F32)
        pl.SPG = (k + 7) / 8;
        pl.G = Kd / 16;
        pl.NDg = (D + kDownRows - 1) / kDownRows;
        if (sh && L.det) return pl;  // the shared FFN's rows join the atomic combine only
        pl.NCg = L.det ? pl.NDg : 0;
        // two logit rows per router block where the grid has room, else four
        // router blocks: the logit rows, and at least one per 256 output rows
        // (store_starts)
        const int nstart = (D + kThreads - 1) / kThreads;
        pl.rb = 2;
        pl.NRg = std::max((E + 15) / 16, (nstart + 7) / 8);
        used = pl.NRg + pl.SPG * pl.G + pl.SPG * pl.NDg + pl.NCg;
        // (the four-row F32 router reads rows of at most 2048)
        if (8 * used > kFusedBlocks && !pl.qrouter && D <= 2048) {
            pl.rb = 4;
            pl.NRg = std::max((E + 31) / 32, (nstart + 7) / 8);
            used = pl.NRg + pl.SPG * pl.G + pl.SPG * pl.NDg + pl.NCg;
        }
        pl.Ewait = E;  // (the start values have flags of their own: flag_starts)
        if (pl.Ewait > 64 * pl.per) return pl;
        if (8 * used > kFusedBlocks) return pl;
        if ((size_t)k * pl.G > (size_t)kFusedBlocks) return pl;            // h record lines
        if ((size_t)k * pl.NDg * 4 > (size_t)kFusedBlocks * 4) return pl;  // partial lines
    } else {
        pl.per = 2;
        pl.rb = 2;
    }
    if (L.gb) {  // the Gemma4 block around the layer: one tail block more in XCD group 0
        if (!moe || sh || L.det || !pl.qrouter || used + 1 > kFusedBlocks / 8) return pl;
        pl.gemma = 1;
    }
    if (sh) {
        // the shared FFN's gate/up rows in blocks of their own (the group's
        // blocks the experts leave free, at most 32 h rows each), its down
        // rows in the experts' down blocks (64 each: NDg * 64 >= D); a dense
        // FFN alone is not in the single launch
        const int S = L.S;
        if (!moe || !L.SU || !L.SD || S % 32 != 0 || S < 256 || S > 4096 || D > kShMaxD) return pl;
        const int slice = 32 * ((S / 32 + 7) / 8);  // h rows of the largest group slice
        const int spare = kFusedBlocks / 8 - used;
        if (spare < 1 || (slice + spare - 1) / spare > 32) return pl;
        pl.NSg = spare;
        pl.sg_rows = (slice + spare - 1) / spare;
        pl.shared = 1;
    }
    size_t lds = 64;
    if (moe) {
        const size_t lds_router = pl.qrouter ? (size_t)2 * 128 * 4 : (size_t)(4 * 512 + 16) * 4;
        const size_t lds_down = (size_t)pl.G * 40;
        size_t lds_gu = 64 + (size_t)D / 4 * 4 * 2 + (size_t)D / 16 * 4 * 2;
        if (L.GU->type == LT_TYPE_Q3_K) lds_gu += (size_t)D;  // the tasks' partial sums
        lds = std::max(lds, std::max(lds_router, std::max(lds_down, lds_gu)));
    }
    if (sh) lds = std::max(lds, std::max((size_t)D * 4, sh_down_lds(L.S)));  // x; shared down weights + h slice
    if (pl.gemma) lds = std::max(lds, (size_t)2 * 128 * 4 + (size_t)D * 4);  // router terms + the prepared x
    if (lds > 40 * 1024) return pl;  // four blocks per CU (160 KB of LDS): the whole grid resident
    pl.lds = lds;
    pl.ok = true;
    return pl;
}

template <int PER, int WIDE, int SH>
static hipError_t launch_fused_t(const FusedArgs &fa, const FusedPlan &pl, hipStream_t s) {
    hipLaunchKernelGGL((k_moe_fused<PER, WIDE, SH>), dim3(kFusedBlocks), dim3(kThreads), pl.lds, s, fa);
    return hipGetLastError();
}

hipError_t launch_moe_fused(const FusedPlan &pl, const FusedLayer &L, const float *bias, const float *x,
                            uint32_t act, uint32_t norm, const float *base, int accumulate, int deterministic,
                            float *out, uint32_t *ids_out, float *w_out, const FusedScratch &sc, hipStream_t s) {
    FusedArgs fa{};
    const bool moe = L.k > 0;
    if (moe) {
        fa.router = reinterpret_cast<const float *>(L.R->p0);
        fa.rq = L.R->p0;
        fa.rd = reinterpret_cast<const uint16_t *>(L.R->p1);
        fa.gu_hdr = L.GU->p0;
        fa.gu_qs = L.GU->p1;
        fa.dn_hdr = L.Dn->p0;
        fa.dn_qs = L.Dn->p1;
        fa.nsb = (int)L.GU->blocks_per_row;
        fa.nsbd = (int)L.Dn->blocks_per_row;
        fa.gu_type = (int)L.GU->type;
        fa.dn_type = (int)L.Dn->type;
        fa.gu_p2 = L.GU->p2;
        fa.gu_p3 = L.GU->p3;
        fa.dn_p2 = L.Dn->p2;
    }
    if (L.SG) {
        fa.sgq = L.SG->p0;
        fa.sgd = reinterpret_cast<const uint16_t *>(L.SG->p1);
        fa.suq = L.SU->p0;
        fa.sud = reinterpret_cast<const uint16_t *>(L.SU->p1);
        fa.sdq = L.SD->p0;
        fa.sdd = reinterpret_cast<const uint16_t *>(L.SD->p1);
    }
    fa.bias = bias;
    fa.x = x;
    fa.base = base;
    fa.out = out;
    fa.ids_out = ids_out;
    fa.w_out = w_out;
    fa.counters = sc.counters;
    fa.lg = sc.lg;
    fa.hl = sc.hl;
    fa.pl = sc.pl;
    fa.err = sc.err;
    fa.stamps = sc.stamps;
    fa.shh = sc.shh;
    fa.qrouter = pl.qrouter;
    fa.S = pl.shared ? L.S : 0;
    fa.NSg = pl.shared ? pl.NSg : 0;
    if (pl.gemma) {
        const GemmaBlock &g = *L.gb;
        fa.gemma = 1;
        fa.g_raw_scale = g.raw_scale;
        fa.g_pre = g.pre_ffw_norm_2;
        fa.g_dscale = g.down_exps_scale;
        fa.g_dense = g.dense;
        fa.g_w2 = g.post_ffw_norm_2;
        fa.g_w = g.post_ffw_norm;
        fa.g_x = g.x;
        fa.g_raw_global = g.raw_global_scale;
        fa.g_eps = g.eps;
        fa.g_out_scale = g.layer_output_scale;
        fa.done = sc.pl;  // (the partial lines: unused without the slot-order combine)
    }
    fa.sg_rows = pl.sg_rows;
    fa.E = moe ? L.E : 0;
    fa.D = L.D;
    fa.F = L.F;
    fa.k = L.k;
    fa.norm = (int)norm;
    fa.act = (int)act;
    fa.accumulate = accumulate;
    fa.det = deterministic;
    fa.local = sc.xcd_local;
    // Down weight loads start 0.7 us (the gate/up blocks' top-k) plus the
    // time 80% of the gate/up weights take at 5 TB/s (the burst rate
    // measured for this stream) after the logits are seen, in 10 ns ticks;
    // tuned on config 3 (14.2 MB: 296 ticks; 200 or 360 are 0.2-0.4 us
    // slower per layer; re-measured on the current kernel, 60% and 100% of
    // the stream instead of 80%: +0.17 and +0.36 us).  With the shared FFN
    // in the launch (its streams run before the experts') 55% is best: on
    // config 4 (17.8 MB) 50-60% measured 0.1-0.2 us faster than 80%, 40%
    // and 100% slower (the Gemma4 block and the APEX instance, whose
    // launches hold no shared FFN, were 0.15 us slower at 55%).
    const double gu_bytes = moe ? (double)L.k * 2.0 * L.F * ((double)L.GU->bytes / (double)L.GU->total_rows) : 0.0;
    fa.dn_delay = 70 + (int)((pl.shared ? 0.55 : 0.8) * gu_bytes / 50000.0);
    fa.NRg = pl.NRg;
    fa.rb = pl.rb;
    fa.SPG = pl.SPG;
    fa.G = pl.G;
    fa.NDg = pl.NDg;
    fa.NCg = pl.NCg;
    fa.Ewait = pl.Ewait;
    // 64 down rows per block (RPG 4): 32-row blocks using the combining
    // blocks' share of the grid (atomic combine) measured 0.15 us slower per
    // layer -- more h record reads and atomics -- though each block's
    // products halve; measured again with both rows' nibbles unpacked before
    // the h records arrive: 12.13 against 11.68 us (the 120 busy blocks per
    // group are dispatched up to 1 us after the first, against 0.3 with 88)
    const int mode = pl.fmt ? 3 : pl.gemma ? 2 : (pl.shared || pl.qrouter) ? 1 : 0;
    if (pl.wide) {
        if (mode == 3) return pl.per == 2 ? launch_fused_t<2, 1, 3>(fa, pl, s) : launch_fused_t<4, 1, 3>(fa, pl, s);
        if (mode == 2) return pl.per == 2 ? launch_fused_t<2, 1, 2>(fa, pl, s) : launch_fused_t<4, 1, 2>(fa, pl, s);
        if (mode == 1) return pl.per == 2 ? launch_fused_t<2, 1, 1>(fa, pl, s) : launch_fused_t<4, 1, 1>(fa, pl, s);
        return pl.per == 2 ? launch_fused_t<2, 1, 0>(fa, pl, s) : launch_fused_t<4, 1, 0>(fa, pl, s);
    }
    if (mode == 3) return pl.per == 2 ? launch_fused_t<2, 0, 3>(fa, pl, s) : launch_fused_t<4, 0, 3>(fa, pl, s);
    if (mode == 2) return pl.per == 2 ? launch_fused_t<2, 0, 2>(fa, pl, s) : launch_fused_t<4, 0, 2>(fa, pl, s);
    if (mode == 1) return pl.per == 2 ? launch_fused_t<2, 0, 1>(fa, pl, s) : launch_fused_t<4, 0, 1>(fa, pl, s);
    return pl.per == 2 ? launch_fused_t<2, 0, 0>(fa, pl, s) : launch_fused_t<4, 0, 0>(fa, pl, s);
}

}  // namespace lt
