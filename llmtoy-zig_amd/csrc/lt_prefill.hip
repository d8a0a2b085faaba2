// lt_prefill.hip -- batched prefill of one MoE layer (Q4_K experts) on MFMA.
//
// The reference prefills one token at a time through the decode path
// (main.zig:1916-1922).  Here T tokens go through the layer together:
//   1. router logits for all tokens with the reference's exact dotf32 order
//      and per-token softmax / top-k (lt_router.hip);
//   2. dispatch: one block counts tokens per expert, lays out per-expert
//      row ranges ("sorted rows"), cuts each range into chunks of at most
//      MC = 128 rows, and scatters (token, slot) assignments into them;
//      X is converted to bf16 once (k_prefill_x_bf16);
//   3. grouped gate/up GEMM: one block per (chunk, 64 output columns); its
//      128 weight rows (64 gate + 64 up) are dequantised from Q4_K to bf16
//      in LDS once per K stage and shared by the chunk's 4 token tiles (one
//      32-row tile per wavefront, v_mfma_f32_32x32x16_bf16, fp32
//      accumulation); gate and up of an output column sit in the same
//      wavefront, so the epilogue act(gate) * up -> H (bf16) needs no
//      exchange;
//   4. grouped down GEMM: one block per (chunk, 128 output rows), the same
//      scheme with H as the A operand -> Y (fp32, sorted rows);
//   5. combine: out[t] = sum over slots in slot order of w[t][s] * Y[pos].
// Both GEMMs run a software pipeline over K stages of 128 (half a Q4_K
// super-block): weight loads are issued two stages ahead into registers,
// A fragments one stage ahead, the dequantised tile is double-buffered in
// LDS, and each stage ends in one barrier.
// A row's result does not depend on which chunk position it lands in, so
// the atomically assigned positions leave the output bit-identical run to
// run.
#include "lt_internal.h"

namespace lt {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float floatx16;

namespace {

constexpr int MC = 128;       // sorted rows per chunk: 4 wavefronts x 32
constexpr int KS = 128;       // K per stage: half a Q4_K super-block
constexpr int LDK = KS + 8;   // padded LDS row (bf16 elements)
constexpr int NB = 128;       // weight rows per block (gate/up: 64 gate + 64 up)
constexpr int BN1 = 64;       // gate/up output columns per block
constexpr int BN2 = 128;      // down output rows (= output columns of Y) per block

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

struct Ws {
    float *logits;
    uint32_t *ids;
    float *w;
    int *offsets;   // [E+1]
    int *chunks;    // [max_chunks][3] = (expert, first row, rows)
    int *n_chunks;  // [1]
    int *perm;      // [T*k] token of each sorted row
    int *pos;       // [T*k] sorted row of assignment t*k + s
    __bf16 *Xb;     // [T][D] X in bf16
    __bf16 *H;      // [T*k][Kd]
    float *Y;       // [T*k][D]
};

int max_chunks(int TK, int E) { return (TK + MC - 1) / MC + E; }

Ws carve(void *base, int T, int k, int E, int Kd, int D) {
    uint8_t *p = (uint8_t *)base;
    const size_t TK = (size_t)T * k;
    Ws w;
    w.logits = (float *)p; p += align256((size_t)T * E * 4);
    w.ids = (uint32_t *)p; p += align256(TK * 4);
    w.w = (float *)p; p += align256(TK * 4);
    w.offsets = (int *)p; p += align256((size_t)(E + 1) * 4);
    w.chunks = (int *)p; p += align256((size_t)max_chunks((int)TK, E) * 12);
    w.n_chunks = (int *)p; p += 256;
    w.perm = (int *)p; p += align256(TK * 4);
    w.pos = (int *)p; p += align256(TK * 4);
    w.Xb = (__bf16 *)p; p += align256((size_t)T * D * 2);
    w.H = (__bf16 *)p; p += align256(TK * Kd * 2);
    w.Y = (float *)p; p += align256(TK * D * 4);
    return w;
}

typedef float float2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));

// Two fp32 values -> a packed bf16 pair (round to nearest even; one
// v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    const float2v v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2v));
}

// 16 fp32 values -> 16 bf16 as two 16-byte words.
__device__ __forceinline__ void store_bf16x16(__bf16 *dst, const float (&v)[16]) {
    uint4 a, b;
    a.x = pack_bf16x2(v[0], v[1]);
    a.y = pack_bf16x2(v[2], v[3]);
    a.z = pack_bf16x2(v[4], v[5]);
    a.w = pack_bf16x2(v[6], v[7]);
    b.x = pack_bf16x2(v[8], v[9]);
    b.y = pack_bf16x2(v[10], v[11]);
    b.z = pack_bf16x2(v[12], v[13]);
    b.w = pack_bf16x2(v[14], v[15]);
    *reinterpret_cast<uint4 *>(dst) = a;
    *reinterpret_cast<uint4 *>(dst + 8) = b;
}

// Q4_K 16-byte chunk cc (0..7) of a super-block with header hdr, dequantised
// (quant/dequant.zig:157-187: (d*sc)*q - dmin*mn) and stored as bf16:
// elements 64p + 16(cc&1) + [0, 16) at lo, the same + 32 at hi (p = cc / 2).
__device__ __forceinline__ void q4k_chunk_to_bf16(uint4 hdr, uint4 q, int cc, __bf16 *lo_dst, __bf16 *hi_dst) {
    const float d = f16_bits_to_f32(hdr.x), dmin = f16_bits_to_f32(hdr.x >> 16);
    const int p = cc >> 1;
    const int sh = (p & 1) * 16;
    const uint32_t ys = hdr.y >> sh, zs = hdr.z >> sh, ws = hdr.w >> sh;
    const uint32_t scp = opaque(p < 2 ? (ys & 0x3f3fu) : ((ws & 0x0f0fu) | ((ys >> 2) & 0x3030u)));
    const uint32_t mnp = opaque(p < 2 ? (zs & 0x3f3fu) : (((ws >> 4) & 0x0f0fu) | ((zs >> 2) & 0x3030u)));
    const float d1 = d * (float)(scp & 0xffu), m1 = dmin * (float)(mnp & 0xffu);
    const float d2 = d * (float)((scp >> 8) & 0xffu), m2 = dmin * (float)((mnp >> 8) & 0xffu);
    const uint32_t wv[4] = {q.x, q.y, q.z, q.w};
    float lo[16], hi[16];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint32_t l = opaque(wv[t] & 0x0f0f0f0fu), h = opaque((wv[t] >> 4) & 0x0f0f0f0fu);
        lo[4 * t + 0] = d1 * (float)(l & 0xffu) - m1;
        lo[4 * t + 1] = d1 * (float)((l >> 8) & 0xffu) - m1;
        lo[4 * t + 2] = d1 * (float)((l >> 16) & 0xffu) - m1;
        lo[4 * t + 3] = d1 * (float)(l >> 24) - m1;
        hi[4 * t + 0] = d2 * (float)(h & 0xffu) - m2;
        hi[4 * t + 1] = d2 * (float)((h >> 8) & 0xffu) - m2;
        hi[4 * t + 2] = d2 * (float)((h >> 16) & 0xffu) - m2;
        hi[4 * t + 3] = d2 * (float)(h >> 24) - m2;
    }
    store_bf16x16(lo_dst, lo);
    store_bf16x16(hi_dst, hi);
}

// One thread's share of a K stage's weight tile: 2 units of (weight row r,
// 16-byte chunk c): r = tid / 4 + 64 j, c = tid % 4.
struct StageRegs {
    uint4 h[2], q[2];
};

__device__ __forceinline__ void stage_load(StageRegs &R, const uint8_t *hdr, const uint8_t *qs, int nsb,
                                           const size_t (&wrow)[2], int ks, int c) {
    const int sb = ks >> 1, cc = (ks & 1) * 4 + c;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const size_t blk = wrow[j] * nsb + sb;
        R.h[j] = ldg16(hdr + blk * 16);
        R.q[j] = ldg16(qs + blk * 128 + cc * 16);
    }
}

// Stage ks's chunk cc = 4 (ks & 1) + c lands at local K 64 (c / 2) + 16 (c & 1)
// (low nibbles) and +32 (high nibbles).
__device__ __forceinline__ void stage_dequant(const StageRegs &R, __bf16 (*Bs)[LDK], int r0, int ks, int c) {
    const int cc = (ks & 1) * 4 + c, local = 64 * (c >> 1) + 16 * (c & 1);
#pragma unroll
    for (int j = 0; j < 2; j++) {
        __bf16 *row = Bs[r0 + 64 * j];
        q4k_chunk_to_bf16(R.h[j], R.q[j], cc, row + local, row + local + 32);
    }
}

// The grouped GEMM of one block over the chunk's rows and the block's NB
// weight rows (ct = 0..3 tiles of 32), K = 128 * NS.  Wavefront w takes
// token tile t = w % (4 / S) and, of every stage's 8 K steps of 16, the
// steps [kb, kb + 8 / S) with kb = (w / (4 / S)) * 8 / S: S = 1 gives each
// of 4 tiles a wavefront of its own; S = 2 / 4 split the K steps of 2 / 1
// tiles over 2 / 4 wavefronts, so a chunk with a single token tile still
// keeps all four wavefronts' MFMA pipes busy.  arow points at this lane's A
// row (row 32 t + lane % 32 of the chunk) plus its K half (lane / 32) * 8.
template <int S>
__device__ __forceinline__ void grouped_gemm(floatx16 (&acc)[4], __bf16 (*Bs)[NB][LDK], const uint8_t *hdr,
                                             const uint8_t *qs, int nsb, const size_t (&wrow)[2], int NS,
                                             const __bf16 *arow, bool wave_on, int kb, int tid, int lane) {
    constexpr int NK = 8 / S;
    const int c = tid & 3, r0 = tid >> 2;
    StageRegs R0, R1;
    bf16x8 a0[NK], a1[NK];
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = floatx16{};
    // Every wavefront issues the same loads on every path (stage indices
    // past the end are clamped and their data left unused; a wavefront
    // without a token tile loads a valid row it does not use): the memory
    // counter waits the compiler derives then cover only the data a step
    // needs, not the prefetches behind it.
    stage_load(R0, hdr, qs, nsb, wrow, 0, c);
    stage_load(R1, hdr, qs, nsb, wrow, 1, c);  // NS = 2 * super-blocks >= 2
#pragma unroll
    for (int i = 0; i < NK; i++) a0[i] = *reinterpret_cast<const bf16x8 *>(arow + (kb + i) * 16);
    stage_dequant(R0, Bs[0], r0, 0, c);
    stage_load(R0, hdr, qs, nsb, wrow, min(2, NS - 1), c);
    __syncthreads();
    // Two stages per trip (NS is even) so the register sets alternate
    // without copies: entering stage ks, Bs[ks & 1] holds it, R1 holds
    // ks + 1 and R0 holds ks + 2.
    for (int ks = 0; ks < NS; ks += 2) {
#pragma unroll
        for (int half = 0; half < 2; half++) {
            const int st = ks + half;
            StageRegs &Rn = half ? R0 : R1;   // stage st + 1
            bf16x8(&acur)[NK] = half ? a1 : a0;
            bf16x8(&anext)[NK] = half ? a0 : a1;
            const size_t sa = (size_t)min(st + 1, NS - 1) * KS;
#pragma unroll
            for (int i = 0; i < NK; i++) anext[i] = *reinterpret_cast<const bf16x8 *>(arow + sa + (kb + i) * 16);
            if (wave_on) {
                __bf16(*B)[LDK] = Bs[st & 1];
#pragma unroll
                for (int i = 0; i < NK; i++)
#pragma unroll
                    for (int ct = 0; ct < 4; ct++) {
                        const bf16x8 b = *reinterpret_cast<const bf16x8 *>(
                            &B[32 * ct + (lane & 31)][(kb + i) * 16 + (lane >> 5) * 8]);
                        acc[ct] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(acur[i], b, acc[ct], 0, 0, 0);
                    }
            }
            if (st + 1 < NS) stage_dequant(Rn, Bs[(st + 1) & 1], r0, st + 1, c);
            stage_load(Rn, hdr, qs, nsb, wrow, min(st + 3, NS - 1), c);
            __syncthreads();
        }
    }
}

// Runs the block's GEMM with K split S and hands every finished C element to
// epi(tile t, element i, values of the 4 column tiles): for S > 1 the S
// partial sums of a tile meet in LDS (the weight buffers, free after the
// last stage) and are added in wavefront order, so results do not depend
// on timing.  acc element i of a 32x32 tile is C[(i / 4) * 8 + (lane / 32) *
// 4 + i % 4][lane % 32].
template <int S, typename Row, typename Epi>
__device__ __forceinline__ void run_block(__bf16 (*Bs)[NB][LDK], const uint8_t *hdr, const uint8_t *qs, int nsb,
                                          const size_t (&wrow)[2], int NS, int mc, Row row_ptr, Epi epi, int tid,
                                          int wave, int lane) {
    constexpr int NT = 4 / S;  // token tiles handled side by side
    const int t = wave % NT, q = wave / NT;
    const int mrow = 32 * t + (lane & 31);
    const bool wave_on = 32 * t < mc;
    const __bf16 *arow = row_ptr(mrow < mc ? mrow : 0) + (lane >> 5) * 8;
    floatx16 acc[4];
    grouped_gemm<S>(acc, Bs, hdr, qs, nsb, wrow, NS, arow, wave_on, q * (8 / S), tid, lane);
    if (S == 1) {
        if (wave_on)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float v[4] = {acc[0][i], acc[1][i], acc[2][i], acc[3][i]};
                epi(t, i, v);
            }
        return;
    }
    float *red = reinterpret_cast<float *>(&Bs[0][0][0]);  // [4 waves][4 ct][16 i][64 lanes]
#pragma unroll
    for (int ct = 0; ct < 4; ct++)
#pragma unroll
        for (int i = 0; i < 16; i++) red[((wave * 4 + ct) * 16 + i) * 64 + lane] = acc[ct][i];
    __syncthreads();
    if (!wave_on) return;
    for (int ii = 0; ii < 16 / S; ii++) {
        const int i = q * (16 / S) + ii;
        float v[4];
#pragma unroll
        for (int ct = 0; ct < 4; ct++) {
            float sum = 0.0f;
#pragma unroll
            for (int qq = 0; qq < S; qq++) sum += red[(((t + NT * qq) * 4 + ct) * 16 + i) * 64 + lane];
            v[ct] = sum;
        }
        epi(t, i, v);
    }
}

}  // namespace

// ---------------------------------------------------------------- dispatch
__global__ void __launch_bounds__(1024) k_prefill_dispatch(const uint32_t *__restrict__ ids, int TK, int k, int E,
                                                           int *__restrict__ offsets, int *__restrict__ chunks,
                                                           int *__restrict__ n_chunks, int *__restrict__ perm,
                                                           int *__restrict__ pos) {
    // Per expert e (thread e): v[0] = its row count, v[1] = its full chunks,
    // v[2 + c] = 1 if its last chunk is partial with c + 1 token tiles.  An
    // inclusive scan over experts gives every expert its row offset and the
    // positions of its chunks in a list ordered by token tiles, largest
    // first: the blocks with the most MFMA work are dispatched first and
    // the short ones fill in behind them.
    __shared__ int cnt[1024], cur[1024];
    __shared__ int scan[2][6][1024];
    const int e = threadIdx.x;
    if (e < E) cnt[e] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < TK; i += blockDim.x) {
        const uint32_t x = ids[i];
        if (x < (uint32_t)E) atomicAdd(&cnt[x], 1);
    }
    __syncthreads();
    const int n = e < E ? cnt[e] : 0, full = n / MC, rem = n % MC, cls = rem ? (rem + 31) / 32 : 0;
    int v[6] = {n, full, cls == 1, cls == 2, cls == 3, cls == 4};
#pragma unroll
    for (int a = 0; a < 6; a++) scan[0][a][e] = v[a];
    __syncthreads();
    int b = 0;
    for (int d = 1; d < (int)blockDim.x; d <<= 1, b ^= 1) {
#pragma unroll
        for (int a = 0; a < 6; a++)
            scan[b ^ 1][a][e] = scan[b][a][e] + (e >= d ? scan[b][a][e - d] : 0);
        __syncthreads();
    }
    const int last = blockDim.x - 1;
    const int tot_full = scan[b][1][last];
    const int tot_p4 = scan[b][5][last], tot_p3 = scan[b][4][last], tot_p2 = scan[b][3][last];
    if (e < E) {
        const int off = scan[b][0][e] - n;
        offsets[e] = off;
        cur[e] = off;
        if (e == E - 1) {
            offsets[E] = off + n;
            *n_chunks = tot_full + tot_p4 + tot_p3 + tot_p2 + scan[b][2][last];
        }
        for (int j = 0; j < full; j++) {
            int *ch = chunks + 3 * (scan[b][1][e] - full + j);
            ch[0] = e;
            ch[1] = j * MC;
            ch[2] = MC;
        }
        if (cls) {
            const int start = cls == 4 ? tot_full : cls == 3 ? tot_full + tot_p4
                                                  : cls == 2 ? tot_full + tot_p4 + tot_p3
                                                             : tot_full + tot_p4 + tot_p3 + tot_p2;
            int *ch = chunks + 3 * (start + scan[b][1 + cls][e] - 1);
            ch[0] = e;
            ch[1] = full * MC;
            ch[2] = rem;
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < TK; i += blockDim.x) {
        const uint32_t x = ids[i];
        if (x < (uint32_t)E) {
            const int p = atomicAdd(&cur[x], 1);
            perm[p] = i / k;
            pos[i] = p;
        } else {
            pos[i] = -1;
        }
    }
}

// X (fp32) -> bf16, 8 elements per thread; n % 8 == 0.
__global__ void __launch_bounds__(256) k_prefill_x_bf16(const float *__restrict__ X, __bf16 *__restrict__ Xb,
                                                        size_t n8) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n8) return;
    const float4 a = ldg16f(X + 8 * i), b = ldg16f(X + 8 * i + 4);
    bf16x8 o;
    o[0] = (__bf16)a.x; o[1] = (__bf16)a.y; o[2] = (__bf16)a.z; o[3] = (__bf16)a.w;
    o[4] = (__bf16)b.x; o[5] = (__bf16)b.y; o[6] = (__bf16)b.z; o[7] = (__bf16)b.w;
    *reinterpret_cast<bf16x8 *>(Xb + 8 * i) = o;
}

// ---------------------------------------------------------------- gate/up
// Block: chunk (expert e, sorted rows base + m0 + [0, mc)) x output columns
// [n0, n0 + 64).  Weight rows 0..63 are gate rows n0.., 64..127 the up rows;
// wavefront w computes token tile w against all 128 (ct 0,1 = gate, 2,3 =
// up), so h = act(gate) * up is formed in registers.
__global__ void __launch_bounds__(256) k_prefill_gate_up(const uint8_t *__restrict__ hdr,
                                                         const uint8_t *__restrict__ qs, int nsb, int F,
                                                         const __bf16 *__restrict__ Xb, int D,
                                                         const int *__restrict__ chunks,
                                                         const int *__restrict__ n_chunks,
                                                         const int *__restrict__ offsets,
                                                         const int *__restrict__ perm, uint32_t act,
                                                         __bf16 *__restrict__ H, int Kd) {
    if ((int)blockIdx.y >= *n_chunks) return;
    const int e = chunks[3 * blockIdx.y], m0 = chunks[3 * blockIdx.y + 1], mc = chunks[3 * blockIdx.y + 2];
    const int base = offsets[e];
    const int n0 = blockIdx.x * BN1;
    __shared__ __attribute__((aligned(16))) __bf16 Bs[2][NB][LDK];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    size_t wrow[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int r = (tid >> 2) + 64 * j;
        wrow[j] = (size_t)e * 2 * F + (r < BN1 ? n0 + r : F + n0 + (r - BN1));
    }
    const int *prow = perm + base + m0;
    auto row_ptr = [&](int m) { return Xb + (size_t)prow[m] * D; };
    // ct 0, 1 = gate columns n0 + [0, 64), ct 2, 3 = the matching up columns
    auto epi = [&](int t, int i, const float (&v)[4]) {
        const int m = 32 * t + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
        if (m < mc) {
            __bf16 *hrow = H + (size_t)(base + m0 + m) * Kd + n0 + (lane & 31);
            hrow[0] = (__bf16)(act_apply(act, v[0]) * v[2]);
            hrow[32] = (__bf16)(act_apply(act, v[1]) * v[3]);
        }
    };
    const int nt = (mc + 31) / 32, NS = 2 * nsb;
    if (nt == 1)
        run_block<4>(Bs, hdr, qs, nsb, wrow, NS, mc, row_ptr, epi, tid, wave, lane);
    else if (nt == 2)
        run_block<2>(Bs, hdr, qs, nsb, wrow, NS, mc, row_ptr, epi, tid, wave, lane);
    else
        run_block<1>(Bs, hdr, qs, nsb, wrow, NS, mc, row_ptr, epi, tid, wave, lane);
    if (blockIdx.x == 0 && Kd > F)  // zero K padding of the down product
        for (int i = tid; i < mc * (Kd - F); i += 256) {
            const int m = i / (Kd - F), col = F + i % (Kd - F);
            H[(size_t)(base + m0 + m) * Kd + col] = (__bf16)0.f;
        }
}

// ---------------------------------------------------------------- down
// Block: chunk x output rows [n0, n0 + 128) of the expert's down matrix
// (= columns of Y); wavefront w computes token tile w, A = H rows (bf16).
__global__ void __launch_bounds__(256) k_prefill_down(const uint8_t *__restrict__ hdr, const uint8_t *__restrict__ qs,
                                                      int nsb, int D, const __bf16 *__restrict__ H, int Kd,
                                                      const int *__restrict__ chunks, const int *__restrict__ n_chunks,
                                                      const int *__restrict__ offsets, float *__restrict__ Y) {
    if ((int)blockIdx.y >= *n_chunks) return;
    const int e = chunks[3 * blockIdx.y], m0 = chunks[3 * blockIdx.y + 1], mc = chunks[3 * blockIdx.y + 2];
    const int base = offsets[e];
    const int n0 = blockIdx.x * BN2;
    __shared__ __attribute__((aligned(16))) __bf16 Bs[2][NB][LDK];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    size_t wrow[2];
#pragma unroll
    for (int j = 0; j < 2; j++) wrow[j] = (size_t)e * D + n0 + (tid >> 2) + 64 * j;
    const __bf16 *hbase = H + (size_t)(base + m0) * Kd;
    auto row_ptr = [&](int m) { return hbase + (size_t)m * Kd; };
    auto epi = [&](int t, int i, const float (&v)[4]) {
        const int m = 32 * t + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
        if (m < mc) {
            float *yrow = Y + (size_t)(base + m0 + m) * D + n0 + (lane & 31);
#pragma unroll
            for (int ct = 0; ct < 4; ct++) yrow[32 * ct] = v[ct];
        }
    };
    const int nt = (mc + 31) / 32, NS = 2 * nsb;
    if (nt == 1)
        run_block<4>(Bs, hdr, qs, nsb, wrow, NS, mc, row_ptr, epi, tid, wave, lane);
    else if (nt == 2)
        run_block<2>(Bs, hdr, qs, nsb, wrow, NS, mc, row_ptr, epi, tid, wave, lane);
    else
        run_block<1>(Bs, hdr, qs, nsb, wrow, NS, mc, row_ptr, epi, tid, wave, lane);
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
           align256((size_t)max_chunks((int)TK, E) * 12) + 256 + 2 * align256(TK * 4) +
           align256((size_t)T * D * 2) + align256(TK * Kd * 2) + align256(TK * D * 4);
}

hipError_t launch_moe_prefill(const DevTensor &R, const DevTensor &GU, const DevTensor &Dn, const float *X, int T,
                              const float *bias, int k, int F, uint32_t act, uint32_t norm, void *ws, float *out,
                              uint32_t *out_ids, float *out_w, hipStream_t s) {
    const int E = (int)GU.n_experts, D = (int)GU.cols, Kd = (int)Dn.cols;
    const int TK = T * k;
    Ws w = carve(ws, T, k, E, Kd, D);
    hipError_t e = launch_router_batched(R, X, T, bias, w.logits, k, norm, w.ids, w.w, s);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_prefill_dispatch, dim3(1), dim3(1024), 0, s, w.ids, TK, k, E, w.offsets, w.chunks,
                       w.n_chunks, w.perm, w.pos);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const size_t n8 = (size_t)T * D / 8;
    hipLaunchKernelGGL(k_prefill_x_bf16, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, s, X, w.Xb, n8);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const int mc = max_chunks(TK, E);
    hipLaunchKernelGGL(k_prefill_gate_up, dim3(F / BN1, mc), dim3(256), 0, s, GU.p0, GU.p1, (int)GU.blocks_per_row,
                       F, w.Xb, D, w.chunks, w.n_chunks, w.offsets, w.perm, act, w.H, Kd);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(k_prefill_down, dim3(D / BN2, mc), dim3(256), 0, s, Dn.p0, Dn.p1, (int)Dn.blocks_per_row, D,
                       w.H, Kd, w.chunks, w.n_chunks, w.offsets, w.Y);
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
