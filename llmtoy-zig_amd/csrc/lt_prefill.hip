// lt_prefill.hip -- batched prefill of one MoE layer (Q4_K experts) on MFMA.
//
// The reference prefills one token at a time through the decode path
// (main.zig:1916-1922).  Here T tokens go through the layer together:
//   1. router logits for all tokens with the reference's exact dotf32 order
//      and per-token softmax / top-k (lt_router.hip);
//   2. dispatch: one block counts tokens per expert, lays out per-expert
//      row ranges ("sorted rows"), cuts each range into chunks of at most
//      MC = 128 rows, and places the (token, slot) assignments into them in
//      assignment order (a stable counting sort);
//      X is converted to f16 once (by the router kernel, or
//      k_prefill_x_f16), each row t divided by r_t = 2^e, a power of two
//      that puts its largest element in [1, 2);
//   3. grouped gate/up GEMM: one block per (chunk, 64 output columns); its
//      128 weight rows (64 gate + 64 up) are dequantised from Q4_K to f16
//      in LDS once per K stage and shared by the chunk's 4 token tiles (one
//      32-row tile per wavefront, v_mfma_f32_32x32x16_f16, fp32
//      accumulation); gate and up of an output column sit in the same
//      wavefront, so the epilogue h = act(gate) * up needs no exchange; it
//      stores H = h / r_t^2 (f16), which |act(g)| <= |g| bounds by the
//      scaled row's products whatever X's magnitude (a value still past
//      f16's range saturates at +-65504 and is counted: the call then
//      reports LT_ERR_DEVICE);
//   4. grouped down GEMM: one block per (chunk, 128 output rows), the same
//      scheme with H as the A operand -> Y (fp32, sorted rows);
//   5. combine: out[t] = r_t^2 * sum over slots in slot order of w[t][s] *
//      Y[pos] (r_t^2 exact).
// Steps 3 and 4 run as one launch when blocks with equal index % 8 share an
// XCD (k_prefill_gemms: a chunk's down blocks take H from its gate/up
// blocks through that XCD's L2), else as two.  Chunks of a single token
// skip the tiles: their blocks stream the weights against int8 limbs of the
// token like the decode kernels (gate_up_tiny, down_tiny).
// Both GEMMs run a software pipeline over K stages of 128 (half a Q4_K
// super-block): weight loads are issued two stages ahead into registers,
// A fragments one stage ahead, the dequantised tile is double-buffered in
// LDS, and each stage ends in one barrier.
// A row's result depends on its chunk only through the chunk's token tiles
// (they pick the K split of the GEMMs, and with it the order of the fp32
// sums), and the stable placement gives every row the same chunk on every
// call, so the output is bit-identical run to run.
//
// f16 rather than bf16 tiles: a Q4_K nibble q becomes the exact f16 1024 + q
// (or 1024 + 16 q) with one v_and_or (its bits in the mantissa under 1024's
// exponent), two such values per dword, so the dequantisation is a packed
// f16 subtract of 1024 and a packed f16 fma (d sc) q - dmin mn per pair of
// weights, with no conversion or packing step -- and f16 keeps 3 more
// mantissa bits than bf16.  The pairs come out as elements (0, 2) and (1, 3) of each aligned
// group of 4, so every K dimension is stored with the middle two of each 4
// swapped (kperm): X and H are written in that order, and the MFMA sums the
// same products.
#include "lt_internal.h"
#include "lt_limbs.h"

#include <stdlib.h>

namespace lt {

typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float floatx16;
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

namespace {

constexpr int MC = 128;       // sorted rows per chunk: 4 wavefronts x 32
constexpr int KS = 128;       // K per stage: half a Q4_K super-block
constexpr int LDK = KS;       // LDS row (f16 elements), units swizzled (bunit)
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
    float *rs;      // [T] row scales: X row t = rs[t] * Xh row t
    _Float16 *Xh;   // [T][D] X / rs in f16, columns in kperm order
    _Float16 *H;    // [T*k][Kd], columns in kperm order
    float *Y;       // [T*k][D]
    int *done;      // [max_chunks] finished gate/up blocks per chunk (fused GEMMs)
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
    w.rs = (float *)p; p += align256((size_t)T * 4);
    w.Xh = (_Float16 *)p; p += align256((size_t)T * D * 2);
    w.H = (_Float16 *)p; p += align256(TK * Kd * 2);
    w.Y = (float *)p; p += align256(TK * D * 4);
    w.done = (int *)p; p += align256((size_t)max_chunks((int)TK, E) * 4);
    return w;
}

// LDS weight tiles: a row's 128 K values are 16 units of 8 f16 (16 bytes);
// unit u of row r is stored at unit bunit(r, u) = u ^ g(r) ^ 4 (u >> 3 & 1),
// g(r) = r & 7 | (r >> 3 ^ r >> 1 & 1) << 3.  g takes 16 distinct values over
// 16 consecutive rows, so the MFMA operand reads (consecutive lanes: rows
// r.., one unit) fall in distinct 16-byte bank groups; the 4 (u >> 3 & 1)
// separates a dequantising quad's units U and 8 + U of one row, so its
// 16-byte writes (a quad per row, four rows per 16 lanes) are conflict-free
// too, whether the LDS serves 8 lanes over 32 banks or 16 over 64.  A
// bijection within each row (XOR with 4 leaves bit 3 alone).  Rows r and
// r + 32 j share g.
__host__ __device__ __forceinline__ int bunit(int r, int u) {
    return u ^ ((r & 7) | (((r >> 3) ^ (r >> 1)) & 1) << 3) ^ (((u >> 3) & 1) << 2);
}

// The K order of every f16 operand: within each aligned group of 4 the
// middle two elements are swapped (an involution).
__host__ __device__ __forceinline__ int kperm(int c) { return (c & ~3) | ((c & 1) << 1) | ((c >> 1) & 1); }

// 4 packed words of (1024 + q 2^j) pairs -> (scale q + neg_min) pairs
// (scale already divided by 2^j), stored as 8 f16 at dst.
__device__ __forceinline__ void q4_pairs_to_f16(const uint32_t (&v)[4], half2v sc, half2v nm, _Float16 *dst) {
    const half2v k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const half2v q = __builtin_bit_cast(half2v, v[i]) - k1024;  // exact: q 2^j, q in 0..15
        o[i] = __builtin_bit_cast(uint32_t, q * sc + nm);
    }
    *reinterpret_cast<uint4 *>(dst) = make_uint4(o[0], o[1], o[2], o[3]);
}

// Q4_K 16-byte chunk cc (0..7) of a super-block with header hdr, dequantised
// (quant/dequant.zig:157-187: (d*sc)*q - dmin*mn) to f16: elements 64p +
// 16(cc&1) + [0, 8) at dst[0], + [8, 16) at dst[1], the same + 32 at dst[2],
// dst[3] (p = cc / 2), each run in kperm order.  Quant byte j holds element j of the low run in its
// low nibble and of the high run in its high nibble.  Under f16's exponent
// of 1024 (0x6400) a nibble in mantissa bits 0-3 reads 1024 + q and one in
// bits 4-7 reads 1024 + 16 q, both exact, so (w & 0x000f000f) | 0x64006400
// is the low-run pair (e0, e2) of the word's bytes 0 and 2, (w & 0x00f000f0)
// | 0x64006400 the high-run pair, and the same of w >> 8 gives (e1, e3):
// one v_and_or per pair (the masks kept in registers so that the compiler
// forms it), the high run's scale divided by 16.
__device__ __forceinline__ void q4k_chunk_to_f16(uint4 hdr, uint4 q, int cc, _Float16 *const (&dst)[4]) {
    const float d = f16_bits_to_f32(hdr.x), dmin = f16_bits_to_f32(hdr.x >> 16);
    const int p = cc >> 1;
    const int sh = (p & 1) * 16;
    const uint32_t ys = hdr.y >> sh, zs = hdr.z >> sh, ws = hdr.w >> sh;
    const uint32_t scp = opaque(p < 2 ? (ys & 0x3f3fu) : ((ws & 0x0f0fu) | ((ys >> 2) & 0x3030u)));
    const uint32_t mnp = opaque(p < 2 ? (zs & 0x3f3fu) : (((ws >> 4) & 0x0f0fu) | ((zs >> 2) & 0x3030u)));
    const _Float16 d1 = (_Float16)(d * (float)(scp & 0xffu)), m1 = (_Float16)(-(dmin * (float)(mnp & 0xffu)));
    const _Float16 d2 = (_Float16)(d * (float)((scp >> 8) & 0xffu) * 0.0625f);
    const _Float16 m2 = (_Float16)(-(dmin * (float)((mnp >> 8) & 0xffu)));
    const uint32_t ml = opaque(0x000f000fu), mh = opaque(0x00f000f0u), ex = opaque(0x64006400u);
    const uint32_t wv[4] = {q.x, q.y, q.z, q.w};
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint32_t w = wv[t], w8 = w >> 8;
        lo[2 * t] = (w & ml) | ex;
        lo[2 * t + 1] = (w8 & ml) | ex;
        hi[2 * t] = (w & mh) | ex;
        hi[2 * t + 1] = (w8 & mh) | ex;
    }
    const uint32_t lo0[4] = {lo[0], lo[1], lo[2], lo[3]}, lo1[4] = {lo[4], lo[5], lo[6], lo[7]};
    const uint32_t hi0[4] = {hi[0], hi[1], hi[2], hi[3]}, hi1[4] = {hi[4], hi[5], hi[6], hi[7]};
    q4_pairs_to_f16(lo0, half2v{d1, d1}, half2v{m1, m1}, dst[0]);
    q4_pairs_to_f16(lo1, half2v{d1, d1}, half2v{m1, m1}, dst[1]);
    q4_pairs_to_f16(hi0, half2v{d2, d2}, half2v{m2, m2}, dst[2]);
    q4_pairs_to_f16(hi1, half2v{d2, d2}, half2v{m2, m2}, dst[3]);
}

// One thread's share of a K stage's weight tile: 2 units of (weight row r,
// 16-byte chunk c): r = tid / 4 + 64 j, c = tid % 4.  The four threads of a
// row (an aligned quad) each load one word of the row's 16-byte header and
// share them over DPP, so a stage in flight holds 10 registers, not 16.
struct StageRegs {
    uint32_t h[2];
    uint4 q[2];
};

__device__ __forceinline__ void stage_load(StageRegs &R, const uint8_t *hdr, const uint8_t *qs, int nsb,
                                           const size_t (&wrow)[2], int ks, int c) {
    const int sb = ks >> 1, cc = (ks & 1) * 4 + c;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const size_t blk = wrow[j] * nsb + sb;
        R.h[j] = *reinterpret_cast<const uint32_t *>(hdr + blk * 16 + 4 * c);
        R.q[j] = ldg16(qs + blk * 128 + cc * 16);
    }
}

template <int CTRL>
__device__ __forceinline__ uint32_t quad_word(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, true);
}

// Stage ks's chunk cc = 4 (ks & 1) + c lands at local K 64 (c / 2) + 16 (c & 1)
// (low nibbles) and +32 (high nibbles): units U, U + 1, U + 4, U + 5 with U
// = 8 (c / 2) + 2 (c & 1), at doff[q] = 8 bunit(r0, unit) (rows r0 + 64 j
// share r0's swizzle).
__device__ __forceinline__ void stage_dequant(const StageRegs &R, _Float16 (*Bs)[LDK], int r0, int ks, int c,
                                              const int (&doff)[4]) {
    const int cc = (ks & 1) * 4 + c;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        _Float16 *row = Bs[r0 + 64 * j];
        const uint4 h = make_uint4(quad_word<0x00>(R.h[j]), quad_word<0x55>(R.h[j]), quad_word<0xAA>(R.h[j]),
                                   quad_word<0xFF>(R.h[j]));
        _Float16 *const dst[4] = {row + doff[0], row + doff[1], row + doff[2], row + doff[3]};
        q4k_chunk_to_f16(h, R.q[j], cc, dst);
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
// wait() runs (in every thread) once the first weight stages are requested
// and before the first A load: the fused kernel's down blocks wait there
// for their chunk's activations.
template <int S, typename Wait>
__device__ __forceinline__ void grouped_gemm(floatx16 (&acc)[4], _Float16 (*Bs)[NB][LDK], const uint8_t *hdr,
                                             const uint8_t *qs, int nsb, const size_t (&wrow)[2], int NS,
                                             const _Float16 *arow, bool wave_on, int kb, int tid, int lane,
                                             Wait wait) {
    constexpr int NK = 8 / S;
    const int c = tid & 3, r0 = tid >> 2;
    int doff[4], boff[NK];  // this thread's swizzled LDS units (f16 offsets in a row)
    {
        const int U = 8 * (c >> 1) + 2 * (c & 1);
        doff[0] = 8 * bunit(r0, U);
        doff[1] = 8 * bunit(r0, U + 1);
        doff[2] = 8 * bunit(r0, U + 4);
        doff[3] = 8 * bunit(r0, U + 5);
#pragma unroll
        for (int i = 0; i < NK; i++) boff[i] = 8 * bunit(lane & 31, 2 * (kb + i) + (lane >> 5));
    }
    StageRegs R[3];
    f16x8 a[2][NK];
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = floatx16{};
    // Every wavefront issues the same loads on every path (stage indices
    // past the end are clamped and their data left unused; a wavefront
    // without a token tile loads a valid row it does not use): the memory
    // counter waits the compiler derives then cover only the data a step
    // needs, not the prefetches behind it.  Three stages' weights are in
    // flight ahead of the one being dequantised.
    stage_load(R[0], hdr, qs, nsb, wrow, 0, c);
    stage_load(R[1], hdr, qs, nsb, wrow, 1, c);  // NS = 2 * super-blocks >= 2
    stage_load(R[2], hdr, qs, nsb, wrow, min(2, NS - 1), c);
    wait();
#pragma unroll
    for (int i = 0; i < NK; i++) a[0][i] = *reinterpret_cast<const f16x8 *>(arow + (kb + i) * 16);
    stage_dequant(R[0], Bs[0], r0, 0, c, doff);
    stage_load(R[0], hdr, qs, nsb, wrow, min(3, NS - 1), c);
    __syncthreads();
    // Six stages per trip, so that the A buffers (stage parity) and the
    // weight register sets (stage mod 3) have fixed names: entering stage
    // st, Bs[st & 1] holds it and R[(st + 1) % 3], R[(st + 2) % 3],
    // R[st % 3] hold stages st + 1, st + 2, st + 3.
    for (int ks = 0; ks < NS; ks += 6) {
#pragma unroll
        for (int u = 0; u < 6; u++) {
            const int st = ks + u;
            if (st >= NS) break;  // (uniform over the block)
            StageRegs &Rn = R[(u + 1) % 3];  // stage st + 1
            f16x8(&acur)[NK] = a[u & 1];
            f16x8(&anext)[NK] = a[(u + 1) & 1];
            const size_t sa = (size_t)min(st + 1, NS - 1) * KS;
#pragma unroll
            for (int i = 0; i < NK; i++) anext[i] = *reinterpret_cast<const f16x8 *>(arow + sa + (kb + i) * 16);
            if (wave_on) {
                _Float16(*B)[LDK] = Bs[st & 1];
#pragma unroll
                for (int i = 0; i < NK; i++)
#pragma unroll
                    for (int ct = 0; ct < 4; ct++) {
                        const f16x8 b = *reinterpret_cast<const f16x8 *>(&B[32 * ct + (lane & 31)][boff[i]]);
                        acc[ct] = __builtin_amdgcn_mfma_f32_32x32x16_f16(acur[i], b, acc[ct], 0, 0, 0);
                    }
            }
            if (st + 1 < NS) stage_dequant(Rn, Bs[(st + 1) & 1], r0, st + 1, c, doff);
            stage_load(Rn, hdr, qs, nsb, wrow, min(st + 4, NS - 1), c);
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
// pre(t, i) gives a value epi receives with element i (the gate/up
// kernel's row scale): all of a wavefront's pre loads are issued before its
// first epi, so that their round trips overlap instead of queueing behind
// each element's stores.
template <int S, typename Row, typename Pre, typename Epi, typename Wait>
__device__ __forceinline__ void run_block(_Float16 (*Bs)[NB][LDK], const uint8_t *hdr, const uint8_t *qs, int nsb,
                                          const size_t (&wrow)[2], int NS, int mc, Row row_ptr, Pre pre, Epi epi,
                                          Wait wait, int tid, int wave, int lane) {
    constexpr int NT = 4 / S;  // token tiles handled side by side
    const int t = wave % NT, q = wave / NT;
    const int mrow = 32 * t + (lane & 31);
    const bool wave_on = 32 * t < mc;
    const _Float16 *arow = row_ptr(mrow < mc ? mrow : 0) + (lane >> 5) * 8;
    floatx16 acc[4];
    grouped_gemm<S>(acc, Bs, hdr, qs, nsb, wrow, NS, arow, wave_on, q * (8 / S), tid, lane, wait);
    constexpr int NI = 16 / S;  // elements this wavefront hands over
    const int i0 = S == 1 ? 0 : q * NI;
    float pv[NI];
    if (S == 1) {
        if (wave_on) {
#pragma unroll
            for (int ii = 0; ii < NI; ii++) pv[ii] = pre(t, ii);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float v[4] = {acc[0][i], acc[1][i], acc[2][i], acc[3][i]};
                epi(t, i, v, pv[i]);
            }
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
#pragma unroll
    for (int ii = 0; ii < NI; ii++) pv[ii] = pre(t, i0 + ii);
#pragma unroll
    for (int ii = 0; ii < NI; ii++) {
        const int i = i0 + ii;
        float v[4];
#pragma unroll
        for (int ct = 0; ct < 4; ct++) {
            float sum = 0.0f;
#pragma unroll
            for (int qq = 0; qq < S; qq++) sum += red[(((t + NT * qq) * 4 + ct) * 16 + i) * 64 + lane];
            v[ct] = sum;
        }
        epi(t, i, v, pv[ii]);
    }
}

}  // namespace

// ---------------------------------------------------------------- dispatch
// The lanes of the wavefront whose id equals this lane's (ids below 2^nb,
// invalid ids >= E in a group of their own): one ballot per id bit.
__device__ __forceinline__ uint64_t match_ids(uint32_t x, bool valid, int nb) {
    uint64_t m = __ballot(1);  // the active lanes
    const uint64_t v = __ballot(valid);
    m &= valid ? v : ~v;
    for (int b = 0; b < nb; b++) {
        const bool on = (x >> b) & 1u;
        const uint64_t bb = __ballot(on);
        m &= on ? bb : ~bb;
    }
    return m;
}

// Lanes of m below this lane.
__device__ __forceinline__ int rank_in(uint64_t m) {
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// One block of 1024 threads.  Assignment i = t k + s goes to sorted row
// offsets[e] + (the number of assignments before i with the same expert e):
// a stable counting sort, so every row's chunk, and with it the row's
// result (the chunk's token tiles pick the GEMM's K split), is the same on
// every call.  Assignments are taken in rounds of 1024 (i = 1024 r + tid),
// a round in 16 segments of 64 (its wavefronts).  Within a wavefront the
// lanes with equal ids find each other with one ballot per id bit
// (match_ids); the first lane of each group adds the group's size to its
// expert's count and, for the placement, writes it to the segment's entry
// of a [segment][expert] table, which P = 1024 / E threads per expert
// turn into each segment's first row (an exclusive scan over segments, the
// experts' running rows carried from one batch of rounds to the next).
// Per expert e (thread e): v[0] = its row count, v[1] = its full chunks,
// v[2 + c] = 1 if its last chunk is partial with c + 1 token tiles.  An
// inclusive scan over experts (wavefront scans, then the wavefront totals)
// gives every expert its row offset and the positions of its chunks in a
// list ordered by token tiles, largest first: the blocks with the most
// MFMA work are dispatched first and the short ones fill in behind them.
// Up to kIdsPer ids per thread are loaded once, all in flight together,
// and kept with their ranks for the placement; longer batches read them
// again.
__global__ void __launch_bounds__(1024) k_prefill_dispatch(const uint32_t *__restrict__ ids, int TK, int k, int E,
                                                           int *__restrict__ offsets, int *__restrict__ chunks,
                                                           int *__restrict__ n_chunks, int *__restrict__ perm,
                                                           int *__restrict__ pos, int *__restrict__ done, int maxc) {
    constexpr int kIdsPer = 8, kTab = 16384;
    __shared__ int cnt[1024], cur[1024], psum[1024];
    __shared__ int tab[kTab];  // [segment][E]: group sizes, then the segment's first rows
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int nb = E > 1 ? 32 - __builtin_clz((unsigned)(E - 1)) : 0;
    const bool cached = TK <= kIdsPer * 1024;
    const int rounds = (TK + 1023) / 1024;
    uint32_t xc[kIdsPer];
    int rk[kIdsPer], gs[kIdsPer];  // cached: rank in the wavefront's group, group size (0: not the group's first)
#pragma unroll
    for (int j = 0; j < kIdsPer; j++) {
        const int i = tid + j * 1024;
        xc[j] = cached && i < TK ? ids[i] : 0xffffffffu;
    }
    // placement in batches of RB rounds (16 RB segments x E in the table)
    const int RB = max(1, min(kIdsPer, kTab / (16 * E)));
    if (tid < E) cnt[tid] = 0;
    for (int i = tid; i < maxc; i += 1024) done[i] = 0;  // the fused GEMMs' per-chunk counts
    for (int q = tid; q < 16 * min(RB, rounds) * E; q += 1024) tab[q] = 0;  // (the first batch's table)
    __syncthreads();
    auto group = [&](uint32_t x, int &rank, int &size) {
        const bool valid = x < (uint32_t)E;
        const uint64_t m = match_ids(x, valid, nb);
        rank = rank_in(m);
        size = valid && rank == 0 ? __popcll(m) : 0;
    };
    // assignment tid + 1024 r: id, rank, group size
    auto get = [&](int r, uint32_t &x, int &rank, int &size) {
        if (cached) {
            x = 0xffffffffu;
            rank = size = 0;
#pragma unroll
            for (int j = 0; j < kIdsPer; j++)
                if (j == r) {
                    x = xc[j];
                    rank = rk[j];
                    size = gs[j];
                }
        } else {
            const int i = tid + 1024 * r;
            x = i < TK ? ids[i] : 0xffffffffu;
            group(x, rank, size);
        }
    };
    if (cached) {
#pragma unroll
        for (int j = 0; j < kIdsPer; j++) {
            if (j < rounds) {
                group(xc[j], rk[j], gs[j]);
                if (gs[j]) atomicAdd(&cnt[xc[j]], gs[j]);
            }
        }
    } else {
        for (int i = tid; i < TK; i += 1024) {
            const uint32_t x = ids[i];
            if (x < (uint32_t)E) atomicAdd(&cnt[x], 1);
        }
    }
    __syncthreads();
    // Experts in order, by wavefront 0: lane l takes experts CH l + [0, CH)
    // (CH = ceil(E / 64)); the lanes' totals of rows, full chunks and
    // partial chunks of each tile count (two 16-bit counts per word) are
    // scanned over the lanes, then each lane lays out its experts' rows and
    // chunks -- full chunks first, then the partial ones by token tiles,
    // largest first: the blocks with the most MFMA work are dispatched
    // first and the short ones fill in behind them.
    if (wave == 0) {
        const int CH = (E + 63) >> 6;
        int t0 = 0, t1 = 0, t12 = 0, t34 = 0;  // rows, full chunks, partial chunks of 1 | 2 << 16, 3 | 4 << 16 tiles
        for (int q = 0; q < CH; q++) {
            const int e = CH * lane + q;
            const int n = e < E ? cnt[e] : 0, rem = n % MC, cls = rem ? (rem + 31) / 32 : 0;
            t0 += n;
            t1 += n / MC;
            t12 += (cls == 1 ? 1 : 0) + (cls == 2 ? 0x10000 : 0);
            t34 += (cls == 3 ? 1 : 0) + (cls == 4 ? 0x10000 : 0);
        }
        int i0 = t0, i1 = t1, i12 = t12, i34 = t34;  // inclusive scans over the lanes
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int a0 = __shfl_up(i0, d, 64), a1 = __shfl_up(i1, d, 64);
            const int a12 = __shfl_up(i12, d, 64), a34 = __shfl_up(i34, d, 64);
            if (lane >= d) {
                i0 += a0;
                i1 += a1;
                i12 += a12;
                i34 += a34;
            }
        }
        const int T1 = __shfl(i1, 63, 64), T12 = __shfl(i12, 63, 64), T34 = __shfl(i34, 63, 64);
        const int tot_full = T1, tot_p4 = T34 >> 16, tot_p3 = T34 & 0xffff, tot_p2 = T12 >> 16, tot_p1 = T12 & 0xffff;
        // first chunk index of each partial class, then this lane's running positions
        int off = i0 - t0, fc = i1 - t1;
        int pc[4] = {tot_full + tot_p4 + tot_p3 + tot_p2 + ((i12 - t12) & 0xffff),
                     tot_full + tot_p4 + tot_p3 + ((i12 - t12) >> 16), tot_full + tot_p4 + ((i34 - t34) & 0xffff),
                     tot_full + ((i34 - t34) >> 16)};
        for (int q = 0; q < CH; q++) {
            const int e = CH * lane + q;
            if (e >= E) break;
            const int n = cnt[e], full = n / MC, rem = n % MC, cls = rem ? (rem + 31) / 32 : 0;
            offsets[e] = off;
            cur[e] = off;
            for (int j = 0; j < full; j++) {
                int *ch = chunks + 3 * (fc + j);
                ch[0] = e;
                ch[1] = j * MC;
                ch[2] = MC;
            }
            fc += full;
            if (cls) {
                int *ch = chunks + 3 * pc[cls - 1];
                ch[0] = e;
                ch[1] = full * MC;
                ch[2] = rem;
                pc[cls - 1]++;
            }
            off += n;
            if (e == E - 1) {
                offsets[E] = off;
                *n_chunks = tot_full + tot_p4 + tot_p3 + tot_p2 + tot_p1;
            }
        }
    }
    __syncthreads();
    // placement: cur[e] = the expert's next free row
    const int P = min(32, 1024 / E), pe = tid % E, pp = tid / E;  // thread pp < P of expert pe
    for (int r0 = 0; r0 < rounds; r0 += RB) {
        const int nr = min(RB, rounds - r0), SB = 16 * nr;
        uint32_t xb[kIdsPer];
        int rkb[kIdsPer];
        if (r0 > 0) {  // (the first batch's table was cleared at the start)
            for (int q = tid; q < SB * E; q += 1024) tab[q] = 0;
            __syncthreads();  // (also: the previous batch's reads of the table and cur's update are done)
        }
#pragma unroll
        for (int rr = 0; rr < kIdsPer; rr++) {
            if (rr < nr) {
                int size;
                get(r0 + rr, xb[rr], rkb[rr], size);
                if (size) tab[(16 * rr + wave) * E + xb[rr]] = size;
            }
        }
        __syncthreads();
        const int SP = (SB + P - 1) / P, s0 = pp * SP, s1 = min(SB, s0 + SP);
        if (pp < P) {
            int loc = 0;
            for (int sg = s0; sg < s1; sg++) loc += tab[sg * E + pe];
            psum[pp * E + pe] = loc;
        }
        __syncthreads();
        int total = 0;
        if (pp < P) {
            int base = cur[pe];
            for (int p2 = 0; p2 < P; p2++) {
                const int ps = psum[p2 * E + pe];
                base += p2 < pp ? ps : 0;
                total += ps;
            }
            for (int sg = s0; sg < s1; sg++) {
                const int c = tab[sg * E + pe];
                tab[sg * E + pe] = base;
                base += c;
            }
        }
        __syncthreads();
        if (pp == 0) cur[pe] += total;  // (read again only after the next batch's first barrier)
#pragma unroll
        for (int rr = 0; rr < kIdsPer; rr++) {
            const int i = tid + 1024 * (r0 + rr);
            if (rr < nr && i < TK) {
                const uint32_t x = xb[rr];
                if (x < (uint32_t)E) {
                    const int p = tab[(16 * rr + wave) * E + x] + rkb[rr];
                    perm[p] = i / k;
                    pos[i] = p;
                } else {
                    pos[i] = -1;
                }
            }
        }
    }
}

// X (fp32) -> f16, one block per token row (prefill_x_exp, prefill_x_store8:
// the row divided by rs = 2^e, stored in kperm order), for the router paths
// that do not write it themselves.  D % 8 == 0; the fp32 row is read twice
// (max, then values).
__global__ void __launch_bounds__(256) k_prefill_x_f16(const float *__restrict__ X, _Float16 *__restrict__ Xh,
                                                       float *__restrict__ rs, int D) {
    const int t = blockIdx.x, tid = threadIdx.x;
    const float *xr = X + (size_t)t * D;
    float m = 0.0f;
    for (int i = 4 * tid; i < D; i += 4 * 256) {
        const float4 v = ldg16f(xr + i);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    __shared__ float s_m[4];
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, __shfl_xor(m, 8, 64));
    m = fmaxf(m, __shfl_xor(m, 4, 64));
    m = fmaxf(m, __shfl_xor(m, 2, 64));
    m = fmaxf(m, __shfl_xor(m, 1, 64));
    if ((tid & 63) == 0) s_m[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(s_m[0], s_m[1]), fmaxf(s_m[2], s_m[3]));
    const int e = prefill_x_exp(m);
    const float inv = ldexpf(1.0f, -e);
    if (tid == 0) rs[t] = ldexpf(1.0f, e);
    _Float16 *hr = Xh + (size_t)t * D;
    for (int i = 8 * tid; i < D; i += 8 * 256) prefill_x_store8(xr, inv, hr, i);
}

// ---------------------------------------------------------------- gate/up
// The activation for the f16 H, branch-free: e^x and 1 / x as one hardware
// instruction each (v_exp_f32 on x log2 e, v_rcp_f32; about 1 ulp of fp32,
// far below the f16 rounding of H that follows).  SiLU g / (1 + e^-g);
// GELU (tanh form) 0.5 g (1 + tanh y) with tanh y = 1 - 2 / (1 + e^2y).
// Limits: g -> -inf gives -0 (SiLU) or 0, +inf gives g; NaN passes.
template <int ACT>
__device__ __forceinline__ float prefill_act(float g) {
    constexpr float kLog2e = 1.4426950408889634f;
    if (ACT == 1) {
        const float y = 0.7978845608028654f * (g + 0.044715f * g * g * g);
        const float t = 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(2.0f * kLog2e * y));
        return 0.5f * g * (1.0f + t);
    }
    return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-kLog2e * g));
}

namespace {

// Arguments of both grouped GEMMs (shared by their separate kernels and the
// fused one).
struct PfArgs {
    const uint8_t *gu_hdr, *gu_qs;  // gate/up planes: [E][2F] rows of gu_nsb super-blocks
    int gu_nsb, F;
    const _Float16 *Xh;
    const float *rs;
    int D;
    const int *chunks, *n_chunks, *offsets, *perm;
    _Float16 *H;
    int Kd;
    const uint8_t *dn_hdr, *dn_qs;  // down planes: [E][D] rows of dn_nsb super-blocks
    int dn_nsb;
    float *Y;
    uint32_t *err;
    int *done;  // fused kernel: finished gate/up blocks per chunk (zeroed by the dispatch)
    int CG;     // fused kernel: chunk slots per XCD group
    const float *X;  // the fp32 input rows (one-token chunks)
    int tiny;        // one-token chunks take the decode-style stream (gate/up rows <= 8, down rows <= 4 super-blocks)
};

struct NoWait {
    __device__ __forceinline__ void operator()() const {}
};

// ---------------------------------------------------------------- chunks of one token
// A chunk of one token streams its weights like the decode path instead of
// dequantising them to f16 tiles for a 32-row MFMA: the f16 tile costs the
// same whatever the chunk's rows, and many one-tile chunks of a skewed
// routing hold a single token (22 of the 63 in a 512-token batch with
// Zipf-biased logits).  (NT = 2 as well needed more registers than two
// waves per SIMD allow.)  A lane owns one Q4_K sub-block pair window
// (position 4 sb + p of a row: K elements 256 sb + 64 p + [0, 64)),
// whose activations it turns into int8 limbs in registers once (limbs16);
// per row it loads the window's 32 quant bytes and its quad's header word
// and meets them with each token's limbs on v_dot4 (q4k_pair_dot); a row's
// window dots meet in LDS and one lane adds them in position order, so
// results do not depend on timing.

struct WinW {
    uint4 q0, q1;
    uint32_t h;
};

__device__ __forceinline__ WinW load_window(const uint8_t *hdr, const uint8_t *qs, size_t blk, int p) {
    WinW w;
    w.q0 = ldg16(qs + blk * 128 + 32 * p);
    w.q1 = ldg16(qs + blk * 128 + 32 * p + 16);
    w.h = *reinterpret_cast<const uint32_t *>(hdr + blk * 16 + 4 * p);
    return w;
}

__device__ __forceinline__ float window_dot(const WinW &w, int p, const Limbs &xl) {
    uint32_t h0, h1, h2, h3;
    quad_header(w.h, h0, h1, h2, h3);
    const PairScale ps = pair_scale(h0, h1, h2, h3, p);
    const uint32_t w8[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
    return q4k_pair_dot(w8, ps, xl);
}

// Gate/up of a chunk of NT tokens (one in use), columns n0 + [0, 64): wavefront
// w takes columns n0 + 16 w + c, one per pass c; lanes 0-31 the gate row,
// 32-63 the up row, lane l & 31 = window position (rows of at most 8
// super-blocks).  Weights two passes ahead; each lane's window dots go to
// LDS (red: [wave][pass][token][lane], the f16 tile's space) and lane c +
// 16 t + 32 half sums the 32 positions of (pass c, token t, gate or up) in
// position order.
template <int ACT, int NT>
__device__ __forceinline__ uint32_t gate_up_tiny(const PfArgs &a, float *red, const int *prow, int e, int row0,
                                                 int n0, int wave, int lane) {
    const int F = a.F, nsb = a.gu_nsb, Kd = a.Kd;
    const int pos = lane & 31, sb = min(pos >> 2, nsb - 1), p = pos & 3;
    const bool on = (pos >> 2) < nsb;
    const int half = lane >> 5;
    Limbs xl[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const float *xr = a.X + (size_t)prow[t] * a.D + 256 * sb + 64 * p;
        float xs[4];
#pragma unroll
        for (int g = 0; g < 4; g++) {  // group by group: 16 values live at a time
            float v[16];
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                const float4 f = ldg16f(xr + 16 * g + i);
                v[i] = f.x; v[i + 1] = f.y; v[i + 2] = f.z; v[i + 3] = f.w;
            }
            limbs16(v, xl[t].a[g], xl[t].b[g], xl[t].sp[g], xs[g]);
        }
        xl[t].xs_lo = xs[0] + xs[1];
        xl[t].xs_hi = xs[2] + xs[3];
    }
    auto blk_of = [&](int c) {
        const int col = n0 + 16 * wave + c;
        return ((size_t)e * 2 * F + (half ? F + col : col)) * nsb + sb;
    };
    WinW w[16];
#pragma unroll
    for (int c = 0; c < 2; c++) w[c] = load_window(a.gu_hdr, a.gu_qs, blk_of(c), p);
    float *rw = red + wave * (16 * NT * 64);
#pragma unroll
    for (int c = 0; c < 16; c++) {
        if (c + 2 < 16) w[c + 2] = load_window(a.gu_hdr, a.gu_qs, blk_of(c + 2), p);
#pragma unroll
        for (int t = 0; t < NT; t++) rw[(c * NT + t) * 64 + lane] = on ? window_dot(w[c], p, xl[t]) : 0.0f;
    }
    __syncthreads();
    const int c = lane & 15, t = (lane >> 4) & 1;
    float v = 0.0f;
    if (t < NT) {
        const float *src = rw + (c * NT + t) * 64 + 32 * half;
#pragma unroll
        for (int q = 0; q < 32; q++) v += src[q];
    }
    const float up = __shfl(v, lane + 32, 64);  // (lanes 0-31: the up row's sum)
    uint32_t sat = 0;
    if (!half && t < NT) {
        // H = act(gate) * up / r^2 (r = 2^k exactly)
        const float r = a.rs[prow[t]];
        const float ri = __builtin_amdgcn_ldexpf(1.0f, 1 - __builtin_amdgcn_frexp_expf(r));
        const float h = prefill_act<ACT>(v) * up * ri * ri;
        const bool big = fabsf(h) > 65504.0f && fabsf(h) <= 3.4e38f;
        sat = big ? 1u : 0u;
        a.H[(size_t)(row0 + t) * Kd + kperm(n0 + 16 * wave + c)] = (_Float16)(big ? copysignf(65504.0f, h) : h);
    }
    return sat;
}

// Down of a chunk of NT tokens (one in use), output rows n0 + [0, 128): lanes
// l & 15 = window position (K of at most 4 super-blocks), lane >> 4 = row
// of the pass; wavefront w takes rows n0 + 32 w + 4 c + (lane >> 4), pass
// c < 8.  The activations are the H rows (f16, K in kperm order).  Lane
// c + 8 rr + 32 t then sums the 16 positions of (pass c, row rr, token t).
template <int NT, typename Wait>
__device__ __forceinline__ void down_tiny(const PfArgs &a, float *red, int e, int row0, int n0, Wait wait, int wave,
                                          int lane) {
    const int nsb = a.dn_nsb, D = a.D, Kd = a.Kd;
    const int pos = lane & 15, sb = min(pos >> 2, nsb - 1), p = pos & 3;
    const bool on = (pos >> 2) < nsb;
    const int rr = lane >> 4;
    auto blk_of = [&](int c) { return ((size_t)e * D + n0 + 32 * wave + 4 * c + rr) * nsb + sb; };
    WinW w[8];
#pragma unroll
    for (int c = 0; c < 2; c++) w[c] = load_window(a.dn_hdr, a.dn_qs, blk_of(c), p);
    wait();
    Limbs xl[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const _Float16 *hr = a.H + (size_t)(row0 + t) * Kd + 256 * sb + 64 * p;
        float xs[4];
#pragma unroll
        for (int g = 0; g < 4; g++) {  // group by group: 16 values live at a time
            float v[16];
#pragma unroll
            for (int i = 0; i < 16; i += 8) {
                const uint4 u = *reinterpret_cast<const uint4 *>(hr + 16 * g + i);  // h[kperm(.. + j)], j < 8
                const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
                _Float16 f[8];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    f[2 * j] = __builtin_bit_cast(_Float16, (uint16_t)(wd[j] & 0xffffu));
                    f[2 * j + 1] = __builtin_bit_cast(_Float16, (uint16_t)(wd[j] >> 16));
                }
#pragma unroll
                for (int j = 0; j < 8; j++) v[i + kperm(j)] = (float)f[j];
            }
            limbs16(v, xl[t].a[g], xl[t].b[g], xl[t].sp[g], xs[g]);
        }
        xl[t].xs_lo = xs[0] + xs[1];
        xl[t].xs_hi = xs[2] + xs[3];
    }
    float *rw = red + wave * (8 * NT * 64);
#pragma unroll
    for (int c = 0; c < 8; c++) {
        if (c + 2 < 8) w[c + 2] = load_window(a.dn_hdr, a.dn_qs, blk_of(c + 2), p);
#pragma unroll
        for (int t = 0; t < NT; t++) rw[(c * NT + t) * 64 + lane] = on ? window_dot(w[c], p, xl[t]) : 0.0f;
    }
    __syncthreads();
    const int c = lane & 7, r4 = (lane >> 3) & 3, t = lane >> 5;
    if (t < NT) {
        const float *src = rw + (c * NT + t) * 64 + 16 * r4;
        float v = 0.0f;
#pragma unroll
        for (int q = 0; q < 16; q++) v += src[q];
        a.Y[(size_t)(row0 + t) * D + n0 + 32 * wave + 4 * c + r4] = v;
    }
}

// Block: chunk (expert e, sorted rows base + m0 + [0, mc)) x output columns
// [n0, n0 + 64).  Weight rows 0..63 are gate rows n0.., 64..127 the up rows;
// wavefront w computes token tile w against all 128 (ct 0,1 = gate, 2,3 =
// up), so h = act(gate) * up is formed in registers.  ACT: the activation
// (0 SiLU, 1 GELU-tanh).  False when the chunk does not exist.
template <int ACT>
__device__ __forceinline__ bool gate_up_body(const PfArgs &a, int bx, int by, _Float16 (*Bs)[NB][LDK]) {
    if (by >= *a.n_chunks) return false;
    const int e = a.chunks[3 * by], m0 = a.chunks[3 * by + 1], mc = a.chunks[3 * by + 2];
    const int base = a.offsets[e];
    const int n0 = bx * BN1, F = a.F, D = a.D, Kd = a.Kd;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    size_t wrow[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int r = (tid >> 2) + 64 * j;
        wrow[j] = (size_t)e * 2 * F + (r < BN1 ? n0 + r : F + n0 + (r - BN1));
    }
    const int *prow = a.perm + base + m0;
    const _Float16 *Xh = a.Xh;
    const float *rs = a.rs;
    _Float16 *H = a.H;
    auto row_ptr = [&](int m) { return Xh + (size_t)prow[m] * D; };
    // ct 0, 1 = gate columns n0 + [0, 64), ct 2, 3 = the matching up columns;
    // with r the row's scale, gate = r v[0] and up = r v[2], and H = act(gate)
    // * up / r^2 = act(r v[0]) * (v[2] / r) (exact scalings) is stored in
    // kperm order (the down GEMM's K); a finite value past f16's range
    // saturates at +-65504 and is counted (inf and NaN pass through)
    uint32_t sat = 0;
    auto sat16 = [&](float h) {  // (no branch: a select and a count)
        const bool big = fabsf(h) > 65504.0f && fabsf(h) <= 3.4e38f;
        sat += big ? 1u : 0u;
        return (_Float16)(big ? copysignf(65504.0f, h) : h);
    };
    auto pre = [&](int t, int i) {  // the row's scale (rows past the chunk: row 0's)
        const int m = 32 * t + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
        return rs[prow[m < mc ? m : 0]];
    };
    auto epi = [&](int t, int i, const float (&v)[4], float r) {
        const int m = 32 * t + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
        if (m < mc) {
            // r = 2^k exactly: frexp gives k + 1, so 1 / r = 2^(1 - (k + 1))
            const float ri = __builtin_amdgcn_ldexpf(1.0f, 1 - __builtin_amdgcn_frexp_expf(r));
            _Float16 *hrow = H + (size_t)(base + m0 + m) * Kd;
            const int c0 = n0 + (lane & 31);
            hrow[kperm(c0)] = sat16(prefill_act<ACT>(v[0] * r) * (v[2] * ri));
            hrow[kperm(c0 + 32)] = sat16(prefill_act<ACT>(v[1] * r) * (v[3] * ri));
        }
    };
    const int nt = (mc + 31) / 32, NS = 2 * a.gu_nsb;
    float *red = reinterpret_cast<float *>(&Bs[0][0][0]);
    if (a.tiny && mc == 1)
        sat = gate_up_tiny<ACT, 1>(a, red, prow, e, base + m0, n0, wave, lane);
    else if (nt == 1)
        run_block<4>(Bs, a.gu_hdr, a.gu_qs, a.gu_nsb, wrow, NS, mc, row_ptr, pre, epi, NoWait{}, tid, wave, lane);
    else if (nt == 2)
        run_block<2>(Bs, a.gu_hdr, a.gu_qs, a.gu_nsb, wrow, NS, mc, row_ptr, pre, epi, NoWait{}, tid, wave, lane);
    else
        run_block<1>(Bs, a.gu_hdr, a.gu_qs, a.gu_nsb, wrow, NS, mc, row_ptr, pre, epi, NoWait{}, tid, wave, lane);
    if (sat) {  // (rare): the count and the error bit, reported at the next synchronising call
        __hip_atomic_fetch_add(a.err + kErrPrefillSat, sat, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        report_timeout(a.err, kErrCodePrefillSat);
    }
    if (bx == 0 && Kd > F)  // zero K padding of the down product
        for (int i = tid; i < mc * (Kd - F); i += 256) {
            const int m = i / (Kd - F), col = F + i % (Kd - F);
            H[(size_t)(base + m0 + m) * Kd + col] = (_Float16)0.f;  // (kperm keeps [F, Kd): F % 4 == 0)
        }
    return true;
}

// Block: chunk x output rows [n0, n0 + 128) of the expert's down matrix
// (= columns of Y); wavefront w computes token tile w, A = H rows (f16).
template <typename Wait>
__device__ __forceinline__ void down_body(const PfArgs &a, int bx, int by, _Float16 (*Bs)[NB][LDK], Wait wait) {
    const int e = a.chunks[3 * by], m0 = a.chunks[3 * by + 1], mc = a.chunks[3 * by + 2];
    const int base = a.offsets[e];
    const int n0 = bx * BN2, D = a.D, Kd = a.Kd;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    size_t wrow[2];
#pragma unroll
    for (int j = 0; j < 2; j++) wrow[j] = (size_t)e * D + n0 + (tid >> 2) + 64 * j;
    const _Float16 *hbase = a.H + (size_t)(base + m0) * Kd;
    float *Y = a.Y;
    auto row_ptr = [&](int m) { return hbase + (size_t)m * Kd; };
    auto pre = [](int, int) { return 0.0f; };
    auto epi = [&](int t, int i, const float (&v)[4], float) {
        const int m = 32 * t + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
        if (m < mc) {
            float *yrow = Y + (size_t)(base + m0 + m) * D + n0 + (lane & 31);
#pragma unroll
            for (int ct = 0; ct < 4; ct++) yrow[32 * ct] = v[ct];
        }
    };
    const int nt = (mc + 31) / 32, NS = 2 * a.dn_nsb;
    float *red = reinterpret_cast<float *>(&Bs[0][0][0]);
    if (a.tiny && mc == 1)
        down_tiny<1>(a, red, e, base + m0, n0, wait, wave, lane);
    else if (nt == 1)
        run_block<4>(Bs, a.dn_hdr, a.dn_qs, a.dn_nsb, wrow, NS, mc, row_ptr, pre, epi, wait, tid, wave, lane);
    else if (nt == 2)
        run_block<2>(Bs, a.dn_hdr, a.dn_qs, a.dn_nsb, wrow, NS, mc, row_ptr, pre, epi, wait, tid, wave, lane);
    else
        run_block<1>(Bs, a.dn_hdr, a.dn_qs, a.dn_nsb, wrow, NS, mc, row_ptr, pre, epi, wait, tid, wave, lane);
}

constexpr uint64_t kPfWaitTicks = 20000000;  // 200 ms of the 100 MHz wall clock

}  // namespace

template <int ACT>
__global__ void __launch_bounds__(256, 2) k_prefill_gate_up(PfArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 Bs[2][NB][LDK];
    gate_up_body<ACT>(a, blockIdx.x, blockIdx.y, Bs);
}

// ---------------------------------------------------------------- down
__global__ void __launch_bounds__(256, 2) k_prefill_down(PfArgs a) {
    if ((int)blockIdx.y >= *a.n_chunks) return;
    __shared__ __attribute__((aligned(16))) _Float16 Bs[2][NB][LDK];
    down_body(a, blockIdx.x, blockIdx.y, Bs, NoWait{});
}

// ---------------------------------------------------------------- both GEMMs in one launch
// Block b of XCD group g = b % 8 (blocks with equal b % 8 share an XCD, as
// probed once per context), in-group index s = b / 8: the first
// (F / 64) CG indices are the gate/up blocks of the group's chunks
// y = g + 8c (c = s / (F / 64), column block s % (F / 64)), the next
// (D / 128) CG the down blocks of the same chunks, in the same chunk order.
// A gate/up block's H rows are ordinary stores that stay in its XCD's L2;
// once they are acknowledged it adds 1 to done[y].  A down block requests
// its first weight stages, then waits until done[y] = F / 64 and reads H
// through the same L2.  So the down blocks of the first chunks run while
// the last gate/up blocks finish, instead of behind the whole gate/up grid.
// A down block only waits for blocks with smaller indices, which are
// dispatched first; the wait is bounded by the wall clock (on expiry the
// error word is set and that call's outputs are wrong).
template <int ACT>
__global__ void __launch_bounds__(256, 2) k_prefill_gemms(PfArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 Bs[2][NB][LDK];
    const int g = blockIdx.x & 7, s = blockIdx.x >> 3;
    const int ngx = a.F / BN1, ngu = ngx * a.CG;
    if (s < ngu) {
        const int y = g + 8 * (s / ngx);
        if (!gate_up_body<ACT>(a, s % ngx, y, Bs)) return;
        // every thread's H stores acknowledged by the L2 before the count
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (threadIdx.x == 0) __hip_atomic_fetch_add(a.done + y, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    const int ndx = a.D / BN2, s2 = s - ngu;
    const int y = g + 8 * (s2 / ndx);
    if (y >= *a.n_chunks) return;
    auto wait = [&] {
        if (threadIdx.x == 0) {
            const uint64_t t0 = wall_clock64();
            int seen;
            while ((seen = __hip_atomic_load(a.done + y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) < ngx) {
                if (wall_clock64() - t0 > kPfWaitTicks) {
                    report_timeout(a.err, kErrCodePrefillWait);
                    report_detail(a.err, (int)blockIdx.x, kErrCodePrefillWait, (uint32_t)y, (uint32_t)seen,
                                  (uint32_t)ngx);
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
        }
        __syncthreads();
    };
    down_body(a, s2 % ndx, y, Bs, wait);
}

// ---------------------------------------------------------------- combine
// Thread: 4 consecutive elements of one token's row (D % 4 == 0); every
// slot's Y row is read with one 16-byte load per thread, all k loads in
// flight before the sum, which runs in slot order; the sum times r_t^2
// (the row scale the activations were divided by, exact).
__global__ void __launch_bounds__(256) k_prefill_combine(const float *__restrict__ Y, const int *__restrict__ pos,
                                                         const float *__restrict__ w, const float *__restrict__ rs,
                                                         int k, int D, float *__restrict__ out) {
    const int t = blockIdx.y, i = 4 * (blockIdx.x * 256 + threadIdx.x);
    if (i >= D) return;
    float4 v[16];
    float ws[16];
#pragma unroll
    for (int s = 0; s < 16; s++) {
        if (s < k) {
            const int p = pos[t * k + s];
            ws[s] = p >= 0 ? w[t * k + s] : 0.0f;
            v[s] = ldg16f(Y + (size_t)(p >= 0 ? p : 0) * D + i);
        }
    }
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int s = 0; s < 16; s++) {
        if (s < k && pos[t * k + s] >= 0) {
            acc.x += ws[s] * v[s].x;
            acc.y += ws[s] * v[s].y;
            acc.z += ws[s] * v[s].z;
            acc.w += ws[s] * v[s].w;
        }
    }
    const float r2 = rs[t] * rs[t];
    acc.x *= r2;
    acc.y *= r2;
    acc.z *= r2;
    acc.w *= r2;
    *reinterpret_cast<float4 *>(out + (size_t)t * D + i) = acc;
}

size_t prefill_workspace_bytes(int T, int k, int E, int Kd, int D) {
    const size_t TK = (size_t)T * k;
    return align256((size_t)T * E * 4) + 2 * align256(TK * 4) + align256((size_t)(E + 1) * 4) +
           align256((size_t)max_chunks((int)TK, E) * 12) + 256 + 2 * align256(TK * 4) + align256((size_t)T * 4) +
           align256((size_t)T * D * 2) + align256(TK * Kd * 2) + align256(TK * D * 4) +
           align256((size_t)max_chunks((int)TK, E) * 4);
}

hipError_t launch_moe_prefill(const DevTensor &R, const DevTensor &GU, const DevTensor &Dn, const float *X, int T,
                              const float *bias, int k, int F, uint32_t act, uint32_t norm, void *ws, float *out,
                              uint32_t *out_ids, float *out_w, uint32_t *err, int xcd_local, hipStream_t s) {
    const int E = (int)GU.n_experts, D = (int)GU.cols, Kd = (int)Dn.cols;
    const int TK = T * k;
    Ws w = carve(ws, T, k, E, Kd, D);
    bool x_done = false;
    hipError_t e = launch_router_batched(R, X, T, bias, w.logits, k, norm, w.ids, w.w, w.Xh, w.rs, &x_done, s);
    if (e != hipSuccess) return e;
    const int mc = max_chunks(TK, E);
    hipLaunchKernelGGL(k_prefill_dispatch, dim3(1), dim3(1024), 0, s, w.ids, TK, k, E, w.offsets, w.chunks,
                       w.n_chunks, w.perm, w.pos, w.done, mc);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (!x_done) {
        hipLaunchKernelGGL(k_prefill_x_f16, dim3((unsigned)T), dim3(256), 0, s, X, w.Xh, w.rs, D);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    PfArgs pa{};
    pa.gu_hdr = (const uint8_t *)GU.p0;
    pa.gu_qs = (const uint8_t *)GU.p1;
    pa.gu_nsb = (int)GU.blocks_per_row;
    pa.F = F;
    pa.Xh = w.Xh;
    pa.rs = w.rs;
    pa.D = D;
    pa.chunks = w.chunks;
    pa.n_chunks = w.n_chunks;
    pa.offsets = w.offsets;
    pa.perm = w.perm;
    pa.H = w.H;
    pa.Kd = Kd;
    pa.dn_hdr = (const uint8_t *)Dn.p0;
    pa.dn_qs = (const uint8_t *)Dn.p1;
    pa.dn_nsb = (int)Dn.blocks_per_row;
    pa.Y = w.Y;
    pa.err = err;
    pa.done = w.done;
    pa.CG = (mc + 7) / 8;
    pa.X = X;
    // (LT_PREFILL_NO_TINY, read at each call: every chunk on the tiles, for testing)
    pa.tiny = GU.blocks_per_row <= 8 && Dn.blocks_per_row <= 4 && !getenv("LT_PREFILL_NO_TINY");
    if (xcd_local) {
        const unsigned nb = 8u * (unsigned)((F / BN1 + D / BN2) * pa.CG);
        hipLaunchKernelGGL(act == 1u ? k_prefill_gemms<1> : k_prefill_gemms<0>, dim3(nb), dim3(256), 0, s, pa);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    } else {
        hipLaunchKernelGGL(act == 1u ? k_prefill_gate_up<1> : k_prefill_gate_up<0>, dim3(F / BN1, mc), dim3(256), 0,
                           s, pa);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        hipLaunchKernelGGL(k_prefill_down, dim3(D / BN2, mc), dim3(256), 0, s, pa);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k_prefill_combine, dim3((D / 4 + 255) / 256, T), dim3(256), 0, s, w.Y, w.pos, w.w, w.rs, k, D,
                       out);
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
