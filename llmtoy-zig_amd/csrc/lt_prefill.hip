// lt_prefill.hip -- batched prefill of one MoE layer (Q4_K experts) on MFMA.
//
// The reference prefills one token at a time through the decode path
// (main.zig:1916-1922).  Here T tokens go through the layer together:
//   1. router logits for all tokens with the reference's exact dotf32 order
//      and per-token softmax / top-k (lt_router.hip);
//   2. dispatch: one block counts tokens per expert, lays out per-expert
//      row ranges ("sorted rows"), cuts each range into chunks of at most
//      MC = 128 rows, and scatters (token, slot) assignments into them;
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
// Both GEMMs run a software pipeline over K stages of 128 (half a Q4_K
// super-block): weight loads are issued two stages ahead into registers,
// A fragments one stage ahead, the dequantised tile is double-buffered in
// LDS, and each stage ends in one barrier.
// A row's result does not depend on which chunk position it lands in, so
// the atomically assigned positions leave the output bit-identical run to
// run.
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
template <int S>
__device__ __forceinline__ void grouped_gemm(floatx16 (&acc)[4], _Float16 (*Bs)[NB][LDK], const uint8_t *hdr,
                                             const uint8_t *qs, int nsb, const size_t (&wrow)[2], int NS,
                                             const _Float16 *arow, bool wave_on, int kb, int tid, int lane) {
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
template <int S, typename Row, typename Pre, typename Epi>
__device__ __forceinline__ void run_block(_Float16 (*Bs)[NB][LDK], const uint8_t *hdr, const uint8_t *qs, int nsb,
                                          const size_t (&wrow)[2], int NS, int mc, Row row_ptr, Pre pre, Epi epi,
                                          int tid, int wave, int lane) {
    constexpr int NT = 4 / S;  // token tiles handled side by side
    const int t = wave % NT, q = wave / NT;
    const int mrow = 32 * t + (lane & 31);
    const bool wave_on = 32 * t < mc;
    const _Float16 *arow = row_ptr(mrow < mc ? mrow : 0) + (lane >> 5) * 8;
    floatx16 acc[4];
    grouped_gemm<S>(acc, Bs, hdr, qs, nsb, wrow, NS, arow, wave_on, q * (8 / S), tid, lane);
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
    // Up to kIdsPer ids per thread are loaded once, all in flight together,
    // and kept for the scatter; longer batches read them again.
    constexpr int kIdsPer = 8;
    __shared__ int cnt[1024], cur[1024];
    __shared__ int scan[2][6][1024];
    const int e = threadIdx.x;
    const bool cached = TK <= kIdsPer * (int)blockDim.x;
    uint32_t xc[kIdsPer];
#pragma unroll
    for (int j = 0; j < kIdsPer; j++) {
        const int i = threadIdx.x + j * blockDim.x;
        xc[j] = cached && i < TK ? ids[i] : 0xffffffffu;
    }
    if (e < E) cnt[e] = 0;
    __syncthreads();
    if (cached) {
#pragma unroll
        for (int j = 0; j < kIdsPer; j++)
            if (xc[j] < (uint32_t)E) atomicAdd(&cnt[xc[j]], 1);
    } else {
        for (int i = threadIdx.x; i < TK; i += blockDim.x) {
            const uint32_t x = ids[i];
            if (x < (uint32_t)E) atomicAdd(&cnt[x], 1);
        }
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
    auto place = [&](int i, uint32_t x) {
        if (x < (uint32_t)E) {
            const int p = atomicAdd(&cur[x], 1);
            perm[p] = i / k;
            pos[i] = p;
        } else {
            pos[i] = -1;
        }
    };
    if (cached) {
#pragma unroll
        for (int j = 0; j < kIdsPer; j++) {
            const int i = threadIdx.x + j * blockDim.x;
            if (i < TK) place(i, xc[j]);
        }
    } else {
        for (int i = threadIdx.x; i < TK; i += blockDim.x) place(i, ids[i]);
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

// Block: chunk (expert e, sorted rows base + m0 + [0, mc)) x output columns
// [n0, n0 + 64).  Weight rows 0..63 are gate rows n0.., 64..127 the up rows;
// wavefront w computes token tile w against all 128 (ct 0,1 = gate, 2,3 =
// up), so h = act(gate) * up is formed in registers.  ACT: the activation
// (0 SiLU, 1 GELU-tanh).
template <int ACT>
__global__ void __launch_bounds__(256) k_prefill_gate_up(const uint8_t *__restrict__ hdr,
                                                         const uint8_t *__restrict__ qs, int nsb, int F,
                                                         const _Float16 *__restrict__ Xh,
                                                         const float *__restrict__ rs, int D,
                                                         const int *__restrict__ chunks,
                                                         const int *__restrict__ n_chunks,
                                                         const int *__restrict__ offsets,
                                                         const int *__restrict__ perm, uint32_t act,
                                                         _Float16 *__restrict__ H, int Kd, uint32_t *err) {
    if ((int)blockIdx.y >= *n_chunks) return;
    const int e = chunks[3 * blockIdx.y], m0 = chunks[3 * blockIdx.y + 1], mc = chunks[3 * blockIdx.y + 2];
    const int base = offsets[e];
    const int n0 = blockIdx.x * BN1;
    __shared__ __attribute__((aligned(16))) _Float16 Bs[2][NB][LDK];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    size_t wrow[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int r = (tid >> 2) + 64 * j;
        wrow[j] = (size_t)e * 2 * F + (r < BN1 ? n0 + r : F + n0 + (r - BN1));
    }
    const int *prow = perm + base + m0;
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
    const int nt = (mc + 31) / 32, NS = 2 * nsb;
    if (nt == 1)
        run_block<4>(Bs, hdr, qs, nsb, wrow, NS, mc, row_ptr, pre, epi, tid, wave, lane);
    else if (nt == 2)
        run_block<2>(Bs, hdr, qs, nsb, wrow, NS, mc, row_ptr, pre, epi, tid, wave, lane);
    else
        run_block<1>(Bs, hdr, qs, nsb, wrow, NS, mc, row_ptr, pre, epi, tid, wave, lane);
    if (sat) {  // (rare): the count and the error bit, reported at the next synchronising call
        __hip_atomic_fetch_add(err + kErrPrefillSat, sat, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        report_timeout(err, kErrCodePrefillSat);
    }
    if (blockIdx.x == 0 && Kd > F)  // zero K padding of the down product
        for (int i = tid; i < mc * (Kd - F); i += 256) {
            const int m = i / (Kd - F), col = F + i % (Kd - F);
            H[(size_t)(base + m0 + m) * Kd + col] = (_Float16)0.f;  // (kperm keeps [F, Kd): F % 4 == 0)
        }
}

// ---------------------------------------------------------------- down
// Block: chunk x output rows [n0, n0 + 128) of the expert's down matrix
// (= columns of Y); wavefront w computes token tile w, A = H rows (f16).
__global__ void __launch_bounds__(256) k_prefill_down(const uint8_t *__restrict__ hdr, const uint8_t *__restrict__ qs,
                                                      int nsb, int D, const _Float16 *__restrict__ H, int Kd,
                                                      const int *__restrict__ chunks, const int *__restrict__ n_chunks,
                                                      const int *__restrict__ offsets, float *__restrict__ Y) {
    if ((int)blockIdx.y >= *n_chunks) return;
    const int e = chunks[3 * blockIdx.y], m0 = chunks[3 * blockIdx.y + 1], mc = chunks[3 * blockIdx.y + 2];
    const int base = offsets[e];
    const int n0 = blockIdx.x * BN2;
    __shared__ __attribute__((aligned(16))) _Float16 Bs[2][NB][LDK];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    size_t wrow[2];
#pragma unroll
    for (int j = 0; j < 2; j++) wrow[j] = (size_t)e * D + n0 + (tid >> 2) + 64 * j;
    const _Float16 *hbase = H + (size_t)(base + m0) * Kd;
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
    const int nt = (mc + 31) / 32, NS = 2 * nsb;
    if (nt == 1)
        run_block<4>(Bs, hdr, qs, nsb, wrow, NS, mc, row_ptr, pre, epi, tid, wave, lane);
    else if (nt == 2)
        run_block<2>(Bs, hdr, qs, nsb, wrow, NS, mc, row_ptr, pre, epi, tid, wave, lane);
    else
        run_block<1>(Bs, hdr, qs, nsb, wrow, NS, mc, row_ptr, pre, epi, tid, wave, lane);
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
           align256((size_t)T * D * 2) + align256(TK * Kd * 2) + align256(TK * D * 4);
}

hipError_t launch_moe_prefill(const DevTensor &R, const DevTensor &GU, const DevTensor &Dn, const float *X, int T,
                              const float *bias, int k, int F, uint32_t act, uint32_t norm, void *ws, float *out,
                              uint32_t *out_ids, float *out_w, uint32_t *err, hipStream_t s) {
    const int E = (int)GU.n_experts, D = (int)GU.cols, Kd = (int)Dn.cols;
    const int TK = T * k;
    Ws w = carve(ws, T, k, E, Kd, D);
    bool x_done = false;
    hipError_t e = launch_router_batched(R, X, T, bias, w.logits, k, norm, w.ids, w.w, w.Xh, w.rs, &x_done, s);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_prefill_dispatch, dim3(1), dim3(1024), 0, s, w.ids, TK, k, E, w.offsets, w.chunks,
                       w.n_chunks, w.perm, w.pos);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (!x_done) {
        hipLaunchKernelGGL(k_prefill_x_f16, dim3((unsigned)T), dim3(256), 0, s, X, w.Xh, w.rs, D);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    const int mc = max_chunks(TK, E);
    hipLaunchKernelGGL(act == 1u ? k_prefill_gate_up<1> : k_prefill_gate_up<0>, dim3(F / BN1, mc), dim3(256), 0, s,
                       GU.p0, GU.p1, (int)GU.blocks_per_row, F, w.Xh, w.rs, D, w.chunks, w.n_chunks, w.offsets, w.perm,
                       act, w.H, Kd, err);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(k_prefill_down, dim3(D / BN2, mc), dim3(256), 0, s, Dn.p0, Dn.p1, (int)Dn.blocks_per_row, D,
                       w.H, Kd, w.chunks, w.n_chunks, w.offsets, w.Y);
    if ((e = hipGetLastError()) != hipSuccess) return e;
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
