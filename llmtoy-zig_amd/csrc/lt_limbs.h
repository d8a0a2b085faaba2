// lt_limbs.h -- activations as two int8 limbs and the Q4_K sub-block pair
// dot product on v_dot4, shared by the single-launch MoE kernel and the
// streaming Q4_K / Q6_K matvecs.
//
// Over a group of 16 activations with m = max|x|:
//   x ~= sp * (256*a + b),  a in [-127, 127], b in [-128, 127],
//   sp = m / (127*256),     |x - sp*(256a + b)| <= m / 65024,
// so a weight byte (a 4-bit or 6-bit unsigned code) meets both limbs in
// v_dot4_i32_i8 (4 exact products per instruction, exact int32 sums) and
// the group's sum is 256*A + B (|.| < 2^23, exact in fp32) times sp.  The
// plain fp32 sum of the group rides along for the format's offset term.
#pragma once

#include "lt_internal.h"

namespace lt {

template <int CTRL>
__device__ __forceinline__ uint32_t dppw(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}

struct Limbs {
    uint32_t a[4][4];  // a[g][m]: bytes = limb a of elements 16g + 4m + 0..3
    uint32_t b[4][4];
    float sp[4];
    float xs_lo, xs_hi;  // exact sums of groups 0+1 and 2+3
};

// Q4_K scale decode of sub-block pair p (2p, 2p+1) from the header words
// (h0 = d | dmin << 16, h1..h3 = scales[0..11]): get_scale_min_k4,
// quant/dequant.zig:289-300.  Returns d*sc and dmin*mn of both sub-blocks.
struct PairScale {
    float dsc0, dsc1, dmn0, dmn1;
};

__device__ __forceinline__ PairScale pair_scale(uint32_t h0, uint32_t h1, uint32_t h2, uint32_t h3, int p) {
    const float d = f16_bits_to_f32(h0);
    const float dmin = f16_bits_to_f32(h0 >> 16);
    const int sh = (p & 1) * 16;
    const uint32_t ys = h1 >> sh, zs = h2 >> sh, ws = h3 >> sh;
    const uint32_t scp = p < 2 ? (ys & 0x3f3fu) : ((ws & 0x0f0fu) | ((ys >> 2) & 0x3030u));
    const uint32_t mnp = p < 2 ? (zs & 0x3f3fu) : (((ws >> 4) & 0x0f0fu) | ((zs >> 2) & 0x3030u));
    PairScale s;
    s.dsc0 = d * (float)(scp & 0xffu);
    s.dsc1 = d * (float)((scp >> 8) & 0xffu);
    s.dmn0 = dmin * (float)(mnp & 0xffu);
    s.dmn1 = dmin * (float)((mnp >> 8) & 0xffu);
    return s;
}

// The four header words of a (row, super-block) from the one word each lane
// of an aligned quad loaded (lane & 3 = word index).
// (quad_perm broadcasts always read a live lane, so no old value is needed:
// v_mov_b32_dpp without a zeroing move first.)
template <int CTRL>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, true);
}

__device__ __forceinline__ void quad_header(uint32_t mine, uint32_t &h0, uint32_t &h1, uint32_t &h2,
                                            uint32_t &h3) {
    h0 = quad_bcast<0x00>(mine);
    h1 = quad_bcast<0x55>(mine);
    h2 = quad_bcast<0xAA>(mine);
    h3 = quad_bcast<0xFF>(mine);
}

// Dot of one Q4_K sub-block pair (64 weights: qs bytes 32p..32p+31 of a
// super-block, w[0..7]) with the limbs of the matching 64 activations; the
// _nib form takes the nibbles already unpacked (lo[m] = w[m] & 0x0f0f0f0f,
// hi[m] = (w[m] >> 4) & 0x0f0f0f0f).
// First product of an accumulator chain: the three-operand v_dot4_i32_i8
// with an inline 0 (the compiler's choice, v_dot4c, needs a v_mov of 0
// first: 8 of the pair's ~56 VALU instructions).
__device__ __forceinline__ int sdot4_first(int a, int b) {
    int r;
    asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

__device__ __forceinline__ float q4k_pair_dot_nib(const uint32_t (&lo)[8], const uint32_t (&hi)[8], const PairScale &s,
                                                  const Limbs &x) {
    int A[4], B[4];
    A[0] = sdot4_first((int)lo[0], (int)x.a[0][0]);
    B[0] = sdot4_first((int)lo[0], (int)x.b[0][0]);
    A[1] = sdot4_first((int)lo[4], (int)x.a[1][0]);
    B[1] = sdot4_first((int)lo[4], (int)x.b[1][0]);
    A[2] = sdot4_first((int)hi[0], (int)x.a[2][0]);
    B[2] = sdot4_first((int)hi[0], (int)x.b[2][0]);
    A[3] = sdot4_first((int)hi[4], (int)x.a[3][0]);
    B[3] = sdot4_first((int)hi[4], (int)x.b[3][0]);
#pragma unroll
    for (int m = 1; m < 4; m++) {
        const uint32_t lo0 = lo[m], hi0 = hi[m];
        const uint32_t lo1 = lo[4 + m], hi1 = hi[4 + m];
        A[0] = __builtin_amdgcn_sdot4((int)lo0, (int)x.a[0][m], A[0], false);
        B[0] = __builtin_amdgcn_sdot4((int)lo0, (int)x.b[0][m], B[0], false);
        A[1] = __builtin_amdgcn_sdot4((int)lo1, (int)x.a[1][m], A[1], false);
        B[1] = __builtin_amdgcn_sdot4((int)lo1, (int)x.b[1][m], B[1], false);
        A[2] = __builtin_amdgcn_sdot4((int)hi0, (int)x.a[2][m], A[2], false);
        B[2] = __builtin_amdgcn_sdot4((int)hi0, (int)x.b[2][m], B[2], false);
        A[3] = __builtin_amdgcn_sdot4((int)hi1, (int)x.a[3][m], A[3], false);
        B[3] = __builtin_amdgcn_sdot4((int)hi1, (int)x.b[3][m], B[3], false);
    }
    float c[4];
#pragma unroll
    for (int g = 0; g < 4; g++) c[g] = (float)((A[g] << 8) + B[g]);  // |.| < 2^23: exact
    const float t_lo = x.sp[0] * c[0] + x.sp[1] * c[1];
    const float t_hi = x.sp[2] * c[2] + x.sp[3] * c[3];
    return (s.dsc0 * t_lo - s.dmn0 * x.xs_lo) + (s.dsc1 * t_hi - s.dmn1 * x.xs_hi);
}

__device__ __forceinline__ float q4k_pair_dot(const uint32_t (&w)[8], const PairScale &s, const Limbs &x) {
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int m = 0; m < 8; m++) {
        lo[m] = w[m] & 0x0f0f0f0fu;
        hi[m] = (w[m] >> 4) & 0x0f0f0f0fu;
    }
    return q4k_pair_dot_nib(lo, hi, s, x);
}

// Limbs of 16 activations v[0..16): a[m] / b[m] hold elements 4m + 0..3 in
// bytes 0..3; xs is their fp32 sum (pairwise order).  A group holding a
// NaN or an infinity gets sp = NaN, so every product that uses it is NaN.
// A group whose largest magnitude is below 2^-100 is scaled by 2^100
// before the division so that 127 / m stays finite.
__device__ __forceinline__ void limbs16(const float (&v)[16], uint32_t (&a)[4], uint32_t (&b)[4], float &sp,
                                        float &xs) {
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) m = fmaxf(m, fabsf(v[i]));
    const float h0 = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    const float h1 = ((v[8] + v[9]) + (v[10] + v[11])) + ((v[12] + v[13]) + (v[14] + v[15]));
    xs = h0 + h1;
    const bool tiny = m < 0x1p-100f;
    const float ms = tiny ? m * 0x1p100f : m;
    const float inv = ms > 0.0f ? 127.0f / ms : 0.0f;
    sp = m * (1.0f / 32512.0f);
    if (!(fabsf(xs) <= 3.0e38f) || !(m <= 3.0e38f)) sp = __int_as_float(0x7fc00000);
#pragma unroll
    for (int w = 0; w < 4; w++) {
        uint32_t pa = 0u, pb = 0u;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float t = (tiny ? v[4 * w + i] * 0x1p100f : v[4 * w + i]) * inv;
            const float fa = rintf(t);
            const float fb = fminf(rintf((t - fa) * 256.0f), 127.0f);
            pa |= ((uint32_t)(int)fa & 0xffu) << (8 * i);
            pb |= ((uint32_t)(int)fb & 0xffu) << (8 * i);
        }
        a[w] = pa;
        b[w] = pb;
    }
}

// Block-wide conversion of x[0..n) (n % 16 == 0, n <= 16 * blockDim.x) to
// limbs in LDS, in two halves so that a kernel can issue its weight loads
// between them and the conversion overlaps those loads (the wait for x
// then does not include them: loads complete in issue order).
// stage_x_load: thread t loads group t (16 activations).
// stage_limbs_store: thread t converts it into la / lb [n / 4] words (word
// i: elements 4i..4i+3) and lsp / lxs [n / 16] (group scale and fp32 sum),
// then a barrier.  Threads past the last group take the last group (the
// same values stored twice): no branch, which would let the compiler sink
// the x loads into it, behind the weight loads.  One group per thread
// instead of each lane converting the 64 activations it uses: a quarter of
// the work per wavefront at n = 4096.
__device__ __forceinline__ int stage_group(int n) {
    return (int)threadIdx.x < n / 16 ? (int)threadIdx.x : n / 16 - 1;
}

__device__ __forceinline__ void stage_x_load(const float *__restrict__ x, int n, float (&v)[16]) {
    const int g = stage_group(n);
#pragma unroll
    for (int t = 0; t < 16; t += 4) {
        const float4 f = ldg16f(x + 16 * g + t);
        v[t] = f.x; v[t + 1] = f.y; v[t + 2] = f.z; v[t + 3] = f.w;
    }
}

__device__ __forceinline__ void stage_limbs_store(const float (&v)[16], int n, uint32_t *la, uint32_t *lb, float *lsp,
                                                  float *lxs) {
    const int g = stage_group(n);
    uint32_t a[4], b[4];
    float sp, xs;
    limbs16(v, a, b, sp, xs);
    *reinterpret_cast<uint4 *>(la + 4 * g) = make_uint4(a[0], a[1], a[2], a[3]);
    *reinterpret_cast<uint4 *>(lb + 4 * g) = make_uint4(b[0], b[1], b[2], b[3]);
    lsp[g] = sp;
    lxs[g] = xs;
    __syncthreads();
}

// The limbs of one group (index g) from stage_limbs_store's arrays.
__device__ __forceinline__ void read_group_limbs(const uint32_t *la, const uint32_t *lb, int g, uint32_t (&a)[4],
                                                 uint32_t (&b)[4]) {
    const uint4 va = *reinterpret_cast<const uint4 *>(la + 4 * g);
    const uint4 vb = *reinterpret_cast<const uint4 *>(lb + 4 * g);
    a[0] = va.x; a[1] = va.y; a[2] = va.z; a[3] = va.w;
    b[0] = vb.x; b[1] = vb.y; b[2] = vb.z; b[3] = vb.w;
}

// A Q4_K sub-block pair's Limbs (groups g0..g0+3, g0 % 4 == 0) from
// stage_limbs_store's arrays.
__device__ __forceinline__ void read_pair_limbs(const uint32_t *la, const uint32_t *lb, const float *lsp,
                                                const float *lxs, int g0, Limbs &xl) {
#pragma unroll
    for (int g = 0; g < 4; g++) read_group_limbs(la, lb, g0 + g, xl.a[g], xl.b[g]);
    const float4 sp4 = *reinterpret_cast<const float4 *>(lsp + g0);
    const float4 xs4 = *reinterpret_cast<const float4 *>(lxs + g0);
    xl.sp[0] = sp4.x; xl.sp[1] = sp4.y; xl.sp[2] = sp4.z; xl.sp[3] = sp4.w;
    xl.xs_lo = xs4.x + xs4.y;
    xl.xs_hi = xs4.z + xs4.w;
}

}  // namespace lt
