// lt_fmt.h -- the 32-element work units of the APEX expert formats (Q5_0,
// Q5_1, IQ4_NL blocks; Q3_K super-block groups) against activations held as
// two int8 limbs per 16-element group (lt_limbs.h), shared by the format
// matvecs (lt_formats.hip) and the single-launch MoE kernel's format roles
// (lt_moe_fused.hip).  The plane layouts are lt_formats.hip's (its header
// comment): Q5_0 / Q5_1 / IQ4_NL qs [R][nb][16], then qh [R][nb][4] and d or
// dm; Q3_K qs [R][nsb][64], hmask [R][nsb][32], scales [R][nsb][12], d
// [R][nsb].
#pragma once

#include "llmtoy_hip.h"
#include "lt_internal.h"
#include "lt_limbs.h"

namespace lt {

// Limbs of n activations: la [n / 4], lb [n / 4] (word i: elements
// 4i..4i+3), then per 16-element group its scale lsp [n / 16] and fp32 sum
// lxs [n / 16].

struct LimbView {
    const uint32_t *la, *lb;
    const float *lsp, *lxs;
};

__device__ __forceinline__ LimbView limb_view(const uint32_t *base, int n) {
    return LimbView{base, base + n / 4, reinterpret_cast<const float *>(base + n / 2),
                    reinterpret_cast<const float *>(base + n / 2 + n / 16)};
}

// The activations of one 32-element unit: groups 0 (elements 0..15) and 1.
struct UnitX {
    uint32_t a[8], b[8];  // a[4g + m]: limb a of elements 16g + 4m + 0..3
    float sp[2], xs[2];
};

__device__ __forceinline__ UnitX load_ux(const LimbView &v, int u) {
    UnitX x;
    const uint4 *pa = reinterpret_cast<const uint4 *>(v.la + 8 * u);
    const uint4 *pb = reinterpret_cast<const uint4 *>(v.lb + 8 * u);
#pragma unroll
    for (int g = 0; g < 2; g++) {
        const uint4 qa = pa[g], qb = pb[g];
        x.a[4 * g] = qa.x; x.a[4 * g + 1] = qa.y; x.a[4 * g + 2] = qa.z; x.a[4 * g + 3] = qa.w;
        x.b[4 * g] = qb.x; x.b[4 * g + 1] = qb.y; x.b[4 * g + 2] = qb.z; x.b[4 * g + 3] = qb.w;
    }
    const float2 sp = *reinterpret_cast<const float2 *>(v.lsp + 2 * u);
    const float2 xs = *reinterpret_cast<const float2 *>(v.lxs + 2 * u);
    x.sp[0] = sp.x; x.sp[1] = sp.y;
    x.xs[0] = xs.x; x.xs[1] = xs.y;
    return x;
}

// Sum over group g of code * x for 16 codes (signed bytes, words c[0..3]):
// sp (256 A + B) with A, B the exact int32 dots against the two limbs
// (|256 A + B| < 2^27 for codes of magnitude <= 127, one fp32 rounding).
__device__ __forceinline__ float group_dot(const uint32_t (&c)[4], const UnitX &x, int g) {
    int A = sdot4_first((int)c[0], (int)x.a[4 * g]);
    int B = sdot4_first((int)c[0], (int)x.b[4 * g]);
#pragma unroll
    for (int m = 1; m < 4; m++) {
        A = __builtin_amdgcn_sdot4((int)c[m], (int)x.a[4 * g + m], A, false);
        B = __builtin_amdgcn_sdot4((int)c[m], (int)x.b[4 * g + m], B, false);
    }
    return x.sp[g] * (float)((A << 8) + B);
}

// Unsigned 5-bit codes of a Q5 block as bytes: word i of the result holds
// elements 4i..4i+3 (low nibbles of qs word i + high bit 4i..4i+3 of qh) and
// word 4 + i elements 16+4i..16+4i+3 (high nibbles + bits 16+4i..).  The
// four high bits of an element group spread into bits 4, 12, 20, 28 with one
// 24-bit multiply: (v * 0x204081) & 0x01010101 puts bit j of v at bit 8j,
// and no two partial products meet.
__device__ __forceinline__ uint32_t spread4(uint32_t v4) { return (__umul24(v4, 0x204081u) & 0x01010101u) << 4; }

// sum over the block of (code) * x: codes 0..31 as bytes, elements 4i..4i+3
// of the low half from qs word i's low nibbles and qh bits 4i..4i+3, of the
// high half from its high nibbles and qh bits 16+4i..
__device__ __forceinline__ float q5u_block_dot(uint4 qv, uint32_t qh, const UnitX &x) {
    const uint32_t w[4] = {qv.x, qv.y, qv.z, qv.w};
    uint32_t cl[4], ch[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        cl[i] = (w[i] & 0x0f0f0f0fu) | spread4((qh >> (4 * i)) & 15u);
        ch[i] = ((w[i] >> 4) & 0x0f0f0f0fu) | spread4((qh >> (16 + 4 * i)) & 15u);
    }
    return group_dot(cl, x, 0) + group_dot(ch, x, 1);
}

// The IQ4_NL table (quant/dequant.zig:607-612) as signed bytes: entries
// 0-3, 4-7, 8-11, 12-15.
constexpr uint32_t kIq4T0 = 0xbfad9881u, kIq4T1 = 0xf6eaddcfu, kIq4T2 = 0x26190d01u, kIq4T3 = 0x71594535u;

// table[n] for the four nibbles in the bytes of n4 (each 0..15):
// v_perm_b32 picks bytes by 3-bit index from the low and high half tables,
// bit 3 chooses between them (v_bfi_b32 on a byte mask).
__device__ __forceinline__ uint32_t iq4_lookup4(uint32_t n4) {
    const uint32_t sel = n4 & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(kIq4T1, kIq4T0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(kIq4T3, kIq4T2, sel);
    const uint32_t b3 = (n4 >> 3) & 0x01010101u;
    const uint32_t m = (b3 << 8) - b3;  // 0x00 or 0xff per byte
    return (hi & m) | (lo & ~m);
}

__device__ __forceinline__ float iq4_block_dot(uint4 qv, const UnitX &x) {
    const uint32_t w[4] = {qv.x, qv.y, qv.z, qv.w};
    uint32_t tl[4], th[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        tl[i] = iq4_lookup4(w[i] & 0x0f0f0f0fu);
        th[i] = iq4_lookup4((w[i] >> 4) & 0x0f0f0f0fu);
    }
    return group_dot(tl, x, 0) + group_dot(th, x, 1);
}

// Q3_K scale i (0..15) from the 12 packed bytes s0, s1, s2 (little-endian
// dwords): low 4 bits from byte i (i < 8) or the high nibble of byte i - 8,
// high 2 bits from bits 2 (i / 4) of byte 8 + i % 4.  The dword is picked by
// a select, not an array index, so the words stay in registers.
__device__ __forceinline__ int q3k_scale(uint32_t s0, uint32_t s1, uint32_t s2, int i) {
    const int b = i & 7;
    const uint32_t lo = (((b & 4) ? s1 : s0) >> (8 * (b & 3) + 4 * (i >> 3))) & 15u;
    const uint32_t hi = (s2 >> (8 * (i & 3) + 2 * (i >> 2))) & 3u;
    return (int)(lo | (hi << 4));
}

// Raw weight words of one unit of one row, loaded before any arithmetic so
// that a lane's loads for several rows are in flight together.
template <int T>
struct UnitW {
    uint4 q;      // qs
    uint32_t qh;  // Q5_0 / Q5_1 high bits
    uint32_t dm;  // f16 d in the low half; Q5_1: f16 m in the high half
};
template <>
struct UnitW<LT_TYPE_Q3_K> {
    uint4 q0, q1;    // qs[32 h ..], qs[32 h + 16 ..] of the unit's half h
    uint4 m0, m1;    // hmask[0 ..], hmask[16 ..]
    uint32_t sc[3];  // the 12 packed scale bytes
    uint32_t d;      // f16 d in the low half
};

// Unit u of `row`: block u, or group u (super-block u / 8, group u % 8).
template <int T>
__device__ __forceinline__ UnitW<T> load_unit(const DevTensor &W, size_t row, int u) {
    const size_t nb = W.blocks_per_row;
    UnitW<T> w;
    if constexpr (T == LT_TYPE_Q3_K) {
        const size_t sb = row * nb + (u >> 3);
        const uint8_t *qs = W.p0 + sb * 64 + 32 * ((u >> 2) & 1);
        w.q0 = *reinterpret_cast<const uint4 *>(qs);
        w.q1 = *reinterpret_cast<const uint4 *>(qs + 16);
        w.m0 = *reinterpret_cast<const uint4 *>(W.p1 + sb * 32);
        w.m1 = *reinterpret_cast<const uint4 *>(W.p1 + sb * 32 + 16);
        const uint32_t *s3 = reinterpret_cast<const uint32_t *>(W.p2 + sb * 12);
        w.sc[0] = s3[0];
        w.sc[1] = s3[1];
        w.sc[2] = s3[2];
        w.d = *reinterpret_cast<const uint16_t *>(W.p3 + sb * 2);
    } else {
        const size_t b = row * nb + u;
        w.q = *reinterpret_cast<const uint4 *>(W.p0 + b * 16);
        if constexpr (T == LT_TYPE_IQ4_NL) {
            w.qh = 0;
            w.dm = *reinterpret_cast<const uint16_t *>(W.p1 + b * 2);
        } else {
            w.qh = *reinterpret_cast<const uint32_t *>(W.p1 + b * 4);
            w.dm = T == LT_TYPE_Q5_1 ? *reinterpret_cast<const uint32_t *>(W.p2 + b * 4)
                                     : (uint32_t)*reinterpret_cast<const uint16_t *>(W.p2 + b * 2);
        }
    }
    return w;
}

// Group u % 8 = 4 h + j of a Q3_K super-block: elements 128 h + 32 j + [0, 32)
// (16 from qs[32 h ..] and hmask[0 ..], 16 from qs[32 h + 16 ..] and
// hmask[16 ..]) against x.  Each element's 3-bit unsigned code
// c = q2 | hbit << 2 (value c - 4) is built four to a dword; the -4 folds
// into the sums of the group's two 16-element halves of x, which are the
// two limb groups, each with its own scale.
__device__ __forceinline__ float q3k_group_dot(const UnitW<LT_TYPE_Q3_K> &w, int u, const UnitX &x) {
    const int h = (u >> 2) & 1, j = u & 3;
    const uint32_t qw[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
    const uint32_t mw[8] = {w.m0.x, w.m0.y, w.m0.z, w.m0.w, w.m1.x, w.m1.y, w.m1.z, w.m1.w};
    const int qsh = 2 * j, msh = j + 4 * h;
    const float d = f16_bits_to_f32((uint16_t)w.d);
    float total = 0.f;
#pragma unroll
    for (int g = 0; g < 2; g++) {
        uint32_t c[4];
        // the high bit moved straight to bit 2 of each byte (a left shift for
        // msh < 2), then one and-or with the two low bits
#pragma unroll
        for (int w4 = 0; w4 < 4; w4++) {
            const uint32_t mb = msh >= 2 ? mw[4 * g + w4] >> (msh - 2) : mw[4 * g + w4] << (2 - msh);
            c[w4] = ((qw[4 * g + w4] >> qsh) & 0x03030303u) | (mb & 0x04040404u);
        }
        const float dot = group_dot(c, x, g);
        total += (d * (float)(q3k_scale(w.sc[0], w.sc[1], w.sc[2], 8 * h + 2 * j + g) - 32)) * (dot - 4.f * x.xs[g]);
    }
    return total;
}

// Contribution of unit u of a row from its weight words and its x (the
// offsets the unsigned codes leave out come back through the group sums).
template <int T>
__device__ __forceinline__ float dot_unit(const UnitW<T> &w, int u, const UnitX &x) {
    if constexpr (T == LT_TYPE_Q3_K) {
        return q3k_group_dot(w, u, x);
    } else {
        const float d = f16_bits_to_f32((uint16_t)w.dm);
        if constexpr (T == LT_TYPE_IQ4_NL) return d * iq4_block_dot(w.q, x);
        const float dot = q5u_block_dot(w.q, w.qh, x);
        const float s0 = x.xs[0] + x.xs[1];
        if constexpr (T == LT_TYPE_Q5_0) return d * (dot - 16.f * s0);                   // codes - 16
        return d * dot + f16_bits_to_f32((uint16_t)(w.dm >> 16)) * s0;                    // Q5_1: d q + m
    }
}

// A 32-element block's codes as signed (IQ4_NL: the table values) or
// unsigned (Q5_0 / Q5_1: 5-bit) bytes, words 0-3 the low half (elements
// 4i..4i+3 in word i), 4-7 the high half, with the block's f16 d (and Q5_1
// m) -- formed from the weights alone, before the activations are there.
struct BlockCodes {
    uint32_t c[8];
    uint32_t dm;
};
template <int T>
__device__ __forceinline__ BlockCodes block_codes(const UnitW<T> &w) {
    static_assert(T == LT_TYPE_IQ4_NL || T == LT_TYPE_Q5_0 || T == LT_TYPE_Q5_1, "32-element block formats");
    BlockCodes b;
    const uint32_t q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if constexpr (T == LT_TYPE_IQ4_NL) {
            b.c[i] = iq4_lookup4(q[i] & 0x0f0f0f0fu);
            b.c[4 + i] = iq4_lookup4((q[i] >> 4) & 0x0f0f0f0fu);
        } else {
            b.c[i] = (q[i] & 0x0f0f0f0fu) | spread4((w.qh >> (4 * i)) & 15u);
            b.c[4 + i] = ((q[i] >> 4) & 0x0f0f0f0fu) | spread4((w.qh >> (16 + 4 * i)) & 15u);
        }
    }
    b.dm = w.dm;
    return b;
}
// The block's contribution from its codes (dot_unit's arithmetic).
template <int T>
__device__ __forceinline__ float block_codes_dot(const BlockCodes &b, const UnitX &x) {
    const uint32_t lo[4] = {b.c[0], b.c[1], b.c[2], b.c[3]}, hi[4] = {b.c[4], b.c[5], b.c[6], b.c[7]};
    const float dot = group_dot(lo, x, 0) + group_dot(hi, x, 1);
    const float d = f16_bits_to_f32((uint16_t)b.dm);
    if constexpr (T == LT_TYPE_IQ4_NL) return d * dot;
    const float s0 = x.xs[0] + x.xs[1];
    if constexpr (T == LT_TYPE_Q5_0) return d * (dot - 16.f * s0);  // codes - 16
    return d * dot + f16_bits_to_f32((uint16_t)(b.dm >> 16)) * s0;   // Q5_1: d q + m
}

template <int T>
__device__ __forceinline__ int units_per_row(const DevTensor &W) {
    return T == LT_TYPE_Q3_K ? 8 * (int)W.blocks_per_row : (int)W.blocks_per_row;
}


}  // namespace lt
