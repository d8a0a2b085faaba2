/*
 * lt_oracle.c -- CPU restatement of llmtoy-zig's decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for the HIP path and the CPU
 * baseline timed by bench.py.  The product library never links or calls it.
 *
 * Source of each function (paths relative to the llmtoy-zig tree) and how it
 * is pinned (tests/test_oracle.py):
 *   lto_f16_to_f32        quant/dequant.zig:302-305  KAT 671-678 (+-1.0), IEEE-754
 *                         closed form over all 65536 encodings (numpy float16).
 *   lto_dequant_q8_0      dequant.zig:42-52          KAT 702-714; brute force.
 *   lto_dot_q8_0          dequant.zig:59-78          KAT 680-700; GPU KAT
 *                         gpu/matvec.zig:3728-3767 (out = i+1); float64 brute force.
 *   lto_dequant_q4_k      dequant.zig:157-187        KAT 760-766 (zero block); GPU KATs
 *                         matvec.zig:3877-3908 (32.0), 3910-3939 (-64.0); independent
 *                         numpy decoder of the ggml block layout on random blocks.
 *   lto_dequant_q6_k      dequant.zig:237-277        independent numpy decoder;
 *                         special cases (q=32 -> 0, sc=0 -> 0, single-element probes).
 *   lto_dotf32            ops/math.zig:96-116        KAT 401-413 (lengths 1,7,8,32,33);
 *                         bitwise vs a numpy float32 restatement of the lane order.
 *   lto_quant_matvec(_par) math.zig:133-171, 277-320 KAT 173-191 (== matvec);
 *                         thread-count invariance (bitwise), brute force.
 *   lto_softmax/silu/gelu math.zig:29-40, 85-88     KATs 378-399; closed forms (float64).
 *   lto_topk              ops/moe.zig:80-91           KAT gemma4/forward.zig:823-829.
 *   lto_topk_softmax_stats, lto_softmax_topk, lto_topk_matvec_f32(_par),
 *   lto_router_topk_softmax  gemma4/forward.zig:598-821  KATs 823-960 and the
 *                         router KAT gpu/matvec.zig:3582-3656.
 *   lto_moe_forward       ops/moe.zig:18-77            closed-form composition of the
 *                         pinned pieces (float64 restatement on small shapes).
 *                         NORM_TOPK and the router bias are BASELINE extensions with
 *                         no reference code: pinned by their closed form only.
 *   lto_ffn_dense         model/forward.zig:301-308, gemma4/forward.zig:392-397  float64
 *                         restatement on an independent Q8_0 decoder (SiLU and GELU-tanh,
 *                         config-1 shape); planted mistakes (gate/up swapped, activation on
 *                         up, the other activation) shown to fail it.
 *   lto_moe_layer_shared  gemma4/forward.zig:392-397, 417, 463-479  composition; float64
 *                         restatement of every term (shared FFN, Q8_0 router, experts).
 *   lto_moe_prefill       T x lto_moe_forward (main.zig:1916-1922 prefills per token).
 *   lto_dequant_q5_0, lto_dot_q5_0, lto_dequant_q5_1, lto_dequant_iq4_nl, lto_dot_iq4_nl,
 *   lto_q3k_scales, lto_dequant_q3_k
 *                         dequant.zig:80-217, 366-486, 607-659.  Decoders written from the
 *                         block layouts (tests/test_oracle_formats.py), the reference's dot
 *                         KATs (716-758), hand-derived accumulation-order cases, float64.
 *   lto_rmsnorm           math.zig:19-25 (rmsnorm), 42-48 (rmsnormRaw: w == NULL) and
 *                         the (1 + w) convention of rmsnorm.glsl.  KATs math.zig:344-354;
 *                         a hand-derived case fixing the sequential sum of squares;
 *                         closed forms on power-of-two vectors; float64.
 *   lto_add_rmsnorm       add_rmsnorm.glsl semantics on the CPU order of
 *                         gemma4/forward.zig:489-490 (a + b, then rmsnorm).  float64,
 *                         equality with lto_rmsnorm of the rounded sum.
 *   lto_rmsnorm_wrs       math.zig:51-82 (rmsnormWeightedAndRawScaled).  KAT math.zig:356-376
 *                         (against separate passes); float64.
 *   lto_gemma4_moe_block  gemma4/forward.zig:403-418, 463-497: router-input prep, router,
 *                         expert loop with down_exps_scale, post_ffw_norm_2, combine with the
 *                         dense FFN, post_ffw_norm, residual, layer_output_scale.  Composition
 *                         of the pinned pieces; float64 restatement; planted-mistake checks.
 *
 * Floating point: every a*b+c below is a rounded multiply followed by a rounded
 * add (the file is compiled with -ffp-contract=off), vector reductions are the
 * ordered lane sums Zig's @reduce(.Add) performs in strict float mode.
 */
#include "lt_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define QK_K 256
#define Q8_0_ELEMS 32
#define Q8_0_BYTES 34
#define Q4_K_BYTES 144
#define Q6_K_BYTES 210
#define Q5_0_BYTES 22
#define Q5_1_BYTES 24
#define IQ4_NL_BYTES 18
#define Q3_K_BYTES 110

/* ------------------------------------------------------------------------ */
/* f16 -> f32, exact (subnormals, signed zero, inf, NaN kept).              */
/* dequant.zig:302-305 does @floatCast(@as(f16, @bitCast(raw))).            */
float lto_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: value = man * 2^-24, exactly representable */
            float v = (float)man * 5.9604644775390625e-08f; /* 2^-24 */
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline float f16_at(const uint8_t *p) { return lto_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* dequant.zig:17-20 */
void lto_dequant_f32(const uint8_t *data, float *out, size_t n) { memcpy(out, data, n * 4); }

/* dequant.zig:24-29 */
void lto_dequant_f16(const uint8_t *data, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = f16_at(data + 2 * i);
}

/* dequant.zig:42-52: val = d * q */
void lto_dequant_q8_0(const uint8_t *data, float *out, size_t n) {
    size_t nb = n / Q8_0_ELEMS;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = data + b * Q8_0_BYTES;
        float d = f16_at(blk);
        for (int i = 0; i < Q8_0_ELEMS; i++) out[b * Q8_0_ELEMS + i] = d * (float)(int8_t)blk[2 + i];
    }
}

/* dequant.zig:59-78: per block, 8 lane accumulators over 4 groups of 8,
 * ordered lane reduce, then total += reduce * d (scale after the sum). */
float lto_dot_q8_0(const uint8_t *data, const float *vec, size_t n) {
    size_t nb = n / Q8_0_ELEMS;
    float total = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = data + b * Q8_0_BYTES;
        float d = f16_at(blk);
        const int8_t *qs = (const int8_t *)(blk + 2);
        const float *v = vec + b * Q8_0_ELEMS;
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 8; l++) {
                float p = (float)qs[8 * j + l] * v[8 * j + l];
                acc[l] = acc[l] + p;
            }
        float r = acc[0];
        for (int l = 1; l < 8; l++) r = r + acc[l];
        float t = r * d;
        total = total + t;
    }
    return total;
}

/* dequant.zig:291-300 (get_scale_min_k4) */
void lto_q4k_scale_min(int j, const uint8_t *s, uint8_t *sc, uint8_t *mn) {
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4));
        *mn = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* dequant.zig:157-187: val = (d*sc)*q - (dmin*mn) */
void lto_dequant_q4_k(const uint8_t *data, float *out, size_t n) {
    size_t nb = n / QK_K;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = data + b * Q4_K_BYTES;
        float d = f16_at(blk), dmin = f16_at(blk + 2);
        const uint8_t *scales = blk + 4, *qs = blk + 16;
        int sub = 0;
        for (int chunk = 0; chunk < QK_K; chunk += 64, sub += 2) {
            uint8_t sc1, mn1, sc2, mn2;
            lto_q4k_scale_min(sub, scales, &sc1, &mn1);
            lto_q4k_scale_min(sub + 1, scales, &sc2, &mn2);
            float d1 = d * (float)sc1, m1 = dmin * (float)mn1;
            float d2 = d * (float)sc2, m2 = dmin * (float)mn2;
            for (int i = 0; i < 32; i++) {
                uint8_t byte = qs[chunk / 2 + i];
                float lo = d1 * (float)(byte & 0x0f);
                float hi = d2 * (float)(byte >> 4);
                out[b * QK_K + chunk + i] = lo - m1;
                out[b * QK_K + chunk + 32 + i] = hi - m2;
            }
        }
    }
}

/* dequant.zig:282-287 */
static inline float q6val(uint8_t ql, uint8_t qh, int qh_shift, int ql_shift) {
    int lo4 = (ql >> ql_shift) & 0x0f;
    int hi2 = (qh >> qh_shift) & 0x03;
    return (float)((lo4 | (hi2 << 4)) - 32);
}

/* dequant.zig:237-277: val = (d*sc)*(q-32) */
void lto_dequant_q6_k(const uint8_t *data, float *out, size_t n) {
    size_t nb = n / QK_K;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = data + b * Q6_K_BYTES;
        const uint8_t *ql = blk, *qh = blk + 128;
        const int8_t *sc = (const int8_t *)(blk + 192);
        float d = f16_at(blk + 208);
        for (int half = 0; half < 2; half++) {
            int ql_off = 64 * half, qh_off = 32 * half, sc_off = 8 * half, chunk = 128 * half;
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                float q1 = q6val(ql[ql_off + l], qh[qh_off + l], 0, 0);
                float q2 = q6val(ql[ql_off + l + 32], qh[qh_off + l], 2, 0);
                float q3 = q6val(ql[ql_off + l], qh[qh_off + l], 4, 4);
                float q4 = q6val(ql[ql_off + l + 32], qh[qh_off + l], 6, 4);
                float s0 = d * (float)sc[sc_off + is + 0];
                float s2 = d * (float)sc[sc_off + is + 2];
                float s4 = d * (float)sc[sc_off + is + 4];
                float s6 = d * (float)sc[sc_off + is + 6];
                size_t base = b * QK_K + chunk + l;
                out[base + 0] = s0 * q1;
                out[base + 32] = s2 * q2;
                out[base + 64] = s4 * q3;
                out[base + 96] = s6 * q4;
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* math.zig:96-116.  4 x 8-lane accumulators over 32-element strides,
 * acc = (acc0+acc1)+(acc2+acc3), 8-wide tail, ordered 8-lane reduce,
 * scalar tail. */
float lto_dotf32(const float *a, const float *b, size_t n) {
    float acc0[8] = {0}, acc1[8] = {0}, acc2[8] = {0}, acc3[8] = {0}, acc[8];
    size_t i = 0;
    for (; i + 32 <= n; i += 32) {
        for (int l = 0; l < 8; l++) {
            float p0 = a[i + l] * b[i + l];
            float p1 = a[i + 8 + l] * b[i + 8 + l];
            float p2 = a[i + 16 + l] * b[i + 16 + l];
            float p3 = a[i + 24 + l] * b[i + 24 + l];
            acc0[l] = acc0[l] + p0;
            acc1[l] = acc1[l] + p1;
            acc2[l] = acc2[l] + p2;
            acc3[l] = acc3[l] + p3;
        }
    }
    for (int l = 0; l < 8; l++) {
        float s01 = acc0[l] + acc1[l];
        float s23 = acc2[l] + acc3[l];
        acc[l] = s01 + s23;
    }
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) {
            float p = a[i + l] * b[i + l];
            acc[l] = acc[l] + p;
        }
    float sum = acc[0];
    for (int l = 1; l < 8; l++) sum = sum + acc[l];
    for (; i < n; i++) {
        float p = a[i] * b[i];
        sum = sum + p;
    }
    return sum;
}

/* math.zig:8-17 */
void lto_matvec_f32(float *out, const float *mat, const float *vec, size_t rows, size_t cols) {
    for (size_t r = 0; r < rows; r++) {
        float sum = 0.0f;
        for (size_t c = 0; c < cols; c++) {
            float p = mat[r * cols + c] * vec[c];
            sum = sum + p;
        }
        out[r] = sum;
    }
}

/* math.zig:194-208 (integer division: a partial trailing block is dropped) */
/* ------------------------------------------------------------------------ */
/* Q5_0 (dequant.zig:189-217): 22 B / 32: d, qh (u32 LE), 16 nibble bytes;   */
/* val = d * ((nib | hb << 4) - 16); element j: low nibble of qs[j], bit j   */
/* of qh; element j + 16: high nibble of qs[j], bit j + 16.                   */
static inline int q5_0_val(const uint8_t *blk, int e) {
    uint32_t qh;
    memcpy(&qh, blk + 2, 4);
    const uint8_t q = blk[6 + (e & 15)];
    const int nib = e < 16 ? (q & 15) : (q >> 4);
    return (nib | (int)(((qh >> e) & 1u) << 4)) - 16;
}

void lto_dequant_q5_0(const uint8_t *data, float *out, size_t n) {
    for (size_t b = 0; b < n / 32; b++) {
        const uint8_t *blk = data + b * Q5_0_BYTES;
        const float d = f16_at(blk);
        for (int e = 0; e < 32; e++) out[b * 32 + e] = d * (float)q5_0_val(blk, e);
    }
}

/* dequant.zig:92-133 dotQ5_0: per block 8 lane accumulators over groups g =
 * 0..3 (elements 8g + l), acc[l] += q5 * v; total += reduce_ordered(acc) * d. */
float lto_dot_q5_0(const uint8_t *data, const float *vec, size_t n) {
    float total = 0.0f;
    for (size_t b = 0; b < n / 32; b++) {
        const uint8_t *blk = data + b * Q5_0_BYTES;
        const float d = f16_at(blk);
        const float *v = vec + b * 32;
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int g = 0; g < 4; g++)
            for (int l = 0; l < 8; l++) {
                float p = (float)q5_0_val(blk, 8 * g + l) * v[8 * g + l];
                acc[l] = acc[l] + p;
            }
        float r = acc[0];
        for (int l = 1; l < 8; l++) r = r + acc[l];
        float t = r * d;
        total = total + t;
    }
    return total;
}

/* Q5_1 (dequant.zig:456-486): 24 B / 32: d, m, qh[4], qs[16];
 * val = d * (nib | hb << 4) + m (rounded multiply, then add). */
void lto_dequant_q5_1(const uint8_t *data, float *out, size_t n) {
    for (size_t b = 0; b < n / 32; b++) {
        const uint8_t *blk = data + b * Q5_1_BYTES;
        const float d = f16_at(blk), m = f16_at(blk + 2);
        const uint8_t *qh = blk + 4, *qs = blk + 8;
        for (int j = 0; j < 16; j++) {
            int hi0 = ((qh[j / 8] >> (j % 8)) & 1) << 4;
            int hi1 = ((qh[(j + 16) / 8] >> ((j + 16) % 8)) & 1) << 4;
            float q0 = (float)((qs[j] & 15) | hi0), q1 = (float)((qs[j] >> 4) | hi1);
            float t0 = d * q0, t1 = d * q1;
            out[b * 32 + j] = t0 + m;
            out[b * 32 + j + 16] = t1 + m;
        }
    }
}

/* IQ4_NL (dequant.zig:607-659): 18 B / 32: d, 16 nibble bytes indexing a
 * fixed non-linear table. */
static const float kIq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

void lto_dequant_iq4_nl(const uint8_t *data, float *out, size_t n) {
    for (size_t b = 0; b < n / 32; b++) {
        const uint8_t *blk = data + b * IQ4_NL_BYTES;
        const float d = f16_at(blk);
        for (int j = 0; j < 16; j++) {
            out[b * 32 + j] = d * kIq4nl[blk[2 + j] & 15];
            out[b * 32 + j + 16] = d * kIq4nl[blk[2 + j] >> 4];
        }
    }
}

/* dequant.zig:642-658 dotIQ4NL: one scalar accumulator per block, adding
 * element j then element j + 16 for j = 0..15; total += d * acc. */
float lto_dot_iq4_nl(const uint8_t *data, const float *vec, size_t n) {
    float total = 0.0f;
    for (size_t b = 0; b < n / 32; b++) {
        const uint8_t *blk = data + b * IQ4_NL_BYTES;
        const float d = f16_at(blk);
        const float *v = vec + b * 32;
        float acc = 0.0f;
        for (int j = 0; j < 16; j++) {
            const uint8_t q = blk[2 + j];
            float p0 = kIq4nl[q & 15] * v[j];
            acc = acc + p0;
            float p1 = kIq4nl[q >> 4] * v[j + 16];
            acc = acc + p1;
        }
        float t = d * acc;
        total = total + t;
    }
    return total;
}

/* Q3_K (dequant.zig:366-454): 110 B / 256: hmask[32], qs[64], 12 packed
 * scale bytes (16 six-bit values, ggml kmask unpacking), f16 d.
 * Element n = 128 h + 32 j + 16 g + l: q2 = (qs[32 h + 16 g + l] >> 2j) & 3,
 * high bit = hmask[16 g + l] & (1 << (j + 4 h)); value = dl * (q2 - 4 * !hi)
 * with dl = d * (sc[8 h + 2 j + g] - 32). */
void lto_q3k_scales(const uint8_t *s, uint8_t *sc) {
    uint32_t a0, a1, tmp, aux[4];
    memcpy(&a0, s, 4);
    memcpy(&a1, s + 4, 4);
    memcpy(&tmp, s + 8, 4);
    const uint32_t k1 = 0x03030303u, k2 = 0x0f0f0f0fu;
    aux[2] = ((a0 >> 4) & k2) | (((tmp >> 4) & k1) << 4);
    aux[3] = ((a1 >> 4) & k2) | (((tmp >> 6) & k1) << 4);
    aux[0] = (a0 & k2) | (((tmp >> 0) & k1) << 4);
    aux[1] = (a1 & k2) | (((tmp >> 2) & k1) << 4);
    memcpy(sc, aux, 16);
}

void lto_dequant_q3_k(const uint8_t *data, float *out, size_t n) {
    for (size_t b = 0; b < n / QK_K; b++) {
        const uint8_t *blk = data + b * Q3_K_BYTES;
        const uint8_t *hmask = blk, *qs = blk + 32;
        const float d = f16_at(blk + 108);
        uint8_t sc[16];
        lto_q3k_scales(blk + 96, sc);
        for (int h = 0; h < 2; h++)
            for (int j = 0; j < 4; j++)
                for (int g = 0; g < 2; g++) {
                    const float dl = d * ((float)sc[8 * h + 2 * j + g] - 32.0f);
                    for (int l = 0; l < 16; l++) {
                        const int q2 = (qs[32 * h + 16 * g + l] >> (2 * j)) & 3;
                        const int hi = (hmask[16 * g + l] >> (j + 4 * h)) & 1;
                        out[b * QK_K + 128 * h + 32 * j + 16 * g + l] = (float)(q2 - (hi ? 0 : 4)) * dl;
                    }
                }
    }
}

size_t lto_row_bytes(uint32_t type, size_t cols) {
    switch (type) {
    case LTO_F32: return cols * 4;
    case LTO_F16: return cols * 2;
    case LTO_Q8_0: return (cols / Q8_0_ELEMS) * Q8_0_BYTES;
    case LTO_Q4_K: return (cols / QK_K) * Q4_K_BYTES;
    case LTO_Q6_K: return (cols / QK_K) * Q6_K_BYTES;
    case LTO_Q5_0: return (cols / 32) * Q5_0_BYTES;
    case LTO_Q5_1: return (cols / 32) * Q5_1_BYTES;
    case LTO_IQ4_NL: return (cols / 32) * IQ4_NL_BYTES;
    case LTO_Q3_K: return (cols / QK_K) * Q3_K_BYTES;
    default: return 0;
    }
}

/* math.zig:211-225 */
int lto_dequant_row(const uint8_t *data, float *out, uint32_t type, size_t cols) {
    switch (type) {
    case LTO_F32: lto_dequant_f32(data, out, cols); return 0;
    case LTO_F16: lto_dequant_f16(data, out, cols); return 0;
    case LTO_Q8_0: lto_dequant_q8_0(data, out, cols); return 0;
    case LTO_Q4_K: lto_dequant_q4_k(data, out, cols); return 0;
    case LTO_Q6_K: lto_dequant_q6_k(data, out, cols); return 0;
    case LTO_Q5_0: lto_dequant_q5_0(data, out, cols); return 0;
    case LTO_Q5_1: lto_dequant_q5_1(data, out, cols); return 0;
    case LTO_IQ4_NL: lto_dequant_iq4_nl(data, out, cols); return 0;
    case LTO_Q3_K: lto_dequant_q3_k(data, out, cols); return 0;
    default: return -1;
    }
}

static inline float row_dot(const uint8_t *row, uint32_t type, const float *vec, size_t cols, float *row_buf) {
    if (type == LTO_Q8_0) return lto_dot_q8_0(row, vec, cols);
    if (type == LTO_Q5_0) return lto_dot_q5_0(row, vec, cols);   /* math.zig:152-155 */
    if (type == LTO_IQ4_NL) return lto_dot_iq4_nl(row, vec, cols); /* math.zig:156-159 */
    if (type == LTO_F32 && ((uintptr_t)row % 4) == 0) return lto_dotf32((const float *)row, vec, cols);
    lto_dequant_row(row, row_buf, type, cols);
    return lto_dotf32(row_buf, vec, cols);
}

static int type_ok(uint32_t t) {
    return t == LTO_F32 || t == LTO_F16 || t == LTO_Q8_0 || t == LTO_Q4_K || t == LTO_Q6_K || t == LTO_Q5_0 ||
           t == LTO_Q5_1 || t == LTO_IQ4_NL || t == LTO_Q3_K;
}

/* math.zig:133-171 */
int lto_quant_matvec(float *out, const uint8_t *mat, uint32_t type, const float *vec, size_t rows, size_t cols,
                     float *row_buf) {
    if (!type_ok(type)) return -1;
    size_t rb = lto_row_bytes(type, cols);
    for (size_t i = 0; i < rows; i++) out[i] = row_dot(mat + i * rb, type, vec, cols, row_buf);
    return 0;
}

/* math.zig:29-35 */
void lto_softmax(float *x, size_t n) {
    float max = x[0];
    for (size_t i = 1; i < n; i++)
        if (x[i] > max) max = x[i];
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - max);
        sum = sum + x[i];
    }
    for (size_t i = 0; i < n; i++) x[i] = x[i] / sum;
}

/* math.zig:38-40 */
float lto_silu(float x) { return x / (1.0f + expf(-x)); }

/* math.zig:85-88: 0.5*x*(1 + tanh(c*(x + 0.044715*x*x*x))) evaluated left to right */
float lto_gelu(float x) {
    const float c = 0.7978845608028654f;
    float x3 = ((0.044715f * x) * x) * x;
    float inner = c * (x + x3);
    float t = tanhf(inner);
    return (0.5f * x) * (1.0f + t);
}

/* ------------------------------------------------------------------------ */
/* Persistent pool (thread_pool.zig:15-112): mutex + condvars over a bounded
 * ring queue; submit() enqueues, wait() blocks until all submitted jobs ran. */
typedef void (*lto_fn)(void *);
typedef struct {
    lto_fn fn;
    void *ctx;
} lto_entry;

struct lto_pool {
    pthread_t *threads;
    int n;
    lto_entry *queue;
    size_t cap, head, tail, pending;
    int shutdown;
    pthread_mutex_t mu;
    pthread_cond_t work_ready, all_done, not_full;
};

static void *pool_worker(void *arg) {
    lto_pool *p = (lto_pool *)arg;
    pthread_mutex_lock(&p->mu);
    for (;;) {
        while (p->head == p->tail && !p->shutdown) pthread_cond_wait(&p->work_ready, &p->mu);
        if (p->shutdown && p->head == p->tail) {
            pthread_mutex_unlock(&p->mu);
            return NULL;
        }
        lto_entry e = p->queue[p->tail % p->cap];
        p->tail++;
        pthread_cond_signal(&p->not_full);
        pthread_mutex_unlock(&p->mu);
        e.fn(e.ctx);
        pthread_mutex_lock(&p->mu);
        p->pending--;
        if (p->pending == 0) pthread_cond_signal(&p->all_done);
    }
}

lto_pool *lto_pool_create(int n) {
    if (n < 1) n = 1;
    lto_pool *p = (lto_pool *)calloc(1, sizeof(*p));
    if (!p) return NULL;
    p->n = n;
    p->cap = (size_t)(n * 4 > 64 ? n * 4 : 64);
    p->queue = (lto_entry *)calloc(p->cap, sizeof(lto_entry));
    p->threads = (pthread_t *)calloc((size_t)n, sizeof(pthread_t));
    pthread_mutex_init(&p->mu, NULL);
    pthread_cond_init(&p->work_ready, NULL);
    pthread_cond_init(&p->all_done, NULL);
    pthread_cond_init(&p->not_full, NULL);
    for (int i = 0; i < n; i++) pthread_create(&p->threads[i], NULL, pool_worker, p);
    return p;
}

void lto_pool_destroy(lto_pool *p) {
    if (!p) return;
    pthread_mutex_lock(&p->mu);
    p->shutdown = 1;
    pthread_cond_broadcast(&p->work_ready);
    pthread_mutex_unlock(&p->mu);
    for (int i = 0; i < p->n; i++) pthread_join(p->threads[i], NULL);
    pthread_mutex_destroy(&p->mu);
    pthread_cond_destroy(&p->work_ready);
    pthread_cond_destroy(&p->all_done);
    pthread_cond_destroy(&p->not_full);
    free(p->queue);
    free(p->threads);
    free(p);
}

int lto_pool_threads(const lto_pool *p) { return p ? p->n : 1; }

static void pool_submit(lto_pool *p, lto_fn fn, void *ctx) {
    pthread_mutex_lock(&p->mu);
    while (p->head - p->tail >= p->cap) pthread_cond_wait(&p->not_full, &p->mu);
    p->queue[p->head % p->cap].fn = fn;
    p->queue[p->head % p->cap].ctx = ctx;
    p->head++;
    p->pending++;
    pthread_cond_signal(&p->work_ready);
    pthread_mutex_unlock(&p->mu);
}

static void pool_wait(lto_pool *p) {
    pthread_mutex_lock(&p->mu);
    while (p->pending > 0) pthread_cond_wait(&p->all_done, &p->mu);
    pthread_mutex_unlock(&p->mu);
}

/* math.zig:228-270 */
typedef struct {
    const uint8_t *mat;
    uint32_t type;
    const float *vec;
    float *out;
    float *row_buf;
    size_t row_start, n_rows, cols;
} row_job;

static void row_job_run(void *arg) {
    row_job *j = (row_job *)arg;
    size_t rb = lto_row_bytes(j->type, j->cols);
    for (size_t i = 0; i < j->n_rows; i++)
        j->out[i] = row_dot(j->mat + (j->row_start + i) * rb, j->type, j->vec, j->cols, j->row_buf);
}

/* math.zig:277-320: nt = min(threads, ceil(rows/64)); the first rows%nt jobs
 * get one extra row.  The reference's job array holds 64 entries, so nt is
 * capped at 64 here (the reference leaves nt > 64 undefined). */
int lto_quant_matvec_par(float *out, const uint8_t *mat, uint32_t type, const float *vec, size_t rows, size_t cols,
                         float *scratch, lto_pool *pool) {
    if (!type_ok(type)) return -1;
    const size_t min_rows = 64;
    size_t n = pool ? (size_t)pool->n : 1;
    size_t nt = (rows + min_rows - 1) / min_rows;
    if (n < nt) nt = n;
    if (nt > 64) nt = 64;
    if (nt <= 1) return lto_quant_matvec(out, mat, type, vec, rows, cols, scratch);
    row_job jobs[64];
    size_t base = rows / nt, extra = rows % nt, row = 0;
    for (size_t t = 0; t < nt; t++) {
        size_t nr = base + (t < extra ? 1 : 0);
        jobs[t].mat = mat;
        jobs[t].type = type;
        jobs[t].vec = vec;
        jobs[t].out = out + row;
        jobs[t].row_buf = scratch + t * cols;
        jobs[t].row_start = row;
        jobs[t].n_rows = nr;
        jobs[t].cols = cols;
        pool_submit(pool, row_job_run, &jobs[t]);
        row += nr;
    }
    pool_wait(pool);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* moe.zig:80-91: O(n*k) selection, strict '>' so the lowest index wins ties. */
void lto_topk(const float *scores, size_t n, size_t *out, size_t k) {
    for (size_t i = 0; i < k; i++) {
        size_t best = 0;
        float best_val = -INFINITY;
        for (size_t j = 0; j < n; j++) {
            int already = 0;
            for (size_t p = 0; p < i; p++)
                if (out[p] == j) {
                    already = 1;
                    break;
                }
            if (!already && scores[j] > best_val) {
                best_val = scores[j];
                best = j;
            }
        }
        out[i] = best;
    }
}

static float act_apply(uint32_t act, float g) { return act == LTO_ACT_GELU_TANH ? lto_gelu(g) : lto_silu(g); }

/* moe.zig:18-77 (see header for the extensions). */
int lto_moe_forward(float *out, const float *router_w, size_t n_experts, const float *router_bias,
                    const uint8_t *gate_up, uint32_t gu_type, const uint8_t *down, uint32_t dn_type, size_t down_cols,
                    const float *x, size_t d_model, size_t k, size_t d_expert, uint32_t act, uint32_t flags,
                    lto_pool *pool, uint32_t *out_ids, float *out_w, int *logit_order_agrees) {
    if (k == 0 || k > n_experts || k > 64 || down_cols < d_expert) return -1;
    if (!type_ok(gu_type) || !type_ok(dn_type)) return -1;
    size_t nthreads = (size_t)lto_pool_threads(pool);
    size_t max_cols = d_model > down_cols ? d_model : down_cols;
    float *gate = (float *)calloc(down_cols, 4);
    float *up = (float *)calloc(d_expert, 4);
    float *dn = (float *)calloc(d_model, 4);
    float *scratch = (float *)calloc(nthreads * max_cols, 4);
    float *scores = (float *)calloc(n_experts, 4);
    float *logits = (float *)calloc(n_experts, 4);
    size_t top[64], top_l[64];
    if (!gate || !up || !dn || !scratch || !scores || !logits) {
        free(gate); free(up); free(dn); free(scratch); free(scores); free(logits);
        return -2;
    }
    /* router: serial quantMatvec over f32 rows (dotf32), moe.zig:47 */
    lto_quant_matvec(scores, (const uint8_t *)router_w, LTO_F32, x, n_experts, d_model, scratch);
    if (router_bias)
        for (size_t e = 0; e < n_experts; e++) scores[e] = scores[e] + router_bias[e];
    memcpy(logits, scores, n_experts * 4);
    lto_softmax(scores, n_experts);
    lto_topk(scores, n_experts, top, k);
    if (logit_order_agrees) {
        lto_topk(logits, n_experts, top_l, k);
        int same = 1;
        for (size_t i = 0; i < k; i++) same &= (top[i] == top_l[i]);
        *logit_order_agrees = same;
    }
    float wsel[64];
    for (size_t i = 0; i < k; i++) wsel[i] = scores[top[i]];
    if (flags & LTO_MOE_NORM_TOPK) {
        float s = 0.0f;
        for (size_t i = 0; i < k; i++) s = s + wsel[i];
        for (size_t i = 0; i < k; i++) wsel[i] = wsel[i] / s;
    }
    size_t gu_rb = lto_row_bytes(gu_type, d_model);
    size_t gu_per_expert = 2 * d_expert * gu_rb;
    size_t dn_rb = lto_row_bytes(dn_type, down_cols);
    size_t dn_per_expert = d_model * dn_rb;
    for (size_t i = 0; i < k; i++) {
        size_t e = top[i];
        float w = wsel[i];
        const uint8_t *gd = gate_up + e * gu_per_expert;
        lto_quant_matvec_par(gate, gd, gu_type, x, d_expert, d_model, scratch, pool);
        lto_quant_matvec_par(up, gd + d_expert * gu_rb, gu_type, x, d_expert, d_model, scratch, pool);
        for (size_t j = 0; j < d_expert; j++) {
            float a = act_apply(act, gate[j]);
            gate[j] = a * up[j];
        }
        for (size_t j = d_expert; j < down_cols; j++) gate[j] = 0.0f; /* zero K padding */
        lto_quant_matvec_par(dn, down + e * dn_per_expert, dn_type, gate, d_model, down_cols, scratch, pool);
        for (size_t j = 0; j < d_model; j++) {
            float t = w * dn[j];
            out[j] = out[j] + t;
        }
        if (out_ids) out_ids[i] = (uint32_t)e;
        if (out_w) out_w[i] = w;
    }
    free(gate); free(up); free(dn); free(scratch); free(scores); free(logits);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* gemma4/forward.zig:598-629: insertion top-k on logits (strict '>', so an
 * earlier index stays ahead on ties) plus an online softmax denominator. */
lto_stats lto_topk_softmax_stats(const float *scores, size_t n, size_t *out, size_t k) {
    float max = scores[0];
    float exp_sum = 0.0f;
    size_t filled = 0;
    for (size_t j = 0; j < n; j++) {
        float s = scores[j];
        if (s > max) {
            float t = exp_sum * expf(max - s);
            exp_sum = t + 1.0f;
            max = s;
        } else {
            exp_sum = exp_sum + expf(s - max);
        }
        if (filled < k) {
            size_t pos = filled++;
            while (pos > 0 && s > scores[out[pos - 1]]) {
                out[pos] = out[pos - 1];
                pos--;
            }
            out[pos] = j;
        } else if (s > scores[out[k - 1]]) {
            size_t pos = k - 1;
            while (pos > 0 && s > scores[out[pos - 1]]) {
                out[pos] = out[pos - 1];
                pos--;
            }
            out[pos] = j;
        }
    }
    lto_stats st = {max, exp_sum};
    return st;
}

/* gemma4/forward.zig:637-643 */
void lto_softmax_topk(float *scores, size_t n, size_t *out, size_t k) {
    lto_stats st = lto_topk_softmax_stats(scores, n, out, k);
    for (size_t i = 0; i < k; i++) scores[out[i]] = expf(scores[out[i]] - st.max) / st.exp_sum;
}

/* gemma4/forward.zig:748-767 */
static void insert_topk(size_t *out, float *sel, size_t k, size_t *filled, size_t idx, float score) {
    if (*filled < k) {
        size_t pos = (*filled)++;
        while (pos > 0 && score > sel[pos - 1]) {
            sel[pos] = sel[pos - 1];
            out[pos] = out[pos - 1];
            pos--;
        }
        sel[pos] = score;
        out[pos] = idx;
    } else if (score > sel[k - 1]) {
        size_t pos = k - 1;
        while (pos > 0 && score > sel[pos - 1]) {
            sel[pos] = sel[pos - 1];
            out[pos] = out[pos - 1];
            pos--;
        }
        sel[pos] = score;
        out[pos] = idx;
    }
}

/* gemma4/forward.zig:672-712 */
lto_stats lto_topk_matvec_f32(const float *w, const float *vec, size_t rows, size_t cols, size_t *out,
                              float *sel, size_t k) {
    float max = -INFINITY, exp_sum = 0.0f;
    size_t filled = 0;
    for (size_t j = 0; j < rows; j++) {
        float score = lto_dotf32(w + j * cols, vec, cols);
        if (score > max) {
            float t = exp_sum * expf(max - score);
            exp_sum = t + 1.0f;
            max = score;
        } else {
            exp_sum = exp_sum + expf(score - max);
        }
        insert_topk(out, sel, k, &filled, j, score);
    }
    lto_stats st = {max, exp_sum};
    return st;
}

typedef struct {
    const float *w, *vec;
    size_t row_start, rows, cols, k;
    size_t idx[16];
    float sc[16];
    lto_stats st;
} router_job;

static void router_job_run(void *arg) {
    router_job *j = (router_job *)arg;
    size_t li[16];
    float ls[16];
    j->st = lto_topk_matvec_f32(j->w + j->row_start * j->cols, j->vec, j->rows, j->cols, li, ls, j->k);
    for (size_t i = 0; i < j->k; i++) {
        j->idx[i] = j->row_start + li[i];
        j->sc[i] = ls[i];
    }
}

/* gemma4/forward.zig:769-821 (row chunks of >= 16, merged in job order) */
lto_stats lto_topk_matvec_f32_par(const float *w, const float *vec, size_t rows, size_t cols, size_t *out,
                                  float *sel, size_t k, lto_pool *pool) {
    size_t n = pool ? (size_t)pool->n : 1;
    size_t nt = (rows + 15) / 16;
    if (n < nt) nt = n;
    if (nt > 64) nt = 64;
    if (nt <= 1 || k > 16) return lto_topk_matvec_f32(w, vec, rows, cols, out, sel, k);
    router_job jobs[64];
    size_t base = rows / nt, extra = rows % nt, row = 0;
    for (size_t t = 0; t < nt; t++) {
        size_t nr = base + (t < extra ? 1 : 0);
        jobs[t].w = w;
        jobs[t].vec = vec;
        jobs[t].row_start = row;
        jobs[t].rows = nr;
        jobs[t].cols = cols;
        jobs[t].k = k;
        pool_submit(pool, router_job_run, &jobs[t]);
        row += nr;
    }
    pool_wait(pool);
    float max = -INFINITY, exp_sum = 0.0f;
    size_t filled = 0;
    for (size_t t = 0; t < nt; t++) {
        if (jobs[t].st.max > max) {
            float s = exp_sum * expf(max - jobs[t].st.max);
            exp_sum = s + jobs[t].st.exp_sum;
            max = jobs[t].st.max;
        } else {
            float s = jobs[t].st.exp_sum * expf(jobs[t].st.max - max);
            exp_sum = exp_sum + s;
        }
        for (size_t i = 0; i < k; i++) insert_topk(out, sel, k, &filled, jobs[t].idx[i], jobs[t].sc[i]);
    }
    lto_stats st = {max, exp_sum};
    return st;
}

/* gemma4/forward.zig:648-668 */
int lto_router_topk_softmax(float *scores, size_t *out, size_t k, const uint8_t *router_w, uint32_t router_type,
                            size_t rows, size_t cols, const float *router_in, float *scratch, lto_pool *pool) {
    if (k == 0 || k > rows || k > 16) return -1;
    if (router_type != LTO_F32 || ((uintptr_t)router_w % 4) != 0) {
        if (lto_quant_matvec_par(scores, router_w, router_type, router_in, rows, cols, scratch, pool)) return -1;
        lto_softmax_topk(scores, rows, out, k);
        return 0;
    }
    float sel[16];
    lto_stats st = lto_topk_matvec_f32_par((const float *)router_w, router_in, rows, cols, out, sel, k, pool);
    for (size_t i = 0; i < k; i++) scores[out[i]] = expf(sel[i] - st.max) / st.exp_sum;
    return 0;
}

/* Dense gated FFN: model/forward.zig:301-308 (SiLU), gemma4/forward.zig:392-397 (GELU). */
int lto_ffn_dense(float *out, const uint8_t *wg, const uint8_t *wu, const uint8_t *wd, uint32_t type, const float *x,
                  size_t d_model, size_t d_ffn, uint32_t act, lto_pool *pool) {
    size_t nthreads = (size_t)lto_pool_threads(pool);
    size_t max_cols = d_model > d_ffn ? d_model : d_ffn;
    float *g = (float *)calloc(d_ffn, 4), *u = (float *)calloc(d_ffn, 4);
    float *scratch = (float *)calloc(nthreads * max_cols, 4);
    if (!g || !u || !scratch) {
        free(g); free(u); free(scratch);
        return -2;
    }
    int rc = lto_quant_matvec_par(g, wg, type, x, d_ffn, d_model, scratch, pool);
    rc |= lto_quant_matvec_par(u, wu, type, x, d_ffn, d_model, scratch, pool);
    for (size_t j = 0; j < d_ffn; j++) {
        float a = act_apply(act, g[j]);
        g[j] = a * u[j];
    }
    rc |= lto_quant_matvec_par(out, wd, type, g, d_model, d_ffn, scratch, pool);
    free(g); free(u); free(scratch);
    return rc ? -1 : 0;
}

/* Config-4 layer: gemma4/forward.zig:392-397 (shared FFN), 417 (router),
 * 463-479 (expert loop, down_exps_scale = 1), 489 (combine). */
int lto_moe_layer_shared(float *out, const float *x, size_t d_model, const uint8_t *router_w, uint32_t router_type,
                         size_t n_experts, const uint8_t *gate_up, uint32_t gu_type, const uint8_t *down,
                         uint32_t dn_type, size_t down_cols, size_t k, size_t d_expert, const uint8_t *sh_gate,
                         const uint8_t *sh_up, const uint8_t *sh_down, uint32_t sh_type, size_t sh_ffn, uint32_t act,
                         lto_pool *pool, uint32_t *out_ids, float *out_w) {
    if (k == 0 || k > 16 || down_cols < d_expert) return -1;
    size_t nthreads = (size_t)lto_pool_threads(pool);
    size_t max_cols = d_model;
    if (down_cols > max_cols) max_cols = down_cols;
    if (sh_ffn > max_cols) max_cols = sh_ffn;
    float *ffn = (float *)calloc(d_model, 4), *moe = (float *)calloc(d_model, 4);
    float *scores = (float *)calloc(n_experts, 4), *scratch = (float *)calloc(nthreads * max_cols, 4);
    float *eg = (float *)calloc(down_cols, 4), *eu = (float *)calloc(d_expert, 4), *ed = (float *)calloc(d_model, 4);
    int rc = -2;
    if (!ffn || !moe || !scores || !scratch || !eg || !eu || !ed) goto done;
    rc = lto_ffn_dense(ffn, sh_gate, sh_up, sh_down, sh_type, x, d_model, sh_ffn, act, pool);
    if (rc) goto done;
    size_t top[16];
    rc = lto_router_topk_softmax(scores, top, k, router_w, router_type, n_experts, d_model, x, scratch, pool);
    if (rc) goto done;
    size_t gu_rb = lto_row_bytes(gu_type, d_model), gu_per = 2 * d_expert * gu_rb;
    size_t dn_rb = lto_row_bytes(dn_type, down_cols), dn_per = d_model * dn_rb;
    for (size_t i = 0; i < k; i++) {
        size_t e = top[i];
        float w_score = scores[e];
        const uint8_t *gd = gate_up + e * gu_per;
        lto_quant_matvec_par(eg, gd, gu_type, x, d_expert, d_model, scratch, pool);
        lto_quant_matvec_par(eu, gd + d_expert * gu_rb, gu_type, x, d_expert, d_model, scratch, pool);
        for (size_t j = 0; j < d_expert; j++) {
            float a = act_apply(act, eg[j]);
            eg[j] = a * eu[j];
        }
        for (size_t j = d_expert; j < down_cols; j++) eg[j] = 0.0f;
        lto_quant_matvec_par(ed, down + e * dn_per, dn_type, eg, d_model, down_cols, scratch, pool);
        float expert_scale = 1.0f * w_score;
        for (size_t j = 0; j < d_model; j++) {
            float t = expert_scale * ed[j];
            moe[j] = moe[j] + t;
        }
        if (out_ids) out_ids[i] = (uint32_t)e;
        if (out_w) out_w[i] = w_score;
    }
    for (size_t j = 0; j < d_model; j++) out[j] = ffn[j] + moe[j];
    rc = 0;
done:
    free(ffn); free(moe); free(scores); free(scratch); free(eg); free(eu); free(ed);
    return rc;
}

int lto_moe_prefill(float *out, const float *X, size_t T, const float *router_w, size_t n_experts,
                    const float *router_bias, const uint8_t *gate_up, uint32_t gu_type, const uint8_t *down,
                    uint32_t dn_type, size_t down_cols, size_t d_model, size_t k, size_t d_expert, uint32_t act,
                    uint32_t flags, lto_pool *pool, uint32_t *out_ids, float *out_w) {
    for (size_t t = 0; t < T; t++) {
        float *o = out + t * d_model;
        memset(o, 0, d_model * 4);
        int rc = lto_moe_forward(o, router_w, n_experts, router_bias, gate_up, gu_type, down, dn_type, down_cols,
                                 X + t * d_model, d_model, k, d_expert, act, flags, pool,
                                 out_ids ? out_ids + t * k : NULL, out_w ? out_w + t * k : NULL, NULL);
        if (rc) return rc;
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* RMS normalisation: math.zig:19-25 (rmsnorm), 42-48 (rmsnormRaw).          */
/* ss is the sequential fp32 sum of v*v in index order; rms_inv =           */
/* 1 / sqrt(ss / n + eps) with correctly rounded sqrt and division; each    */
/* output is (v * rms_inv) * w.  one_plus_w uses (1 + w) (rmsnorm.glsl      */
/* flag bit 0); w == NULL multiplies by nothing (rmsnormRaw).               */
static float rms_inv_of(const float *x, size_t n, float eps) {
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float sq = x[i] * x[i];
        ss = ss + sq;
    }
    return 1.0f / sqrtf(ss / (float)n + eps);
}

void lto_rmsnorm(float *out, const float *x, const float *w, size_t n, float eps, int one_plus_w) {
    const float r = rms_inv_of(x, n, eps);
    const float bias = one_plus_w ? 1.0f : 0.0f;
    for (size_t i = 0; i < n; i++) {
        float v = x[i] * r;
        out[i] = w ? v * (bias + w[i]) : v;
    }
}

/* out = rmsnorm(a + b, w): the sum is rounded first (gemma4/forward.zig:489-490). */
void lto_add_rmsnorm(float *out, const float *a, const float *b, const float *w, size_t n, float eps,
                     int one_plus_w) {
    float *v = (float *)malloc(n * 4);
    if (!v) return;
    for (size_t i = 0; i < n; i++) v[i] = a[i] + b[i];
    lto_rmsnorm(out, v, w, n, eps, one_plus_w);
    free(v);
}

/* math.zig:51-82: one ss for both outputs; weighted = (x * rms_inv) * w,
 * raw = (x * (rms_inv * raw_global_scale)) * raw_scale. */
void lto_rmsnorm_wrs(float *weighted_out, float *raw_scaled_out, const float *x, const float *w,
                     const float *raw_scale, float raw_global_scale, size_t n, float eps) {
    const float r = rms_inv_of(x, n, eps);
    const float raw_base = r * raw_global_scale;
    for (size_t i = 0; i < n; i++) {
        float a = x[i] * r;
        float b = x[i] * raw_base;
        weighted_out[i] = a * w[i];
        raw_scaled_out[i] = b * raw_scale[i];
    }
}

/* The MoE tail alone (gemma4/forward.zig:482-497): moe = rmsnorm(moe, w2);
 * ffn = ffn + moe; ffn = rmsnorm(ffn, w); x = x + ffn; x *= los (if != 1).
 * moe and ffn are overwritten as in the reference. */
void lto_moe_tail(float *x, float *moe, float *ffn, const float *post_ffw_norm_2, const float *post_ffw_norm,
                  float layer_output_scale, size_t n, float eps) {
    lto_rmsnorm(moe, moe, post_ffw_norm_2, n, eps, 0);
    for (size_t i = 0; i < n; i++) ffn[i] = ffn[i] + moe[i];
    lto_rmsnorm(ffn, ffn, post_ffw_norm, n, eps, 0);
    for (size_t i = 0; i < n; i++) x[i] = x[i] + ffn[i];
    if (layer_output_scale != 1.0f)
        for (size_t i = 0; i < n; i++) x[i] = x[i] * layer_output_scale;
}

/* Gemma4 MoE block after the dense FFN (gemma4/forward.zig:403-497).
 * x [d] is the residual stream (updated in place); dense_ffn [d] the dense
 * FFN output after post_ffw_norm_1 (not modified here: copied).
 * down_exps_scale may be NULL (all ones). */
int lto_gemma4_moe_block(float *x, const float *dense_ffn, size_t d_model, const uint8_t *router_w,
                         uint32_t router_type, size_t n_experts, const uint8_t *gate_up, uint32_t gu_type,
                         const uint8_t *down, uint32_t dn_type, size_t down_cols, size_t k, size_t d_expert,
                         const float *pre_ffw_norm_2, const float *router_scale, const float *down_exps_scale,
                         const float *post_ffw_norm_2, const float *post_ffw_norm, float layer_output_scale,
                         float eps, uint32_t act, lto_pool *pool, uint32_t *out_ids, float *out_w) {
    if (k == 0 || k > 16 || down_cols < d_expert) return -1;
    size_t nthreads = (size_t)lto_pool_threads(pool);
    size_t max_cols = d_model > down_cols ? d_model : down_cols;
    float *moe_in = (float *)calloc(d_model, 4), *router_in = (float *)calloc(d_model, 4);
    float *moe = (float *)calloc(d_model, 4), *ffn = (float *)calloc(d_model, 4);
    float *scores = (float *)calloc(n_experts, 4), *scratch = (float *)calloc(nthreads * max_cols, 4);
    float *eg = (float *)calloc(down_cols, 4), *eu = (float *)calloc(d_expert, 4), *ed = (float *)calloc(d_model, 4);
    int rc = -2;
    if (!moe_in || !router_in || !moe || !ffn || !scores || !scratch || !eg || !eu || !ed) goto done;
    {
        /* 403-418: shared residual RMS for the expert and router inputs */
        const float inv_sqrt_d = 1.0f / sqrtf((float)d_model);
        lto_rmsnorm_wrs(moe_in, router_in, x, pre_ffw_norm_2, router_scale, inv_sqrt_d, d_model, eps);
        size_t top[16];
        rc = lto_router_topk_softmax(scores, top, k, router_w, router_type, n_experts, d_model, router_in, scratch,
                                     pool);
        if (rc) goto done;
        /* 463-479: expert loop */
        size_t gu_rb = lto_row_bytes(gu_type, d_model), gu_per = 2 * d_expert * gu_rb;
        size_t dn_rb = lto_row_bytes(dn_type, down_cols), dn_per = d_model * dn_rb;
        for (size_t i = 0; i < k; i++) {
            size_t e = top[i];
            float w_score = scores[e];
            const uint8_t *gd = gate_up + e * gu_per;
            lto_quant_matvec_par(eg, gd, gu_type, moe_in, d_expert, d_model, scratch, pool);
            lto_quant_matvec_par(eu, gd + d_expert * gu_rb, gu_type, moe_in, d_expert, d_model, scratch, pool);
            for (size_t j = 0; j < d_expert; j++) {
                float a = act_apply(act, eg[j]);
                eg[j] = a * eu[j];
            }
            for (size_t j = d_expert; j < down_cols; j++) eg[j] = 0.0f;
            lto_quant_matvec_par(ed, down + e * dn_per, dn_type, eg, d_model, down_cols, scratch, pool);
            float expert_scale = (down_exps_scale ? down_exps_scale[e] : 1.0f) * w_score;
            for (size_t j = 0; j < d_model; j++) {
                float t = expert_scale * ed[j];
                moe[j] = moe[j] + t;
            }
            if (out_ids) out_ids[i] = (uint32_t)e;
            if (out_w) out_w[i] = w_score;
        }
        /* 482-497: the tail */
        memcpy(ffn, dense_ffn, d_model * 4);
        lto_moe_tail(x, moe, ffn, post_ffw_norm_2, post_ffw_norm, layer_output_scale, d_model, eps);
        rc = 0;
    }
done:
    free(moe_in); free(router_in); free(moe); free(ffn); free(scores); free(scratch); free(eg); free(eu); free(ed);
    return rc;
}
