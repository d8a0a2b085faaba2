/*
 * lt_oracle.h -- CPU restatement of llmtoy-zig's decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path and the timed CPU baseline in bench.py.  Only tests/, the smoke entry
 * point and bench.py's cpu_baseline leg may load it.  The product library
 * (libllmtoy_hip.so) never links or calls it.
 *
 * Every function restates a reference function (cited file:line, paths
 * relative to the llmtoy-zig source tree) with the same floating-point
 * operation order: separate multiply and add (no FMA contraction), ordered
 * vector reductions, glibc expf/tanhf in place of Zig's @exp/std.math.tanh.
 * Build flags: -O2 -ffp-contract=off -fno-fast-math (see oracle/Makefile).
 *
 * Pinning status of each function is listed in the header comment of
 * lt_oracle.c and checked by tests/test_oracle.py.
 */
#ifndef LT_ORACLE_H
#define LT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GgmlType ids, src/gguf/types.zig:23-53 */
enum { LTO_F32 = 0, LTO_F16 = 1, LTO_Q5_0 = 6, LTO_Q5_1 = 7, LTO_Q8_0 = 8, LTO_Q3_K = 11, LTO_Q4_K = 12,
       LTO_Q6_K = 14, LTO_IQ4_NL = 20 };

/* activations for the gated FFN (src/ops/math.zig:37-40, 84-88) */
enum { LTO_ACT_SILU = 0, LTO_ACT_GELU_TANH = 1 };

/* moe flags */
enum {
    LTO_MOE_NORM_TOPK = 1u << 0, /* renormalise the selected weights (BASELINE extension) */
};

typedef struct {
    float max;
    float exp_sum;
} lto_stats;

typedef struct lto_pool lto_pool;

/* ---- formats: src/quant/dequant.zig ------------------------------------- */
float lto_f16_to_f32(uint16_t raw);                                   /* 302-305 */
void lto_dequant_f32(const uint8_t *data, float *out, size_t n);      /* 17-20 */
void lto_dequant_f16(const uint8_t *data, float *out, size_t n);      /* 24-29 */
void lto_dequant_q8_0(const uint8_t *data, float *out, size_t n);     /* 42-52 */
float lto_dot_q8_0(const uint8_t *data, const float *vec, size_t n);  /* 59-78 */
void lto_dequant_q4_k(const uint8_t *data, float *out, size_t n);     /* 157-187 */
void lto_dequant_q6_k(const uint8_t *data, float *out, size_t n);     /* 237-277 */
void lto_q4k_scale_min(int j, const uint8_t *scales, uint8_t *sc, uint8_t *mn); /* 291-300 */

/* ---- ops: src/ops/math.zig ---------------------------------------------- */
/* the Gemma4 APEX expert formats: dequant.zig:189-217 (Q5_0, dotQ5_0 92-133),
 * 366-454 (Q3_K), 456-486 (Q5_1), 607-659 (IQ4_NL, dotIQ4NL 642-658)      */
void lto_dequant_q5_0(const uint8_t *data, float *out, size_t n);
float lto_dot_q5_0(const uint8_t *data, const float *vec, size_t n);
void lto_dequant_q5_1(const uint8_t *data, float *out, size_t n);
void lto_dequant_iq4_nl(const uint8_t *data, float *out, size_t n);
float lto_dot_iq4_nl(const uint8_t *data, const float *vec, size_t n);
void lto_q3k_scales(const uint8_t *scales12, uint8_t *sc16);
void lto_dequant_q3_k(const uint8_t *data, float *out, size_t n);
float lto_dotf32(const float *a, const float *b, size_t n);           /* 96-116 */
size_t lto_row_bytes(uint32_t type, size_t cols);                     /* 194-208 (0 = unsupported) */
int lto_dequant_row(const uint8_t *data, float *out, uint32_t type, size_t cols); /* 211-225 */
void lto_matvec_f32(float *out, const float *mat, const float *vec, size_t rows, size_t cols); /* 8-17 */
int lto_quant_matvec(float *out, const uint8_t *mat, uint32_t type, const float *vec,
                     size_t rows, size_t cols, float *row_buf);       /* 133-171 */
void lto_softmax(float *x, size_t n);                                 /* 29-35 */
float lto_silu(float x);                                              /* 38-40 */
float lto_gelu(float x);                                              /* 85-88 */

/* persistent pool + row-parallel matvec: thread_pool.zig:15-112, math.zig:277-320 */
lto_pool *lto_pool_create(int n_threads);
void lto_pool_destroy(lto_pool *pool);
int lto_pool_threads(const lto_pool *pool);
int lto_quant_matvec_par(float *out, const uint8_t *mat, uint32_t type, const float *vec,
                         size_t rows, size_t cols, float *scratch, lto_pool *pool);

/* ---- MoE: src/ops/moe.zig ----------------------------------------------- */
void lto_topk(const float *scores, size_t n, size_t *out, size_t k);  /* moe.zig:80-91 */

/* moeForward (moe.zig:18-77), extended with:
 *   - optional per-expert logit bias (router_bias, may be NULL),
 *   - LTO_MOE_NORM_TOPK,
 *   - act selects SiLU (reference) or GELU-tanh,
 *   - down_cols >= d_expert (zero-padded K for the down product).
 * out must be pre-zeroed by the caller (as in the reference).
 * out_ids/out_w (may be NULL) receive the selection in selection order.
 * *logit_order_agrees (may be NULL) is set to 1 when selecting the top-k on
 * the raw logits (lowest index wins ties) gives the same ids as selecting on
 * the probabilities, which is how the GPU router selects.                   */
int lto_moe_forward(float *out, const float *router_w, size_t n_experts,
                    const float *router_bias,
                    const uint8_t *gate_up, uint32_t gu_type,
                    const uint8_t *down, uint32_t dn_type, size_t down_cols,
                    const float *x, size_t d_model, size_t k, size_t d_expert,
                    uint32_t act, uint32_t flags, lto_pool *pool,
                    uint32_t *out_ids, float *out_w, int *logit_order_agrees);

/* ---- Gemma4 router: src/model/gemma4/forward.zig ------------------------- */
lto_stats lto_topk_softmax_stats(const float *scores, size_t n, size_t *out, size_t k); /* 598-629 */
void lto_softmax_topk(float *scores, size_t n, size_t *out, size_t k);                  /* 637-643 */
lto_stats lto_topk_matvec_f32(const float *w, const float *vec, size_t rows, size_t cols,
                              size_t *out, float *sel_scores, size_t k);                /* 672-712 */
lto_stats lto_topk_matvec_f32_par(const float *w, const float *vec, size_t rows, size_t cols,
                                  size_t *out, float *sel_scores, size_t k, lto_pool *pool); /* 769-821 */
/* routerTopKSoftmax (648-668): scores[rows] receives the selected probabilities
 * at the selected indices (other entries: logits or untouched as in the ref). */
int lto_router_topk_softmax(float *scores, size_t *out, size_t k, const uint8_t *router_w,
                            uint32_t router_type, size_t rows, size_t cols,
                            const float *router_in, float *scratch, lto_pool *pool);

/* Gemma4-like layer (config 4): routerTopKSoftmax + CPU expert loop
 * (forward.zig:463-479) with down_exps_scale = 1, plus a shared dense FFN.
 * out = shared_ffn(x) + sum_k p_k * expert_k(x).  out is overwritten.      */
int lto_moe_layer_shared(float *out, const float *x, size_t d_model,
                         const uint8_t *router_w, uint32_t router_type, size_t n_experts,
                         const uint8_t *gate_up, uint32_t gu_type,
                         const uint8_t *down, uint32_t dn_type, size_t down_cols,
                         size_t k, size_t d_expert,
                         const uint8_t *sh_gate, const uint8_t *sh_up, const uint8_t *sh_down,
                         uint32_t sh_type, size_t sh_ffn, uint32_t act, lto_pool *pool,
                         uint32_t *out_ids, float *out_w);

/* Dense gated FFN (model/forward.zig:301-308, gemma4/forward.zig:392-397):
 * out = Wd * (act(Wg x) * (Wu x)).  out is overwritten.                     */
int lto_ffn_dense(float *out, const uint8_t *wg, const uint8_t *wu, const uint8_t *wd,
                  uint32_t type, const float *x, size_t d_model, size_t d_ffn,
                  uint32_t act, lto_pool *pool);

/* Batched prefill oracle: T independent lto_moe_forward evaluations
 * (the reference prefills one token at a time, main.zig:1916-1922).
 * out[T*d_model] is overwritten. out_ids[T*k], out_w[T*k] may be NULL.     */
int lto_moe_prefill(float *out, const float *X, size_t T, const float *router_w, size_t n_experts,
                    const float *router_bias,
                    const uint8_t *gate_up, uint32_t gu_type,
                    const uint8_t *down, uint32_t dn_type, size_t down_cols,
                    size_t d_model, size_t k, size_t d_expert, uint32_t act, uint32_t flags,
                    lto_pool *pool, uint32_t *out_ids, float *out_w);

/* ---- RMS norms and the Gemma4 MoE block: src/ops/math.zig, gemma4/forward.zig ---- */
/* math.zig:19-25 / 42-48 (w == NULL); one_plus_w: out = x*r*(1+w)          */
void lto_rmsnorm(float *out, const float *x, const float *w, size_t n, float eps, int one_plus_w);
/* rmsnorm(a + b, w) with the sum rounded first                              */
void lto_add_rmsnorm(float *out, const float *a, const float *b, const float *w, size_t n, float eps,
                     int one_plus_w);
/* math.zig:51-82 rmsnormWeightedAndRawScaled                                */
void lto_rmsnorm_wrs(float *weighted_out, float *raw_scaled_out, const float *x, const float *w,
                     const float *raw_scale, float raw_global_scale, size_t n, float eps);
/* gemma4/forward.zig:482-497; moe and ffn are overwritten                   */
void lto_moe_tail(float *x, float *moe, float *ffn, const float *post_ffw_norm_2, const float *post_ffw_norm,
                  float layer_output_scale, size_t n, float eps);
/* gemma4/forward.zig:403-497: x (in/out) through the MoE block; dense_ffn is
 * the dense FFN output after post_ffw_norm_1. down_exps_scale may be NULL.  */
int lto_gemma4_moe_block(float *x, const float *dense_ffn, size_t d_model, const uint8_t *router_w,
                         uint32_t router_type, size_t n_experts, const uint8_t *gate_up, uint32_t gu_type,
                         const uint8_t *down, uint32_t dn_type, size_t down_cols, size_t k, size_t d_expert,
                         const float *pre_ffw_norm_2, const float *router_scale, const float *down_exps_scale,
                         const float *post_ffw_norm_2, const float *post_ffw_norm, float layer_output_scale,
                         float eps, uint32_t act, lto_pool *pool, uint32_t *out_ids, float *out_w);

#ifdef __cplusplus
}
#endif
#endif
