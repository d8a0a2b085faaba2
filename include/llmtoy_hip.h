/*
 * llmtoy_hip.h -- C ABI of the MI355X (gfx950) decode hot path.
 *
 * Stands in for llmtoy-zig's src/gpu Vulkan backend on the batch-1 decode
 * path: GGUF block-quantised matvec (Q8_0, Q4_K, Q6_K, F32) and the MoE layer
 * around it.  Plain C types only; one context per device; a context is not
 * thread-safe and launches everything on one HIP stream.
 *
 * Pointers passed to compute calls are device pointers unless LT_HOST_IO is
 * set, in which case they are host pointers, the call stages them through
 * context-owned device buffers and returns after the results are copied back.
 * Without LT_HOST_IO a call returns once the work is enqueued on the
 * context's stream (lt_sync waits for it).
 *
 * Graph capture.  Calls with device pointers (no LT_HOST_IO) may be captured
 * into a HIP graph on the context's stream (lt_stream).  Make one call with
 * the same shapes before capturing: the first call sizes the context's
 * scratch, and the first single-launch MoE call runs a one-time device probe
 * that cannot be captured (such a call returns LT_ERR_INVALID).  Scratch is
 * never freed before lt_destroy -- a later call with larger shapes gets new
 * buffers and retires the old ones -- so a captured graph stays valid for the
 * life of the context.  Replays of a graph and direct calls share scratch, so
 * they must not run concurrently (use the context's stream).
 *
 * Errors found on the device.  The single-launch MoE kernel bounds each of
 * its waits (200 ms); a wait that runs out makes that call's outputs NaN and
 * sets an error word.  A device-pointer call returns before that is known:
 * the next lt_sync (or LT_HOST_IO call) returns LT_ERR_DEVICE and clears it.
 * Callers that use device pointers should check lt_sync.
 *
 * Reference citations are paths in the llmtoy-zig tree.
 */
#ifndef LLMTOY_HIP_H
#define LLMTOY_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  The reference reports these conditions through Zig error
 * unions and null sessions that send the caller to its CPU path
 * (gemma4/forward.zig:434-480, gpu/matvec.zig:564-577). */
typedef enum {
    LT_OK = 0,
    LT_ERR_UNSUPPORTED = 1, /* type or shape the device path does not cover: use the CPU path */
    LT_ERR_INVALID = 2,     /* bad argument (null pointer, size mismatch, k out of range) */
    LT_ERR_DEVICE = 3,      /* HIP runtime error or no device */
    LT_ERR_OOM = 4          /* device allocation failed */
} lt_status;

/* GgmlType ids, gguf/types.zig:23-53 */
enum {
    LT_TYPE_F32 = 0,
    LT_TYPE_F16 = 1,
    LT_TYPE_Q8_0 = 8,
    LT_TYPE_Q4_K = 12,
    LT_TYPE_Q6_K = 14,
    /* the Gemma4 APEX expert formats (quant/dequant.zig:189-217, 366-486, 607-659) */
    LT_TYPE_Q5_0 = 6,
    LT_TYPE_Q5_1 = 7,
    LT_TYPE_Q3_K = 11,
    LT_TYPE_IQ4_NL = 20
};

/* Gated-FFN activation: SiLU (ops/math.zig:37-40) or GELU-tanh (math.zig:84-88). */
enum { LT_ACT_SILU = 0, LT_ACT_GELU_TANH = 1 };

enum {
    LT_HOST_IO = 1u << 0,       /* pointers are host memory; the call is synchronous */
    LT_MOE_NORM_TOPK = 1u << 1, /* renormalise the k selected weights to sum to 1 */
    LT_MOE_ACCUMULATE = 1u << 2, /* out += result (moeForward's contract, ops/moe.zig:17) */
    LT_MOE_UNFUSED = 1u << 3,    /* lt_moe_forward: run router, gate/up and down as separate launches
                                    instead of the single-launch kernel (same results to tolerance) */
    LT_MOE_DETERMINISTIC = 1u << 4 /* lt_moe_forward: add the k expert outputs in slot order (bit-identical
                                      results run to run, like the reference's moeForward, ops/moe.zig:67-76);
                                      without it the single-launch kernel adds them with float atomics in
                                      arrival order (faster; last bits may vary between runs) */,
    LT_NORM_PRECISE = 1u << 5,     /* RMS norms: sum the squares sequentially in index order on one lane,
                                      the reference's CPU order (math.zig:19-25), so results are bit-exact
                                      with it; default: a fixed-shape tree sum (same bits every run, within
                                      a few ulp of the CPU order; n dependent adds saved).  The reference's
                                      GPU norms offer the same choice (rmsnorm.glsl flag bit 1) */
    LT_NORM_ONE_PLUS_W = 1u << 6   /* lt_rmsnorm / lt_add_rmsnorm: multiply by (1 + w) instead of w
                                      (rmsnorm.glsl flag bit 0) */
};

typedef struct lt_ctx lt_ctx;
typedef struct lt_tensor lt_tensor;

/* Replaces GpuContext.init / deinit (gpu/context.zig:270-) and
 * GpuWeights.init / deinit (gemma4/gpu_weights.zig:373, 1065).
 * Environment: LT_FORCE_NO_DEVICE=1 makes lt_init fail with LT_ERR_DEVICE,
 * which callers treat like the reference's failed GpuContext.init
 * (main.zig:1889-1892): fall back to the CPU path. */
int lt_init(int device, lt_ctx **out_ctx);
void lt_destroy(lt_ctx *ctx);
/* Text of the last error on this context ("" if none). */
const char *lt_last_error(const lt_ctx *ctx);
/* Wait for all work enqueued on the context's stream. */
int lt_sync(lt_ctx *ctx);
/* The hipStream_t the context launches on (for events and interop). */
void *lt_stream(lt_ctx *ctx);

/* Upload one GGUF tensor (raw block bytes) into device memory the context
 * owns.  Replaces MatvecSession.initFromRaw (gpu/matvec.zig:564-577) and the
 * expert uploads of GpuWeights (gemma4/gpu_weights.zig:3660-3777).
 *   rows, cols : per-expert matrix shape (RawMatrix.rows/cols,
 *                model/model_weights.zig:17-22); cols is the GGUF row length.
 *   n_experts  : 1 for a 2-D tensor; E for the flattened 3-D expert tensors
 *                (gemma4/loader.zig:277-292): expert e's rows start at byte
 *                e * rows * rowBytes(type, cols).
 *   nbytes     : must equal n_experts * rows * rowBytes(type, cols)
 *                (ops/math.zig:194-208).
 * cols must be a multiple of the block size (32 for Q8_0, 256 for K-quants);
 * pad shorter rows with zero blocks.  The host buffer may be freed after the
 * call returns.  The device copy is repacked into a planar layout with the
 * same byte count: the GGUF bytes cross PCIe in 4 MiB pieces through pinned
 * staging buffers (up to 8 in flight) and a device kernel splits them into
 * the planes.  The context keeps that staging (up to 64 MiB pinned host and
 * 64 MiB device memory) until lt_destroy. */
int lt_tensor_upload(lt_ctx *ctx, const void *host_bytes, size_t nbytes, uint32_t ggml_type, size_t rows,
                     size_t cols, size_t n_experts, lt_tensor **out_tensor);
/* Read an uploaded tensor back as GGUF block bytes (nbytes must equal
 * lt_tensor_bytes); the inverse of lt_tensor_upload.  No counterpart in the
 * reference (its uploads are write-only); it lets a caller verify an upload
 * byte for byte. */
int lt_tensor_read(lt_ctx *ctx, const lt_tensor *t, void *host_bytes, size_t nbytes);
/* Copy an uploaded tensor (same layout) to a new device allocation; used to
 * rotate weight copies so that timing is not served from the 256 MB cache. */
int lt_tensor_clone(lt_ctx *ctx, const lt_tensor *src, lt_tensor **out_tensor);
int lt_tensor_free(lt_ctx *ctx, lt_tensor *t);
/* Read nbytes (a positive multiple of 16) of device memory at buf (16-byte
 * aligned) once, with a streaming kernel of 16-byte loads, on the context's
 * stream.  No counterpart in the reference: bench.py times it as the read
 * ceiling of one launch that the decode kernels' streams are set against. */
int lt_stream_read(lt_ctx *ctx, const void *buf, size_t nbytes);
/* Device bytes held by the tensor (equal to the GGUF byte count). */
size_t lt_tensor_bytes(const lt_tensor *t);

/* out[rows] = W[rows x cols] * x[cols], fp32 accumulation.  Activations are
 * fp32, except for Q4_K and Q6_K rows of 1, 2, 4, 8 or 16 super-blocks
 * (cols 256..4096, powers of two): there each group of 16 activations is
 * split into two int8 limbs, x ~= sp * (256 a + b) with sp = max|x| / 32512
 * (|error| <= max|x| / 65024 per element, about 2e-5 rel-L2 on the dot
 * product), which meet the weight codes in v_dot4; a group holding a NaN or
 * an infinity makes every output NaN.
 * Replaces quantMatvec / quantMatvecPar (ops/math.zig:133-171, 277-320) and
 * MatvecSession.run / runQ8_1Mv (gpu/matvec.zig:497-647,
 * gemma4/gpu_weights.zig:1573-1607).  W must be a 2-D tensor. */
int lt_matvec(lt_ctx *ctx, float *out, const lt_tensor *W, const float *x, uint32_t flags);

/* Dense gated FFN: out[d_model] = Wd * (act(Wg x) * (Wu x)).
 * Replaces the dense-FFN matvec chain (model/forward.zig:301-308,
 * gemma4/forward.zig:392-397; GPU: runLayerDenseFfnQ8_1, gpu_weights.zig).
 * Q8_0 weights with d_model <= 2048 and d_ffn <= 8192 (multiples of 32,
 * down K == d_ffn) run as one launch whose 8 partial sums per output row
 * meet through float atomics (last bits may vary run to run); LT_MOE_UNFUSED
 * runs gate/up and down as two launches instead.  flags: LT_HOST_IO,
 * LT_MOE_UNFUSED. */
int lt_ffn_dense(lt_ctx *ctx, float *out, const lt_tensor *Wg, const lt_tensor *Wu, const lt_tensor *Wd,
                 const float *x, uint32_t act, uint32_t flags);

/* Router logits, softmax and top-k (selection on the logits: strict '>', the
 * lowest index wins ties).  ids[k], weights[k] in selection order.
 * scores (may be NULL) receives n_experts values as routerTopKSoftmax leaves
 * its scores buffer: the logit of every unselected expert, the (unnormalised)
 * softmax probability of every selected one.
 * weights = exp(l - max) / sum_all exp(l - max), or renormalised over the
 * selection with LT_MOE_NORM_TOPK.  bias (may be NULL) is added to each logit.
 * F32 routers reproduce dotf32's accumulation order bit for bit
 * (ops/math.zig:96-116); Q8_0 routers reproduce dotQ8_0's
 * (quant/dequant.zig:59-78).  Replaces routerTopKSoftmax / softmaxTopK
 * (gemma4/forward.zig:637-668) and MoeRouterTopKPipeline
 * (gpu/matvec.zig:2630-2721). */
int lt_moe_router_topk(lt_ctx *ctx, const lt_tensor *router, const float *x, const float *bias, uint32_t k,
                       uint32_t flags, uint32_t *ids, float *weights, float *scores);

/* Expert-indexed gate/up: h[s][j] = act(G_e x)[j] * (U_e x)[j] for slot s,
 * e = ids[s], j < d_expert; h rows are padded with zeros to down_cols.
 * gate_up is the flattened [E, 2*d_expert, d_model] tensor (gate rows then
 * up rows per expert, ops/moe.zig:55-73).  h is [k, down_cols] fp32.  A
 * device pointer x must be 16-byte aligned.
 * Replaces ExpertGateUpIdPipeline (gpu/matvec.zig:1348-1460). */
int lt_expert_gate_up_id(lt_ctx *ctx, const lt_tensor *gate_up, const float *x, const uint32_t *ids, uint32_t k,
                         uint32_t d_expert, uint32_t down_cols, uint32_t act, float *h, uint32_t flags);

/* Expert-indexed down with the weighted combine fused:
 * out[i] = sum_{s<k, in slot order} weights[s] * (D_{ids[s]} h[s])[i]
 * (plus the previous out[i] with LT_MOE_ACCUMULATE).  A device pointer h
 * must be 16-byte aligned.
 * Replaces ExpertDownIdPipeline + AccumPipeline (gpu/matvec.zig:1465-1610,
 * 833-1008). */
int lt_expert_down_id(lt_ctx *ctx, const lt_tensor *down, const float *h, const uint32_t *ids,
                      const float *weights, uint32_t k, float *out, uint32_t flags);

/* One MoE layer for one token: router -> top-k -> expert gate/up -> down ->
 * weighted combine, optionally plus a shared dense FFN (sh_* non-NULL):
 * out = shared_ffn(x) + sum_s w_s * expert_s(x).
 * Replaces moeForward (ops/moe.zig:18-77) and GpuWeights.runExpertBatch
 * (gemma4/gpu_weights.zig:2748-3149).  out_ids / out_w (may be NULL)
 * receive the routing.  d_expert is the expert FFN width; down's cols may be
 * larger (zero-padded K).  One launch of the single-launch kernel where the
 * layer fits it (F32 or Q8_0 router, d_model 256..4096, down K <= 1024, <=
 * 256 experts, k <= 16): Q4_K experts (with a Q8_0 shared FFN in the same
 * launch), or Q3_K / Q4_K gate_up with IQ4_NL, Q5_0 or Q5_1 down (atomic
 * combine, the shared FFN then first, as the base); other expert types and
 * LT_MOE_UNFUSED run router, gate/up and down as separate launches. */
int lt_moe_forward(lt_ctx *ctx, float *out, const float *x, const lt_tensor *router, const float *router_bias,
                   const lt_tensor *gate_up, const lt_tensor *down, const lt_tensor *sh_gate,
                   const lt_tensor *sh_up, const lt_tensor *sh_down, uint32_t k, uint32_t d_expert, uint32_t act,
                   uint32_t flags, uint32_t *out_ids, float *out_w);

/* lt_moe_forward without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory -- code
 * under HIP graph capture, serving loops that forbid hipMalloc.  Same
 * arguments and results as lt_moe_forward, on the single-launch kernel only:
 * F32 or Q8_0 router, Q4_K gate_up and down, d_model 256..4096 (a multiple
 * of 256), down K <= 1024, <= 256 experts, k <= 16, optionally a Q8_0 shared
 * FFN with down K == d_ffn in 256..4096 (then without LT_MOE_DETERMINISTIC),
 * device pointers only (flags: LT_MOE_NORM_TOPK, LT_MOE_ACCUMULATE,
 * LT_MOE_DETERMINISTIC); any other shape, type or flag returns
 * LT_ERR_UNSUPPORTED or LT_ERR_INVALID.  Its scratch is the library's static
 * device array of 762,368 bytes per GPU (held until the process ends, set up
 * by lt_init): all calls on one GPU share it, so calls that overlap on one
 * GPU (several streams or contexts at once) race. */
int lt_moe_forward_noalloc(lt_ctx *ctx, float *out, const float *x, const lt_tensor *router,
                           const float *router_bias, const lt_tensor *gate_up, const lt_tensor *down,
                           const lt_tensor *sh_gate, const lt_tensor *sh_up, const lt_tensor *sh_down, uint32_t k,
                           uint32_t d_expert, uint32_t act, uint32_t flags, uint32_t *out_ids, float *out_w);

/* Batched prefill of one MoE layer over T tokens (X, out: [T, d_model]):
 * per-token routing as lt_moe_router_topk, tokens sorted per expert, grouped
 * expert GEMM with f16 MFMA (fp32 accumulation) over Q4_K weights
 * dequantised in LDS, then a combine in slot order.  The reference prefills
 * one token at a time through the decode path (main.zig:1916-1922); results
 * match per-token lt_moe_forward to f16 tolerance.  Each X row is divided by
 * a power of two 2^e that puts its largest element in [1, 2) and the expert
 * activations between the two GEMMs are kept divided by 2^(2e) (f16 tiles,
 * exact rescaling), so rows of any magnitude stay inside f16's range; an
 * activation that still passes +-65504 saturates there, is counted, and the
 * call (LT_HOST_IO) or the next lt_sync returns LT_ERR_DEVICE naming the
 * count.  Device pointers X and out must be 16-byte aligned. */
int lt_moe_prefill(lt_ctx *ctx, float *out, const float *X, uint32_t T, const lt_tensor *router,
                   const float *router_bias, const lt_tensor *gate_up, const lt_tensor *down, uint32_t k,
                   uint32_t d_expert, uint32_t act, uint32_t flags, uint32_t *out_ids, float *out_w);

/* Profiling (the counterpart of the reference's GpuProfiler, gpu/context.zig:
 * 34-268, enabled there by LLMTOY_GPU_PROFILE).  With LT_PROFILE set when
 * lt_init runs, every call records a HIP event pair around the device work it
 * enqueues (not while the stream is being captured); LT_PROFILE=timeline also
 * makes the single-launch MoE kernel record, per workgroup, the wall-clock
 * time at which each phase of its role ended (router: first row data, logit
 * published; gate/up: logits seen, expert known, dot products done, h
 * published; down: logits seen, weight loads issued, h read, adds issued).
 * Events and stamps are collected at synchronising calls (lt_sync, LT_HOST_IO
 * calls): the stamps of the last single-launch MoE kernel before each.
 * lt_profile_report writes a text table (per-call counts and times, per-phase
 * medians) into buf (NUL-terminated, truncated to len) and returns the full
 * length; 0 when LT_PROFILE is off.  No counterpart of the allocation-free
 * entry point's spans: lt_moe_forward_noalloc records phase stamps only. */
size_t lt_profile_report(lt_ctx *ctx, char *buf, size_t len);

/* ---- RMS norms and the Gemma4 MoE block (Gemma4's steps around the MoE layer) ----
 * Row length n <= 16384 floats; eps in [0, 1].  Every product and sum is a
 * separately rounded fp32 operation and rms_inv = 1 / sqrt(ss / n + eps)
 * with correctly rounded division and square root, as in the reference.
 * flags: LT_HOST_IO, LT_NORM_PRECISE (and where noted LT_NORM_ONE_PLUS_W). */

/* math.rmsnorm (ops/math.zig:19-25): out = x * rms_inv(x) * w; w == NULL is
 * rmsnormRaw (42-48).  Each of rows rows of n floats is normalised on its
 * own (the reference normalises one vector: rows = 1).  out may equal x.
 * Also takes LT_NORM_ONE_PLUS_W.  Replaces the rmsnorm pipeline
 * (gpu/shaders/rmsnorm.glsl). */
int lt_rmsnorm(lt_ctx *ctx, float *out, const float *x, const float *w, uint32_t rows, uint32_t n, float eps,
               uint32_t flags);
/* out = rmsnorm(a + b, w), the sum rounded first (gemma4/forward.zig:489-490;
 * gpu/shaders/add_rmsnorm.glsl).  Also takes LT_NORM_ONE_PLUS_W. */
int lt_add_rmsnorm(lt_ctx *ctx, float *out, const float *a, const float *b, const float *w, uint32_t rows,
                   uint32_t n, float eps, uint32_t flags);
/* math.rmsnormWeightedAndRawScaled (ops/math.zig:51-82): one RMS of x;
 * weighted_out = x * rms_inv * w, raw_scaled_out = x * (rms_inv *
 * raw_global_scale) * raw_scale.  Gemma4 uses it for the expert and router
 * inputs (gemma4/forward.zig:403-414). */
int lt_rmsnorm_weighted_raw_scaled(lt_ctx *ctx, float *weighted_out, float *raw_scaled_out, const float *x,
                                   const float *w, const float *raw_scale, float raw_global_scale, uint32_t n,
                                   float eps, uint32_t flags);
/* The Gemma4 MoE tail in one launch (gemma4/forward.zig:482-497; on the
 * reference's GPU, GpuWeights.recordMoeResidualTail, gemma4/gpu_weights.zig:
 * 3349-3410):  m = rmsnorm(moe, post_ffw_norm_2); c = dense_ffn + m;
 * x = x + rmsnorm(c, post_ffw_norm); then x *= layer_output_scale unless it
 * is 1.  x is read and written. */
int lt_moe_tail(lt_ctx *ctx, float *x, const float *moe, const float *dense_ffn, const float *post_ffw_norm_2,
                const float *post_ffw_norm, float layer_output_scale, uint32_t n, float eps, uint32_t flags);
/* The whole Gemma4 MoE block of one decode token after the dense FFN
 * (gemma4/forward.zig:403-497; GpuWeights.runExpertBatch with MoeTailParams,
 * gemma4/gpu_weights.zig:2748-3149):
 *   moe_in, router_in = rmsnormWeightedAndRawScaled(x, pre_ffw_norm_2,
 *                       router_scale, 1 / sqrt(d_model))
 *   routerTopKSoftmax(router, router_in) -> k ids, softmax probabilities p
 *   moe = sum_k down_exps_scale[id] * p * down_id(act(gate_id moe_in) * up_id moe_in)
 *   x   = lt_moe_tail(x, moe, dense_ffn, ...)
 * x [d_model] is updated in place; dense_ffn is the dense FFN output after
 * post_ffw_norm_1.  down_exps_scale [n_experts] may be NULL (all ones).
 * router: F32 or Q8_0; experts: Q4_K, Q3_K, Q5_0, Q5_1 or IQ4_NL (device x:
 * 16-byte aligned).  With a Q8_0 router, Q4_K or Q3_K gate/up, Q4_K,
 * IQ4_NL, Q5_0 or Q5_1 down and the default tree sums the whole block is
 * one launch of the single-launch MoE kernel
 * (router-input prep in its router blocks, the expert input in its gate/up
 * blocks, the tail in one block after the down blocks); otherwise the
 * router-input prep runs inside the Q8_0 router kernel, or in a norm
 * kernel, and the experts and the tail in launches of their own.  The
 * single launch adds the experts' rows with float atomics, so the last bits
 * of x may differ run to run (as lt_moe_forward's default combine).  flags:
 * LT_HOST_IO, LT_NORM_PRECISE, LT_MOE_NORM_TOPK, LT_MOE_UNFUSED (separate
 * launches), LT_MOE_DETERMINISTIC (the separate launches, whose down kernel
 * adds in slot order: bit-identical run to run).  out_ids / out_w (may be
 * NULL) get the selection and its probabilities (router_out at the selected
 * ids). */
int lt_gemma4_moe_block(lt_ctx *ctx, float *x, const float *dense_ffn, const lt_tensor *router,
                        const lt_tensor *gate_up, const lt_tensor *down, const float *pre_ffw_norm_2,
                        const float *router_scale, const float *down_exps_scale, const float *post_ffw_norm_2,
                        const float *post_ffw_norm, float layer_output_scale, float eps, uint32_t k,
                        uint32_t d_expert, uint32_t act, uint32_t flags, uint32_t *out_ids, float *out_w);

#ifdef __cplusplus
}
#endif
#endif /* LLMTOY_HIP_H */
