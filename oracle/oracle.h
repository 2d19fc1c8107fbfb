/*
 * oracle.h -- CPU fp32 restatement of rustane's transformer forward token loop.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path (librustane_hip.so) and the timed CPU baseline.  Only the test suite,
 * the smoke check and the benchmark's CPU-baseline leg load it.  The product
 * path never links, loads or calls anything in this directory.
 *
 * Every function follows a file of the reference (whiskeypolitik/rustane,
 * crates/engine/src/...), cited next to its declaration.  The reference keeps
 * activations channel-first [D, S] (x[d*S + s]); the oracle does the same for
 * the functions that mirror the reference's CPU ops, and uses token-major
 * [S, *] internally where that only changes the loop order, not the
 * arithmetic.
 *
 * vDSP / cblas calls in the reference (cpu/vdsp.rs) map to portable C++
 * loops with the same contracts: vsma out = a*s + b, vsub out = b - a,
 * sgemm_at C += A * B^T (beta = 1), mtrans.
 *
 * Parity pins (what checks each function; tests/test_oracle_kats.py and
 * tests/test_golden_losses.py):
 *   orc_random_vec            bit-exact vs an independent numpy LCG; golden losses
 *   orc_embedding_forward     reference KATs (cpu/embedding.rs:46-94)
 *   orc_rmsnorm_*             reference KATs + closed form (cpu/rmsnorm.rs:244-369)
 *   orc_silu_gate             reference KATs + closed form (cpu/silu.rs:48-109)
 *   orc_cross_entropy_*       reference KATs, gradients sum to 0, numerical gradient
 *                             (cpu/cross_entropy.rs:98-155), logsumexp via numpy
 *   orc_vsma/vsub/mtrans/sgemm_at  reference KATs (cpu/vdsp.rs:404-483) + numpy matmul
 *   orc_rope_table / orc_sdpa_fwd  textbook brute force in float64 on tiny shapes;
 *                             p = 0 identity; norm preservation; causality
 *   orc_forward (tail)        reference-held golden losses (results/forward_utilization/
 *                             scale_ladder.json, results/2026-03-18_1830_param-sweep.md)
 *   orc_forward (body)        layer = independent numpy float64 restatement on tiny shapes;
 *                             FFN/attention branch linearity in Wo and W2
 *   orc_decode_*              decode logits at position p == orc_forward logits at p
 *   orc_forward_backward      every gradient vs float64 autograd of an independent
 *                             torch restatement of the forward (tiny shapes, softcap on
 *                             and off, loss_scale); accumulation (+=) across calls
 *   orc_rmsnorm_backward_*, orc_silu_gate_backward
 *                             reference numerical-gradient KATs (cpu/rmsnorm.rs:278-316,
 *                             cpu/silu.rs:68-90) + float64 autograd
 *   orc_adam_step_fused       the reference's Adam unit tests (cpu/adam.rs:138-190:
 *                             moves toward the minimum, weight decay alone shrinks,
 *                             m = 0.1 and v = 0.001 after one unit-gradient step) +
 *                             closed form of the first step (|update| = 1 when wd = 0)
 *   orc_learning_rate         closed form at the warmup and cosine end points
 *   orc_sdpa_backward, orc_rope_backward
 *                             float64 autograd of the textbook forward; RoPE backward
 *                             is the inverse rotation (round trip to identity)
 *
 * Parity unpinned: the ANE's bit-level fp16 numerics (accumulation order, its
 * softmax) that the reference executes inside the un-vendored `ane` crate; no
 * vectors for them exist, only the reference's tolerances, so this
 * restatement is fp32 and the GPU path is held to those tolerances.
 */
#ifndef RUSTANE_ORACLE_H
#define RUSTANE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ModelConfig (crates/engine/src/model.rs:5-17); MHA only (kv_heads == heads). */
typedef struct {
    int32_t dim, hidden, heads, head_dim, nlayers, vocab;
    float rms_eps;   /* 1e-5, cpu/rmsnorm.rs:10 */
    float rope_base; /* 1e4,  kernels/sdpa_fwd.rs:29 */
    float softcap;   /* 0 = off, full_model.rs:75 */
    /* 0: fp32 throughout (the reference's CPU arithmetic).  Otherwise a set
     * of ORC_F16_* bits: the forward and decode round to fp16 (round to
     * nearest even) at those points, which are where an fp16-operand device
     * path must round (ORC_F16_ALL).  Used to separate kernel error from the
     * fp16 operand precision at full depth; not used by the backward pass. */
    int32_t fp16_operands;
} orc_config;

#define ORC_F16_XN 1     /* first RMSNorm output (QKV operand)                  */
#define ORC_F16_Q 2      /* q after RoPE                                        */
#define ORC_F16_K 4      /* k after RoPE (the K cache)                          */
#define ORC_F16_V 8      /* v (the V cache)                                     */
#define ORC_F16_P 16     /* unnormalised probabilities into P.V, multi-token passes only; row sums stay fp32 */
#define ORC_F16_ATTN 32  /* attention output (Wo operand)                       */
#define ORC_F16_XN2 64   /* second RMSNorm output (W1|W3 operand)               */
#define ORC_F16_GATE 128 /* SwiGLU gate (W2 operand)                            */
#define ORC_F16_XF 256   /* final RMSNorm output (logits operand)               */
#define ORC_F16_ALL 511

/* ModelWeights (full_model.rs:19-23) + LayerWeights (layer.rs:52-63), fp32 host
 * arrays in the reference orientation.  layers[9*l + j], j in RSTK order:
 *   0 wq [D, D] (in x out)   1 wk [D, D]   2 wv [D, D]   3 wo [D, D] (q_dim x D)
 *   4 w1 [D, F]              5 w3 [D, F]   6 w2 [D, F] (out x in, used transposed)
 *   7 gamma1 [D]             8 gamma2 [D]                                       */
typedef struct {
    const float* embed;       /* [V, D] */
    const float* gamma_final; /* [D]    */
    const float* const* layers;
} orc_weights;

/* ---- vDSP / cblas contracts (cpu/vdsp.rs:150-402) ---- */
void orc_vsma(const float* a, float s, const float* b, float* out, size_t n);
void orc_vsub(const float* a, const float* b, float* out, size_t n);
void orc_mtrans(const float* a, size_t a_cols, float* c, size_t c_cols, size_t m, size_t n);
void orc_sgemm_at(const float* a, size_t m, size_t k, const float* b, size_t n, float* c);

/* ---- CPU ops ---- */
void orc_random_vec(float* out, size_t n, float scale);
void orc_embedding_forward(const float* table, size_t dim, const uint32_t* ids, size_t seq,
                           float* out);
float orc_rmsnorm_forward(const float* x, const float* gamma, float* out, size_t dim, float eps);
void orc_rmsnorm_forward_channel_first(const float* x, const float* gamma, float* out,
                                       float* rms_inv, size_t dim, size_t seq, float eps);
void orc_silu_gate(const float* gate, const float* up, float* out, size_t n);
float orc_cross_entropy_forward(const float* logits, size_t vocab, uint32_t target,
                                float* log_sm /* nullable [vocab] */);
float orc_cross_entropy_forward_backward_batch(const float* logits, const uint32_t* targets,
                                               size_t seq, size_t vocab, float* dlogits,
                                               float inv_seq);

/* ---- attention (kernels/sdpa_fwd.rs) ---- */
void orc_rope_table(size_t seq, size_t hd, float base, float* cos_buf, float* sin_buf);
/* xnorm [D, S] channel-first; outputs [D, S] channel-first (q_rope, k_rope, v
 * nullable). */
void orc_sdpa_fwd(const orc_config* cfg, size_t seq, const float* xnorm, const float* wq,
                  const float* wk, const float* wv, float* attn_out, float* q_rope,
                  float* k_rope, float* v);

/* ---- layer / model ---- */
/* layer::forward (layer.rs:4409-4624): x [D, S] -> x_next [D, S]. */
void orc_layer_forward(const orc_config* cfg, size_t seq, const float* const* lw,
                       const float* x, float* x_next);
/* full_model::forward / forward_losses (full_model.rs:915-991, 1603-1660) for
 * `batch` independent sequences of length `seq` (the multistream model,
 * multistream.rs:54-161).  Returns 0 on success.
 *   logits_out        nullable [B, S, V]
 *   token_losses_out  nullable [B, S]
 *   mean_loss_out     nullable [B]   (total / S, cross_entropy.rs:58-96 + full_model.rs:987) */
int orc_forward(const orc_config* cfg, const orc_weights* w, const uint32_t* tokens,
                const uint32_t* targets, int batch, int seq, float* logits_out,
                float* token_losses_out, float* mean_loss_out);

/* ---- backward (the training pass) ---- */
/* ModelGrads (full_model.rs) + LayerGrads: the shapes and orientation of
 * orc_weights, every array accumulated into (+=), as the reference does. */
typedef struct {
    float* dembed;       /* [V, D] */
    float* dgamma_final; /* [D]    */
    float* const* layers; /* layers[9*l + j], RSTK order as in orc_weights */
} orc_grads;
/* full_model::forward then backward_ws (full_model.rs:915-991, 592-702;
 * layer::backward_into, layer.rs:7037-7366) for `batch` independent
 * sequences; each adds loss_scale x its gradient of its mean loss into g.
 * mean_loss_out nullable [B].  Returns 0 on success. */
int orc_forward_backward(const orc_config* cfg, const orc_weights* w, const uint32_t* tokens,
                         const uint32_t* targets, int batch, int seq, float loss_scale,
                         const orc_grads* g, float* mean_loss_out);
/* rmsnorm::backward_channel_first (cpu/rmsnorm.rs:185-240): [dim, seq]. */
void orc_rmsnorm_backward_channel_first(const float* dy, const float* x, const float* gamma,
                                        const float* rms_inv, float* dx, float* dgamma, size_t dim,
                                        size_t seq);
/* SiLU-gate backward of layer::backward_into (layer.rs:7083-7104). */
void orc_silu_gate_backward(const float* dgate, const float* h1, const float* h3, float* dh1,
                            float* dh3, size_t n);
/* sdpa_bwd graphs (kernels/sdpa_bwd.rs:44-300), token-major [seq, D] (q, k
 * after RoPE); dq, dk, dv are overwritten. */
void orc_sdpa_backward(const orc_config* cfg, size_t seq, const float* q, const float* k,
                       const float* v, const float* da, float* dq, float* dk, float* dv);
/* rope_backward_inplace (layer.rs:7389-7407), token-major [seq, D]. */
void orc_rope_backward(const orc_config* cfg, float* dx, size_t seq);

/* ---- optimizer (the training step's update) ---- */
/* AdamW step_fused (cpu/adam.rs:95-132; the Metal shader metal_adam.rs:16-40
 * computes the same): g = grad*grad_scale; m = b1*m + (1-b1)*g;
 * v = b2*v + (1-b2)*g*g; update = (m*bc1) / (sqrt(v*bc2) + eps);
 * param -= lr*(update + wd*param), bc1 = 1/(1 - b1^t), bc2 = 1/(1 - b2^t).
 * grad may be NULL (treated as zeros). */
void orc_adam_step_fused(float* param, const float* grad, float* m, float* v, size_t n, uint32_t t, float lr,
                         float beta1, float beta2, float eps, float weight_decay, float grad_scale);
/* b^t by repeated squaring in fp32 (the f32::powi of the bias corrections). */
float orc_powi(float b, uint32_t t);
/* vDSP_svesq (cpu/vdsp.rs:329-335): sum of squares in fp32. */
float orc_svesq(const float* x, size_t n);
/* learning_rate (full_model.rs:903-913): linear warmup, then cosine to
 * max_lr * min_lr_frac. */
float orc_learning_rate(uint32_t step, float max_lr, float min_lr_frac, uint32_t warmup_steps,
                        uint32_t total_steps);

/* ---- single-token decode with a KV cache (no reference implementation;
 *      contract: logits at step p equal the forward's logits at position p) ---- */
typedef struct orc_kv orc_kv;
orc_kv* orc_kv_create(const orc_config* cfg, int max_ctx);
void orc_kv_destroy(orc_kv* kv);
int orc_kv_pos(const orc_kv* kv);
/* Runs the prompt through the model, filling the cache; logits of the last
 * prompt position into last_logits (nullable [V]). */
int orc_prefill(const orc_config* cfg, const orc_weights* w, orc_kv* kv, const uint32_t* tokens,
                int len, float* last_logits);
/* One token at position kv->pos; logits_out [V]; returns argmax (ties -> lowest). */
int orc_decode_step(const orc_config* cfg, const orc_weights* w, orc_kv* kv, uint32_t token,
                    float* logits_out);

/* Threads the oracle's OpenMP loops use. */
/* B sequences with their own caches in one pass (the layers' GEMMs over all
 * B*len rows at once, attention per sequence); same results as B separate
 * orc_prefill / orc_decode_step calls up to fp32 summation order.
 * tokens [B*len] (sequence-major); last_logits nullable [B, V];
 * decode: tokens [B], logits_out [B, V], argmax_out nullable [B]. */
int orc_prefill_batch(const orc_config* cfg, const orc_weights* w, orc_kv* const* kvs, int B,
                      const uint32_t* tokens, int len, float* last_logits);
int orc_decode_step_batch(const orc_config* cfg, const orc_weights* w, orc_kv* const* kvs, int B,
                          const uint32_t* tokens, float* logits_out, int32_t* argmax_out);
int orc_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
