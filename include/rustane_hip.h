/*
 * rustane_hip.h -- C-ABI of librustane_hip.so, the MI355X (gfx950) forward
 * token loop and greedy decode path for rustane's engine.
 *
 * This library takes the place of the reference's device bridge: the `ane`
 * crate re-exported by crates/ane-bridge/src/lib.rs:1-9 (MIL graph build,
 * Graph::compile, Executable::run_cached_direct, fp16 IOSurface TensorData)
 * plus the Accelerate calls of crates/engine/src/cpu/vdsp.rs that the forward
 * makes.  Above it, the engine's forward/loss API (full_model::forward,
 * forward_ws, forward_only_ws, forward_losses) keeps its signatures and
 * weight layout; a Rust `hip-bridge` crate binds these symbols.
 *
 * Conventions (mirroring the reference's full_model.rs / layer.rs):
 *  - All functions return RH_OK (0) on success or a negative RH_E* code; the
 *    message is available from rh_last_error().  Nothing throws across the
 *    boundary.
 *  - Host pointers are owned by the caller and are only read or written
 *    during the call.  Device pointers (the *_dev entry points) must stay
 *    valid until the context's stream has drained (rh_sync).
 *  - A context owns one GPU, one HIP stream and all device memory (fp16
 *    weights, KV cache, workspaces); training adds a second stream of its
 *    own for the weight gradients, joined back into the context stream
 *    before rh_forward_backward returns.  A context is driven by one thread
 *    at a time; separate contexts may run concurrently (multistream.rs:54-161).
 *  - Activations are token-major inside the library; the weight tensors come
 *    in and go out in the reference orientation (layer.rs:52-63).
 */
#ifndef RUSTANE_HIP_H
#define RUSTANE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RH_OK 0
#define RH_EINVAL -1     /* bad argument / unsupported shape            */
#define RH_ERANGE -2     /* token id >= vocab, batch or length too big   */
#define RH_ENOMEM -3     /* device allocation failed                     */
#define RH_EDEVICE -4    /* HIP runtime error                            */
#define RH_ESTATE -5     /* call out of order (e.g. decode before prefill) */
#define RH_EIO -6        /* file missing, unreadable or not in the format */

/* ModelConfig (crates/engine/src/model.rs:5-17).  MHA only: kv_heads must
 * equal heads (the reference reshapes K/V with `heads`, sdpa_fwd.rs:162-181).
 * head_dim is 64 or 128; dim % 128 == 0, dim <= 8192; hidden % 128 == 0; vocab % 4 == 0. */
typedef struct rh_config {
    int32_t dim, hidden, heads, kv_heads, head_dim, seq, nlayers, vocab;
    float rms_eps;   /* 1e-5  (cpu/rmsnorm.rs:10)                */
    float rope_base; /* 1e4   (kernels/sdpa_fwd.rs:29)           */
    float softcap;   /* 0=off (full_model.rs:75, :569-576)       */
} rh_config;

typedef struct rh_ctx rh_ctx;

/* Replaces CompiledKernels::{compile, try_compile, compile_forward_only}
 * (layer.rs:843-969) + KernelBuffers::allocate* (layer.rs:170-641): binds a
 * device, creates the stream, allocates fp16 weights and the KV cache for
 * max_batch sequences of up to max_ctx positions (max_ctx = 0: no cache).
 * No JIT: kernels are precompiled for gfx950. */
int rh_create(const rh_config* cfg, int device, int max_batch, int max_ctx, rh_ctx** out);
void rh_destroy(rh_ctx* ctx);
/* Last error message of the context; with ctx NULL, of the calling thread's
 * last context-free call (token files, checkpoint header, compute_bpb). */
const char* rh_last_error(const rh_ctx* ctx);
/* The context's configuration and capacities (any output may be NULL). */
int rh_context_info(const rh_ctx* ctx, rh_config* cfg_out, int* max_batch_out, int* max_ctx_out);

/* Uploads ModelWeights (full_model.rs:19-23) in the reference orientation,
 * fp32 -> fp16 for matrices, fp32 for gammas; replaces the per-call weight
 * staging of layer.rs:4670-4705 (done once here).  layer_tensors holds
 * nlayers*9 pointers in RSTK order (bin/train.rs:238-345):
 *   wq[D,D] wk[D,D] wv[D,D] wo[D,D] w1[D,F] w3[D,F] w2[D,F] gamma1[D] gamma2[D]
 * (wq/wk/wv/wo/w1/w3 are in x out; w2 is out x in, used transposed).
 * Each matrix passes through a device staging buffer the size of the
 * largest tensor.  When the context keeps fp32 master weights
 * (rh_set_fp32_masters, or once an optimizer state exists) the matrices
 * land in them instead, so rh_read_weights_f32 returns them exactly and
 * training continues from the exact values; any optimizer moments restart
 * from zero (ModelOptState::zeros after load_checkpoint,
 * bin/train.rs:444-449). */
int rh_load_weights_f32(rh_ctx* ctx, const float* embed, const float* gamma_final,
                        const float* const* layer_tensors);

/* Whether the context keeps fp32 master weights on the device (4 bytes per
 * parameter: 26.4 GB at 7B, twice the fp16 weights).  Off by default, so
 * forward-only and decode contexts hold the fp16 weights alone.  keep = 1
 * allocates them now (holding the current weights widened from fp16) and
 * makes later fp32 loads write through them; a training run calls it right
 * after rh_create, where the reference compiles its kernels before
 * load_checkpoint / ModelWeights::random (bin/train.rs:427-448), so the
 * optimizer starts from the exact fp32 weights.  keep = 0 frees them
 * (RH_ESTATE once the optimizer state exists, which owns them).  Without
 * masters, the first rh_update_weights creates them from the fp16 device
 * weights.  No counterpart in the reference, whose weights are host fp32. */
int rh_set_fp32_masters(rh_ctx* ctx, int keep);

/* Downloads the weights in the reference orientation: the fp32 masters when
 * they hold the current weights (after an fp32 load or an optimizer step),
 * otherwise the fp16 device copy widened; same argument layout as
 * rh_load_weights_f32, but writable.  Any pointer may be NULL to skip that
 * tensor. */
int rh_read_weights_f32(rh_ctx* ctx, float* embed, float* gamma_final,
                        float* const* layer_tensors);

/* Synthetic weights generated on the device: every matrix (embed, wq..w2)
 * i.i.d. N(0, std^2) from Philox4x32-10 keyed by (seed, tensor id), gammas
 * = 1.  No counterpart in the reference, whose init is ModelWeights::random
 * (full_model.rs:132-141); it exists so multi-GB configs need no host copy. */
int rh_init_weights_normal(rh_ctx* ctx, uint64_t seed, float std);

/* full_model::forward / forward_only_ws / forward_losses
 * (full_model.rs:378-472, 915-991, 1603-1660) for `batch` independent
 * sequences of `seq` tokens (multistream.rs semantics, one launch).
 * tokens/targets [batch*seq] (targets may be NULL if no loss is wanted).
 *   logits_out       nullable [batch, seq, vocab] fp32 (post-softcap)
 *   token_losses_out nullable [batch, seq]  (forward_losses)
 *   mean_loss_out    nullable [batch]        (forward: total/seq)     */
int rh_forward(rh_ctx* ctx, const uint32_t* tokens, const uint32_t* targets, int batch, int seq,
               float* logits_out, float* token_losses_out, float* mean_loss_out);

/* Same as rh_forward with every pointer in device memory, enqueued on the
 * context stream without synchronising (no counterpart in the reference:
 * it is the HBM-resident form a serving loop uses).  Token ids are clamped to
 * the vocabulary on the device and counted; rh_sync reports RH_ERANGE if any
 * were out of range. */
int rh_forward_dev(rh_ctx* ctx, const uint32_t* tokens, const uint32_t* targets, int batch,
                   int seq, float* logits_out, float* token_losses_out, float* mean_loss_out);

/* Training pass: full_model::forward then full_model::backward / backward_ws
 * (full_model.rs:592-702, 915-991; layer::backward_into, layer.rs:7037-7366)
 * for `batch` independent sequences of `seq` tokens.  Adds loss_scale times
 * the gradient of each sequence's mean loss to the context's fp32 gradients
 * (they accumulate across calls, as the reference's ModelGrads do; see
 * rh_zero_grads).  The first call allocates the gradients (the parameter
 * count in fp32), transposed fp16 weight copies and per-layer activation
 * caches, and creates the weight-gradient stream.  Synchronises before
 * returning.  mean_loss_out nullable [batch].  Needs hidden % 64 == 0. */
int rh_forward_backward(rh_ctx* ctx, const uint32_t* tokens, const uint32_t* targets, int batch, int seq,
                        float loss_scale, float* mean_loss_out);
/* The same pass in two calls, for callers of full_model::forward ->
 * ForwardResult (full_model.rs:120-129, 915-991) followed by
 * full_model::backward(&fwd, tokens, softcap, loss_scale, grads)
 * (full_model.rs:996-1010), e.g. crates/engine/tests/phase4_training.rs:61-72.
 * rh_forward_train runs the training forward with logit softcap `softcap`
 * (mean_loss_out nullable [batch]) and keeps its caches on the device; *out
 * receives a handle to them (free it with rh_forward_result_free).
 * rh_backward adds loss_scale times the gradient of that forward to the
 * gradients (as rh_forward_backward does: forward then backward gives the
 * same gradients bit for bit) and, when grad_norm_out is not NULL, writes
 * the L2 norm of the accumulated gradients (rh_grad_norm), the reference
 * backward's return value.  tokens (the forward's input tokens) and softcap
 * must equal the forward's (RH_EINVAL otherwise).  The caches live in the
 * context: any later call that runs a forward on it (rh_forward*,
 * rh_prefill, rh_validate, rh_forward_backward, another rh_forward_train)
 * makes the handle stale and rh_backward returns RH_ESTATE.  A handle may
 * be consumed more than once, each backward accumulating again. */
typedef struct rh_forward_result rh_forward_result;
int rh_forward_train(rh_ctx* ctx, const uint32_t* tokens, const uint32_t* targets, int batch, int seq,
                     float softcap, float* mean_loss_out, rh_forward_result** out);
int rh_backward(rh_ctx* ctx, const rh_forward_result* fwd, const uint32_t* tokens, float softcap, float loss_scale,
                float* grad_norm_out);
void rh_forward_result_free(rh_forward_result* fwd);
/* ModelGrads::zero_out: sets every gradient to 0. */
int rh_zero_grads(rh_ctx* ctx);
/* Copies the gradients to host fp32 arrays in the orientation and RSTK order
 * of rh_load_weights_f32 (every pointer nullable; layer_grads[9*l + j] may be
 * NULL to skip a tensor).  RH_ESTATE before the first rh_forward_backward. */
int rh_read_grads_f32(rh_ctx* ctx, float* dembed, float* dgamma_final, float* const* layer_grads);

/* Fills the KV cache from `batch` prompts of `len` tokens (planned
 * metal-decode path, crates/metal-decode/src/lib.rs:1-8) and sets the decode
 * position to len.  next_tok_out (nullable [batch]) receives the argmax of
 * the last position's logits, last_logits_out (nullable [batch, vocab]) the
 * logits themselves.  batch <= min(max_batch, 16). */
int rh_prefill(rh_ctx* ctx, const uint32_t* tokens, int batch, int len, uint32_t* next_tok_out,
               float* last_logits_out);

/* One greedy decode step for the batch set by rh_prefill (batch must equal
 * it, RH_EINVAL otherwise; the arrays hold exactly batch entries): embeds
 * in_tok [batch] at the current position, appends K/V, returns the argmax
 * token (ties -> lowest id) in out_tok [batch] and optionally logits
 * [batch, vocab].  Contract: logits equal the forward's logits at that
 * position. */
int rh_decode_step(rh_ctx* ctx, int batch, const uint32_t* in_tok, uint32_t* out_tok, float* logits_out);

/* rh_decode_step without any allocation: no counterpart in the reference.
 * For callers that cannot allocate device memory or runtime objects (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  in_tok [batch], out_tok [batch] and logits_out (nullable
 * [batch, vocab]) are DEVICE pointers (in_tok may equal out_tok: each step
 * then feeds its argmax to the next); batch must equal the prefill batch.
 * The step is enqueued on the context stream (rh_stream) without
 * synchronising; rh_sync waits and reports clamped out-of-range ids.  The
 * step reads and advances the context's device-side position, so a step
 * captured into a graph (on the context stream) moves forward on every
 * replay; the next rh_decode_step, rh_decode or rh_decode_pos re-reads that
 * position.  A replay at a full cache writes nothing to it and its outputs
 * are undefined (rh_sync then returns RH_ERANGE).  Its scratch
 * (activations, attention and argmax partials; the logits too when
 * logits_out is NULL) lives in a fixed 64 MiB device array per GPU, cut
 * into four 16 MiB slots: a context takes one at its first call and keeps
 * it until rh_destroy, so up to four contexts per GPU use this entry point
 * at once (RH_ERANGE for a fifth), and no two share scratch.  RH_ERANGE
 * when the batch and model need more than a slot (7B at batch 16 needs
 * about 4 MiB). */
int rh_decode_step_noalloc(rh_ctx* ctx, int batch, const uint32_t* in_tok, uint32_t* out_tok,
                           float* logits_out);

/* nsteps greedy steps run entirely on the device (each step's argmax is the
 * next step's input); out_tokens [nsteps, batch].  Starts from in_tok
 * [batch]; batch must equal the prefill batch. */
int rh_decode(rh_ctx* ctx, int batch, const uint32_t* in_tok, int nsteps, uint32_t* out_tokens);

/* Logit softcap c for later calls (c * tanh(z / c), 0 = off); the reference
 * passes it per forward call (full_model.rs:569-576). */
int rh_set_softcap(rh_ctx* ctx, float softcap);

/* Current decode position (tokens in the cache). */
int rh_decode_pos(rh_ctx* ctx, int* pos_out);

/* Waits for the context stream; returns the first deferred device error. */
int rh_sync(rh_ctx* ctx);
/* The context's hipStream_t, for callers that time or order work on it. */
void* rh_stream(rh_ctx* ctx);

/* Per-kernel-class timing with HIP events on the context stream: while
 * enabled, every launch of `kernel_class` in the forward, prefill and decode calls is
 * timed by an event pair (bracketing the launch; for RH_K_GEMM_W13 stamped at
 * the GEMM kernel's own start and end); rh_profile_read returns the summed
 * time and the launch count since rh_profile_enable.  Not a reference
 * interface: it serves the benchmark's per-kernel roofline figure.  Classes: */
#define RH_K_GEMM_QKV 0
#define RH_K_GEMM_WO 1
#define RH_K_GEMM_W13 2
#define RH_K_GEMM_W2 3
#define RH_K_GEMM_LOGITS 4
#define RH_K_ATTN 5
#define RH_K_GEMV_QKV 6
#define RH_K_GEMV_WO 7
#define RH_K_GEMV_W13 8
#define RH_K_GEMV_W2 9
#define RH_K_GEMV_LOGITS 10
#define RH_K_DECODE_ATTN 11
#define RH_K_NCLASSES 12
int rh_profile_enable(rh_ctx* ctx, int kernel_class, int enable);
int rh_profile_read(rh_ctx* ctx, int kernel_class, double* total_ms, int64_t* launches);

/* Forward calls (one graph per batch, seq and loss/no-loss, built on first
 * use) and decode steps as captured HIP graphs (1, default), or eager
 * launches (0).  While a kernel class is being timed (rh_profile_enable)
 * forwards launch eagerly. */
int rh_set_graphs(rh_ctx* ctx, int enable);

/* ---- on-disk formats either side of the forward ----------------------- */

/* RSTK v1 checkpoint (bin/train.rs:238-345): "RSTK", then version, step, dim,
 * nlayers, vocab, seq as little-endian u32 (28 bytes), then fp32 tensors
 * embed[V*D], gamma_final[D] and per layer wq wk wv wo w1 w3 w2 gamma1
 * gamma2 in the rh_load_weights_f32 orientation.  hidden is not stored. */
typedef struct rh_ckpt_info {
    uint32_t version, step, dim, nlayers, vocab, seq;
    uint64_t file_bytes;
} rh_ckpt_info;
/* Reads the header only (context-free). */
int rh_checkpoint_info(const char* path, rh_ckpt_info* out);
/* load_checkpoint (bin/train.rs:296-345): maps the file and uploads its
 * weights.  The header's dim/nlayers/vocab must match the context and the
 * file must hold exactly the tensors of the context's config; step_out
 * (nullable) receives the stored step. */
int rh_load_checkpoint(rh_ctx* ctx, const char* path, uint32_t* step_out);
/* save_checkpoint (bin/train.rs:238-275) of the device weights (fp16
 * widened to fp32; seq = the context's seq); written to path.tmp, renamed. */
int rh_save_checkpoint(rh_ctx* ctx, const char* path, uint32_t step);

/* TokenData (data.rs:11-44): a memory-mapped flat little-endian uint16 token
 * file (a trailing odd byte is ignored). */
typedef struct rh_tokens rh_tokens;
int rh_tokens_open(const char* path, rh_tokens** out);
void rh_tokens_close(rh_tokens* tokens);
int64_t rh_tokens_len(const rh_tokens* tokens);
/* tokens(start, len) widened to u32; RH_ERANGE past the end. */
int rh_tokens_read(const rh_tokens* tokens, int64_t start, int len, uint32_t* out);

/* compute_bpb (data.rs:75-91): over the n (loss, target) pairs whose
 * token_bytes[target] > 0, bpb = sum(loss) / (ln 2 * sum(bytes)), summed in
 * order in fp32 (0 when no bytes).  token_bytes holds `vocab` int32 entries
 * (token_bytes.bin, data.rs:46-71).  Any output may be NULL. */
int rh_compute_bpb(const float* losses, const uint32_t* targets, int64_t n, const int32_t* token_bytes,
                   int vocab, float* bpb_out, float* total_nats_out, int64_t* total_bytes_out);

/* validate (bin/train.rs:196-236): `steps` windows of the context's seq at
 * pos = (s * seq) % (len - seq - 1), input tokens(pos, seq), targets
 * tokens(pos + 1, seq); per-token losses by the forward (forward_losses,
 * full_model.rs:1603-1660), up to max_batch windows per launch.
 * avg_loss_out = sum of losses / tokens; bpb_out = compute_bpb over all
 * windows when token_bytes ([vocab]) is given, else 0.  Needs
 * len >= seq + 2. */
int rh_validate(rh_ctx* ctx, const rh_tokens* val, const int32_t* token_bytes, int steps,
                float* avg_loss_out, float* bpb_out);

/* ---- optimizer and training step ---- */
/* TrainConfig (full_model.rs:42-78). */
typedef struct {
    float max_lr, min_lr_frac;
    uint32_t warmup_steps, total_steps;
    float beta1, beta2, eps, weight_decay, matrix_lr_scale, embed_lr_scale, loss_scale;
    uint32_t accum_steps;
    float grad_clip, softcap;
} rh_train_config;
/* TrainConfig::default (full_model.rs:59-78). */
void rh_train_config_default(rh_train_config* out);
/* learning_rate (full_model.rs:903-913): linear warmup, cosine decay to
 * max_lr * min_lr_frac. */
float rh_learning_rate(uint32_t step, const rh_train_config* tc);
/* grad_norm (full_model.rs:1403-1450): L2 norm of all gradients (per-block
 * fp32 sums of squares of every tensor, added in double on the device; 0
 * while the gradients are zero). */
int rh_grad_norm(rh_ctx* ctx, float* norm_out);
/* update_weights (full_model.rs:1123-1400): one AdamW step_fused
 * (cpu/adam.rs:95-132) at step count t >= 1 over every parameter, gradients
 * multiplied by grad_scale: the embedding at lr * embed_lr_scale and the
 * gammas at lr without weight decay, the seven matrices per layer at
 * lr * matrix_lr_scale with weight_decay.  The first call allocates the
 * optimizer state: first and second moments (zero) and, unless
 * rh_set_fp32_masters made them, the fp32 master weights (read from the
 * fp16 device weights).  With masters, rh_load_weights_f32 and
 * rh_load_checkpoint write them exactly, rh_init_weights_normal leaves them
 * to be re-read from the fp16 copy; every weight write restarts the moments
 * from zero.  After an update rh_read_weights_f32 (and rh_save_checkpoint)
 * return the fp32 masters. */
int rh_update_weights(rh_ctx* ctx, uint32_t t, float lr, const rh_train_config* tc, float grad_scale);
/* train_step / train_step_with_options (full_model.rs:1488-1600): zero the
 * gradients; accum_steps sequences of the context's seq from `data` at
 * pos = (step * 7919 + micro * 104729) % (len - seq - 1) (inputs
 * tokens(pos, seq), targets shifted by one), forward + backward with
 * tc->loss_scale (up to max_batch sequences per launch); clip by the global
 * norm (combined scale = grad_clip / norm when norm / (accum_steps *
 * loss_scale) > grad_clip, else 1 / (accum_steps * loss_scale)); AdamW at
 * t = step + 1 with learning_rate(step).  The training forward uses
 * tc->softcap; the context's own softcap is unchanged afterwards.  loss_out: mean loss of the microbatches;
 * grad_norm_out: the norm divided by accum_steps * loss_scale. */
int rh_train_step(rh_ctx* ctx, const rh_tokens* data, uint32_t step, const rh_train_config* tc, float* loss_out,
                  float* grad_norm_out);

/* ---- request scheduler (multistream::ForwardScheduler, multistream.rs:54-161) ----
 * One worker thread owns the context and serves a bounded FIFO in batches:
 * up to max_batch forward requests of equal length run as one rh_forward,
 * generation requests of equal prompt length and step count as one
 * rh_prefill + rh_decode (batch <= 16).  The worker waits up to max_wait_us
 * after the oldest request for a batch to fill (0: serve what is queued).
 * While a scheduler exists only its worker may use the context. */
#define RH_JOB_FORWARD 0   /* tokens/targets [len] -> loss (forward_only_ws)   */
#define RH_JOB_GENERATE 1  /* prompt [len] -> nsteps greedy tokens (out_tokens) */
typedef struct rh_sched rh_sched;
typedef struct rh_sched_config {
    int max_batch;       /* requests per launch (also capped by the context)  */
    int queue_capacity;  /* submit blocks while this many are queued           */
    int max_wait_us;
} rh_sched_config;
typedef struct rh_sched_request {
    uint64_t request_id;
    int kind, len, nsteps;
    const uint32_t* tokens;   /* copied at submit                              */
    const uint32_t* targets;  /* forward only, copied at submit                */
    uint32_t* out_tokens;     /* generate only: written before the result is posted */
} rh_sched_request;
typedef struct rh_sched_result {   /* ForwardBenchResult (multistream.rs:35-42) + batch/status */
    uint64_t request_id;
    int kind, status;         /* status: RH_OK or the failing call's code      */
    float loss;               /* forward: mean CE over the request's tokens    */
    int batch;                /* requests served in the same launch            */
    float queue_wait_ms, service_ms, total_ms;
    char message[128];        /* error text when status != RH_OK               */
} rh_sched_result;
int rh_sched_create(rh_ctx* ctx, const rh_sched_config* cfg, rh_sched** out);
/* Drains the queue, then stops the worker. */
void rh_sched_destroy(rh_sched* sched);
int rh_sched_submit(rh_sched* sched, const rh_sched_request* request);
/* Blocks for the next finished request (RH_ESTATE if none is outstanding). */
int rh_sched_wait(rh_sched* sched, rh_sched_result* out);
/* ForwardScheduler::run_batch: submits n requests, waits for all, results
 * sorted by request id (no other requests may be outstanding). */
int rh_sched_run_batch(rh_sched* sched, const rh_sched_request* requests, int n,
                       rh_sched_result* results);

#ifdef __cplusplus
}
#endif
#endif
