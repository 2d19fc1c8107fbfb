// rh_kernels.h -- host-side launchers for the gfx950 kernels (internal).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

typedef _Float16 f16;

namespace rh {

// ---------------- prefill GEMM:  Y[m][n] = sum_k X[m][k] * W[n][k] -------------
// EPI_SWIGLU_SAVE is EPI_SWIGLU that also stores the fp16 pre-activations
// h1, h3 (planes [M][F] at h13 and h13 + M*F) for the backward pass.
enum GemmEpi { EPI_F32 = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_QKV = 3, EPI_SWIGLU_SAVE = 4, EPI_SILU_BWD = 5 };

struct GemmArgs {
    const f16* W;  // [N, K] weights ("out x in"), fragment order (frag_off), rows padded to 16
    const f16* X;  // [M, K] activations (token-major), fragment order, rows padded to 16
    int M, N, K;
    float* out_f32;  // EPI_F32: [M, ldo]; EPI_RESID: residual x [M, ldo], updated in place
    f16* out_f16;    // EPI_SWIGLU: gate [M, ldo] in fragment order
    int ldo;
    float alpha;     // EPI_RESID: x += alpha * acc; EPI_F32: out = alpha * acc (0 = unscaled)
    const float* resid_in;  // EPI_RESID: the residual read, [M, ldo] (null: out_f32, in place)
    float softcap;   // EPI_F32: c * tanh(acc / c) when c > 0
    // EPI_QKV: N = 3*D rows ordered q | k | v; RoPE on q and k.
    f16* q;          // [B][H][S][hd]
    f16* kc;         // [B][H][ctx][hd]
    f16* vc;         // [B][H][ctx][hd]
    const float2* rope;  // [pos][hd/2] (cos, sin)
    int S, D, H, hd, ctx, pos0;
    f16* h13;        // EPI_SWIGLU_SAVE (written) / EPI_SILU_BWD (read): h1 | h3 planes, [2][M][ldo] fp16
                     // row-major.  EPI_SILU_BWD: acc is the gate gradient [M][ldo = N]; out_f16 gets
                     // dh1 | dh3 in fragment order [M][2N]
    // Stream-K workspace (optional): fp32 partial tiles.
    float* sk_part;
    size_t sk_part_floats;
    int force_cfg;  // 0 = heuristic; otherwise a GemmCfg value (tuning)
    bool nt_out;    // EPI_F32 / EPI_RESID: nontemporal output stores (data read much later)
    // Optional timing: stamped at the kernel's own start and end by the
    // one-block-per-tile launch (hipExtLaunchKernelGGL), recorded around the
    // launches otherwise.
    hipEvent_t prof_start, prof_stop;
};
// Tile configurations of the prefill GEMM (all: direct-to-LDS 4-stage
// pipeline; waves x per-wave tile).
enum GemmCfg {
    GCFG_AUTO = 0,
    GCFG_D8_256x256 = 6,     // 8 waves (128x64 each)
    GCFG_D8_256x256_SK = 7,  // ... stream-K
    GCFG_D4_128x128 = 8,     // 4 waves (64x64 each)
    GCFG_D4_128x128_SK = 9,
    GCFG_D8_256x128 = 10,    // 8 waves (64x64 each), 16x16x32 MFMA
    GCFG_D8_256x128_SK = 11,
    GCFG_D4_256x256 = 12,    // 4 waves (128x128 each, accumulators in AGPRs)
    GCFG_D4_256x256_SK = 13,
    GCFG_D4_256x128 = 14,    // 4 waves (128x64 each)
    GCFG_D4_256x128_SK = 15,
    GCFG_D4_192x128 = 16,    // 4 waves (96x64 each)
    GCFG_D4_192x128_SK = 17,
    GCFG_D8_192x256 = 18,    // 8 waves (96x64 each), 16x16x32 MFMA
    GCFG_D8_192x256_SK = 19,
    GCFG_D4_192x256 = 20,    // 4 waves (96x128 each, accumulators in AGPRs)
    GCFG_D4_192x256_SK = 21,
    GCFG_D8_192x128 = 24,    // 8 waves (96x32 each), 16x16x32 MFMA
    GCFG_D8_192x128_SK = 25,
    GCFG_D8_128x128 = 26,    // 8 waves (64x32 each), 16x16x32 MFMA
    GCFG_D8_128x128_SK = 27,
};
// Floats of stream-K workspace any prefill GEMM needs.
size_t gemm_sk_part_floats();
hipError_t launch_gemm(int epi, const GemmArgs& a, hipStream_t st);
// Residual projection followed by the next RMSNorm:
//   x [M, N] += alpha * (X W^T)            (a.out_f32 = x, a.ldo = N; with
//                                           a.resid_in set, x = resid_in + ...)
//   xn = rmsnorm(x) * gamma, fp16 in fragment order (skipped when gamma is null).
// With few output tiles (narrow N, small M) K is split: every split writes an
// fp32 partial into a.sk_part and one row kernel sums the partials in split
// order (deterministic), adds the residual and normalises -- no stream-K
// fix-up kernel and no separate norm pass.  Otherwise the GEMM's own residual
// epilogue runs, then the norm.  Needs N % 8 == 0 and N <= 8192.
hipError_t launch_gemm_resid_norm(const GemmArgs& a, const float* gamma, float eps, f16* xn,
                                  hipStream_t st);
// X W^T as *nsplit >= 2 fp32 partials [M][N] at a.sk_part + s * M * N, to be
// summed in split order by the consumer, when the output has too few tiles
// to fill the CUs (the same split as launch_gemm_resid_norm); otherwise
// *nsplit = 0 and nothing is launched.  Needs K % 128 == 0, N % 8 == 0.
hipError_t launch_gemm_partials(const GemmArgs& a, int* nsplit, hipStream_t st);
// Weight-gradient GEMM for a short K (the token count): out [M][ldo] fp32 =
// alpha * X W^T (alpha 0: unscaled), or += when accumulate; persistent blocks
// whose store waves write each 128x128 tile while the next one is computed.
// Needs K % 128 == 0, N % 4 == 0.
hipError_t launch_gemm_wgrad(const GemmArgs& a, bool accumulate, hipStream_t st);

// ---------------- attention ----------------
// Causal prefill attention: q [B][H][S][hd], k/v [B][H][ctx][hd] (positions
// 0..S-1), out token-major [B*S][H*hd] in fragment order (rows padded to 16).
// lse (nullable) [B][H][S]: per query log2-sum-exp2 of the scaled scores.
hipError_t launch_attn_prefill(const f16* q, const f16* k, const f16* v, f16* out, int B, int H,
                               int S, int hd, int ctx, hipStream_t st, float* lse = nullptr);
// Decode attention over positions 0..*pos (the current token is at *pos):
// q [B][H*hd], K/V caches [B][H][ctx][hd], out [B][H*hd] fp16.  The cache is
// split into nch = attn_decode_chunks(B, H, ctx) chunks per (b, h) (a
// positive nch forces that many equal chunks: tuning); with more than one,
// per-chunk partials (m, l, o[hd]) go to part_* ([B][H][nch] entries) and a
// merge kernel writes out.  out_frag: out in fragment order (frag_off over
// H*hd columns, 16 rows), the decode GEMV's x_frag input.
constexpr int ATTN_DEC_CHUNK = 128;
hipError_t launch_attn_decode(const f16* q, const f16* k, const f16* v, const int* pos,
                              float* part_m, float* part_l, float* part_o, f16* out, int B, int H,
                              int hd, int ctx, hipStream_t st, int nch = 0, bool out_frag = false);
int attn_decode_chunks(int B, int H, int ctx);

// ---------------- decode GEMV (B <= 16 tokens) ----------------
enum GemvEpi { GV_F32 = 0, GV_RESID = 1, GV_SWIGLU = 2, GV_QKV = 3 };
struct GemvArgs {
    const f16* W;  // [N, K]
    const f16* X;  // [B, K]
    int B, N, K;
    float* out_f32;  // GV_F32 [B, ldo], GV_RESID x [B, ldo]
    f16* out_f16;    // GV_SWIGLU gate [B, ldo]; GV_QKV q [B, D]
    int ldo;
    float alpha, softcap;
    f16* kc; f16* vc;  // GV_QKV: [B][H][ctx][hd]
    const float2* rope;
    const int* pos;    // device position
    int D, H, hd, ctx;
    // GV_F32 only (optional): per-block argmax partials [B][gemv_argmax_blocks(N)]
    float* am_val;
    int* am_idx;
    int cfg;           // 0 = default (waves, depth) variant; 1..gemv_num_variants() forces one
    // Optional in-kernel RMSNorm (not GV_RESID): X is ignored and the input is
    // rmsnorm(xres [B, K] fp32) * gamma, eps; needs gemv_norm_fits(B, K).
    const float* xres;
    const float* gamma;
    float eps;
    // Optional, GV_RESID: also write the next RMSNorm's input as
    // xg_out [B, N] = fp16(x_new * gnext) and this block's per-token sum of
    // x_new^2 over its 16 rows, ssq_out[blockIdx * 16 + token].
    f16* xg_out;
    const float* gnext;
    float* ssq_out;
    // Optional, not GV_RESID: X holds such fp16(x * gamma) rows; each
    // token's 1/rms comes from rs_n blocks of ssq partials (rs_part) and eps,
    // and scales the accumulators before the epilogue.
    const float* rs_part;
    int rs_n;
    // Fragment-order activations (frag_off, 16 rows; rows >= B are read and
    // their results dropped, so the buffer must hold 16 rows): x_frag for X,
    // out_frag for the fp16 rows a later GEMV reads (GV_RESID's xg_out,
    // GV_SWIGLU's gate).  Every X load then reads 1 KB contiguous (8 cache
    // lines), where a row-major one touches a line per live token.
    bool x_frag, out_frag;
};
// W is fp16 [N, K] in fragment order (frag_off), rows padded to a multiple of 16.
hipError_t launch_gemv(int epi, const GemvArgs& a, hipStream_t st);
// Decode batches whose GEMV inputs (attention output, gate, x * gamma) go in
// fragment order, 16 rows.  A row-major X load touches one cache line per
// live token (lane row r reads token r; rows past B reread token 0), a
// fragment-order one always 8: standalone, the W2 GEMV takes 15.9 us
// row-major up to 8 tokens, then 0.45 us more per token (17.2 at 11, 19.1 at
// 16), and 17.2 us in fragment order at any count.
constexpr bool gemv_frag_inputs(int B) { return B >= 12; }
int gemv_num_variants();
constexpr size_t GEMV_NORM_LDS = 32768;  // bytes of normalised rows a block may stage
bool gemv_norm_fits(int B, int K);
int gemv_argmax_blocks(int N);
// Greedy token from the logits GEMV's argmax partials (ties -> lowest id):
// writes out[b], next_in[b] (nullable), seq_out[state[1]*B + b] (nullable),
// then state[0] += 1, state[1] += 1 when advance is set and state[0] < limit
// (else ERR_PAST_CACHE is or-ed into *err, when err is not null).
hipError_t launch_argmax_final(const float* pv, const int* pi, int nblk, int B, uint32_t* out,
                               uint32_t* next_in, uint32_t* seq_out, int* state, bool advance, int limit,
                               int* err, hipStream_t st);
// Bit of the context's device error word: a decode step ran at a position
// past the KV cache (its other bits count clamped token ids).
constexpr int ERR_PAST_CACHE = 1 << 30;

// ---------------- row ops ----------------
hipError_t launch_embed(const uint32_t* tok, const f16* E, float* x, int rows, int D, int V,
                        int* err, hipStream_t st);
// out [rows, D] row-major, or in fragment order (frag_off, rows padded to 16)
// when frag is set (the layout of every prefill GEMM operand).
hipError_t launch_rmsnorm(const float* x, const float* gamma, f16* out, int rows, int D,
                          float eps, hipStream_t st, bool frag = false);
// rmsnorm of rows x[(r*stride + offset)] -> out[r]  (last-position gather)
hipError_t launch_rmsnorm_strided(const float* x, const float* gamma, f16* out, int rows, int D,
                                  float eps, int stride_rows, int offset_rows, hipStream_t st);
// x [rows, D] = xin + alpha * sum_s part[s*split_stride + row*D ...] (s =
// 0..S-1 in order; xin may be x), then out = rmsnorm(x) * gamma in fragment
// order when gamma is set.  D % 8 == 0, D <= 8192.
hipError_t launch_resid_norm(const float* xin, float* x, const float* part, int S, size_t split_stride,
                             float alpha, const float* gamma, float eps, f16* out, int rows, int D,
                             hipStream_t st);
hipError_t launch_cross_entropy(const float* logits, const uint32_t* targets, float* loss,
                                int rows, int V, int* err, hipStream_t st);
hipError_t launch_mean_rows(const float* loss, float* mean, int B, int S, hipStream_t st);
hipError_t launch_set_state(int* state, int pos, int step, hipStream_t st);
hipError_t launch_fill_f32(float* p, float v, size_t n, hipStream_t st);

// ---------------- training (backward pass) ----------------
// Backward activations are held in internal units: the CE gradient is stored
// as (softmax - onehot) * GRAD_UNIT (see rh_trainops.hip).
constexpr float GRAD_UNIT = 16.0f;
// dl [rows][ldd] fp16 fragment order (zero in columns V..ldd-1) from the
// (softcapped when softcap > 0) logits [rows][V] and targets.
hipError_t launch_ce_backward(const float* logits, const uint32_t* targets, f16* dl, int rows, int V, int ldd,
                              float softcap, float unit, hipStream_t st);
// dst [C][Rp] (fragment order) = transpose of src [R][C] (fragment order),
// zero in columns R..Rp-1; map 1 reads the W1|W3 interleaved SwiGLU weight
// as [W1 rows | W3 rows].  C % 128 == 0, Rp % 128 == 0.
hipError_t launch_transpose_frag(const f16* src, f16* dst, int R, int C, int Rp, int map, hipStream_t st);
// Two map-0 transposes with the same padded token count in one launch.
hipError_t launch_transpose_frag2(const f16* src0, f16* dst0, int R0, int C0, const f16* src1, f16* dst1, int R1,
                                  int C1, int Rp, hipStream_t st);
// RMSNorm backward over M rows: dx = rmsnorm'(x)^T dy (+ dres), optional
// fp16 fragment-order copy of hscale * dx, per-block dgamma partials
// [rms_backward_blocks(M)][D].  dy is the sum of nsplit (1..8) fp32 partials
// [M][D] split_stride floats apart, added in order.  dx may alias dres.
int rms_backward_blocks(int M);
hipError_t launch_rms_backward(const float* dy, int nsplit, size_t split_stride, const float* x,
                               const float* gamma, const float* dres, float* dx, f16* outh, float hscale,
                               float* dg_part, int M, int D, float eps, hipStream_t st);
// dgamma[d] += kappa * sum_b part[b][d]  (= instead of += when store is set)
hipError_t launch_dgamma_reduce(const float* part, int nblk, int D, float kappa, float* dgamma, bool store,
                                hipStream_t st);
// dembed[utok[u]] += kappa * dy[idx[j]] for j in [start[u], start[u+1]).
hipError_t launch_embed_backward(const float* dy, const uint32_t* utok, const int* start, const int* idx, int nuniq,
                                 float kappa, float* dembed, int D, hipStream_t st);
// Causal attention backward: q, k, v [B][H][S][hd] fp16 (q, k after RoPE), o
// the forward output (fragment order [B*S][H*hd]), dOf [B*S][H*hd] fp32 as
// the sum of nsplit (1..8) partials split_stride floats apart, lse from the
// forward.  Workspace dOh (fp16 [B][H][S][hd]) and Drow ([B][H][S]).
// Writes dqkv, the dX GEMM's operand: fp16 in fragment order [B*S][3*H*hd]
// (dq | dk | dv, the RoPE backward applied to dq and dk with the table rope
// [S][hd/2]).
hipError_t launch_attn_backward(const f16* q, const f16* k, const f16* v, const f16* o, const float* dOf,
                                int nsplit, size_t split_stride, const float* lse, f16* dOh, float* Drow,
                                f16* dqkv, const float2* rope, int B, int H, int S, int hd, hipStream_t st);

// ---------------- optimizer ----------------
// One AdamW step (step_fused) with its constants: omb1 = 1 - beta1,
// omb2 = 1 - beta2, bc1 = 1/(1 - beta1^t), bc2 = 1/(1 - beta2^t), gradients
// multiplied by gscale.
struct AdamArgs {
    float lr, beta1, beta2, omb1, omb2, eps, wd, gscale, bc1, bc2;
};
// Elementwise AdamW over n fp32 values (grad null = zeros); when dst is set
// also writes the fp16 row-packed copy (fragment order, K columns).
hipError_t launch_adam_rows(float* p, const float* g, float* m, float* v, size_t n, const AdamArgs& a, f16* dst,
                            int K, hipStream_t st);
// AdamW over a [R][C] tensor whose fp16 copy is transposed (the packing of
// launch_pack_transpose: row dst_row(c), k = r, K = ldd).
hipError_t launch_adam_transpose(float* p, const float* g, float* m, float* v, int R, int C, const AdamArgs& a,
                                 f16* dst, int ldd, int map, int row_off, hipStream_t st);
// Per-block sums of squares of x[0..n) into part[0..sumsq_blocks(n)).
int sumsq_blocks(size_t n);
hipError_t launch_sumsq(const float* x, size_t n, float* part, hipStream_t st);
// *out = the sum of part[0..n) in double (one block; a fixed order).
hipError_t launch_sum_parts(const float* part, size_t n, double* out, hipStream_t st);

// ---------------- weight packing ----------------
// Device weights are fp16 [N, K] in fragment order (frag_off in rh_device.h),
// N padded to a multiple of 16.
// Transposing pack: element (row_map(c), k = r) = half(src[r*C + c]) for a
// [R][C] fp32 source, K = ldd.  map: 0 identity rows (dst row = row_off + c),
// 1 = W1/W3 interleave in 16-row groups (dst row = 32*(c/16) + c%16 + row_off,
// row_off 0 for W1 and 16 for W3).
hipError_t launch_pack_transpose(const float* src, f16* dst, int R, int C, int ldd, int map,
                                 int row_off, hipStream_t st);
hipError_t launch_unpack_transpose(const f16* src, float* dst, int R, int C, int lds, int map,
                                   int row_off, hipStream_t st);
// Row pack: element (row, k) = half(src[row*K + k]) for a [R][K] source.
hipError_t launch_pack_rows(const float* src, f16* dst, int R, int K, hipStream_t st);
hipError_t launch_unpack_rows(const f16* src, float* dst, int R, int K, hipStream_t st);
hipError_t launch_convert_f32_f16(const float* src, f16* dst, size_t n, hipStream_t st);
hipError_t launch_convert_f16_f32(const f16* src, float* dst, size_t n, hipStream_t st);
hipError_t launch_init_normal(float* dst, size_t n, uint64_t seed, uint32_t tensor_id, float std,
                              hipStream_t st);

}  // namespace rh
