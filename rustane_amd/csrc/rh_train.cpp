// rh_train.cpp -- the training pass behind include/rustane_hip.h:
// full_model::forward + backward_ws (full_model.rs:915-991, 592-702) with
// layer::backward_into (layer.rs:7037-7366) per layer.
//
// The forward is the inference forward's kernels with every activation the
// backward needs kept per layer (the ForwardCache of layer.rs:79-126): the
// layer input and post-attention residuals (fp32), the normalised GEMM
// operands, q/k/v, the attention output and its log-sum-exp, the SwiGLU
// pre-activations and gate.  The backward then runs, per layer in reverse:
//
//   dW2 += dffn^T gate          dgate = dffn W2          (SiLU backward) -> dh1|dh3
//   dx_ffn = dh1 W1^T + dh3 W3^T    dW1, dW3 += x2n^T dh{1,3}
//   dx2 = RMSNorm2'(dx_ffn) + dy    da = (a dx2) Wo^T    dWo += attn^T (a dx2)
//   attention backward -> dq, dk, dv   (RoPE backward on dq, dk)
//   dxn = dq Wq^T + dk Wk^T + dv Wv^T   dWq, dWk, dWv += xn^T d{q,k,v}
//   dy' = RMSNorm1'(dxn) + dx2
//
// Every product is an NT GEMM of the forward's kernel: the data-gradient
// GEMMs stream transposed copies of the weights (built once per weight
// version), the weight-gradient GEMMs contract over tokens and take
// token-inner (transposed) copies of their operands, and accumulate into the
// fp32 gradients in their epilogue (C += kappa * acc).  Gradients keep the
// reference's tensor shapes and orientation and accumulate across calls.
#include "rh_ctx.h"

#include <algorithm>
#include <array>
#include <cmath>
#include <cstring>
#include <map>
#include <vector>

namespace rhrt {

struct TrainState {
    // M: token capacity of the buffers; Mp: this call's token count B * S
    // rounded up to 128 (the K of the weight-gradient GEMMs, <= capacity's)
    int M = 0, Mp = 0, B = 0, S = 0;
    uint64_t packs_gen = 0;            // weight version the transposed copies hold
    bool zero = true;  // every gradient is 0: the weight-gradient GEMMs store instead of accumulating
    // fp32 gradients, reference orientation (RSTK order per layer)
    float *dembed = nullptr, *dgf = nullptr;
    std::vector<std::array<float*, 9>> dlay;
    // transposed fp16 weights (fragment order)
    f16* embed_t = nullptr;  // [D][Vp]
    struct WT { f16 *qkvt, *ot, *w13t, *w2t; };
    std::vector<WT> wt;
    // per-layer forward caches
    struct Cache {
        float *xin, *x2, *lse;
        f16 *xn, *q, *k, *v, *attn, *x2n, *h13, *gate;
    };
    std::vector<Cache> c;
    float* xlast = nullptr;  // residual after the last layer
    f16* xf = nullptr;       // final RMSNorm rows (fragment order)
    // backward workspace
    // Activation gradients in fp16 fragment order, one buffer per role so each
    // is rewritten only once per layer: H1 = the layer's output gradient times
    // alpha (dffn), H1m = alpha * dx2, H2 = [dh1 | dh3], H2q = [dq | dk | dv].
    f16 *dlh = nullptr, *dlT = nullptr, *H1 = nullptr, *H1m = nullptr, *H2 = nullptr, *H2q = nullptr;
    // The weight-gradient GEMMs run on the side stream in four groups per
    // layer (0: dW2, 1: dW1 dW3, 2: dWo, 3: dWq dWk dWv), each after its
    // token-inner operand copies tx[g] (written on the side stream too, from
    // the activation gradient above and a forward cache).  ready[g] (main):
    // group g's activation gradient is written; read[g] (side): the copy has
    // read it, so the main stream may rewrite that buffer a layer later.
    f16* tx[4][2] = {};
    hipStream_t side = nullptr;
    hipEvent_t ready[5] = {}, read[4] = {};  // ready[4]: the logits gradient
    f16* dOh = nullptr;
    float *gout = nullptr, *dres = nullptr, *Drow = nullptr, *dgp = nullptr;
    uint32_t* utok = nullptr;
    int *ustart = nullptr, *uidx = nullptr;
    // optimizer: the fp32 master weights (created by the first fp32 weight
    // load or optimizer call) and ModelOptState's moments (first optimizer call)
    struct Opt {
        float* emb = nullptr;                  // master embedding [V][D]
        std::vector<std::array<float*, 7>> w;  // masters of the 7 matrices per layer
        uint64_t synced = 0;                   // weight version the masters hold
        bool moments = false;                  // moments and norm partials allocated
        float *emb_m = nullptr, *emb_v = nullptr, *gf_m = nullptr, *gf_v = nullptr;
        std::vector<std::array<float*, 9>> m, v;
    };
    Opt* opt = nullptr;
    // gradient norm: per-block sums of squares of every gradient tensor, their sum
    float* norm_part = nullptr;
    double* norm_sum = nullptr;
    // The kept forward (ForwardResult, full_model.rs:120-129): the caches
    // above, ctx->logits and ctx->d_tgt hold the forward of fwd_B sequences of
    // fwd_S tokens run at ctx->work_epoch == fwd_epoch with logit softcap
    // fwd_softcap; utok/ustart/uidx hold the embedding backward's index.
    uint64_t fwd_epoch = 0, fwd_id = 0;
    int fwd_B = 0, fwd_S = 0, fwd_nuniq = 0;
    float fwd_softcap = 0.f;
    std::vector<uint32_t> fwd_tokens;
    ~TrainState() {
        if (side) {
            (void)hipStreamSynchronize(side);
            (void)hipStreamDestroy(side);
        }
        for (hipEvent_t e : ready)
            if (e) (void)hipEventDestroy(e);
        for (hipEvent_t e : read)
            if (e) (void)hipEventDestroy(e);
        delete opt;
    }
};

void train_state_free(TrainState* t) { delete t; }

int zero_moments(rh_ctx* ctx);

int weights_written(rh_ctx* ctx, bool masters_hold_them) {
    TrainState* T = ctx->train;
    if (!T || !T->opt) return RH_OK;
    if (masters_hold_them) T->opt->synced = ctx->wgen;
    if (T->opt->moments) RCK(zero_moments(ctx));
    return RH_OK;
}

const float* train_master(const rh_ctx* ctx, int l, int j) {
    const TrainState* T = ctx->train;
    if (!T || !T->opt || T->opt->synced != ctx->wgen) return nullptr;
    return j < 0 ? T->opt->emb : T->opt->w[l][j];
}

}  // namespace rhrt

using namespace rhrt;

namespace {

size_t round_up(size_t x, size_t m) { return (x + m - 1) / m * m; }

// The host side of the training state (no device memory yet).
int ensure_train_host(rh_ctx* ctx) {
    if (ctx->train) return RH_OK;
    ctx->train = new (std::nothrow) TrainState;
    return ctx->train ? RH_OK : fail(ctx, RH_ENOMEM, "out of host memory");
}

// Gradients and transposed weights: allocated once per context.
int ensure_train_static(rh_ctx* ctx) {
    RCK(ensure_train_host(ctx));
    TrainState* T = ctx->train;
    if (T->dembed) return RH_OK;
    const rh_config& c = ctx->cfg;
    const size_t D = c.dim, F = c.hidden, V = c.vocab, Vp = round_up(V, 128);
    if (!T->side) {  // the weight-gradient GEMMs' stream (default priority, like the context's)
        HCK(hipStreamCreateWithFlags(&T->side, hipStreamNonBlocking));
        for (hipEvent_t& e : T->ready) HCK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
        for (hipEvent_t& e : T->read) HCK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    }
    RCK(dalloc(ctx, &T->dembed, V * D));
    RCK(dalloc(ctx, &T->dgf, D));
    T->dlay.resize(c.nlayers);
    const size_t sz[9] = {D * D, D * D, D * D, D * D, D * F, D * F, D * F, D, D};
    size_t nparts = rh::sumsq_blocks(V * D) + rh::sumsq_blocks(D);
    for (auto& g : T->dlay)
        for (int j = 0; j < 9; ++j) {
            RCK(dalloc(ctx, &g[j], sz[j]));
            nparts += rh::sumsq_blocks(sz[j]);
        }
    RCK(dalloc(ctx, &T->norm_part, nparts));
    RCK(dalloc(ctx, &T->norm_sum, 1));
    RCK(dalloc(ctx, &T->embed_t, D * Vp));
    T->wt.resize(c.nlayers);
    for (auto& w : T->wt) {
        RCK(dalloc(ctx, &w.qkvt, D * 3 * D));
        RCK(dalloc(ctx, &w.ot, D * D));
        RCK(dalloc(ctx, &w.w13t, D * 2 * F));
        RCK(dalloc(ctx, &w.w2t, F * D));
    }
    T->zero = true;
    return RH_OK;
}

// Caches and workspace for B sequences of S tokens (grow-only).
int ensure_train_ws(rh_ctx* ctx, int B, int S) {
    TrainState* T = ctx->train;
    const int M = B * S;
    if (M <= T->M) {  // every buffer is indexed with the current B, S: any B*S within capacity fits
        T->B = B;
        T->S = S;
        T->Mp = (int)round_up((size_t)M, 128);
        return RH_OK;
    }
    HCK(hipStreamSynchronize(ctx->stream));
    if (T->side) HCK(hipStreamSynchronize(T->side));  // the weight-gradient stream reads some of them
    // free the old per-shape buffers
    for (auto& cc : T->c) {
        void* ps[] = {cc.xin, cc.x2, cc.lse, cc.xn, cc.q, cc.k, cc.v, cc.attn, cc.x2n, cc.h13, cc.gate};
        for (void* p : ps) dfree(ctx, p);
    }
    {
        void* ps[] = {T->xlast, T->xf, T->dlh, T->dlT, T->H1, T->H1m, T->H2, T->H2q, T->dOh,
                      T->gout, T->dres, T->Drow, T->dgp, T->utok, T->ustart, T->uidx};
        for (void* p : ps) dfree(ctx, p);
        for (auto& pr : T->tx)
            for (f16*& p : pr) {
                dfree(ctx, p);
                p = nullptr;
            }
    }
    const rh_config& c = ctx->cfg;
    const size_t D = c.dim, F = c.hidden, V = c.vocab, Vp = round_up(V, 128);
    const size_t m = M, m16 = round_up(m, 16), mp = round_up(m, 128);
    T->c.assign(c.nlayers, TrainState::Cache{});
    for (auto& cc : T->c) {
        RCK(dalloc(ctx, &cc.xin, m * D));
        RCK(dalloc(ctx, &cc.x2, m * D));
        RCK(dalloc(ctx, &cc.lse, (size_t)M * c.heads));
        RCK(dalloc(ctx, &cc.xn, m16 * D));
        RCK(dalloc(ctx, &cc.q, m * D));
        RCK(dalloc(ctx, &cc.k, m * D));
        RCK(dalloc(ctx, &cc.v, m * D));
        RCK(dalloc(ctx, &cc.attn, m16 * D));
        RCK(dalloc(ctx, &cc.x2n, m16 * D));
        RCK(dalloc(ctx, &cc.h13, 2 * m * F));
        RCK(dalloc(ctx, &cc.gate, m16 * F));
    }
    RCK(dalloc(ctx, &T->xlast, m * D));
    RCK(dalloc(ctx, &T->xf, m16 * D));
    RCK(dalloc(ctx, &T->dlh, m16 * Vp));
    RCK(dalloc(ctx, &T->dlT, Vp * mp));
    RCK(dalloc(ctx, &T->H1, m16 * D));
    RCK(dalloc(ctx, &T->H1m, m16 * D));
    RCK(dalloc(ctx, &T->H2, m16 * 2 * F));
    RCK(dalloc(ctx, &T->H2q, m16 * 3 * D));
    const size_t txr[4][2] = {{D, F}, {2 * F, D}, {D, D}, {3 * D, D}};  // rows of each copy
    for (int g = 0; g < 4; ++g)
        for (int i = 0; i < 2; ++i) RCK(dalloc(ctx, &T->tx[g][i], txr[g][i] * mp));
    RCK(dalloc(ctx, &T->dOh, m * D));
    RCK(dalloc(ctx, &T->gout, m * D));  // an unsplit data-gradient product [M][D]
    RCK(dalloc(ctx, &T->dres, m * D));
    RCK(dalloc(ctx, &T->Drow, (size_t)M * c.heads));
    RCK(dalloc(ctx, &T->dgp, (size_t)rh::rms_backward_blocks(M) * D));
    RCK(dalloc(ctx, &T->utok, m));
    RCK(dalloc(ctx, &T->ustart, m + 1));
    RCK(dalloc(ctx, &T->uidx, m));
    T->M = M;
    T->Mp = (int)mp;
    T->B = B;
    T->S = S;
    return RH_OK;
}

// Transposed weight copies for the data-gradient GEMMs, rebuilt when the
// weights changed since they were made.
int ensure_packs(rh_ctx* ctx) {
    TrainState* T = ctx->train;
    if (T->packs_gen == ctx->wgen) return RH_OK;
    const rh_config& c = ctx->cfg;
    const int D = c.dim, F = c.hidden, V = c.vocab, Vp = (int)round_up(V, 128);
    hipStream_t st = ctx->stream;
    LCK(rh::launch_transpose_frag(ctx->embed, T->embed_t, V, D, Vp, 0, st));
    for (int l = 0; l < c.nlayers; ++l) {
        const Layer& W = ctx->L[l];
        LCK(rh::launch_transpose_frag(W.wqkv, T->wt[l].qkvt, 3 * D, D, 3 * D, 0, st));
        LCK(rh::launch_transpose_frag(W.wo, T->wt[l].ot, D, D, D, 0, st));
        LCK(rh::launch_transpose_frag(W.w13, T->wt[l].w13t, 2 * F, D, 2 * F, 1, st));
        LCK(rh::launch_transpose_frag(W.w2, T->wt[l].w2t, D, F, D, 0, st));
    }
    T->packs_gen = ctx->wgen;
    return RH_OK;
}

// The forward token loop of enqueue_body with the caches kept per layer.
int enqueue_forward_train(rh_ctx* ctx, int B, int S) {
    TrainState* T = ctx->train;
    const rh_config& c = ctx->cfg;
    const int M = B * S, D = c.dim, F = c.hidden;
    const float alpha = 1.0f / std::sqrt(2.0f * (float)c.nlayers);
    hipStream_t st = ctx->stream;
    // The residual stream moves out of place through the per-layer caches the
    // backward reads: xin[l] -> (Wo) x2[l] -> (W2) xin[l + 1] ... -> xlast.
    LCK(rh::launch_embed(ctx->d_tok, ctx->embed, T->c[0].xin, M, D, c.vocab, ctx->d_err, st));
    LCK(rh::launch_rmsnorm(T->c[0].xin, ctx->L[0].g1, T->c[0].xn, M, D, c.rms_eps, st, true));
    for (int l = 0; l < c.nlayers; ++l) {
        const Layer& W = ctx->L[l];
        const TrainState::Cache& cc = T->c[l];
        rh::GemmArgs g{};
        g.W = W.wqkv; g.X = cc.xn; g.M = M; g.N = 3 * D; g.K = D;
        g.q = cc.q; g.kc = cc.k; g.vc = cc.v; g.rope = ctx->rope;
        g.S = S; g.D = D; g.H = c.heads; g.hd = c.head_dim; g.ctx = S; g.pos0 = 0;
        set_sk(ctx, g);
        RCK(timed(ctx, RH_K_GEMM_QKV, [&] { return rh::launch_gemm(rh::EPI_QKV, g, st); }));
        RCK(timed(ctx, RH_K_ATTN, [&] {
            return rh::launch_attn_prefill(cc.q, cc.k, cc.v, cc.attn, B, c.heads, S, c.head_dim, S, st, cc.lse);
        }));
        g = rh::GemmArgs{};
        g.W = W.wo; g.X = cc.attn; g.M = M; g.N = D; g.K = D;
        g.resid_in = cc.xin; g.out_f32 = cc.x2; g.ldo = D; g.alpha = alpha;
        set_sk(ctx, g);
        RCK(timed(ctx, RH_K_GEMM_WO, [&] { return rh::launch_gemm_resid_norm(g, W.g2, c.rms_eps, cc.x2n, st); }));
        g = rh::GemmArgs{};
        g.W = W.w13; g.X = cc.x2n; g.M = M; g.N = 2 * F; g.K = D;
        g.out_f16 = cc.gate; g.ldo = F; g.h13 = cc.h13;
        set_sk(ctx, g);
        RCK(timed(ctx, RH_K_GEMM_W13, [&](hipEvent_t t0, hipEvent_t t1) {
            g.prof_start = t0; g.prof_stop = t1;
            return rh::launch_gemm(rh::EPI_SWIGLU_SAVE, g, st);
        }));
        const bool last = l + 1 == c.nlayers;
        g = rh::GemmArgs{};
        g.W = W.w2; g.X = cc.gate; g.M = M; g.N = D; g.K = F;
        g.resid_in = cc.x2; g.out_f32 = last ? T->xlast : T->c[l + 1].xin; g.ldo = D; g.alpha = alpha;
        set_sk(ctx, g);
        const float* ng = last ? ctx->gfinal : ctx->L[l + 1].g1;
        f16* nxn = last ? T->xf : T->c[l + 1].xn;
        RCK(timed(ctx, RH_K_GEMM_W2, [&] { return rh::launch_gemm_resid_norm(g, ng, c.rms_eps, nxn, st); }));
    }
    return enqueue_tail(ctx, B, S, true, T->xf, T->fwd_softcap);
}

// dgamma (+)= kappa * the partial sums of rms_backward (stores while the
// gradients are logically zero).
int gamma_grad(rh_ctx* ctx, int nblk, int D, float kappa, float* dgamma) {
    LCK(rh::launch_dgamma_reduce(ctx->train->dgp, nblk, D, kappa, dgamma, ctx->train->zero, ctx->stream));
    return RH_OK;
}

// C[rows][cols] += kappa * X W^T with X [rows][Mp], W [cols][Mp] (token-inner).
// When every gradient is still zero the epilogue stores kappa * acc instead
// (the same values; it skips reading the fp32 gradient back).  K is the
// token count, short next to the fp32 output these GEMMs write, so the tile
// is picked from MI355X timings at K = 512 / 2048 / 8192 (store | accumulate
// epilogue, us) rather than by the FLOP model:
//   4096 x 4096:  256x128 8-wave 29.6 | 39.1, 73.7 | 79.1  (192x128 4-wave
//                 34 | 55, 84 | 97); at K 8192 the model's pick, 280 | 297
//   4096 x 11008: 192x256 8-wave 80 | 105, 220 | 242, 744 | 790  (192x128
//                 4-wave 88 | 124, 263 | 278)
//   32000 x 4096 (tied embedding): 192x256 256 | 364, 694 | 772; at K 8192
//                 256x128 2079 | 2164
// On the side stream (st != the context's stream) no stream-K: its workspace
// belongs to the main stream's GEMMs.
int grad_gemm(rh_ctx* ctx, const f16* X, const f16* W, int rows, int cols, float kappa, float* out,
              hipStream_t st) {
    rh::GemmArgs g{};
    g.X = X; g.W = W; g.M = rows; g.N = cols; g.K = ctx->train->Mp;
    g.out_f32 = out; g.ldo = cols; g.alpha = kappa;
    g.nt_out = true;  // read only by the optimizer
    const bool long_k = g.K >= 8192;
    if (ctx->train->zero && g.K <= 1024 && (size_t)rows * cols >= (size_t)4096 * 4096) {
        LCK(rh::launch_gemm_wgrad(g, false, st));
        return RH_OK;
    }
    if (cols > 4096)
        g.force_cfg = rh::GCFG_D8_192x256;
    else if (rows > 4096)
        g.force_cfg = long_k ? rh::GCFG_D8_256x128 : rh::GCFG_D8_192x256;
    else
        g.force_cfg = long_k ? rh::GCFG_AUTO : rh::GCFG_D8_256x128;
    if (st == ctx->stream) set_sk(ctx, g);
    LCK(rh::launch_gemm(ctx->train->zero ? rh::EPI_F32 : rh::EPI_RESID, g, st));
    return RH_OK;
}

// out [M][N] fp32 = A W^T with A [M][K] and W [N][K] (fragment order).
// As the sum of *nsplit fp32 partials at *parts, M * N floats apart: K split
// into the stream-K workspace when the output has too few tiles to fill the
// CUs (the consuming row kernel adds them up, so no fix-up kernel runs),
// otherwise the whole product in out (*nsplit = 1).
int data_gemm(rh_ctx* ctx, const f16* A, const f16* W, int M, int N, int K, float* out, const float** parts,
              int* nsplit) {
    rh::GemmArgs g{};
    g.X = A; g.W = W; g.M = M; g.N = N; g.K = K;
    g.out_f32 = out; g.ldo = N;
    set_sk(ctx, g);
    LCK(rh::launch_gemm_partials(g, nsplit, ctx->stream));
    if (*nsplit >= 2) {
        *parts = ctx->sk_part;
        return RH_OK;
    }
    LCK(rh::launch_gemm(rh::EPI_F32, g, ctx->stream));
    *parts = out;
    *nsplit = 1;
    return RH_OK;
}

int enqueue_backward(rh_ctx* ctx, int B, int S, float loss_scale, int nuniq) {
    TrainState* T = ctx->train;
    const rh_config& c = ctx->cfg;
    const int M = B * S, D = c.dim, F = c.hidden, V = c.vocab, Vp = (int)round_up(V, 128), Mp = T->Mp;
    const int H = c.heads, hd = c.head_dim;
    const float alpha = 1.0f / std::sqrt(2.0f * (float)c.nlayers);
    const float kappa = loss_scale / ((float)S * rh::GRAD_UNIT);
    const int nblk = rh::rms_backward_blocks(M);
    hipStream_t st = ctx->stream;
    // Main stream: the chain through the data gradients.  Side stream: the
    // weight gradients, each group from its own copies, after the activation
    // gradient it reads is written (ready) and before that buffer is rewritten
    // a layer later (read).  No buffer either stream writes is touched by the
    // other until the event that orders them.
    hipStream_t sd = T->side;
    for (hipEvent_t e : T->read) HCK(hipEventRecord(e, sd));  // nothing read yet
    auto publish = [&](int g) -> int {  // main -> side: group g's input is written
        HCK(hipEventRecord(T->ready[g], st));
        HCK(hipStreamWaitEvent(sd, T->ready[g], 0));
        return RH_OK;
    };
    auto rewrite = [&](int g) -> int {  // main waits: the side has copied group g's input
        HCK(hipStreamWaitEvent(st, T->read[g], 0));
        return RH_OK;
    };
    // CE gradient (internal units), dx_final = dl E, dembed += dl^T x_final
    LCK(rh::launch_ce_backward(ctx->logits, ctx->d_tgt, T->dlh, M, V, Vp, T->fwd_softcap, rh::GRAD_UNIT, st));
    RCK(publish(4));
    LCK(rh::launch_transpose_frag2(T->dlh, T->dlT, M, Vp, T->xf, T->tx[0][0], M, D, Mp, sd));
    RCK(grad_gemm(ctx, T->dlT, T->tx[0][0], V, D, kappa, T->dembed, sd));
    const size_t MD = (size_t)M * D;  // stride of the data-gradient partials
    const float* dp;
    int ns;
    RCK(data_gemm(ctx, T->dlh, T->embed_t, M, D, Vp, T->gout, &dp, &ns));
    // final RMSNorm backward: dy -> dres, a*dy -> H1 (the last layer's dffn)
    LCK(rh::launch_rms_backward(dp, ns, MD, T->xlast, ctx->gfinal, nullptr, T->dres, T->H1, alpha, T->dgp, M, D,
                                c.rms_eps, st));
    RCK(gamma_grad(ctx, nblk, D, kappa, T->dgf));
    for (int l = c.nlayers - 1; l >= 0; --l) {
        const Layer& W = ctx->L[l];
        const TrainState::Cache& cc = T->c[l];
        const TrainState::WT& wt = T->wt[l];
        float* const* G = T->dlay[l].data();
        f16* const* X0 = T->tx[0];
        f16* const* X1 = T->tx[1];
        f16* const* X2 = T->tx[2];
        f16* const* X3 = T->tx[3];
        // dW2 += dffn^T gate (side); dgate = dffn W2 with the SiLU backward -> [dh1 | dh3]
        RCK(publish(0));
        LCK(rh::launch_transpose_frag2(T->H1, X0[0], M, D, cc.gate, X0[1], M, F, Mp, sd));
        HCK(hipEventRecord(T->read[0], sd));
        RCK(grad_gemm(ctx, X0[0], X0[1], D, F, kappa, G[6], sd));
        RCK(rewrite(1));
        {
            rh::GemmArgs g{};
            g.X = T->H1; g.W = wt.w2t; g.M = M; g.N = F; g.K = D;
            g.h13 = cc.h13; g.out_f16 = T->H2; g.ldo = F;
            set_sk(ctx, g);
            LCK(rh::launch_gemm(rh::EPI_SILU_BWD, g, st));
        }
        // dx_ffn = [dh1 | dh3] [W1 | W3]^T; dW1, dW3 += x2n^T dh (side)
        RCK(publish(1));
        LCK(rh::launch_transpose_frag2(T->H2, X1[0], M, 2 * F, cc.x2n, X1[1], M, D, Mp, sd));
        HCK(hipEventRecord(T->read[1], sd));
        RCK(grad_gemm(ctx, X1[1], X1[0], D, F, kappa, G[4], sd));
        RCK(grad_gemm(ctx, X1[1], X1[0] + (size_t)F * Mp, D, F, kappa, G[5], sd));
        RCK(data_gemm(ctx, T->H2, wt.w13t, M, D, 2 * F, T->gout, &dp, &ns));
        // dx2 = RMSNorm2'(dx_ffn) + dy (in place in dres); a*dx2 -> H1m
        RCK(rewrite(2));
        LCK(rh::launch_rms_backward(dp, ns, MD, cc.x2, W.g2, T->dres, T->dres, T->H1m, alpha, T->dgp, M, D,
                                    c.rms_eps, st));
        RCK(gamma_grad(ctx, nblk, D, kappa, G[8]));
        // da = (a dx2) Wo^T; dWo += attn^T (a dx2) (side)
        RCK(publish(2));
        LCK(rh::launch_transpose_frag2(T->H1m, X2[0], M, D, cc.attn, X2[1], M, D, Mp, sd));
        HCK(hipEventRecord(T->read[2], sd));
        RCK(grad_gemm(ctx, X2[1], X2[0], D, D, kappa, G[3], sd));
        RCK(data_gemm(ctx, T->H1m, wt.ot, M, D, D, T->gout, &dp, &ns));
        // attention backward -> dq | dk | dv with the RoPE backward, as the fp16
        // operand H2q (rewritten: the side stream has copied the previous layer's)
        RCK(rewrite(3));
        LCK(rh::launch_attn_backward(cc.q, cc.k, cc.v, cc.attn, dp, ns, MD, cc.lse, T->dOh, T->Drow, T->H2q,
                                     ctx->rope, B, H, S, hd, st));
        // dxn = dqkv [Wq | Wk | Wv]^T; dWq, dWk, dWv += xn^T d{q,k,v} (side)
        RCK(publish(3));
        LCK(rh::launch_transpose_frag2(T->H2q, X3[0], M, 3 * D, cc.xn, X3[1], M, D, Mp, sd));
        HCK(hipEventRecord(T->read[3], sd));
        for (int j = 0; j < 3; ++j)
            RCK(grad_gemm(ctx, X3[1], X3[0] + (size_t)j * D * Mp, D, D, kappa, G[j], sd));
        RCK(data_gemm(ctx, T->H2q, wt.qkvt, M, D, 3 * D, T->gout, &dp, &ns));
        // dy' = RMSNorm1'(dxn) + dx2 (in place); a*dy' -> H1 (the next layer's dffn)
        RCK(rewrite(0));
        LCK(rh::launch_rms_backward(dp, ns, MD, cc.xin, W.g1, T->dres, T->dres, T->H1, alpha, T->dgp, M, D,
                                    c.rms_eps, st));
        RCK(gamma_grad(ctx, nblk, D, kappa, G[7]));
    }
    // every weight gradient is written before anything after the backward reads them
    HCK(hipEventRecord(T->ready[4], sd));
    HCK(hipStreamWaitEvent(st, T->ready[4], 0));
    LCK(rh::launch_embed_backward(T->dres, T->utok, T->ustart, T->uidx, nuniq, kappa, T->dembed, D, st));
    T->zero = false;
    return RH_OK;
}

const size_t* tensor_sizes(const rh_config& c, size_t out[9]) {
    const size_t D = c.dim, F = c.hidden;
    const size_t sz[9] = {D * D, D * D, D * D, D * D, D * F, D * F, D * F, D, D};
    std::copy(sz, sz + 9, out);
    return out;
}

}  // namespace

// fp32 master weights (reference orientation), allocated together: the
// tensors are published only once every allocation has succeeded, so a
// failed call leaves no partial set behind for a later call to mistake for
// a complete one.
int rhrt::ensure_masters(rh_ctx* ctx) {
    RCK(ensure_train_host(ctx));
    TrainState* T = ctx->train;
    if (!T->opt) {
        T->opt = new (std::nothrow) TrainState::Opt;
        if (!T->opt) return fail(ctx, RH_ENOMEM, "out of host memory");
    }
    auto* o = T->opt;
    if (o->emb) return RH_OK;
    const rh_config& c = ctx->cfg;
    size_t sz[9];
    tensor_sizes(c, sz);
    float* emb = nullptr;
    std::vector<std::array<float*, 7>> w(c.nlayers);
    for (auto& a : w) a.fill(nullptr);
    int rc = dalloc(ctx, &emb, (size_t)c.vocab * c.dim);
    for (int l = 0; l < c.nlayers && rc == RH_OK; ++l)
        for (int j = 0; j < 7 && rc == RH_OK; ++j) rc = dalloc(ctx, &w[l][j], sz[j]);
    if (rc != RH_OK) {
        dfree(ctx, emb);
        for (auto& a : w)
            for (float* p : a) dfree(ctx, p);
        return rc;
    }
    o->w = std::move(w);
    o->emb = emb;
    o->synced = 0;  // nothing written yet
    return RH_OK;
}

bool rhrt::have_masters(const rh_ctx* ctx) { return ctx->train && ctx->train->opt && ctx->train->opt->emb; }

float* rhrt::master_ptr(rh_ctx* ctx, int l, int j) {
    return j < 0 ? ctx->train->opt->emb : ctx->train->opt->w[l][j];
}

// Frees the masters (no optimizer moments may exist: they belong together).
int rhrt::drop_masters(rh_ctx* ctx) {
    if (!have_masters(ctx)) return RH_OK;
    auto* o = ctx->train->opt;
    if (o->moments) return fail(ctx, RH_ESTATE, "the optimizer state holds the fp32 masters");
    HCK(hipStreamSynchronize(ctx->stream));
    dfree(ctx, o->emb);
    o->emb = nullptr;
    for (auto& a : o->w)
        for (float* p : a) dfree(ctx, p);
    o->w.clear();
    o->synced = 0;
    return RH_OK;
}

// Zeroes the moments (ModelOptState::zeros).
int rhrt::zero_moments(rh_ctx* ctx) {
    auto* o = ctx->train->opt;
    const rh_config& c = ctx->cfg;
    size_t sz[9];
    tensor_sizes(c, sz);
    hipStream_t st = ctx->stream;
    const size_t VD = (size_t)c.vocab * c.dim;
    LCK(rh::launch_fill_f32(o->emb_m, 0.f, VD, st));
    LCK(rh::launch_fill_f32(o->emb_v, 0.f, VD, st));
    LCK(rh::launch_fill_f32(o->gf_m, 0.f, c.dim, st));
    LCK(rh::launch_fill_f32(o->gf_v, 0.f, c.dim, st));
    for (int l = 0; l < c.nlayers; ++l)
        for (int j = 0; j < 9; ++j) {
            LCK(rh::launch_fill_f32(o->m[l][j], 0.f, sz[j], st));
            LCK(rh::launch_fill_f32(o->v[l][j], 0.f, sz[j], st));
        }
    return RH_OK;
}

namespace {

// Optimizer state: masters, moments (zeroed when created) and the norm's
// partials.  Masters older than the device weights (rh_init_weights_normal)
// are re-read from the fp16 device copy.
int ensure_opt(rh_ctx* ctx) {
    RCK(ensure_train_static(ctx));
    RCK(ensure_masters(ctx));
    TrainState* T = ctx->train;
    auto* o = T->opt;
    const rh_config& c = ctx->cfg;
    const size_t D = c.dim, V = c.vocab;
    size_t sz[9];
    tensor_sizes(c, sz);
    hipStream_t st = ctx->stream;
    if (!o->moments) {
        RCK(dalloc(ctx, &o->emb_m, V * D));
        RCK(dalloc(ctx, &o->emb_v, V * D));
        RCK(dalloc(ctx, &o->gf_m, D));
        RCK(dalloc(ctx, &o->gf_v, D));
        o->m.resize(c.nlayers);
        o->v.resize(c.nlayers);
        for (int l = 0; l < c.nlayers; ++l)
            for (int j = 0; j < 9; ++j) {
                RCK(dalloc(ctx, &o->m[l][j], sz[j]));
                RCK(dalloc(ctx, &o->v[l][j], sz[j]));
            }
        o->moments = true;
        RCK(zero_moments(ctx));
    }
    if (o->synced != ctx->wgen) {
        LCK(rh::launch_unpack_rows(ctx->embed, o->emb, (int)V, (int)D, st));
        for (int l = 0; l < c.nlayers; ++l)
            for (int j = 0; j < 7; ++j) {
                const TensorMap mp = layer_map(ctx, l, j);
                if (mp.map < 0) {
                    LCK(rh::launch_unpack_rows(mp.dst, o->w[l][j], mp.R, mp.C, st));
                } else {
                    LCK(rh::launch_unpack_transpose(mp.dst, o->w[l][j], mp.R, mp.C, mp.ldd, mp.map, mp.row_off, st));
                }
            }
        o->synced = ctx->wgen;
    }
    return RH_OK;
}

// 1 - b^t in fp32 by repeated squaring (f32::powi of the bias corrections).
float powi_f32(float b, uint32_t t) {
    float r = 1.0f, x = b;
    for (uint32_t e = t; e; e >>= 1) {
        if (e & 1u) r *= x;
        x *= x;
    }
    return r;
}

}  // namespace

extern "C" {

void rh_train_config_default(rh_train_config* tc) {
    if (!tc) return;
    *tc = rh_train_config{3e-4f, 0.1f, 100u, 10000u, 0.9f, 0.95f, 1e-8f, 0.1f, 0.05f, 5.0f, 256.0f, 10u, 1.0f, 0.0f};
}

float rh_learning_rate(uint32_t step, const rh_train_config* tc) {
    if (!tc) return 0.f;
    if (step < tc->warmup_steps) return tc->max_lr * (float)(step + 1) / (float)tc->warmup_steps;
    const float decay = (float)(step - tc->warmup_steps) / (float)(tc->total_steps - tc->warmup_steps);
    const float min_lr = tc->max_lr * tc->min_lr_frac;
    return min_lr + 0.5f * (1.0f + std::cos(3.14159265358979323846f * decay)) * (tc->max_lr - min_lr);
}

int rh_grad_norm(rh_ctx* ctx, float* norm_out) {
    if (!ctx || !norm_out) return fail(ctx, RH_EINVAL, "null argument");
    TrainState* T = ctx->train;
    if (!T || !T->dembed || T->zero) {
        *norm_out = 0.f;
        return RH_OK;
    }
    HCK(hipSetDevice(ctx->device));
    const rh_config& c = ctx->cfg;
    size_t sz[9];
    tensor_sizes(c, sz);
    hipStream_t st = ctx->stream;
    // grad_norm's tensor order (full_model.rs:1403-1450)
    std::vector<std::pair<const float*, size_t>> ts{{T->dembed, (size_t)c.vocab * c.dim}, {T->dgf, (size_t)c.dim}};
    for (int l = 0; l < c.nlayers; ++l)
        for (int j = 0; j < 9; ++j) ts.emplace_back(T->dlay[l][j], sz[j]);
    // per-block partials of every tensor, then their sum in double on the device
    size_t off = 0;
    for (auto& t : ts) {
        LCK(rh::launch_sumsq(t.first, t.second, T->norm_part + off, st));
        off += rh::sumsq_blocks(t.second);
    }
    LCK(rh::launch_sum_parts(T->norm_part, off, T->norm_sum, st));
    double total = 0.0;
    HCK(hipMemcpyAsync(&total, T->norm_sum, sizeof(double), hipMemcpyDeviceToHost, st));
    HCK(hipStreamSynchronize(st));
    *norm_out = (float)std::sqrt(total);
    return RH_OK;
}

int rh_update_weights(rh_ctx* ctx, uint32_t t, float lr, const rh_train_config* tc, float grad_scale) {
    if (!ctx || !tc) return fail(ctx, RH_EINVAL, "null argument");
    if (t == 0) return fail(ctx, RH_EINVAL, "the Adam step count t starts at 1");
    HCK(hipSetDevice(ctx->device));
    RCK(ensure_opt(ctx));
    TrainState* T = ctx->train;
    auto* o = T->opt;
    const rh_config& c = ctx->cfg;
    const size_t D = c.dim, V = c.vocab;
    size_t sz[9];
    tensor_sizes(c, sz);
    hipStream_t st = ctx->stream;
    const bool zg = T->zero;  // gradients logically zero: no grad reads
    rh::AdamArgs a{};
    a.beta1 = tc->beta1;
    a.beta2 = tc->beta2;
    a.omb1 = 1.0f - tc->beta1;
    a.omb2 = 1.0f - tc->beta2;
    a.eps = tc->eps;
    a.gscale = grad_scale;
    a.bc1 = 1.0f / (1.0f - powi_f32(tc->beta1, t));
    a.bc2 = 1.0f / (1.0f - powi_f32(tc->beta2, t));
    // update_weights (full_model.rs:1123-1241): embed at lr * embed_lr_scale, gamma_final at lr, no decay
    rh::AdamArgs ae = a;
    ae.lr = lr * tc->embed_lr_scale;
    ae.wd = 0.f;
    LCK(rh::launch_adam_rows(o->emb, zg ? nullptr : T->dembed, o->emb_m, o->emb_v, V * D, ae, ctx->embed, (int)D,
                             st));
    rh::AdamArgs ag = a;
    ag.lr = lr;
    ag.wd = 0.f;
    LCK(rh::launch_adam_rows(ctx->gfinal, zg ? nullptr : T->dgf, o->gf_m, o->gf_v, D, ag, nullptr, 0, st));
    // update_layer (:1243-1400): matrices at lr * matrix_lr_scale with decay, gammas at lr without
    rh::AdamArgs am = a;
    am.lr = lr * tc->matrix_lr_scale;
    am.wd = tc->weight_decay;
    for (int l = 0; l < c.nlayers; ++l) {
        for (int j = 0; j < 7; ++j) {
            const TensorMap mp = layer_map(ctx, l, j);
            const float* g = zg ? nullptr : T->dlay[l][j];
            if (mp.map < 0) {
                LCK(rh::launch_adam_rows(o->w[l][j], g, o->m[l][j], o->v[l][j], sz[j], am, mp.dst, mp.C, st));
            } else {
                LCK(rh::launch_adam_transpose(o->w[l][j], g, o->m[l][j], o->v[l][j], mp.R, mp.C, am, mp.dst,
                                              mp.ldd, mp.map, mp.row_off, st));
            }
        }
        LCK(rh::launch_adam_rows(ctx->L[l].g1, zg ? nullptr : T->dlay[l][7], o->m[l][7], o->v[l][7], D, ag,
                                 nullptr, 0, st));
        LCK(rh::launch_adam_rows(ctx->L[l].g2, zg ? nullptr : T->dlay[l][8], o->m[l][8], o->v[l][8], D, ag,
                                 nullptr, 0, st));
    }
    HCK(hipStreamSynchronize(st));
    ++ctx->wgen;  // the transposed copies of the backward are rebuilt on its next call
    o->synced = ctx->wgen;
    return RH_OK;
}

}  // extern "C"

namespace {
int train_step_body(rh_ctx* ctx, const rh_tokens* data, uint32_t step, const rh_train_config* tc,
                    uint64_t max_pos, float* loss_out, float* grad_norm_out);
int forward_backward_impl(rh_ctx* ctx, const uint32_t* tokens, const uint32_t* targets, int batch, int seq,
                          float softcap, float loss_scale, float* mean_loss_out);
}  // namespace

extern "C" {

int rh_train_step(rh_ctx* ctx, const rh_tokens* data, uint32_t step, const rh_train_config* tc, float* loss_out,
                  float* grad_norm_out) {
    if (!ctx || !data || !tc) return fail(ctx, RH_EINVAL, "null argument");
    if (tc->accum_steps == 0 || !(tc->loss_scale > 0.f))
        return fail(ctx, RH_EINVAL, "accum_steps must be >= 1 and loss_scale > 0");
    const int S = ctx->cfg.seq;
    const int64_t n = rh_tokens_len(data);
    if (n < (int64_t)S + 2) return fail(ctx, RH_ERANGE, "token data shorter than seq + 2");
    const uint64_t max_pos = (uint64_t)(n - S - 1);
    // The training forward uses tc->softcap; the context's own softcap (the
    // one forwards and decodes use) is not touched.
    const int rc = train_step_body(ctx, data, step, tc, max_pos, loss_out, grad_norm_out);
    return rc;
}

}  // extern "C"

namespace {

int train_step_body(rh_ctx* ctx, const rh_tokens* data, uint32_t step, const rh_train_config* tc,
                    uint64_t max_pos, float* loss_out, float* grad_norm_out) {
    const int S = ctx->cfg.seq;
    RCK(rh_zero_grads(ctx));
    // train_step_with_options (full_model.rs:1510-1600): accum_steps sequences
    // at pseudo-random positions (step*7919 + micro*104729) % max_pos, run as
    // batches of up to max_batch independent sequences.
    const int mb = std::max(1, std::min<int>((int)tc->accum_steps, ctx->max_batch));
    std::vector<uint32_t> buf((size_t)S + 1), tok((size_t)mb * S), tgt((size_t)mb * S);
    std::vector<float> losses(mb);
    float total = 0.f;
    for (uint32_t i0 = 0; i0 < tc->accum_steps; i0 += mb) {
        const int nb = std::min<int>(mb, (int)(tc->accum_steps - i0));
        for (int j = 0; j < nb; ++j) {
            const uint64_t pos = ((uint64_t)step * 7919u + (uint64_t)(i0 + j) * 104729u) % max_pos;
            RCK(rh_tokens_read(data, (int64_t)pos, S + 1, buf.data()));
            std::memcpy(&tok[(size_t)j * S], buf.data(), (size_t)S * 4);
            std::memcpy(&tgt[(size_t)j * S], buf.data() + 1, (size_t)S * 4);
        }
        RCK(forward_backward_impl(ctx, tok.data(), tgt.data(), nb, S, tc->softcap, tc->loss_scale, losses.data()));
        for (int j = 0; j < nb; ++j) total += losses[j];
    }
    const float gsc = 1.0f / ((float)tc->accum_steps * tc->loss_scale);
    float raw = 0.f;
    RCK(rh_grad_norm(ctx, &raw));
    const float scaled = raw * gsc;
    const float combined = scaled > tc->grad_clip ? tc->grad_clip / raw : gsc;
    RCK(rh_update_weights(ctx, step + 1, rh_learning_rate(step, tc), tc, combined));
    if (loss_out) *loss_out = total / (float)tc->accum_steps;
    if (grad_norm_out) *grad_norm_out = scaled;
    return RH_OK;
}

}  // namespace

extern "C" {

// Zeroing is logical: the next backward's weight-gradient GEMMs and gamma
// reductions store instead of accumulating, and reads return zeros until
// then, so no pass over the gradient memory is needed.
int rh_zero_grads(rh_ctx* ctx) {
    if (!ctx) return RH_EINVAL;
    TrainState* T = ctx->train;
    if (!T) return RH_OK;  // nothing allocated yet: the first backward starts from zero
    T->zero = true;
    return RH_OK;
}

}  // extern "C"

namespace {

// Host-built index of the embedding backward: every distinct token and its
// positions, in increasing order.
struct TokenIndex {
    std::vector<uint32_t> utok;
    std::vector<int> start{0}, idx;
};

// Checks a training forward's arguments and sizes every buffer it needs.
int prepare_train(rh_ctx* ctx, const uint32_t* tokens, const uint32_t* targets, int batch, int seq, float softcap) {
    if (!ctx || !tokens || !targets) return fail(ctx, RH_EINVAL, "null argument");
    if (batch <= 0 || seq <= 0 || batch > ctx->max_batch)
        return fail(ctx, RH_ERANGE, "batch must be in [1, max_batch] and seq >= 1");
    if (!(softcap >= 0.f) || !std::isfinite(softcap)) return fail(ctx, RH_EINVAL, "softcap must be >= 0");
    const rh_config& c = ctx->cfg;
    if (c.hidden % 64 != 0) return fail(ctx, RH_EINVAL, "the backward pass needs hidden % 64 == 0");
    const size_t M = (size_t)batch * seq;
    RCK(check_tokens(ctx, tokens, M));
    RCK(check_tokens(ctx, targets, M));
    HCK(hipSetDevice(ctx->device));
    RCK(ensure_workspace(ctx, (int)M));
    RCK(ensure_rope(ctx, seq));
    RCK(ensure_train_static(ctx));
    RCK(ensure_train_ws(ctx, batch, seq));
    RCK(ensure_packs(ctx));
    return RH_OK;
}

// Uploads the tokens, targets and the embedding backward's index (ix must
// stay alive until the stream has drained) and enqueues the training forward
// whose caches the backward reads; records it as the kept forward.
int enqueue_kept_forward(rh_ctx* ctx, const uint32_t* tokens, const uint32_t* targets, int batch, int seq,
                         float softcap, TokenIndex& ix) {
    TrainState* T = ctx->train;
    hipStream_t st = ctx->stream;
    const size_t M = (size_t)batch * seq;
    std::map<uint32_t, std::vector<int>> pos;
    for (size_t i = 0; i < M; ++i) pos[tokens[i]].push_back((int)i);
    for (auto& kv : pos) {
        ix.utok.push_back(kv.first);
        ix.idx.insert(ix.idx.end(), kv.second.begin(), kv.second.end());
        ix.start.push_back((int)ix.idx.size());
    }
    HCK(hipMemcpyAsync(ctx->d_tok, tokens, M * sizeof(uint32_t), hipMemcpyHostToDevice, st));
    HCK(hipMemcpyAsync(ctx->d_tgt, targets, M * sizeof(uint32_t), hipMemcpyHostToDevice, st));
    HCK(hipMemcpyAsync(T->utok, ix.utok.data(), ix.utok.size() * sizeof(uint32_t), hipMemcpyHostToDevice, st));
    HCK(hipMemcpyAsync(T->ustart, ix.start.data(), ix.start.size() * sizeof(int), hipMemcpyHostToDevice, st));
    HCK(hipMemcpyAsync(T->uidx, ix.idx.data(), ix.idx.size() * sizeof(int), hipMemcpyHostToDevice, st));
    T->fwd_softcap = softcap;
    T->fwd_B = batch;
    T->fwd_S = seq;
    T->fwd_nuniq = (int)ix.utok.size();
    T->fwd_tokens.assign(tokens, tokens + M);
    T->fwd_epoch = ctx->work_epoch;
    T->fwd_id += 1;
    RCK(enqueue_forward_train(ctx, batch, seq));
    return RH_OK;
}

// The backward of the kept forward, accumulating into the gradients.
int enqueue_kept_backward(rh_ctx* ctx, float loss_scale) {
    TrainState* T = ctx->train;
    const int rc = enqueue_backward(ctx, T->fwd_B, T->fwd_S, loss_scale, T->fwd_nuniq);
    if (rc != RH_OK) (void)hipStreamSynchronize(T->side);  // leave no weight-gradient work behind
    return rc;
}

int forward_backward_impl(rh_ctx* ctx, const uint32_t* tokens, const uint32_t* targets, int batch, int seq,
                          float softcap, float loss_scale, float* mean_loss_out) {
    RCK(prepare_train(ctx, tokens, targets, batch, seq, softcap));
    if (!(loss_scale > 0.f) || !std::isfinite(loss_scale)) return fail(ctx, RH_EINVAL, "loss_scale must be > 0");
    TokenIndex ix;
    RCK(enqueue_kept_forward(ctx, tokens, targets, batch, seq, softcap, ix));
    RCK(enqueue_kept_backward(ctx, loss_scale));
    hipStream_t st = ctx->stream;
    if (mean_loss_out) HCK(hipMemcpyAsync(mean_loss_out, ctx->mean, batch * sizeof(float), hipMemcpyDeviceToHost, st));
    HCK(hipStreamSynchronize(st));
    return check_err_flag(ctx);
}

}  // namespace

struct rh_forward_result {
    const rh_ctx* ctx;
    uint64_t id;
};

extern "C" {

int rh_forward_backward(rh_ctx* ctx, const uint32_t* tokens, const uint32_t* targets, int batch, int seq,
                        float loss_scale, float* mean_loss_out) {
    if (!ctx) return RH_EINVAL;
    return forward_backward_impl(ctx, tokens, targets, batch, seq, ctx->cfg.softcap, loss_scale, mean_loss_out);
}

int rh_forward_train(rh_ctx* ctx, const uint32_t* tokens, const uint32_t* targets, int batch, int seq,
                     float softcap, float* mean_loss_out, rh_forward_result** out) {
    if (!out) return fail(ctx, RH_EINVAL, "null argument");
    *out = nullptr;
    RCK(prepare_train(ctx, tokens, targets, batch, seq, softcap));
    auto* r = new (std::nothrow) rh_forward_result{ctx, 0};
    if (!r) return fail(ctx, RH_ENOMEM, "out of host memory");
    TokenIndex ix;
    int rc = enqueue_kept_forward(ctx, tokens, targets, batch, seq, softcap, ix);
    hipStream_t st = ctx->stream;
    if (rc == RH_OK && mean_loss_out &&
        hipMemcpyAsync(mean_loss_out, ctx->mean, batch * sizeof(float), hipMemcpyDeviceToHost, st) != hipSuccess)
        rc = fail(ctx, RH_EDEVICE, "hipMemcpyAsync of the losses failed");
    if (hipStreamSynchronize(st) != hipSuccess && rc == RH_OK) rc = fail(ctx, RH_EDEVICE, "stream synchronize failed");
    if (rc == RH_OK) rc = check_err_flag(ctx);
    if (rc != RH_OK) {
        ctx->train->fwd_id += 1;  // nothing may consume a failed forward
        delete r;
        return rc;
    }
    r->id = ctx->train->fwd_id;
    *out = r;
    return RH_OK;
}

int rh_backward(rh_ctx* ctx, const rh_forward_result* fwd, const uint32_t* tokens, float softcap, float loss_scale,
                float* grad_norm_out) {
    if (!ctx || !fwd || !tokens) return fail(ctx, RH_EINVAL, "null argument");
    if (!(loss_scale > 0.f) || !std::isfinite(loss_scale)) return fail(ctx, RH_EINVAL, "loss_scale must be > 0");
    TrainState* T = ctx->train;
    if (fwd->ctx != ctx || !T || fwd->id != T->fwd_id || T->fwd_epoch != ctx->work_epoch)
        return fail(ctx, RH_ESTATE,
                    "the forward result is stale: another forward, prefill or validation has run on this "
                    "context since it was made, or it belongs to another context");
    if (softcap != T->fwd_softcap) return fail(ctx, RH_EINVAL, "softcap differs from the forward's");
    if (!std::equal(T->fwd_tokens.begin(), T->fwd_tokens.end(), tokens))
        return fail(ctx, RH_EINVAL, "tokens differ from the forward's input tokens");
    HCK(hipSetDevice(ctx->device));
    RCK(ensure_packs(ctx));  // the weights may have changed since the forward
    RCK(enqueue_kept_backward(ctx, loss_scale));
    HCK(hipStreamSynchronize(ctx->stream));
    if (grad_norm_out) RCK(rh_grad_norm(ctx, grad_norm_out));
    return RH_OK;
}

void rh_forward_result_free(rh_forward_result* fwd) { delete fwd; }

int rh_read_grads_f32(rh_ctx* ctx, float* dembed, float* dgamma_final, float* const* layer_grads) {
    if (!ctx) return RH_EINVAL;
    TrainState* T = ctx->train;
    if (!T || !T->dembed) return fail(ctx, RH_ESTATE, "no gradients: run rh_forward_backward first");
    HCK(hipSetDevice(ctx->device));
    const rh_config& c = ctx->cfg;
    const size_t D = c.dim, F = c.hidden, V = c.vocab;
    hipStream_t st = ctx->stream;
    const size_t sz[9] = {D * D, D * D, D * D, D * D, D * F, D * F, D * F, D, D};
    if (T->zero) {
        if (dembed) std::memset(dembed, 0, V * D * sizeof(float));
        if (dgamma_final) std::memset(dgamma_final, 0, D * sizeof(float));
        if (layer_grads)
            for (int l = 0; l < c.nlayers; ++l)
                for (int j = 0; j < 9; ++j)
                    if (layer_grads[9 * l + j]) std::memset(layer_grads[9 * l + j], 0, sz[j] * sizeof(float));
        return RH_OK;
    }
    if (dembed) HCK(hipMemcpyAsync(dembed, T->dembed, V * D * sizeof(float), hipMemcpyDeviceToHost, st));
    if (dgamma_final) HCK(hipMemcpyAsync(dgamma_final, T->dgf, D * sizeof(float), hipMemcpyDeviceToHost, st));
    if (layer_grads)
        for (int l = 0; l < c.nlayers; ++l)
            for (int j = 0; j < 9; ++j)
                if (layer_grads[9 * l + j])
                    HCK(hipMemcpyAsync(layer_grads[9 * l + j], T->dlay[l][j], sz[j] * sizeof(float),
                                       hipMemcpyDeviceToHost, st));
    HCK(hipStreamSynchronize(st));
    return RH_OK;
}

}  // extern "C"
