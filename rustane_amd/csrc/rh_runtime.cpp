// rh_runtime.cpp -- host runtime behind include/rustane_hip.h.
//
// Owns the device, one HIP stream, the fp16 weights (repacked once at upload
// to the [out, in] layout the kernels stream), the KV cache and the
// workspaces, and sequences the kernels of the forward token loop:
//
//   embed -> L x [rmsnorm -> QKV GEMM (+RoPE, K/V store) -> causal attention
//                 -> Wo GEMM (+x += a*o) -> rmsnorm -> W1|W3 GEMM (+SwiGLU)
//                 -> W2 GEMM (+x += a*f)] -> rmsnorm -> tied logits GEMM
//   -> cross-entropy rows -> per-sequence mean
//
// which is layer::forward (layer.rs:4409-4624) and full_model::forward
// (full_model.rs:915-991) with a = 1/sqrt(2L) (layer.rs:4640).  The decode
// step runs the same chain on B <= 16 tokens with GEMV kernels and a KV cache,
// and is replayed as a captured HIP graph.
#include "rh_ctx.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <vector>

namespace rhrt {

int fail(rh_ctx* c, int code, const std::string& m) {
    if (c) c->err = m;
    return code;
}

void dfree(rh_ctx* ctx, void* p) {
    if (!p) return;
    auto it = std::find(ctx->allocs.begin(), ctx->allocs.end(), p);
    if (it != ctx->allocs.end()) ctx->allocs.erase(it);
    (void)hipFree(p);
}

size_t D_(const rh_ctx* c) { return (size_t)c->cfg.dim; }
size_t F_(const rh_ctx* c) { return (size_t)c->cfg.hidden; }
size_t V_(const rh_ctx* c) { return (size_t)c->cfg.vocab; }

// RoPE table, theta = p / base^(2i/hd) in fp32 (kernels/sdpa_fwd.rs:24-39).
int ensure_rope(rh_ctx* ctx, int npos) {
    if (npos <= ctx->rope_len) return RH_OK;
    const int hd = ctx->cfg.head_dim;
    std::vector<float2> t((size_t)npos * (hd / 2));
    for (int p = 0; p < npos; ++p)
        for (int i = 0; i < hd / 2; ++i) {
            const float th = (float)p / std::pow(ctx->cfg.rope_base, 2.0f * (float)i / (float)hd);
            t[(size_t)p * (hd / 2) + i] = make_float2(std::cos(th), std::sin(th));
        }
    HCK(hipStreamSynchronize(ctx->stream));
    drop_graphs(ctx);  // captured steps hold the old table's address
    dfree(ctx, ctx->rope);
    ctx->rope = nullptr;
    RCK(dalloc(ctx, &ctx->rope, t.size()));
    HCK(hipMemcpy(ctx->rope, t.data(), t.size() * sizeof(float2), hipMemcpyHostToDevice));
    ctx->rope_len = npos;
    return RH_OK;
}

// Destroys every captured graph, after the stream has drained any replay of
// them still in flight.
void drop_graphs(rh_ctx* ctx) {
    if (!ctx->dgraph && ctx->fgraphs.empty()) return;
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->dgraph) (void)hipGraphExecDestroy(ctx->dgraph);
    ctx->dgraph = nullptr;
    ctx->dgraph_B = 0;
    for (auto& g : ctx->fgraphs) (void)hipGraphExecDestroy(g.exec);
    ctx->fgraphs.clear();
}

int ensure_workspace(rh_ctx* ctx, int M) {
    ctx->work_epoch += 1;  // every caller writes the workspace next
    if (M <= ctx->ws_M) return RH_OK;
    HCK(hipStreamSynchronize(ctx->stream));
    drop_graphs(ctx);  // captured forwards hold the old buffers' addresses
    void* olds[] = {ctx->x, ctx->xn, ctx->q, ctx->kbuf, ctx->vbuf, ctx->attn, ctx->gate,
                    ctx->logits, ctx->tok_loss, ctx->mean, ctx->d_tok, ctx->d_tgt};
    for (void* p : olds) dfree(ctx, p);
    const size_t D = D_(ctx), F = F_(ctx), V = V_(ctx), m = (size_t)M;
    // GEMM operands (xn, attn, gate) are in fragment order: rows padded to 16
    const size_t m16 = (m + 15) / 16 * 16;
    RCK(dalloc(ctx, &ctx->x, m * D));
    RCK(dalloc(ctx, &ctx->xn, m16 * D));
    RCK(dalloc(ctx, &ctx->q, m * D));
    RCK(dalloc(ctx, &ctx->kbuf, m * D));
    RCK(dalloc(ctx, &ctx->vbuf, m * D));
    RCK(dalloc(ctx, &ctx->attn, m16 * D));
    RCK(dalloc(ctx, &ctx->gate, m16 * F));
    RCK(dalloc(ctx, &ctx->logits, m * V));
    RCK(dalloc(ctx, &ctx->tok_loss, m));
    RCK(dalloc(ctx, &ctx->mean, m));
    RCK(dalloc(ctx, &ctx->d_tok, m));
    RCK(dalloc(ctx, &ctx->d_tgt, m));
    if (!ctx->sk_part) {
        ctx->sk_part_floats = rh::gemm_sk_part_floats();
        RCK(dalloc(ctx, &ctx->sk_part, ctx->sk_part_floats));
    }
    ctx->ws_M = M;
    return RH_OK;
}

int ensure_staging(rh_ctx* ctx, size_t elems) {
    if (elems <= ctx->staging_elems) return RH_OK;
    HCK(hipStreamSynchronize(ctx->stream));
    dfree(ctx, ctx->staging);
    ctx->staging = nullptr;
    RCK(dalloc(ctx, &ctx->staging, elems));
    ctx->staging_elems = elems;
    return RH_OK;
}

void set_sk(const rh_ctx* ctx, rh::GemmArgs& g) {
    g.sk_part = ctx->sk_part;
    g.sk_part_floats = ctx->sk_part_floats;
}

}  // namespace rhrt

using namespace rhrt;

namespace {

// ---- the forward token loop -----------------------------------------------
// kv_k/kv_v: per-layer K/V destination base and ctx stride.  For a plain
// forward they are the scratch buffers (ctx = S); for a prefill they are the
// cache layers (ctx = max_ctx).
// Every residual GEMM (Wo, W2) also produces the next RMSNorm's output in xn:
// Wo the layer's second norm, W2 the next layer's first norm -- or, after the
// last layer, the final norm when final_norm is set (the forward's logits).
int enqueue_body(rh_ctx* ctx, int B, int S, bool to_cache, bool final_norm) {
    const rh_config& c = ctx->cfg;
    const int M = B * S, D = c.dim, F = c.hidden;
    const float alpha = 1.0f / std::sqrt(2.0f * (float)c.nlayers);
    hipStream_t st = ctx->stream;
    LCK(rh::launch_embed(ctx->d_tok, ctx->embed, ctx->x, M, D, c.vocab, ctx->d_err, st));
    LCK(rh::launch_rmsnorm(ctx->x, ctx->L[0].g1, ctx->xn, M, D, c.rms_eps, st, true));
    for (int l = 0; l < c.nlayers; ++l) {
        const Layer& W = ctx->L[l];
        f16* kc = to_cache ? ctx->kcache + (size_t)l * ctx->kv_layer : ctx->kbuf;
        f16* vc = to_cache ? ctx->vcache + (size_t)l * ctx->kv_layer : ctx->vbuf;
        const int kvctx = to_cache ? ctx->max_ctx : S;
        const float* next_gamma = l + 1 < c.nlayers ? ctx->L[l + 1].g1 : (final_norm ? ctx->gfinal : nullptr);
        rh::GemmArgs g{};
        g.W = W.wqkv; g.X = ctx->xn; g.M = M; g.N = 3 * D; g.K = D;
        g.q = ctx->q; g.kc = kc; g.vc = vc; g.rope = ctx->rope;
        g.S = S; g.D = D; g.H = c.heads; g.hd = c.head_dim; g.ctx = kvctx; g.pos0 = 0;
        set_sk(ctx, g);
        RCK(timed(ctx, RH_K_GEMM_QKV, [&] { return rh::launch_gemm(rh::EPI_QKV, g, st); }));
        RCK(timed(ctx, RH_K_ATTN, [&] {
            return rh::launch_attn_prefill(ctx->q, kc, vc, ctx->attn, B, c.heads, S, c.head_dim, kvctx, st);
        }));
        g = rh::GemmArgs{};
        g.W = W.wo; g.X = ctx->attn; g.M = M; g.N = D; g.K = D;
        g.out_f32 = ctx->x; g.ldo = D; g.alpha = alpha;
        set_sk(ctx, g);
        RCK(timed(ctx, RH_K_GEMM_WO, [&] { return rh::launch_gemm_resid_norm(g, W.g2, c.rms_eps, ctx->xn, st); }));
        g = rh::GemmArgs{};
        g.W = W.w13; g.X = ctx->xn; g.M = M; g.N = 2 * F; g.K = D;
        g.out_f16 = ctx->gate; g.ldo = F;
        set_sk(ctx, g);
        RCK(timed(ctx, RH_K_GEMM_W13, [&](hipEvent_t t0, hipEvent_t t1) {
            g.prof_start = t0; g.prof_stop = t1;
            return rh::launch_gemm(rh::EPI_SWIGLU, g, st);
        }));
        g = rh::GemmArgs{};
        g.W = W.w2; g.X = ctx->gate; g.M = M; g.N = D; g.K = F;
        g.out_f32 = ctx->x; g.ldo = D; g.alpha = alpha;
        set_sk(ctx, g);
        RCK(timed(ctx, RH_K_GEMM_W2,
                  [&] { return rh::launch_gemm_resid_norm(g, next_gamma, c.rms_eps, ctx->xn, st); }));
    }
    return RH_OK;
}

// Logits + loss from xn, which enqueue_body(final_norm = true) left holding
// the final RMSNorm of every row.
}  // namespace

int rhrt::enqueue_tail(rh_ctx* ctx, int B, int S, bool with_loss, const f16* xf, float softcap) {
    const rh_config& c = ctx->cfg;
    const int M = B * S, D = c.dim;
    hipStream_t st = ctx->stream;
    rh::GemmArgs g{};
    g.W = ctx->embed; g.X = xf ? xf : ctx->xn; g.M = M; g.N = c.vocab; g.K = D;
    g.out_f32 = ctx->logits; g.ldo = c.vocab; g.softcap = softcap < 0.f ? c.softcap : softcap;
    set_sk(ctx, g);
    RCK(timed(ctx, RH_K_GEMM_LOGITS, [&] { return rh::launch_gemm(rh::EPI_F32, g, st); }));
    if (with_loss) {
        LCK(rh::launch_cross_entropy(ctx->logits, ctx->d_tgt, ctx->tok_loss, M, c.vocab, ctx->d_err, st));
        LCK(rh::launch_mean_rows(ctx->tok_loss, ctx->mean, B, S, st));
    }
    return RH_OK;
}

namespace {

bool profiling(const rh_ctx* ctx) {
    for (const auto& p : ctx->prof)
        if (p.on) return true;
    return false;
}

// The forward over d_tok (and d_tgt): enqueue_body + enqueue_tail, replayed
// from a captured graph per (B, S, loss) -- about 226 launches at 7B become
// one -- or launched eagerly when graphs are off or a kernel class is being
// timed (per-launch events need the eager launches).
constexpr size_t kMaxFwdGraphs = 8;
int run_forward(rh_ctx* ctx, int B, int S, bool with_loss) {
    if (!ctx->use_graphs || profiling(ctx)) {
        RCK(enqueue_body(ctx, B, S, false, true));
        return enqueue_tail(ctx, B, S, with_loss);
    }
    auto& gs = ctx->fgraphs;
    auto it = std::find_if(gs.begin(), gs.end(),
                           [&](const FwdGraph& g) { return g.B == B && g.S == S && g.loss == with_loss; });
    if (it == gs.end()) {
        if (gs.size() >= kMaxFwdGraphs) {
            HCK(hipStreamSynchronize(ctx->stream));  // the evicted graph may still be replaying
            (void)hipGraphExecDestroy(gs.front().exec);
            gs.erase(gs.begin());
        }
        hipGraph_t graph = nullptr;
        HCK(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
        ctx->events_off = true;
        int rc = enqueue_body(ctx, B, S, false, true);
        if (rc == RH_OK) rc = enqueue_tail(ctx, B, S, with_loss);
        ctx->events_off = false;
        const hipError_t ec = hipStreamEndCapture(ctx->stream, &graph);
        if (rc != RH_OK) {
            if (graph) (void)hipGraphDestroy(graph);
            return rc;
        }
        HCK(ec);
        FwdGraph g;
        g.B = B; g.S = S; g.loss = with_loss;
        const hipError_t ei = hipGraphInstantiate(&g.exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        HCK(ei);
        gs.push_back(g);
        it = gs.end() - 1;
    }
    HCK(hipGraphLaunch(it->exec, ctx->stream));
    return RH_OK;
}

}  // namespace

// One decode step for B tokens at position b.state[0].  For small B the
// RMSNorms run inside the QKV / W1|W3 / logits GEMVs (one launch fewer per
// norm); otherwise a row kernel writes the normalised rows first.
int rhrt::enqueue_decode_step(rh_ctx* ctx, int B, const DecodeBufs& b) {
    const rh_config& c = ctx->cfg;
    const int D = c.dim, F = c.hidden;
    const float alpha = 1.0f / std::sqrt(2.0f * (float)c.nlayers);
    const bool fuse_norm = rh::gemv_norm_fits(B, D);
    const bool xfrag = rh::gemv_frag_inputs(B);  // fp16 GEMV inputs in fragment order
    hipStream_t st = ctx->stream;
    // Input of a normed GEMV.  Small B: the GEMV normalises x itself (xres +
    // gamma).  Larger B: the residual GEMV before it left fp16(x * gamma) in
    // dxn and per-block sums of squares in ssq, and the GEMV scales by 1/rms
    // (xg); the first norm of the step, after the embedding, is a row kernel.
    bool xg = false;
    auto normed = [&](rh::GemvArgs& g, const float* gamma) -> int {
        if (fuse_norm) {
            g.xres = b.dx; g.gamma = gamma; g.eps = c.rms_eps;
        } else if (xg) {
            g.X = b.dxn; g.rs_part = b.ssq; g.rs_n = D / 16; g.eps = c.rms_eps;
        } else {
            LCK(rh::launch_rmsnorm(b.dx, gamma, b.dxn, B, D, c.rms_eps, st, xfrag));
            g.X = b.dxn;
        }
        g.x_frag = xfrag && !fuse_norm;
        return RH_OK;
    };
    auto produce = [&](rh::GemvArgs& g, const float* gnext) {
        if (fuse_norm || !b.ssq) return;
        g.xg_out = b.dxn; g.gnext = gnext; g.ssq_out = b.ssq; g.out_frag = xfrag;
        xg = true;
    };
    LCK(rh::launch_embed(b.tok_in, ctx->embed, b.dx, B, D, c.vocab, ctx->d_err, st));
    for (int l = 0; l < c.nlayers; ++l) {
        const Layer& W = ctx->L[l];
        f16* kc = ctx->kcache + (size_t)l * ctx->kv_layer;
        f16* vc = ctx->vcache + (size_t)l * ctx->kv_layer;
        rh::GemvArgs g{};
        RCK(normed(g, W.g1));
        g.W = W.wqkv; g.B = B; g.N = 3 * D; g.K = D;
        g.out_f16 = b.dq; g.kc = kc; g.vc = vc; g.rope = ctx->rope; g.pos = b.state;
        g.D = D; g.H = c.heads; g.hd = c.head_dim; g.ctx = ctx->max_ctx;
        RCK(timed(ctx, RH_K_GEMV_QKV, [&] { return rh::launch_gemv(rh::GV_QKV, g, st); }));
        RCK(timed(ctx, RH_K_DECODE_ATTN, [&] {
            return rh::launch_attn_decode(b.dq, kc, vc, b.state, b.pm, b.pl, b.po, b.dattn, B, c.heads,
                                          c.head_dim, ctx->max_ctx, st, 0, xfrag);
        }));
        g = rh::GemvArgs{};
        g.W = W.wo; g.X = b.dattn; g.B = B; g.N = D; g.K = D; g.x_frag = xfrag;
        g.out_f32 = b.dx; g.ldo = D; g.alpha = alpha;
        produce(g, W.g2);
        RCK(timed(ctx, RH_K_GEMV_WO, [&] { return rh::launch_gemv(rh::GV_RESID, g, st); }));
        g = rh::GemvArgs{};
        RCK(normed(g, W.g2));
        g.W = W.w13; g.B = B; g.N = 2 * F; g.K = D;
        g.out_f16 = b.dgate; g.ldo = F; g.out_frag = xfrag;
        RCK(timed(ctx, RH_K_GEMV_W13, [&] { return rh::launch_gemv(rh::GV_SWIGLU, g, st); }));
        g = rh::GemvArgs{};
        g.W = W.w2; g.X = b.dgate; g.B = B; g.N = D; g.K = F; g.x_frag = xfrag;
        g.out_f32 = b.dx; g.ldo = D; g.alpha = alpha;
        produce(g, l + 1 < c.nlayers ? ctx->L[l + 1].g1 : ctx->gfinal);
        RCK(timed(ctx, RH_K_GEMV_W2, [&] { return rh::launch_gemv(rh::GV_RESID, g, st); }));
    }
    rh::GemvArgs g{};
    RCK(normed(g, ctx->gfinal));
    g.W = ctx->embed; g.B = B; g.N = c.vocab; g.K = D;
    g.out_f32 = b.dlogits; g.ldo = c.vocab; g.softcap = c.softcap;
    g.am_val = b.am_v; g.am_idx = b.am_i;
    RCK(timed(ctx, RH_K_GEMV_LOGITS, [&] { return rh::launch_gemv(rh::GV_F32, g, st); }));
    LCK(rh::launch_argmax_final(b.am_v, b.am_i, rh::gemv_argmax_blocks(c.vocab), B, b.tok_out, b.next_in, b.seq,
                                b.state, true, ctx->max_ctx, ctx->d_err, st));
    return RH_OK;
}

rhrt::DecodeBufs rhrt::ctx_decode_bufs(rh_ctx* ctx) {
    DecodeBufs b{};
    b.dx = ctx->dx; b.dxn = ctx->dxn; b.dq = ctx->dq; b.dattn = ctx->dattn; b.dgate = ctx->dgate;
    b.dlogits = ctx->dlogits; b.pm = ctx->pm; b.pl = ctx->pl; b.po = ctx->po;
    b.am_v = ctx->dam_v; b.am_i = ctx->dam_i; b.state = ctx->dstate; b.ssq = ctx->dssq;
    b.tok_in = ctx->dtok; b.tok_out = ctx->dout; b.next_in = ctx->dtok; b.seq = ctx->dseq;
    return b;
}

namespace {

int run_decode_step(rh_ctx* ctx, int B) {
    const DecodeBufs bufs = ctx_decode_bufs(ctx);
    if (!ctx->use_graphs) return enqueue_decode_step(ctx, B, bufs);
    if (!ctx->dgraph || ctx->dgraph_B != B) {
        if (ctx->dgraph) {
            HCK(hipGraphExecDestroy(ctx->dgraph));
            ctx->dgraph = nullptr;
        }
        hipGraph_t graph = nullptr;
        HCK(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
        ctx->events_off = true;
        const int rc = enqueue_decode_step(ctx, B, bufs);
        ctx->events_off = false;
        const hipError_t ec = hipStreamEndCapture(ctx->stream, &graph);
        if (rc != RH_OK) {
            if (graph) (void)hipGraphDestroy(graph);
            return rc;
        }
        HCK(ec);
        const hipError_t ei = hipGraphInstantiate(&ctx->dgraph, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        HCK(ei);
        ctx->dgraph_B = B;
    }
    HCK(hipGraphLaunch(ctx->dgraph, ctx->stream));
    return RH_OK;
}

}  // namespace

rhrt::TensorMap rhrt::layer_map(rh_ctx* ctx, int l, int j) {
    const int D = ctx->cfg.dim, F = ctx->cfg.hidden;
    Layer& W = ctx->L[l];
    switch (j) {
        case 0: return {D, D, 0, 0, W.wqkv, D};
        case 1: return {D, D, 0, D, W.wqkv, D};
        case 2: return {D, D, 0, 2 * D, W.wqkv, D};
        case 3: return {D, D, 0, 0, W.wo, D};
        case 4: return {D, F, 1, 0, W.w13, D};
        case 5: return {D, F, 1, 16, W.w13, D};
        case 6: return {D, F, -1, 0, W.w2, F};
    }
    return {0, 0, -1, 0, nullptr, 0};
}

int rhrt::check_err_flag(rh_ctx* ctx) {
    int h = 0;
    HCK(hipMemcpyAsync(&h, ctx->d_err, sizeof(int), hipMemcpyDeviceToHost, ctx->stream));
    HCK(hipStreamSynchronize(ctx->stream));
    if (h != 0) {
        const int z = 0;
        HCK(hipMemcpy(ctx->d_err, &z, sizeof(int), hipMemcpyHostToDevice));
        if (h & rh::ERR_PAST_CACHE)
            return fail(ctx, RH_ERANGE, "a decode step ran past the end of the KV cache; its outputs are undefined");
        return fail(ctx, RH_ERANGE, std::to_string(h) + " token id(s) >= vocab were clamped to 0");
    }
    return RH_OK;
}

int rhrt::check_tokens(rh_ctx* ctx, const uint32_t* t, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (t[i] >= (uint32_t)ctx->cfg.vocab)
            return fail(ctx, RH_ERANGE, "token id " + std::to_string(t[i]) + " at index " +
                                            std::to_string(i) + " >= vocab " + std::to_string(ctx->cfg.vocab));
    return RH_OK;
}

namespace {

// src (fp32, reference orientation, on the device) -> device fp16 layout
int pack_from(rh_ctx* ctx, const float* src, const TensorMap& m) {
    if (m.map < 0) {
        LCK(rh::launch_pack_rows(src, m.dst, m.R, m.C, ctx->stream));
    } else {
        LCK(rh::launch_pack_transpose(src, m.dst, m.R, m.C, m.ldd, m.map, m.row_off, ctx->stream));
    }
    return RH_OK;
}

int unpack_to_staging(rh_ctx* ctx, const TensorMap& m) {
    if (m.map < 0) {
        LCK(rh::launch_unpack_rows(m.dst, ctx->staging, m.R, m.C, ctx->stream));
    } else {
        LCK(rh::launch_unpack_transpose(m.dst, ctx->staging, m.R, m.C, m.ldd, m.map, m.row_off, ctx->stream));
    }
    return RH_OK;
}

// Re-reads the decode position from the device once allocation-free steps
// have run since the prefill: a captured one may be replayed at any time,
// so the device's copy stays the authority until the next prefill.
int sync_pos(rh_ctx* ctx) {
    if (!ctx->pos_on_device) return RH_OK;
    HCK(hipSetDevice(ctx->device));
    int st[2] = {0, 0};
    HCK(hipMemcpyAsync(st, ctx->dstate, sizeof st, hipMemcpyDeviceToHost, ctx->stream));
    HCK(hipStreamSynchronize(ctx->stream));
    ctx->host_pos = st[0];
    return RH_OK;
}

void destroy_ctx(rh_ctx* ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    drop_graphs(ctx);
    for (auto& p : ctx->prof)
        for (auto& e : p.ev) { (void)hipEventDestroy(e.first); (void)hipEventDestroy(e.second); }
    rhrt::train_state_free(ctx->train);
    rhrt::noalloc_release(ctx);
    for (void* p : ctx->allocs) (void)hipFree(p);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

}  // namespace

extern "C" {

const char* rh_last_error(const rh_ctx* ctx) { return ctx ? ctx->err.c_str() : rh_internal_tls_error(); }

}  // extern "C"
int rh_internal_fail(rh_ctx* ctx, int code, const std::string& msg) { return fail(ctx, code, msg); }
extern "C" {

int rh_context_info(const rh_ctx* ctx, rh_config* cfg_out, int* max_batch_out, int* max_ctx_out) {
    if (!ctx) return RH_EINVAL;
    if (cfg_out) *cfg_out = ctx->cfg;
    if (max_batch_out) *max_batch_out = ctx->max_batch;
    if (max_ctx_out) *max_ctx_out = ctx->max_ctx;
    return RH_OK;
}

int rh_create(const rh_config* cfg, int device, int max_batch, int max_ctx, rh_ctx** out) {
    if (!cfg || !out) return RH_EINVAL;
    *out = nullptr;
    const rh_config& c = *cfg;
    if (c.dim <= 0 || c.dim % 128 || c.dim > 8192 || c.hidden <= 0 || c.hidden % 128 || c.heads <= 0 ||
        c.kv_heads != c.heads || !(c.head_dim == 64 || c.head_dim == 128) ||
        c.heads * c.head_dim != c.dim || c.nlayers <= 0 || c.vocab <= 0 || c.vocab % 4 ||
        c.seq <= 0 || max_batch <= 0 || max_ctx < 0 || !(c.rms_eps > 0.f) || !(c.rope_base > 0.f) ||
        c.softcap < 0.f)
        return RH_EINVAL;
    rh_ctx* ctx = new (std::nothrow) rh_ctx;
    if (!ctx) return RH_ENOMEM;
    ctx->cfg = c;
    ctx->device = device;
    ctx->max_batch = max_batch;
    ctx->max_ctx = max_ctx;
    auto bail = [&](int rc) { destroy_ctx(ctx); return rc; };
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev) return bail(RH_EDEVICE);
    if (hipSetDevice(device) != hipSuccess) return bail(RH_EDEVICE);
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) return bail(RH_EDEVICE);
    int rc0 = noalloc_init(ctx);  // device address of rh_decode_step_noalloc's scratch
    if (rc0) return bail(rc0);

    const size_t D = c.dim, F = c.hidden, V = c.vocab;
    int rc = RH_OK;
    // the embedding table doubles as the logits weight: fragment order, rows padded to 16
    const size_t V16 = (V + 15) / 16 * 16;
    if ((rc = dalloc(ctx, &ctx->embed, V16 * D)) || (rc = dalloc(ctx, &ctx->gfinal, D))) return bail(rc);
    if (hipMemset(ctx->embed, 0, V16 * D * sizeof(f16)) != hipSuccess) return bail(RH_EDEVICE);
    ctx->L.resize(c.nlayers);
    for (auto& W : ctx->L) {
        if ((rc = dalloc(ctx, &W.wqkv, 3 * D * D)) || (rc = dalloc(ctx, &W.wo, D * D)) ||
            (rc = dalloc(ctx, &W.w13, 2 * F * D)) || (rc = dalloc(ctx, &W.w2, D * F)) ||
            (rc = dalloc(ctx, &W.g1, D)) || (rc = dalloc(ctx, &W.g2, D)))
            return bail(rc);
    }
    if ((rc = dalloc(ctx, &ctx->d_err, 1))) return bail(rc);
    if (hipMemset(ctx->d_err, 0, sizeof(int)) != hipSuccess) return bail(RH_EDEVICE);
    if ((rc = ensure_rope(ctx, std::max(c.seq, max_ctx)))) return bail(rc);
    if (max_ctx > 0) {
        const int Bd = std::min(max_batch, 16);
        ctx->kv_layer = (size_t)max_batch * c.heads * (size_t)max_ctx * c.head_dim;
        const int nch = rh::attn_decode_chunks(1, c.heads, max_ctx);  // decode attention partials per (sequence, head)
        if ((rc = dalloc(ctx, &ctx->kcache, ctx->kv_layer * c.nlayers)) ||
            (rc = dalloc(ctx, &ctx->vcache, ctx->kv_layer * c.nlayers)) ||
            (rc = dalloc(ctx, &ctx->dx, 16 * D)) || (rc = dalloc(ctx, &ctx->dxn, 16 * D)) ||
            (rc = dalloc(ctx, &ctx->dq, 16 * D)) || (rc = dalloc(ctx, &ctx->dattn, 16 * D)) ||
            (rc = dalloc(ctx, &ctx->dgate, 16 * F)) || (rc = dalloc(ctx, &ctx->dlogits, 16 * V)) ||
            (rc = dalloc(ctx, &ctx->pm, (size_t)Bd * c.heads * nch)) ||
            (rc = dalloc(ctx, &ctx->pl, (size_t)Bd * c.heads * nch)) ||
            (rc = dalloc(ctx, &ctx->po, (size_t)Bd * c.heads * nch * c.head_dim)) ||
            (rc = dalloc(ctx, &ctx->dstate, 2)) || (rc = dalloc(ctx, &ctx->dtok, 16)) ||
            (rc = dalloc(ctx, &ctx->dssq, D)) ||
            (rc = dalloc(ctx, &ctx->dout, 16)) || (rc = dalloc(ctx, &ctx->dseq, (size_t)max_ctx * 16)) ||
            (rc = dalloc(ctx, &ctx->dam_v, (size_t)rh::gemv_argmax_blocks(c.vocab) * 16)) ||
            (rc = dalloc(ctx, &ctx->dam_i, (size_t)rh::gemv_argmax_blocks(c.vocab) * 16)))
            return bail(rc);
        // GEMV B operand rows >= B are never read, but keep them defined.
        if (hipMemset(ctx->dxn, 0, 16 * D * sizeof(f16)) != hipSuccess) return bail(RH_EDEVICE);
    }
    // weights start as N(0, 0.02) with unit gammas so a context is usable at once
    if ((rc = rh_init_weights_normal(ctx, 0, 0.02f))) return bail(rc);
    *out = ctx;
    return RH_OK;
}

void rh_destroy(rh_ctx* ctx) { destroy_ctx(ctx); }

int rh_load_weights_f32(rh_ctx* ctx, const float* embed, const float* gamma_final,
                        const float* const* layer_tensors) {
    if (!ctx || !embed || !gamma_final || !layer_tensors) return fail(ctx, RH_EINVAL, "null argument");
    HCK(hipSetDevice(ctx->device));
    const rh_config& c = ctx->cfg;
    const size_t D = c.dim, F = c.hidden, V = c.vocab;
    for (int i = 0; i < 9 * c.nlayers; ++i)
        if (!layer_tensors[i]) return fail(ctx, RH_EINVAL, "null layer tensor " + std::to_string(i));
    // With fp32 masters (rh_set_fp32_masters, or an optimizer state) each
    // matrix lands in its master copy, which is then packed to the fp16
    // device layout; otherwise it passes through a staging buffer the size
    // of the largest tensor.
    const bool masters = have_masters(ctx);
    if (!masters) RCK(ensure_staging(ctx, std::max({V * D, D * F, D * D})));
    hipStream_t st = ctx->stream;
    float* mst = masters ? master_ptr(ctx, 0, -1) : ctx->staging;
    HCK(hipMemcpyAsync(mst, embed, V * D * sizeof(float), hipMemcpyHostToDevice, st));
    LCK(rh::launch_pack_rows(mst, ctx->embed, (int)V, (int)D, st));
    HCK(hipMemcpyAsync(ctx->gfinal, gamma_final, D * sizeof(float), hipMemcpyHostToDevice, st));
    for (int l = 0; l < c.nlayers; ++l) {
        const float* const* t = layer_tensors + 9 * l;
        for (int j = 0; j < 7; ++j) {
            const TensorMap m = layer_map(ctx, l, j);
            mst = masters ? master_ptr(ctx, l, j) : ctx->staging;
            HCK(hipMemcpyAsync(mst, t[j], (size_t)m.R * m.C * sizeof(float), hipMemcpyHostToDevice, st));
            RCK(pack_from(ctx, mst, m));
        }
        HCK(hipMemcpyAsync(ctx->L[l].g1, t[7], D * sizeof(float), hipMemcpyHostToDevice, st));
        HCK(hipMemcpyAsync(ctx->L[l].g2, t[8], D * sizeof(float), hipMemcpyHostToDevice, st));
    }
    HCK(hipStreamSynchronize(st));
    ++ctx->wgen;
    RCK(weights_written(ctx, masters));
    return RH_OK;
}

int rh_set_fp32_masters(rh_ctx* ctx, int keep) {
    if (!ctx) return RH_EINVAL;
    HCK(hipSetDevice(ctx->device));
    if (!keep) return drop_masters(ctx);
    if (have_masters(ctx)) return RH_OK;
    RCK(ensure_masters(ctx));
    // until the next fp32 load they hold the current fp16 device weights
    const rh_config& c = ctx->cfg;
    hipStream_t st = ctx->stream;
    LCK(rh::launch_unpack_rows(ctx->embed, master_ptr(ctx, 0, -1), c.vocab, c.dim, st));
    for (int l = 0; l < c.nlayers; ++l)
        for (int j = 0; j < 7; ++j) {
            const TensorMap m = layer_map(ctx, l, j);
            if (m.map < 0) {
                LCK(rh::launch_unpack_rows(m.dst, master_ptr(ctx, l, j), m.R, m.C, st));
            } else {
                LCK(rh::launch_unpack_transpose(m.dst, master_ptr(ctx, l, j), m.R, m.C, m.ldd, m.map, m.row_off, st));
            }
        }
    HCK(hipStreamSynchronize(st));
    return weights_written(ctx, true);
}

int rh_read_weights_f32(rh_ctx* ctx, float* embed, float* gamma_final, float* const* layer_tensors) {
    if (!ctx) return RH_EINVAL;
    HCK(hipSetDevice(ctx->device));
    const rh_config& c = ctx->cfg;
    const size_t D = c.dim, F = c.hidden, V = c.vocab;
    RCK(ensure_staging(ctx, std::max({V * D, D * F, D * D})));
    hipStream_t st = ctx->stream;
    // After optimizer steps the fp32 masters are the weights; otherwise
    // widen the fp16 device copy.
    if (embed) {
        const float* src = train_master(ctx, 0, -1);
        if (!src) {
            LCK(rh::launch_unpack_rows(ctx->embed, ctx->staging, (int)V, (int)D, st));
            src = ctx->staging;
        }
        HCK(hipMemcpyAsync(embed, src, V * D * sizeof(float), hipMemcpyDeviceToHost, st));
        HCK(hipStreamSynchronize(st));
    }
    if (gamma_final) HCK(hipMemcpyAsync(gamma_final, ctx->gfinal, D * sizeof(float), hipMemcpyDeviceToHost, st));
    if (layer_tensors) {
        for (int l = 0; l < c.nlayers; ++l) {
            float* const* t = layer_tensors + 9 * l;
            for (int j = 0; j < 7; ++j) {
                if (!t[j]) continue;
                const TensorMap m = layer_map(ctx, l, j);
                const float* src = train_master(ctx, l, j);
                if (!src) {
                    RCK(unpack_to_staging(ctx, m));
                    src = ctx->staging;
                }
                HCK(hipMemcpyAsync(t[j], src, (size_t)m.R * m.C * sizeof(float), hipMemcpyDeviceToHost, st));
                HCK(hipStreamSynchronize(st));
            }
            if (t[7]) HCK(hipMemcpyAsync(t[7], ctx->L[l].g1, D * sizeof(float), hipMemcpyDeviceToHost, st));
            if (t[8]) HCK(hipMemcpyAsync(t[8], ctx->L[l].g2, D * sizeof(float), hipMemcpyDeviceToHost, st));
        }
    }
    HCK(hipStreamSynchronize(st));
    (void)F;
    return RH_OK;
}

int rh_init_weights_normal(rh_ctx* ctx, uint64_t seed, float std_) {
    if (!ctx) return RH_EINVAL;
    HCK(hipSetDevice(ctx->device));
    const rh_config& c = ctx->cfg;
    const size_t D = c.dim, F = c.hidden, V = c.vocab;
    RCK(ensure_staging(ctx, std::max({V * D, D * F, D * D})));
    hipStream_t st = ctx->stream;
    LCK(rh::launch_init_normal(ctx->staging, V * D, seed, 0u, std_, st));
    LCK(rh::launch_pack_rows(ctx->staging, ctx->embed, (int)V, (int)D, st));
    LCK(rh::launch_fill_f32(ctx->gfinal, 1.0f, D, st));
    for (int l = 0; l < c.nlayers; ++l) {
        for (int j = 0; j < 7; ++j) {
            const TensorMap m = layer_map(ctx, l, j);
            LCK(rh::launch_init_normal(ctx->staging, (size_t)m.R * m.C, seed, 1u + 9u * l + j, std_, st));
            RCK(pack_from(ctx, ctx->staging, m));
        }
        LCK(rh::launch_fill_f32(ctx->L[l].g1, 1.0f, D, st));
        LCK(rh::launch_fill_f32(ctx->L[l].g2, 1.0f, D, st));
    }
    HCK(hipStreamSynchronize(st));
    ++ctx->wgen;
    RCK(weights_written(ctx, false));
    (void)F;
    return RH_OK;
}

int rh_forward_dev(rh_ctx* ctx, const uint32_t* tokens, const uint32_t* targets, int batch, int seq,
                   float* logits_out, float* token_losses_out, float* mean_loss_out) {
    if (!ctx || !tokens) return fail(ctx, RH_EINVAL, "null argument");
    if (batch <= 0 || seq <= 0 || batch > ctx->max_batch)
        return fail(ctx, RH_ERANGE, "batch must be in [1, max_batch] and seq >= 1");
    if ((token_losses_out || mean_loss_out) && !targets)
        return fail(ctx, RH_EINVAL, "losses requested without targets");
    HCK(hipSetDevice(ctx->device));
    const int M = batch * seq;
    RCK(ensure_workspace(ctx, M));
    RCK(ensure_rope(ctx, seq));
    hipStream_t st = ctx->stream;
    HCK(hipMemcpyAsync(ctx->d_tok, tokens, (size_t)M * sizeof(uint32_t), hipMemcpyDeviceToDevice, st));
    if (targets)
        HCK(hipMemcpyAsync(ctx->d_tgt, targets, (size_t)M * sizeof(uint32_t), hipMemcpyDeviceToDevice, st));
    RCK(run_forward(ctx, batch, seq, targets != nullptr));
    const size_t V = V_(ctx);
    if (logits_out)
        HCK(hipMemcpyAsync(logits_out, ctx->logits, (size_t)M * V * sizeof(float), hipMemcpyDeviceToDevice, st));
    if (token_losses_out)
        HCK(hipMemcpyAsync(token_losses_out, ctx->tok_loss, (size_t)M * sizeof(float), hipMemcpyDeviceToDevice, st));
    if (mean_loss_out)
        HCK(hipMemcpyAsync(mean_loss_out, ctx->mean, (size_t)batch * sizeof(float), hipMemcpyDeviceToDevice, st));
    return RH_OK;
}

int rh_forward(rh_ctx* ctx, const uint32_t* tokens, const uint32_t* targets, int batch, int seq,
               float* logits_out, float* token_losses_out, float* mean_loss_out) {
    if (!ctx || !tokens) return fail(ctx, RH_EINVAL, "null argument");
    if (batch <= 0 || seq <= 0 || batch > ctx->max_batch)
        return fail(ctx, RH_ERANGE, "batch must be in [1, max_batch] and seq >= 1");
    if ((token_losses_out || mean_loss_out) && !targets)
        return fail(ctx, RH_EINVAL, "losses requested without targets");
    const size_t M = (size_t)batch * seq;
    RCK(check_tokens(ctx, tokens, M));
    if (targets) RCK(check_tokens(ctx, targets, M));
    HCK(hipSetDevice(ctx->device));
    RCK(ensure_workspace(ctx, (int)M));
    RCK(ensure_rope(ctx, seq));
    hipStream_t st = ctx->stream;
    HCK(hipMemcpyAsync(ctx->d_tok, tokens, M * sizeof(uint32_t), hipMemcpyHostToDevice, st));
    if (targets) HCK(hipMemcpyAsync(ctx->d_tgt, targets, M * sizeof(uint32_t), hipMemcpyHostToDevice, st));
    RCK(run_forward(ctx, batch, seq, targets != nullptr));
    const size_t V = V_(ctx);
    if (logits_out) HCK(hipMemcpyAsync(logits_out, ctx->logits, M * V * sizeof(float), hipMemcpyDeviceToHost, st));
    if (token_losses_out)
        HCK(hipMemcpyAsync(token_losses_out, ctx->tok_loss, M * sizeof(float), hipMemcpyDeviceToHost, st));
    if (mean_loss_out) HCK(hipMemcpyAsync(mean_loss_out, ctx->mean, batch * sizeof(float), hipMemcpyDeviceToHost, st));
    HCK(hipStreamSynchronize(st));
    return check_err_flag(ctx);
}

int rh_prefill(rh_ctx* ctx, const uint32_t* tokens, int batch, int len, uint32_t* next_tok_out,
               float* last_logits_out) {
    if (!ctx || !tokens) return fail(ctx, RH_EINVAL, "null argument");
    if (ctx->max_ctx <= 0) return fail(ctx, RH_ESTATE, "context was created without a KV cache");
    if (batch <= 0 || batch > std::min(ctx->max_batch, 16) || len <= 0 || len > ctx->max_ctx)
        return fail(ctx, RH_ERANGE, "prefill needs 1 <= batch <= min(max_batch, 16), 1 <= len <= max_ctx");
    const size_t M = (size_t)batch * len;
    RCK(check_tokens(ctx, tokens, M));
    HCK(hipSetDevice(ctx->device));
    RCK(ensure_workspace(ctx, (int)M));
    hipStream_t st = ctx->stream;
    HCK(hipMemcpyAsync(ctx->d_tok, tokens, M * sizeof(uint32_t), hipMemcpyHostToDevice, st));
    RCK(enqueue_body(ctx, batch, len, true, false));
    const rh_config& c = ctx->cfg;
    LCK(rh::launch_rmsnorm_strided(ctx->x, ctx->gfinal, ctx->dxn, batch, c.dim, c.rms_eps, len, len - 1, st));
    rh::GemvArgs g{};
    g.W = ctx->embed; g.X = ctx->dxn; g.B = batch; g.N = c.vocab; g.K = c.dim;
    g.out_f32 = ctx->dlogits; g.ldo = c.vocab; g.softcap = c.softcap;
    g.am_val = ctx->dam_v; g.am_idx = ctx->dam_i;
    RCK(timed(ctx, RH_K_GEMV_LOGITS, [&] { return rh::launch_gemv(rh::GV_F32, g, st); }));
    LCK(rh::launch_set_state(ctx->dstate, len, 0, st));
    LCK(rh::launch_argmax_final(ctx->dam_v, ctx->dam_i, rh::gemv_argmax_blocks(c.vocab), batch, ctx->dout,
                                ctx->dtok, nullptr, ctx->dstate, false, ctx->max_ctx, nullptr, st));
    if (next_tok_out) HCK(hipMemcpyAsync(next_tok_out, ctx->dout, batch * sizeof(uint32_t), hipMemcpyDeviceToHost, st));
    if (last_logits_out)
        HCK(hipMemcpyAsync(last_logits_out, ctx->dlogits, (size_t)batch * c.vocab * sizeof(float),
                           hipMemcpyDeviceToHost, st));
    HCK(hipStreamSynchronize(st));
    ctx->dec_B = batch;
    ctx->host_pos = len;
    ctx->pos_on_device = false;
    ctx->have_prefill = true;
    return check_err_flag(ctx);
}

int rh_decode_step(rh_ctx* ctx, int batch, const uint32_t* in_tok, uint32_t* out_tok, float* logits_out) {
    if (!ctx || !in_tok) return fail(ctx, RH_EINVAL, "null argument");
    if (!ctx->have_prefill) return fail(ctx, RH_ESTATE, "rh_decode_step before rh_prefill");
    RCK(sync_pos(ctx));
    if (batch != ctx->dec_B)
        return fail(ctx, RH_EINVAL, "batch " + std::to_string(batch) + " differs from the prefill batch " +
                                        std::to_string(ctx->dec_B));
    if (ctx->host_pos >= ctx->max_ctx) return fail(ctx, RH_ERANGE, "KV cache is full");
    const int B = ctx->dec_B;
    RCK(check_tokens(ctx, in_tok, B));
    HCK(hipSetDevice(ctx->device));
    hipStream_t st = ctx->stream;
    HCK(hipMemcpyAsync(ctx->dtok, in_tok, B * sizeof(uint32_t), hipMemcpyHostToDevice, st));
    LCK(rh::launch_set_state(ctx->dstate, ctx->host_pos, 0, st));
    RCK(run_decode_step(ctx, B));
    if (out_tok) HCK(hipMemcpyAsync(out_tok, ctx->dout, B * sizeof(uint32_t), hipMemcpyDeviceToHost, st));
    if (logits_out)
        HCK(hipMemcpyAsync(logits_out, ctx->dlogits, (size_t)B * ctx->cfg.vocab * sizeof(float),
                           hipMemcpyDeviceToHost, st));
    HCK(hipStreamSynchronize(st));
    ctx->host_pos += 1;
    return check_err_flag(ctx);
}

int rh_decode(rh_ctx* ctx, int batch, const uint32_t* in_tok, int nsteps, uint32_t* out_tokens) {
    if (!ctx || !in_tok || !out_tokens) return fail(ctx, RH_EINVAL, "null argument");
    if (!ctx->have_prefill) return fail(ctx, RH_ESTATE, "rh_decode before rh_prefill");
    RCK(sync_pos(ctx));
    if (batch != ctx->dec_B)
        return fail(ctx, RH_EINVAL, "batch " + std::to_string(batch) + " differs from the prefill batch " +
                                        std::to_string(ctx->dec_B));
    if (nsteps <= 0 || ctx->host_pos + nsteps > ctx->max_ctx)
        return fail(ctx, RH_ERANGE, "nsteps must be >= 1 and fit in the KV cache");
    const int B = ctx->dec_B;
    RCK(check_tokens(ctx, in_tok, B));
    HCK(hipSetDevice(ctx->device));
    hipStream_t st = ctx->stream;
    HCK(hipMemcpyAsync(ctx->dtok, in_tok, B * sizeof(uint32_t), hipMemcpyHostToDevice, st));
    LCK(rh::launch_set_state(ctx->dstate, ctx->host_pos, 0, st));
    for (int s = 0; s < nsteps; ++s) RCK(run_decode_step(ctx, B));
    HCK(hipMemcpyAsync(out_tokens, ctx->dseq, (size_t)nsteps * B * sizeof(uint32_t), hipMemcpyDeviceToHost, st));
    HCK(hipStreamSynchronize(st));
    ctx->host_pos += nsteps;
    return check_err_flag(ctx);
}

int rh_set_softcap(rh_ctx* ctx, float softcap) {
    if (!ctx) return RH_EINVAL;
    if (!(softcap >= 0.f)) return fail(ctx, RH_EINVAL, "softcap must be >= 0");
    if (softcap != ctx->cfg.softcap) drop_graphs(ctx);  // captured launches bake the softcap in
    ctx->cfg.softcap = softcap;
    return RH_OK;
}

int rh_decode_pos(rh_ctx* ctx, int* pos_out) {
    if (!ctx || !pos_out) return RH_EINVAL;
    RCK(sync_pos(ctx));
    *pos_out = ctx->host_pos;
    return RH_OK;
}

int rh_sync(rh_ctx* ctx) {
    if (!ctx) return RH_EINVAL;
    HCK(hipSetDevice(ctx->device));
    HCK(hipStreamSynchronize(ctx->stream));
    return check_err_flag(ctx);
}

void* rh_stream(rh_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int rh_profile_enable(rh_ctx* ctx, int cls, int enable) {
    if (!ctx || cls < 0 || cls >= RH_K_NCLASSES) return RH_EINVAL;
    Prof& p = ctx->prof[cls];
    for (auto& e : p.ev) { (void)hipEventDestroy(e.first); (void)hipEventDestroy(e.second); }
    p.ev.clear();
    p.ms = 0;
    p.n = 0;
    p.on = enable != 0;
    return RH_OK;
}

int rh_profile_read(rh_ctx* ctx, int cls, double* total_ms, int64_t* launches) {
    if (!ctx || cls < 0 || cls >= RH_K_NCLASSES) return RH_EINVAL;
    HCK(hipSetDevice(ctx->device));
    HCK(hipStreamSynchronize(ctx->stream));
    Prof& p = ctx->prof[cls];
    for (auto& e : p.ev) {
        float ms = 0.f;
        HCK(hipEventElapsedTime(&ms, e.first, e.second));
        p.ms += ms;
        p.n += 1;
        (void)hipEventDestroy(e.first);
        (void)hipEventDestroy(e.second);
    }
    p.ev.clear();
    if (total_ms) *total_ms = p.ms;
    if (launches) *launches = p.n;
    return RH_OK;
}

int rh_set_graphs(rh_ctx* ctx, int enable) {
    if (!ctx) return RH_EINVAL;
    ctx->use_graphs = enable != 0;
    return RH_OK;
}

}  // extern "C"
