// rh_ctx.h -- the context object and the host helpers shared by the
// runtime's translation units (forward/decode runtime, training pass).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <utility>
#include <type_traits>
#include <vector>

#include "../../include/rustane_hip.h"
#include "rh_internal.h"
#include "rh_kernels.h"

namespace rhrt {

struct Layer {
    f16 *wqkv = nullptr, *wo = nullptr, *w13 = nullptr, *w2 = nullptr;
    float *g1 = nullptr, *g2 = nullptr;
};

struct Prof {
    bool on = false;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> ev;
    double ms = 0;
    int64_t n = 0;
};

// A captured forward (body + logits/loss tail) for one (batch, seq, loss).
struct FwdGraph {
    int B = 0, S = 0;
    bool loss = false;
    hipGraphExec_t exec = nullptr;
};

struct TrainState;                 // rh_train.cpp
void train_state_free(TrainState* t);  // host side only; device buffers are context allocations

}  // namespace rhrt

struct rh_ctx {
    rh_config cfg{};
    int device = 0, max_batch = 0, max_ctx = 0;
    hipStream_t stream = nullptr;
    std::string err;
    std::vector<void*> allocs;

    f16* embed = nullptr;
    float* gfinal = nullptr;
    std::vector<rhrt::Layer> L;
    float2* rope = nullptr;
    int rope_len = 0;

    // forward / prefill workspace (grow-only, sized for M = B*S rows);
    // work_epoch counts the calls that write it (a kept training forward is
    // valid while the count is unchanged)
    int ws_M = 0;
    uint64_t work_epoch = 0;
    float *x = nullptr, *logits = nullptr, *tok_loss = nullptr, *mean = nullptr;
    f16 *xn = nullptr, *q = nullptr, *kbuf = nullptr, *vbuf = nullptr, *attn = nullptr, *gate = nullptr;
    uint32_t *d_tok = nullptr, *d_tgt = nullptr;
    size_t logits_rows = 0;
    int* d_err = nullptr;

    // KV cache [L][max_batch][H][max_ctx][hd]
    f16 *kcache = nullptr, *vcache = nullptr;
    size_t kv_layer = 0;

    // decode (B <= 16)
    float *dx = nullptr, *dlogits = nullptr, *pm = nullptr, *pl = nullptr, *po = nullptr;
    f16 *dxn = nullptr, *dq = nullptr, *dattn = nullptr, *dgate = nullptr;
    int* dstate = nullptr;
    float* dssq = nullptr;  // [D/16][16] sums of squares from the residual GEMVs (B > fused-norm limit)
    uint32_t *dtok = nullptr, *dout = nullptr, *dseq = nullptr;
    float* dam_v = nullptr;  // [argmax blocks][16] argmax partials of the logits GEMV
    int* dam_i = nullptr;
    int dec_B = 0, host_pos = 0;
    // an allocation-free step ran since the prefill (a captured one may be
    // replayed any time): host-side calls re-read the position from dstate
    bool pos_on_device = false;
    bool have_prefill = false;
    bool use_graphs = true;
    hipGraphExec_t dgraph = nullptr;
    int dgraph_B = 0;
    std::vector<rhrt::FwdGraph> fgraphs;  // forward graphs, most recent last
    // no profiling events while set: a graph is being captured, or the call
    // must not create runtime objects (rh_decode_step_noalloc)
    bool events_off = false;

    float* staging = nullptr;
    size_t staging_elems = 0;

    // stream-K workspace of the prefill GEMMs (fp32 partial tiles)
    float* sk_part = nullptr;
    size_t sk_part_floats = 0;

    rhrt::Prof prof[RH_K_NCLASSES];

    // bumped whenever the weights change (derived copies are rebuilt lazily)
    uint64_t wgen = 1;
    // training state (rh_train.cpp), allocated by the first backward call
    rhrt::TrainState* train = nullptr;
};


namespace rhrt {

// Records m as the context's last error and returns code.
int fail(rh_ctx* c, int code, const std::string& m);

#define HCK(expr)                                                                     \
    do {                                                                              \
        hipError_t e_ = (expr);                                                       \
        if (e_ != hipSuccess)                                                         \
            return rhrt::fail(ctx, RH_EDEVICE, std::string(#expr) + ": " + hipGetErrorString(e_)); \
    } while (0)

#define RCK(expr)                   \
    do {                            \
        int r_ = (expr);            \
        if (r_ != RH_OK) return r_; \
    } while (0)

#define LCK(expr)                                                                              \
    do {                                                                                       \
        hipError_t e_ = (expr);                                                                \
        if (e_ != hipSuccess)                                                                  \
            return rhrt::fail(ctx, RH_EDEVICE, std::string("launch ") + #expr + ": " + hipGetErrorString(e_)); \
    } while (0)

// Device allocation owned by the context (freed with it).
template <typename T>
int dalloc(rh_ctx* ctx, T** p, size_t elems) {
    void* q = nullptr;
    if (elems == 0) elems = 1;
    if (hipMalloc(&q, elems * sizeof(T)) != hipSuccess) {
        (void)hipGetLastError();
        return fail(ctx, RH_ENOMEM, "hipMalloc of " + std::to_string(elems * sizeof(T)) + " bytes failed");
    }
    ctx->allocs.push_back(q);
    *p = (T*)q;
    return RH_OK;
}
void dfree(rh_ctx* ctx, void* p);

// Launches fn(); when profiling class cls is on (and no graph is being
// captured) times it with an event pair.  A launcher that takes the two
// events (fn(start, stop); both null when off) stamps them at its kernel's
// own start and end, so the time excludes the dispatch; otherwise the events
// are recorded around fn().
template <typename Fn>
int timed(rh_ctx* ctx, int cls, Fn&& fn) {
    Prof& p = ctx->prof[cls];
    const bool on = p.on && !ctx->events_off;
    constexpr bool attached = std::is_invocable_v<Fn, hipEvent_t, hipEvent_t>;
    hipEvent_t a = nullptr, b = nullptr;
    if (on) {
        HCK(hipEventCreate(&a));
        HCK(hipEventCreate(&b));
        if constexpr (!attached) HCK(hipEventRecord(a, ctx->stream));
    }
    hipError_t e;
    if constexpr (attached)
        e = fn(a, b);
    else
        e = fn();
    if (e != hipSuccess) return fail(ctx, RH_EDEVICE, std::string("kernel launch: ") + hipGetErrorString(e));
    if (on) {
        if constexpr (!attached) HCK(hipEventRecord(b, ctx->stream));
        p.ev.emplace_back(a, b);
    }
    return RH_OK;
}

// Where weight tensor j (RSTK order, 0..6) of layer l lives on the device:
// reference orientation [R][C] and its fp16 packing (map -1: rows as is,
// K = C; map 0/1: transposed to rows dst_row(c), K = ldd, row_off).
struct TensorMap {
    int R, C, map, row_off;
    f16* dst;
    int ldd;
};
TensorMap layer_map(rh_ctx* ctx, int l, int j);
// The fp32 master copy of weight tensor j of layer l (j = -1: the
// embedding) kept by the optimizer, or null when there is none or the
// device weights changed since it was written.
const float* train_master(const rh_ctx* ctx, int l, int j);
// The fp32 master weights: whether they exist, where tensor j of layer l
// (j = -1: the embedding) lives among them, their allocation (all or none)
// and their release (refused while optimizer moments exist).
bool have_masters(const rh_ctx* ctx);
float* master_ptr(rh_ctx* ctx, int l, int j);
int ensure_masters(rh_ctx* ctx);
int drop_masters(rh_ctx* ctx);
// After a weight write (wgen already bumped): the masters hold the new
// weights when masters_hold_them is set (an fp32 load), otherwise they are
// stale; the moments restart from zero (ModelOptState::zeros).
int weights_written(rh_ctx* ctx, bool masters_hold_them);
// Destroys the captured graphs (their kernel arguments hold buffer addresses).
void drop_graphs(rh_ctx* ctx);

void set_sk(const rh_ctx* ctx, rh::GemmArgs& g);
int ensure_rope(rh_ctx* ctx, int npos);
int ensure_workspace(rh_ctx* ctx, int M);
int check_tokens(rh_ctx* ctx, const uint32_t* t, size_t n);
int check_err_flag(rh_ctx* ctx);
// Logits (+ CE loss rows and per-sequence means) from the final-norm rows in
// ctx->xn, or in xf when given; softcap < 0: the context's.
int enqueue_tail(rh_ctx* ctx, int B, int S, bool with_loss, const f16* xf = nullptr, float softcap = -1.f);

// Device buffers one greedy decode step uses besides the weights and the KV
// cache: the residual rows, normalised rows, q, attention output and gate of
// the B tokens, the logits, the attention's per-chunk partials, the logits
// GEMV's argmax partials, the position state, and the token in/out arrays.
struct DecodeBufs {
    float* dx;                 // [B][D] fp32 residual stream
    f16 *dxn, *dq, *dattn;     // [B][D]
    f16* dgate;                // [B][F]
    float* dlogits;            // [B][V]
    float *pm, *pl, *po;       // [B][H][chunks] (m, l), [B][H][chunks][hd] o
    float* ssq;                // [D/16][16] per-block sums of squares of x (norm without a row kernel)
    float* am_v;               // [gemv_argmax_blocks(V)][16]
    int* am_i;
    int* state;                // [2]: position, step
    const uint32_t* tok_in;    // [B] token ids of this step
    uint32_t* tok_out;         // [B] argmax ids
    uint32_t* next_in;         // nullable: argmax ids again, as the next step's input
    uint32_t* seq;             // nullable: argmax ids at seq[state[1] * B + b]
};
// The context's own decode buffers (allocated by rh_create).
DecodeBufs ctx_decode_bufs(rh_ctx* ctx);
// One decode step for B tokens at position state[0] (then state += 1).
int enqueue_decode_step(rh_ctx* ctx, int B, const DecodeBufs& b);
// Resolves the device address of the fixed scratch array of
// rh_decode_step_noalloc on ctx->device (once per device; the device must be
// current).  Called by rh_create.
int noalloc_init(rh_ctx* ctx);
// Frees the context's scratch slot (rh_destroy).
void noalloc_release(const rh_ctx* ctx);

}  // namespace rhrt
