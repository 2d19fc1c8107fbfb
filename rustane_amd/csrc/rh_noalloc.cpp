// rh_noalloc.cpp -- rh_decode_step_noalloc: the greedy decode step with its
// scratch memory in one fixed device array instead of context allocations.
//
// The step's scratch (residual rows, normalised rows, q, attention output,
// gate, logits when the caller passes none, the attention's per-chunk
// partials, the logits GEMV's argmax partials and the position state) is
// carved out of `scratch`, a file-scope device array of kScratchBytes.  Each
// GPU the library runs on holds its own copy of it until the process ends.
// Host code never uses the array's name as an address: rh_create resolves
// the device address once per device with hipGetSymbolAddress (with that
// device current) and the entry point passes that address to the kernels.
//
// Every call on one GPU shares that GPU's array, whatever the context: calls
// whose work overlaps on the GPU (two contexts' streams, or two host threads)
// race.  Nothing in the array has to start at zero: every buffer the step
// reads is written earlier in the same step, and the position state is set
// by a kernel at the start of each call.
#include "rh_ctx.h"

#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

namespace {

constexpr size_t kScratchBytes = (size_t)64 << 20;  // 64 MiB per GPU
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};  // device address of `scratch`, per device

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Lays the step's buffers out from base (null: only sizes them); returns the
// bytes used.  own_logits: the caller gave no logits buffer, so the logits
// GEMV writes into the scratch.
size_t layout(const rh_ctx* ctx, int B, bool own_logits, unsigned char* base, rhrt::DecodeBufs* b) {
    const rh_config& c = ctx->cfg;
    const size_t D = c.dim, F = c.hidden, V = c.vocab;
    const size_t nch = (size_t)rh::attn_decode_chunks(B, c.heads, ctx->max_ctx);
    const size_t part = (size_t)B * c.heads * nch;
    const size_t am = (size_t)rh::gemv_argmax_blocks(c.vocab) * 16;
    size_t off = 0;
    auto take = [&](size_t bytes) -> unsigned char* {
        unsigned char* p = base ? base + off : nullptr;
        off += align256(bytes);
        return p;
    };
    b->dx = (float*)take((size_t)B * D * 4);
    b->dxn = (f16*)take((size_t)B * D * 2);
    b->dq = (f16*)take((size_t)B * D * 2);
    b->dattn = (f16*)take((size_t)B * D * 2);
    b->dgate = (f16*)take((size_t)B * F * 2);
    b->dlogits = own_logits ? (float*)take((size_t)B * V * 4) : nullptr;
    b->pm = (float*)take(part * 4);
    b->pl = (float*)take(part * 4);
    b->po = (float*)take(part * c.head_dim * 4);
    b->am_v = (float*)take(am * 4);
    b->am_i = (int*)take(am * 4);
    b->state = (int*)take(2 * 4);
    b->ssq = (float*)take(D * 4);
    return off;
}

}  // namespace

int rhrt::noalloc_init(rh_ctx* ctx) {
    if (ctx->device < 0 || ctx->device >= kMaxDevices)
        return fail(ctx, RH_EDEVICE, "device index beyond the scratch table");
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_scratch[ctx->device]) return RH_OK;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
        return fail(ctx, RH_EDEVICE, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch[ctx->device] = p;
    return RH_OK;
}

extern "C" {

int rh_decode_step_noalloc(rh_ctx* ctx, int batch, const uint32_t* in_tok, uint32_t* out_tok, float* logits_out) {
    using namespace rhrt;
    if (!ctx || !in_tok || !out_tok) return fail(ctx, RH_EINVAL, "null argument");
    if (batch < 1 || batch > 16) return fail(ctx, RH_ERANGE, "batch must be in [1, 16]");
    DecodeBufs b{};
    const size_t need = layout(ctx, batch, logits_out == nullptr, nullptr, &b);
    if (need > kScratchBytes)
        return fail(ctx, RH_ERANGE,
                    "rh_decode_step_noalloc: batch " + std::to_string(batch) + " at this model and max_ctx " +
                        std::to_string(ctx->max_ctx) + " needs " + std::to_string(need) +
                        " bytes of scratch; the fixed scratch holds " + std::to_string(kScratchBytes));
    if (!ctx->have_prefill) return fail(ctx, RH_ESTATE, "rh_decode_step_noalloc before rh_prefill");
    if (batch != ctx->dec_B)
        return fail(ctx, RH_EINVAL, "batch " + std::to_string(batch) + " differs from the prefill batch " +
                                        std::to_string(ctx->dec_B));
    if (ctx->host_pos >= ctx->max_ctx) return fail(ctx, RH_ERANGE, "KV cache is full");
    HCK(hipSetDevice(ctx->device));
    RCK(noalloc_init(ctx));  // no-op once rh_create resolved it for this device
    void* base = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        base = g_scratch[ctx->device];
    }
    layout(ctx, batch, logits_out == nullptr, (unsigned char*)base, &b);
    if (logits_out) b.dlogits = logits_out;
    b.tok_in = in_tok;
    b.tok_out = out_tok;
    b.next_in = nullptr;
    b.seq = nullptr;
    LCK(rh::launch_set_state(b.state, ctx->host_pos, 0, ctx->stream));
    ctx->events_off = true;  // no profiling events: they are runtime allocations too
    const int rc = enqueue_decode_step(ctx, batch, b);
    ctx->events_off = false;
    RCK(rc);
    ctx->host_pos += 1;
    return RH_OK;
}

}  // extern "C"
