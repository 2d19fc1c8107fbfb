// rh_noalloc.cpp -- rh_decode_step_noalloc: the greedy decode step with its
// scratch memory in one fixed device array instead of context allocations.
//
// The step's scratch (residual rows, normalised rows, q, attention output,
// gate, logits when the caller passes none, the attention's per-chunk
// partials and the logits GEMV's argmax partials) is carved out of
// `scratch`, a file-scope device array of kSlots * kSlotBytes.  Each GPU the
// library runs on holds its own copy of it until the process ends.  Host
// code never uses the array's name as an address: rh_create resolves the
// device address once per device with hipGetSymbolAddress (with that device
// current) and the entry point passes addresses inside it to the kernels.
//
// The array is cut into kSlots slots; a context takes a free slot of its
// device at its first call and keeps it until rh_destroy, so contexts on one
// GPU never share scratch (a fifth context using this entry point on one GPU
// at the same time is refused).  Calls of one context run in its stream
// order.  Nothing in a slot has to start at zero: every buffer the step
// reads is written earlier in the same step.
//
// The position is the context's own device-side decode state (allocated by
// rh_create), read and advanced by the step's kernels, so a captured step
// moves forward on every replay; the host-side entry points re-read it
// before their next use of the position.
#include "rh_ctx.h"

#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

namespace {

constexpr int kSlots = 4;
constexpr size_t kSlotBytes = (size_t)16 << 20;  // 16 MiB per context, 64 MiB per GPU
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kSlots * kSlotBytes];

std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};              // device address of `scratch`, per device
const rh_ctx* g_owner[kMaxDevices][kSlots] = {};  // the context holding each slot

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
    const size_t R = rh::gemv_frag_inputs(B) ? 16 : (size_t)B;  // fragment-order inputs hold 16 rows
    b->dx = (float*)take((size_t)B * D * 4);
    b->dxn = (f16*)take(R * D * 2);
    b->dq = (f16*)take((size_t)B * D * 2);
    b->dattn = (f16*)take(R * D * 2);
    b->dgate = (f16*)take(R * F * 2);
    b->dlogits = own_logits ? (float*)take((size_t)B * V * 4) : nullptr;
    b->pm = (float*)take(part * 4);
    b->pl = (float*)take(part * 4);
    b->po = (float*)take(part * c.head_dim * 4);
    b->am_v = (float*)take(am * 4);
    b->am_i = (int*)take(am * 4);
    b->ssq = (float*)take(D * 4);
    return off;
}

// The context's slot of its device's scratch (taken on first use), or null
// when every slot is held by another context.
unsigned char* slot_of(const rh_ctx* ctx) {
    std::lock_guard<std::mutex> lk(g_mu);
    unsigned char* base = (unsigned char*)g_scratch[ctx->device];
    if (!base) return nullptr;
    int freeslot = -1;
    for (int i = 0; i < kSlots; ++i) {
        if (g_owner[ctx->device][i] == ctx) return base + (size_t)i * kSlotBytes;
        if (!g_owner[ctx->device][i] && freeslot < 0) freeslot = i;
    }
    if (freeslot < 0) return nullptr;
    g_owner[ctx->device][freeslot] = ctx;
    return base + (size_t)freeslot * kSlotBytes;
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

void rhrt::noalloc_release(const rh_ctx* ctx) {
    if (ctx->device < 0 || ctx->device >= kMaxDevices) return;
    std::lock_guard<std::mutex> lk(g_mu);
    for (int i = 0; i < kSlots; ++i)
        if (g_owner[ctx->device][i] == ctx) g_owner[ctx->device][i] = nullptr;
}

extern "C" {

int rh_decode_step_noalloc(rh_ctx* ctx, int batch, const uint32_t* in_tok, uint32_t* out_tok, float* logits_out) {
    using namespace rhrt;
    if (!ctx || !in_tok || !out_tok) return fail(ctx, RH_EINVAL, "null argument");
    if (batch < 1 || batch > 16) return fail(ctx, RH_ERANGE, "batch must be in [1, 16]");
    DecodeBufs b{};
    const size_t need = layout(ctx, batch, logits_out == nullptr, nullptr, &b);
    if (need > kSlotBytes)
        return fail(ctx, RH_ERANGE,
                    "rh_decode_step_noalloc: batch " + std::to_string(batch) + " at this model and max_ctx " +
                        std::to_string(ctx->max_ctx) + " needs " + std::to_string(need) +
                        " bytes of scratch; a context's slot holds " + std::to_string(kSlotBytes));
    if (!ctx->have_prefill) return fail(ctx, RH_ESTATE, "rh_decode_step_noalloc before rh_prefill");
    if (batch != ctx->dec_B)
        return fail(ctx, RH_EINVAL, "batch " + std::to_string(batch) + " differs from the prefill batch " +
                                        std::to_string(ctx->dec_B));
    if (ctx->host_pos >= ctx->max_ctx) return fail(ctx, RH_ERANGE, "KV cache is full");
    HCK(hipSetDevice(ctx->device));
    RCK(noalloc_init(ctx));  // no-op once rh_create resolved it for this device
    unsigned char* base = slot_of(ctx);
    if (!base)
        return fail(ctx, RH_ERANGE, "rh_decode_step_noalloc: every scratch slot of this GPU is held by another "
                                    "context (" + std::to_string(kSlots) + " slots)");
    layout(ctx, batch, logits_out == nullptr, base, &b);
    if (logits_out) b.dlogits = logits_out;
    b.state = ctx->dstate;  // the context's position, advanced by the step itself
    b.tok_in = in_tok;
    b.tok_out = out_tok;
    b.next_in = nullptr;
    b.seq = nullptr;
    ctx->events_off = true;  // no profiling events: they are runtime allocations too
    const int rc = enqueue_decode_step(ctx, batch, b);
    ctx->events_off = false;
    RCK(rc);
    ctx->host_pos += 1;         // eager calls: one step each
    ctx->pos_on_device = true;  // replays of a captured step advance only the device's copy
    return RH_OK;
}

}  // extern "C"
