// rh_gemv.hip -- decode projections for B <= 16 tokens (HBM-bound).
//
// y[b][n] = sum_k W[n][k] * x[b][k] with W [N, K] fp16 streamed exactly once,
// stored in fragment order (frag_off in rh_device.h) so every load
// instruction reads 1 KB contiguous.  A block owns 16 weight rows (two
// 16-row tiles for the SwiGLU pair) and its NW waves split K in 128-wide
// chunks, chunk c going to wave c % NW.  The MFMA's k order within a chunk is
// k = 32u + 8g + e (u = MFMA step, g = lane group, e = element), which is the
// order the fragments are stored in.  Each wave keeps DEPTH chunks in flight:
// HBM needs about bandwidth x latency bytes outstanding, and a decode GEMV
// has only N/16 blocks to supply them.  Loads are unconditional (chunk indexes
// past the wave's last chunk are clamped to a valid chunk and multiplied by
// zero), which keeps the load/wait schedule branch-free.
// The product runs on 16x16x32 MFMA with the tokens as the B operand (token
// rows >= B read row 0 and are discarded), which keeps the VALU free and
// handles B 1..16 with one kernel.  Epilogues mirror the prefill GEMM's:
// RoPE + KV-cache append, residual, SwiGLU, logits (+ per-block argmax
// partials for greedy decode).
//
// Larger batches (the normalised rows exceed the LDS budget): the residual
// GEMV that updates x also writes fp16(x * gamma_next) and per-block sums of
// x^2 per token; the next GEMV sums those partials in a fixed order, takes
// x * gamma as its fp16 input and scales its accumulators by each token's
// 1/rms -- the RMSNorm (rmsnorm::forward_channel_first, cpu/rmsnorm.rs:149-183)
// with no launch of its own (rs_part / ssq_out): rmsnorm(x) * gamma . W =
// (1/rms) * ((x * gamma) . W), rounded to fp16 before instead of after the
// 1/rms factor.  The fp16 input is x * gamma * XG_SCALE (a power of two, so
// the scaling is exact) and the consumer multiplies by 1/(rms * XG_SCALE):
// the unnormalised residual then stays finite up to |x * gamma| = 2^20
// instead of fp16's 65504, while values down to 2^-10 keep full fp16
// precision (smaller ones, subnormal after the scale, are off by at most
// 2^-21 in absolute terms).
//
// NORM: the input is the fp32 residual stream and the block applies the
// RMSNorm itself (rmsnorm::forward_channel_first, cpu/rmsnorm.rs:149-183)
// into LDS while its first weight chunks are in flight, in the same
// summation order as the standalone row kernel, so the normalised fp16 rows
// are bit-identical and one launch per norm disappears.
#include "rh_device.h"
#include "rh_kernels.h"

namespace rh {
namespace {

constexpr float XG_SCALE = 1.0f / 16.0f;

template <int EPI, int RT, int NW, int DEPTH, bool NORM, bool XF = false>
__global__ __launch_bounds__(NW * 64) void gemv_kernel(GemvArgs a) {
    __shared__ f32x4 sred[NW][RT][64];
    extern __shared__ __attribute__((aligned(16))) f16 sx[];  // NORM: normalised rows [B][K]
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int K = a.K, N = a.N;
    int rows[RT];
    if constexpr (EPI == GV_SWIGLU) {
        // W1|W3 interleaved in 16-row groups: block b owns features 16b..16b+15
        rows[0] = 32 * blockIdx.x;
        rows[1] = 32 * blockIdx.x + 16;
    } else {
        rows[0] = blockIdx.x * 16;
    }
    const f16* wp[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) wp[t] = a.W + (size_t)(rows[t] >> 4) * K * 16 + lane * 8;
    const bool xvalid = r < a.B;
    const int xrow = xvalid ? r : 0;
    const f16* xp = a.X + (size_t)xrow * K + 8 * g;
    const f16* xf = a.X + lane * 8;  // XF (x_frag): lane l's 16 bytes of each 1 KB fragment

    f32x4 acc[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t] = f32x4{};

    const int nch = K / 128;
    // chunks of this wave: w, w + NW, ... (< nch)
    const int my = w < nch ? (nch - 1 - w) / NW + 1 : 0;
    constexpr int XD = NORM ? 1 : DEPTH;  // X from LDS is read at use, not prefetched
    f16x8 wb[DEPTH][RT][4], xb[XD][4];
    auto wload = [&](int i, f16x8 (&wr)[RT][4]) {
        const size_t c = (size_t)min(w + i * NW, nch - 1);
#pragma unroll
        for (int t = 0; t < RT; ++t)
#pragma unroll
            for (int u = 0; u < 4; ++u) wr[t][u] = ld_stream((const f16x8*)(wp[t] + c * 2048 + 512 * u));
    };
    auto xload = [&](int i, f16x8 (&xr)[4]) {
        const int off = min(w + i * NW, nch - 1) * 128;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if constexpr (NORM)
                xr[u] = *(const f16x8*)&sx[xrow * K + off + 32 * u + 8 * g];
            else
                xr[u] = *(const f16x8*)(XF ? xf + (size_t)(off >> 7) * 2048 + 512 * u : xp + off + 32 * u);
        }
    };
    auto mac = [&](const f16x8 (&wr)[RT][4], const f16x8 (&xr)[4], bool live) {
        const f16x8 z = {};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const f16x8 xv = live ? xr[u] : z;
#pragma unroll
            for (int t = 0; t < RT; ++t) acc[t] = mfma16(wr[t][u], xv, acc[t]);
        }
    };
    // rs_part: token t's sum of squares over the producer's rs_n (<= 512)
    // blocks, as 16 strided slices summed in order and then the slices in
    // order.  Loaded ahead of the weight prefetch and reduced after the k
    // loop: only the epilogue needs 1/rms, so the loads' latency and the
    // reduction stay off the weight stream.
    constexpr bool RS = !NORM && EPI != GV_RESID;
    float pv[RS ? 32 : 1];
    if constexpr (RS) {
        if (a.rs_part && tid < 256) {
            const int t = tid & 15, q = tid >> 4;
#pragma unroll
            for (int k = 0; k < 32; ++k) {
                const int i = q + 16 * k;
                pv[k] = i < a.rs_n && t < a.B ? a.rs_part[i * 16 + t] : 0.f;
            }
        }
    }
#pragma unroll
    for (int s = 0; s < DEPTH; ++s) {
        wload(s, wb[s]);
        if constexpr (!NORM) xload(s, xb[s]);
    }
    if constexpr (NORM) {
        // r = 1/sqrt(sum(x^2) * (1/K) + eps), out = (x * r) * gamma: threads
        // 0..255 sum in the row kernel's order, the whole block writes
        __shared__ float red[NW];
        for (int t = 0; t < a.B; ++t) {
            const float* xr = a.xres + (size_t)t * K;
            float ss = 0.f;
            if (tid < 256)
                for (int i = tid * 4; i < K; i += 1024) {
                    const f32x4 v = *(const f32x4*)(xr + i);
                    ss += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
                }
            ss = wave_sum(ss);
            __syncthreads();
            if (lane == 0) red[w] = ss;
            __syncthreads();
            const float rs = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) * (1.0f / (float)K) + a.eps);
            for (int i = tid * 4; i < K; i += NW * 256) {
                const f32x4 v = *(const f32x4*)(xr + i);
                const f32x4 gm = *(const f32x4*)(a.gamma + i);
                *(f16x4*)&sx[t * K + i] = f16x4{(f16)(v[0] * rs * gm[0]), (f16)(v[1] * rs * gm[1]),
                                                (f16)(v[2] * rs * gm[2]), (f16)(v[3] * rs * gm[3])};
            }
        }
        __syncthreads();
    }
    int i = 0;
    for (; i + DEPTH < my; i += DEPTH) {
#pragma unroll
        for (int s = 0; s < DEPTH; ++s) {
            if constexpr (NORM) {
                xload(i + s, xb[0]);
                mac(wb[s], xb[0], true);
            } else {
                mac(wb[s], xb[s], true);
                xload(i + s + DEPTH, xb[s]);
            }
            wload(i + s + DEPTH, wb[s]);
        }
    }
#pragma unroll
    for (int s = 0; s < DEPTH; ++s) {
        if constexpr (NORM) {
            xload(i + s, xb[0]);
            mac(wb[s], xb[0], i + s < my);
        } else {
            mac(wb[s], xb[s], i + s < my);
        }
    }

#pragma unroll
    for (int t = 0; t < RT; ++t) sred[w][t][lane] = acc[t];
    __shared__ float s_sq[RS ? 16 : 1][16];
    if constexpr (RS) {
        if (a.rs_part && tid < 256) {
            float ss = 0.f;
#pragma unroll
            for (int k = 0; k < 32; ++k) ss += pv[k];
            s_sq[tid >> 4][tid & 15] = ss;
        }
    }
    __syncthreads();
    if (w != 0) return;
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        f32x4 s = sred[0][t][lane];
#pragma unroll
        for (int v = 1; v < NW; ++v) s += sred[v][t][lane];
        acc[t] = s;
    }
    if constexpr (RS) {
        if (a.rs_part) {
            float ss = 0.f;  // token r's slices, in order
#pragma unroll
            for (int q = 0; q < 16; ++q) ss += s_sq[q][r];
            const float rs = 1.0f / sqrtf(ss * (1.0f / (float)K) + a.eps) * (1.0f / XG_SCALE);
#pragma unroll
            for (int t = 0; t < RT; ++t) acc[t] *= rs;
        }
    }
    const int tok = r;
    // lane holds rows rows[t] + 4g + (0..3) for token `tok`
    if constexpr (EPI == GV_SWIGLU) {
        if (!xvalid) return;
        const int f = 16 * blockIdx.x + 4 * g;
        f16x4 gv;
#pragma unroll
        for (int e = 0; e < 4; ++e) gv[e] = (f16)(silu_f(acc[0][e]) * acc[1][e]);
        *(f16x4*)(a.out_f16 + (a.out_frag ? frag_off(tok, f, a.ldo) : (size_t)tok * a.ldo + f)) = gv;
    } else {
        const int n = rows[0] + 4 * g;
        float v0 = acc[0][0], v1 = acc[0][1], v2 = acc[0][2], v3 = acc[0][3];
        if constexpr (EPI == GV_F32) {
            if (a.softcap > 0.f) {
                const float cc = a.softcap, ic = 1.0f / cc;
                v0 = tanhf(v0 * ic) * cc; v1 = tanhf(v1 * ic) * cc;
                v2 = tanhf(v2 * ic) * cc; v3 = tanhf(v3 * ic) * cc;
            }
            if (xvalid && n < N)
                *(f32x4*)(a.out_f32 + (size_t)tok * a.ldo + n) = f32x4{v0, v1, v2, v3};
            if (a.am_val) {
                // best of this lane's 4 rows (ties -> lowest row), then across the
                // 4 lane groups of the token; rows >= N never win
                float bv = -INFINITY;
                int bi = 0x7fffffff;
                if (n < N) {
                    bv = v0; bi = n;
                    if (v1 > bv) { bv = v1; bi = n + 1; }
                    if (v2 > bv) { bv = v2; bi = n + 2; }
                    if (v3 > bv) { bv = v3; bi = n + 3; }
                }
#pragma unroll
                for (int o = 16; o < 64; o <<= 1) {
                    const float ov = __shfl_xor(bv, o, RH_WAVE);
                    const int oi = __shfl_xor(bi, o, RH_WAVE);
                    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
                }
                if (g == 0 && xvalid) {  // token-major, so each token's reduction reads contiguously
                    a.am_val[(size_t)tok * gridDim.x + blockIdx.x] = bv;
                    a.am_idx[(size_t)tok * gridDim.x + blockIdx.x] = bi;
                }
            }
        } else if constexpr (EPI == GV_RESID) {
            const bool live = xvalid && n < N;
            f32x4 x = f32x4{};
            if (live) {
                f32x4* px = (f32x4*)(a.out_f32 + (size_t)tok * a.ldo + n);
                x = *px;
                x[0] = v0 * a.alpha + x[0]; x[1] = v1 * a.alpha + x[1];
                x[2] = v2 * a.alpha + x[2]; x[3] = v3 * a.alpha + x[3];
                *px = x;
            }
            if (a.ssq_out) {  // the next RMSNorm's input and partial sums (all 64 lanes)
                if (live) {
                    const f32x4 gm = *(const f32x4*)(a.gnext + n);
                    *(f16x4*)(a.xg_out + (a.out_frag ? frag_off(tok, n, N) : (size_t)tok * N + n)) =
                        f16x4{(f16)(x[0] * gm[0] * XG_SCALE), (f16)(x[1] * gm[1] * XG_SCALE),
                              (f16)(x[2] * gm[2] * XG_SCALE), (f16)(x[3] * gm[3] * XG_SCALE)};
                }
                // the token's 4 lane groups, in a fixed order
                const float ss = xrow_sum4((x[0] * x[0] + x[1] * x[1]) + (x[2] * x[2] + x[3] * x[3]));
                if (g == 0) a.ssq_out[(size_t)blockIdx.x * 16 + r] = ss;
            }
        } else {  // GV_QKV
            if (!xvalid || n >= N) return;
            // a position past the cache (a captured step replayed too often):
            // RoPE at the last slot, no K/V write
            const int pos = *a.pos, pr = min(pos, a.ctx - 1);
            const int sec = n / a.D, cc = n - sec * a.D;
            const int h = cc / a.hd, d = cc - h * a.hd;
            if (sec > 0 && pos >= a.ctx) return;
            if (sec < 2) {
                const float2 cs0 = a.rope[(size_t)pr * (a.hd / 2) + d / 2];
                const float2 cs1 = a.rope[(size_t)pr * (a.hd / 2) + d / 2 + 1];
                const float r0 = v0 * cs0.x + (-v1) * cs0.y, r1 = v1 * cs0.x + v0 * cs0.y;
                const float r2 = v2 * cs1.x + (-v3) * cs1.y, r3 = v3 * cs1.x + v2 * cs1.y;
                v0 = r0; v1 = r1; v2 = r2; v3 = r3;
            }
            f16* dst;
            if (sec == 0)
                dst = a.out_f16 + (size_t)tok * a.D + cc;
            else
                dst = (sec == 1 ? a.kc : a.vc) + (((size_t)tok * a.H + h) * a.ctx + pos) * a.hd + d;
            *(f16x4*)dst = f16x4{(f16)v0, (f16)v1, (f16)v2, (f16)v3};
        }
    }
}

// Reduce the per-block (value, index) partials of the logits GEMV ([B][nblk],
// token-major); ties -> lowest index.  16 waves: 16/B per token (B <= 16),
// each strided over its token's partials with 8 coalesced loads of each
// array in flight, then the token's waves merge through LDS.
// Writes out[b], next_in[b] and seq_out[state[1] * B + b]; then (advance)
// state[0] += 1, state[1] += 1 while the position is inside the cache
// (state[0] < limit); a step run at a position past it (a captured step
// replayed too often) wrote nothing to the cache and sets ERR_PAST_CACHE in
// *err instead.
__global__ __launch_bounds__(1024) void argmax_final_kernel(const float* pv, const int* pi, int nblk,
                                                            int B, uint32_t* out, uint32_t* next_in,
                                                            uint32_t* seq_out, int* state, int advance,
                                                            int limit, int* err) {
    __shared__ float sv[16];
    __shared__ int si[16];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int wpt = 16 / B;  // waves per token
    const int b = w / wpt, sub = w - b * wpt;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    auto take = [&](float v, int ix) {
        if (v > bv || (v == bv && ix < bi)) { bv = v; bi = ix; }
    };
    if (b < B) {
        const int step = wpt * 64;
        int p = sub * 64 + lane;
        const float* tv = pv + (size_t)b * nblk;
        const int* ti = pi + (size_t)b * nblk;
        for (; p + 7 * step < nblk; p += 8 * step) {
            float v[8];
            int ix[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                v[q] = tv[p + q * step];
                ix[q] = ti[p + q * step];
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) take(v[q], ix[q]);
        }
        for (; p < nblk; p += step) take(tv[p], ti[p]);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) take(__shfl_xor(bv, o, RH_WAVE), __shfl_xor(bi, o, RH_WAVE));
        if (lane == 0) { sv[w] = bv; si[w] = bi; }
    }
    __syncthreads();
    if (b < B && sub == 0 && lane == 0) {
        for (int v = 1; v < wpt; ++v) take(sv[w + v], si[w + v]);
        if (bi == 0x7fffffff) bi = 0;  // all logits NaN
        out[b] = (uint32_t)bi;
        if (next_in) next_in[b] = (uint32_t)bi;
        if (seq_out) seq_out[(size_t)state[1] * B + b] = (uint32_t)bi;
    }
    if (!advance) return;
    __syncthreads();  // every token's writer has read state[1]
    if (threadIdx.x == 0) {
        if (state[0] < limit) {
            state[0] += 1;
            state[1] += 1;
        } else if (err) {
            atomicOr(err, ERR_PAST_CACHE);
        }
    }
}

// (NW, DEPTH) variants selectable through GemvArgs::cfg (1-based).
struct Variant { int nw, depth; };
constexpr Variant kVariants[] = {{4, 2}, {4, 3}, {4, 4}, {8, 2}, {8, 3}, {8, 4}, {16, 2}};
constexpr int kNumVariants = sizeof(kVariants) / sizeof(kVariants[0]);

template <int EPI, int RT, int NW, int DEPTH>
hipError_t launch_one(const GemvArgs& a, int nblk, hipStream_t st) {
    if constexpr (EPI != GV_RESID) {
        if (a.xres) {
            const size_t lds = (size_t)a.B * a.K * sizeof(f16);
            hipLaunchKernelGGL((gemv_kernel<EPI, RT, NW, DEPTH, true>), dim3(nblk), dim3(NW * 64), lds, st, a);
            return hipSuccess;
        }
    }
    if (a.x_frag)
        hipLaunchKernelGGL((gemv_kernel<EPI, RT, NW, DEPTH, false, true>), dim3(nblk), dim3(NW * 64), 0, st, a);
    else
        hipLaunchKernelGGL((gemv_kernel<EPI, RT, NW, DEPTH, false>), dim3(nblk), dim3(NW * 64), 0, st, a);
    return hipSuccess;
}

template <int EPI, int RT>
hipError_t launch_variant(int v, const GemvArgs& a, int nblk, hipStream_t st) {
    switch (v) {
        case 1: return launch_one<EPI, RT, 4, 2>(a, nblk, st);
        case 2: return launch_one<EPI, RT, 4, 3>(a, nblk, st);
        case 3: if constexpr (RT == 1) return launch_one<EPI, RT, 4, 4>(a, nblk, st); else break;
        case 4: return launch_one<EPI, RT, 8, 2>(a, nblk, st);
        case 5: return launch_one<EPI, RT, 8, 3>(a, nblk, st);
        case 6: if constexpr (RT == 1) return launch_one<EPI, RT, 8, 4>(a, nblk, st); else break;
        case 7: return launch_one<EPI, RT, 16, 2>(a, nblk, st);
        default: break;
    }
    return hipErrorInvalidValue;
}

// Default variant per shape, from sweeps of the 7B decode shapes on MI355X
// with fragment-ordered weights streamed from HBM by nontemporal loads
// (footprint > 2 GiB): 4 waves x 2 deep everywhere except the tall
// matrices at few tokens (QKV, logits: 8 x 2) and the SwiGLU pair rows at
// 16 tokens (8 x 2).  B 1: QKV 17.8 us, W1|W3 29.1, W2 15.4, Wo 7.3,
// logits 40.1 (5.5 - 6.5 TB/s).
int pick_variant(int epi, const GemvArgs& a) {
    if (epi == GV_SWIGLU) return a.B > 4 ? 4 : 1;
    if (a.K > 4096) return 1;
    if (a.N >= 8192) return a.B >= 8 ? 1 : 4;
    return 1;
}

}  // namespace

int gemv_num_variants() { return kNumVariants; }

bool gemv_norm_fits(int B, int K) { return (size_t)B * K * sizeof(f16) <= GEMV_NORM_LDS; }

hipError_t launch_gemv(int epi, const GemvArgs& a, hipStream_t st) {
    if (a.K % 128 != 0 || a.B < 1 || a.B > 16 || a.N % 4 != 0) return hipErrorInvalidValue;
    if (a.am_val && (epi != GV_F32 || !a.am_idx)) return hipErrorInvalidValue;
    if (a.xres && (epi == GV_RESID || !a.gamma || !gemv_norm_fits(a.B, a.K))) return hipErrorInvalidValue;
    if (a.ssq_out && (epi != GV_RESID || !a.xg_out || !a.gnext)) return hipErrorInvalidValue;
    if (a.rs_part && (epi == GV_RESID || a.xres || a.rs_n < 1 || a.rs_n > 512)) return hipErrorInvalidValue;
    if (a.x_frag && a.xres) return hipErrorInvalidValue;  // the in-kernel norm reads xres, not X
    // fragment-order outputs: whole 128-column chunks (GV_RESID's xg_out, GV_SWIGLU's gate)
    if (a.out_frag && !((epi == GV_RESID && a.N % 128 == 0) || (epi == GV_SWIGLU && a.ldo % 128 == 0)))
        return hipErrorInvalidValue;
    const int v = a.cfg > 0 ? a.cfg : pick_variant(epi, a);
    if (v > kNumVariants) return hipErrorInvalidValue;
    const int nblk = (a.N + 15) / 16;
    hipError_t e;
    switch (epi) {
        case GV_F32: e = launch_variant<GV_F32, 1>(v, a, nblk, st); break;
        case GV_RESID: e = launch_variant<GV_RESID, 1>(v, a, nblk, st); break;
        case GV_QKV: e = launch_variant<GV_QKV, 1>(v, a, nblk, st); break;
        case GV_SWIGLU:
            if (a.N % 32 != 0) return hipErrorInvalidValue;
            e = launch_variant<GV_SWIGLU, 2>(v, a, a.N / 32, st);
            break;
        default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess) return e;
    return hipGetLastError();
}

int gemv_argmax_blocks(int N) { return (N + 15) / 16; }

hipError_t launch_argmax_final(const float* pv, const int* pi, int nblk, int B, uint32_t* out,
                               uint32_t* next_in, uint32_t* seq_out, int* state, bool advance, int limit,
                               int* err, hipStream_t st) {
    if (B < 1 || B > 16 || nblk < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(1024), 0, st, pv, pi, nblk, B, out, next_in,
                       seq_out, state, advance ? 1 : 0, limit, err);
    return hipGetLastError();
}

}  // namespace rh
