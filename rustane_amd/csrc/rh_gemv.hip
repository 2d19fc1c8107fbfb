// rh_gemv.hip -- decode projections for B <= 16 tokens (HBM-bound).
//
// y[b][n] = sum_k W[n][k] * x[b][k] with W [N, K] fp16 streamed exactly once.
// A block owns 16 weight rows (two 16-row tiles for the SwiGLU pair) and its
// 4 waves split K in 128-wide chunks.  The MFMA's k order within a chunk is
// k = 32u + 8g + e (u = MFMA step, g = lane group, e = element), so the four
// lane groups of one row read 64 contiguous bytes per load instruction; the
// next chunk is loaded before the current one is consumed. 
// The product is done on 16x16x32 MFMA with the tokens as the B
// operand (rows >= B are zero), which keeps the VALU free and handles B 1..16
// with one kernel; MFMA throughput is far above what HBM can feed.  Epilogues
// mirror the prefill GEMM's: RoPE + KV-cache append, residual, SwiGLU, logits.
#include "rh_device.h"
#include "rh_kernels.h"

namespace rh {
namespace {

template <int EPI, int RT>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
    __shared__ f32x4 sred[4][RT][64];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int K = a.K, N = a.N;
    int rows[RT];
    if constexpr (EPI == GV_SWIGLU) {
        const int jb = blockIdx.x >> 1, u = blockIdx.x & 1;
        rows[0] = 64 * jb + 16 * u;
        rows[1] = 64 * jb + 32 + 16 * u;
    } else {
        rows[0] = blockIdx.x * 16;
    }
    const f16x8 z = {};
    const f16* wp[RT];
    bool wvalid[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        wvalid[t] = rows[t] + r < N;
        wp[t] = a.W + (size_t)(wvalid[t] ? rows[t] + r : 0) * K + 8 * g;
    }
    const bool xvalid = r < a.B;
    const f16* xp = a.X + (size_t)(xvalid ? r : 0) * K + 8 * g;

    f32x4 acc[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t] = f32x4{};

    const int nch = K / 128;
    f16x8 wa[RT][4], xa[4], wb[RT][4], xb[4];
    auto load = [&](int c, f16x8 (&wr)[RT][4], f16x8 (&xr)[4]) {
        const size_t off = (size_t)c * 128;
#pragma unroll
        for (int t = 0; t < RT; ++t)
#pragma unroll
            for (int u = 0; u < 4; ++u)
                wr[t][u] = wvalid[t] ? *(const f16x8*)(wp[t] + off + 32 * u) : z;
#pragma unroll
        for (int u = 0; u < 4; ++u) xr[u] = xvalid ? *(const f16x8*)(xp + off + 32 * u) : z;
    };
    auto mac = [&](const f16x8 (&wr)[RT][4], const f16x8 (&xr)[4]) {
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int t = 0; t < RT; ++t) acc[t] = mfma16(wr[t][u], xr[u], acc[t]);
    };
    int c = w;
    if (c < nch) load(c, wa, xa);
    while (c < nch) {
        const int c2 = c + 4;
        if (c2 < nch) load(c2, wb, xb);
        mac(wa, xa);
        if (c2 >= nch) break;
        const int c3 = c2 + 4;
        if (c3 < nch) load(c3, wa, xa);
        mac(wb, xb);
        c = c3;
    }
#pragma unroll
    for (int t = 0; t < RT; ++t) sred[w][t][lane] = acc[t];
    __syncthreads();
    if (w != 0) return;
#pragma unroll
    for (int t = 0; t < RT; ++t)
        acc[t] = (sred[0][t][lane] + sred[1][t][lane]) + (sred[2][t][lane] + sred[3][t][lane]);
    if (!xvalid) return;
    const int tok = r;
    // lane holds rows rows[t] + 4g + (0..3) for token `tok`
    if constexpr (EPI == GV_SWIGLU) {
        const int jb = blockIdx.x >> 1, u = blockIdx.x & 1;
        const int f = 32 * jb + 16 * u + 4 * g;
        f16x4 gv;
#pragma unroll
        for (int i = 0; i < 4; ++i) gv[i] = (f16)(silu_f(acc[0][i]) * acc[1][i]);
        *(f16x4*)(a.out_f16 + (size_t)tok * a.ldo + f) = gv;
    } else {
        const int n = rows[0] + 4 * g;
        if (n >= N) return;
        float v0 = acc[0][0], v1 = acc[0][1], v2 = acc[0][2], v3 = acc[0][3];
        if constexpr (EPI == GV_F32) {
            if (a.softcap > 0.f) {
                const float cc = a.softcap, ic = 1.0f / cc;
                v0 = tanhf(v0 * ic) * cc; v1 = tanhf(v1 * ic) * cc;
                v2 = tanhf(v2 * ic) * cc; v3 = tanhf(v3 * ic) * cc;
            }
            *(f32x4*)(a.out_f32 + (size_t)tok * a.ldo + n) = f32x4{v0, v1, v2, v3};
        } else if constexpr (EPI == GV_RESID) {
            f32x4* px = (f32x4*)(a.out_f32 + (size_t)tok * a.ldo + n);
            f32x4 x = *px;
            x[0] = v0 * a.alpha + x[0]; x[1] = v1 * a.alpha + x[1];
            x[2] = v2 * a.alpha + x[2]; x[3] = v3 * a.alpha + x[3];
            *px = x;
        } else {  // GV_QKV
            const int pos = *a.pos;
            const int sec = n / a.D, cc = n - sec * a.D;
            const int h = cc / a.hd, d = cc - h * a.hd;
            if (sec < 2) {
                const float2 cs0 = a.rope[(size_t)pos * (a.hd / 2) + d / 2];
                const float2 cs1 = a.rope[(size_t)pos * (a.hd / 2) + d / 2 + 1];
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

}  // namespace

hipError_t launch_gemv(int epi, const GemvArgs& a, hipStream_t st) {
    if (a.K % 128 != 0 || a.B < 1 || a.B > 16 || a.N % 4 != 0) return hipErrorInvalidValue;
    const int nblk = (a.N + 15) / 16;
    switch (epi) {
        case GV_F32: hipLaunchKernelGGL((gemv_kernel<GV_F32, 1>), dim3(nblk), dim3(256), 0, st, a); break;
        case GV_RESID: hipLaunchKernelGGL((gemv_kernel<GV_RESID, 1>), dim3(nblk), dim3(256), 0, st, a); break;
        case GV_QKV: hipLaunchKernelGGL((gemv_kernel<GV_QKV, 1>), dim3(nblk), dim3(256), 0, st, a); break;
        case GV_SWIGLU:
            if (a.N % 64 != 0) return hipErrorInvalidValue;
            hipLaunchKernelGGL((gemv_kernel<GV_SWIGLU, 2>), dim3(a.N / 32), dim3(256), 0, st, a);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace rh
