// rh_gemm.hip -- prefill GEMMs on fp16 MFMA (gfx950) with fused epilogues.
//
// One kernel shape serves every projection of the forward token loop
// (kernels/sdpa_fwd.rs:115-117 QKV, dyn_matmul.rs:15-75 Wo, ffn_fused.rs:80-160
// W1/W3/W2, full_model.rs:555-567 tied logits):
//     Y[m][n] = sum_k X[m][k] * W[n][k]
// X is the token-major fp16 activation [M, K]; W is the weight repacked at
// upload to [N, K] ("out x in"), so both operands stream along k.  The MFMA
// computes the transposed tile (A = weight rows, B = token rows): each lane's
// accumulator then holds 4 consecutive output features of one token, which
// makes the RoPE pairs (2i, 2i+1) and 16-byte fp32 stores lane-local.
//
// Block tile 128 (features) x BM (tokens) x 64 (k), 4 waves in 2 x 2, each
// wave 64 x BM/2 as 32x32x16 MFMA tiles.  Global -> register prefetch of the
// next k-slab overlaps the MFMAs of the current one; LDS is double-buffered
// with rows padded by 16 bytes so the 16-byte fragment reads are
// bank-conflict free.  Tiles are remapped so the BM-slices that share a
// weight panel run on the same XCD (one L2).
#include "rh_device.h"
#include "rh_kernels.h"

namespace rh {
namespace {

constexpr int BN = 128, BK = 64, LDK = BK + 8;

template <int BM, int EPI>
__global__ __launch_bounds__(256) void gemm_nt_kernel(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) f16 sW[2][BN * LDK];
    __shared__ __attribute__((aligned(16))) f16 sX[2][BM * LDK];
    constexpr int WCH = BN * BK / 8 / 256;  // 16-byte chunks per thread, weight slab
    constexpr int XCH = BM * BK / 8 / 256;  // 16-byte chunks per thread, token slab
    constexpr int MT = BM / 64;             // 32-token MFMA tiles per wave

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wn = wv & 1, wm = wv >> 1;
    const int N = a.N, M = a.M, K = a.K;
    const int nbN = (N + BN - 1) / BN, nbM = (M + BM - 1) / BM;
    const int logical = xcd_remap(blockIdx.x, nbN * nbM);
    const int nb = logical / nbM, mb = logical - nb * nbM;
    const int n0 = nb * BN, m0 = mb * BM;

    f16x8 rw[WCH], rx[XCH];
    const f16x8 zero8 = {};
    auto gload = [&](int k0) {
#pragma unroll
        for (int p = 0; p < WCH; ++p) {
            const int c = tid + 256 * p, row = c >> 3, col = (c & 7) * 8;
            const int n = n0 + row;
            rw[p] = n < N ? *(const f16x8*)(a.W + (size_t)n * K + k0 + col) : zero8;
        }
#pragma unroll
        for (int p = 0; p < XCH; ++p) {
            const int c = tid + 256 * p, row = c >> 3, col = (c & 7) * 8;
            const int m = m0 + row;
            rx[p] = m < M ? *(const f16x8*)(a.X + (size_t)m * K + k0 + col) : zero8;
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int p = 0; p < WCH; ++p) {
            const int c = tid + 256 * p, row = c >> 3, col = (c & 7) * 8;
            *(f16x8*)&sW[buf][row * LDK + col] = rw[p];
        }
#pragma unroll
        for (int p = 0; p < XCH; ++p) {
            const int c = tid + 256 * p, row = c >> 3, col = (c & 7) * 8;
            *(f16x8*)&sX[buf][row * LDK + col] = rx[p];
        }
    };

    f32x16 acc[2][MT];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < MT; ++j) acc[i][j] = f32x16{};

    const int KT = K / BK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < KT) gload((kt + 1) * BK);
        const f16* ws = sW[cur];
        const f16* xs = sX[cur];
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) {
            const int kc = kk * 16 + 8 * (lane >> 5);
            f16x8 af[2], bf[MT];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *(const f16x8*)&ws[(wn * 64 + i * 32 + (lane & 31)) * LDK + kc];
#pragma unroll
            for (int j = 0; j < MT; ++j)
                bf[j] = *(const f16x8*)&xs[(wm * (BM / 2) + j * 32 + (lane & 31)) * LDK + kc];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < MT; ++j) acc[i][j] = mfma32(af[i], bf[j], acc[i][j]);
        }
        if (kt + 1 < KT) sstore(cur ^ 1);
        __syncthreads();
    }

    // ---- epilogue: lane holds token m = .. + lane%32 and, per q4, the four
    // consecutive features n = .. + 8*q4 + 4*(lane/32) + (0..3).
#pragma unroll
    for (int j = 0; j < MT; ++j) {
        const int m = m0 + wm * (BM / 2) + j * 32 + (lane & 31);
        if (m >= M) continue;
        if constexpr (EPI == EPI_SWIGLU) {
            // The wave's 64 weight rows are 32 W1 rows (tile 0) followed by the
            // matching 32 W3 rows (tile 1) of feature block fb.
            const int fb = (n0 + wn * 64) >> 6;
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const int f = 32 * fb + 8 * q4 + 4 * (lane >> 5);
                f16x4 g;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float h1 = acc[0][j][4 * q4 + r], h3 = acc[1][j][4 * q4 + r];
                    g[r] = (f16)(silu_f(h1) * h3);
                }
                *(f16x4*)(a.out_f16 + (size_t)m * a.ldo + f) = g;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const int n = n0 + wn * 64 + i * 32 + 8 * q4 + 4 * (lane >> 5);
                    if (n >= N) continue;
                    float v0 = acc[i][j][4 * q4 + 0], v1 = acc[i][j][4 * q4 + 1];
                    float v2 = acc[i][j][4 * q4 + 2], v3 = acc[i][j][4 * q4 + 3];
                    if constexpr (EPI == EPI_F32) {
                        if (a.softcap > 0.f) {
                            const float c = a.softcap, ic = 1.0f / c;
                            v0 = tanhf(v0 * ic) * c; v1 = tanhf(v1 * ic) * c;
                            v2 = tanhf(v2 * ic) * c; v3 = tanhf(v3 * ic) * c;
                        }
                        *(f32x4*)(a.out_f32 + (size_t)m * a.ldo + n) = f32x4{v0, v1, v2, v3};
                    } else if constexpr (EPI == EPI_RESID) {
                        f32x4* px = (f32x4*)(a.out_f32 + (size_t)m * a.ldo + n);
                        f32x4 x = *px;
                        x[0] = v0 * a.alpha + x[0]; x[1] = v1 * a.alpha + x[1];
                        x[2] = v2 * a.alpha + x[2]; x[3] = v3 * a.alpha + x[3];
                        *px = x;
                    } else {  // EPI_QKV
                        const int sec = n / a.D, c = n - sec * a.D;
                        const int h = c / a.hd, d = c - h * a.hd;
                        const int b = m / a.S, s = m - b * a.S, pos = a.pos0 + s;
                        if (sec < 2) {
                            const float2 cs0 = a.rope[(size_t)pos * (a.hd / 2) + d / 2];
                            const float2 cs1 = a.rope[(size_t)pos * (a.hd / 2) + d / 2 + 1];
                            const float r0 = v0 * cs0.x + (-v1) * cs0.y, r1 = v1 * cs0.x + v0 * cs0.y;
                            const float r2 = v2 * cs1.x + (-v3) * cs1.y, r3 = v3 * cs1.x + v2 * cs1.y;
                            v0 = r0; v1 = r1; v2 = r2; v3 = r3;
                        }
                        f16* dst;
                        if (sec == 0)
                            dst = a.q + (((size_t)b * a.H + h) * a.S + s) * a.hd + d;
                        else
                            dst = (sec == 1 ? a.kc : a.vc) + (((size_t)b * a.H + h) * a.ctx + pos) * a.hd + d;
                        *(f16x4*)dst = f16x4{(f16)v0, (f16)v1, (f16)v2, (f16)v3};
                    }
                }
        }
    }
}

template <int EPI>
hipError_t launch_epi(const GemmArgs& a, hipStream_t st) {
    const int nbN = (a.N + BN - 1) / BN;
    const int tiles128 = nbN * ((a.M + 127) / 128);
    if (tiles128 >= 512) {
        hipLaunchKernelGGL((gemm_nt_kernel<128, EPI>), dim3(tiles128), dim3(256), 0, st, a);
    } else {
        const int tiles64 = nbN * ((a.M + 63) / 64);
        hipLaunchKernelGGL((gemm_nt_kernel<64, EPI>), dim3(tiles64), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(int epi, const GemmArgs& a, hipStream_t st) {
    if (a.K % BK != 0 || a.N % 4 != 0 || a.M <= 0) return hipErrorInvalidValue;
    switch (epi) {
        case EPI_F32: return launch_epi<EPI_F32>(a, st);
        case EPI_RESID: return launch_epi<EPI_RESID>(a, st);
        case EPI_SWIGLU:
            if (a.N % 64 != 0) return hipErrorInvalidValue;
            return launch_epi<EPI_SWIGLU>(a, st);
        case EPI_QKV: return launch_epi<EPI_QKV>(a, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace rh
