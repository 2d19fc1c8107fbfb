// rh_trainops.hip -- row and elementwise kernels of the backward pass.
//
// Gradient units.  Backward activations that feed a GEMM are fp16, and a
// sequence's true gradients are O(1/S) small (the CE gradient carries 1/S,
// full_model.rs:325), below fp16's normal range for typical weights.  So the
// backward runs in internal units: the CE gradient is stored as
// (softmax - onehot) * GRAD_UNIT, and every quantity downstream is the true
// one divided by kappa = loss_scale / (S * GRAD_UNIT).  Weight gradients are
// scaled back by kappa where they are accumulated (GEMM epilogue alpha, the
// gamma reductions, the embedding scatter), in fp32.
#include <algorithm>

#include "rh_device.h"
#include "rh_kernels.h"

namespace rh {
namespace {

// Softmax cross-entropy gradient of one logits row (cross_entropy.rs:58-96
// without the 1/S, which kappa carries): dl = (softmax - onehot) * unit, times
// 1 - (z/c)^2 when the logits z were softcapped (full_model.rs:608-615), fp16
// in fragment order [rows][ldd], zero in columns V..ldd-1.
__global__ __launch_bounds__(256) void ce_backward_kernel(const float* __restrict__ logits,
                                                          const uint32_t* __restrict__ targets,
                                                          f16* __restrict__ dl, int V, int ldd, float softcap,
                                                          float unit) {
    __shared__ float sm[4], ss[4];
    const int row = blockIdx.x, tid = threadIdx.x;
    const float* l = logits + (size_t)row * V;
    float m = -INFINITY, s = 0.f;
    for (int i = tid * 4; i < V; i += 1024) {
        const f32x4 v = *(const f32x4*)(l + i);
        const float vm = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
        if (vm > m) { s *= __expf(m - vm); m = vm; }
        s += __expf(v[0] - m) + __expf(v[1] - m) + __expf(v[2] - m) + __expf(v[3] - m);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float om = __shfl_xor(m, o, RH_WAVE), os = __shfl_xor(s, o, RH_WAVE);
        const float nm = fmaxf(m, om);
        s = (m == -INFINITY ? 0.f : s * __expf(m - nm)) + (om == -INFINITY ? 0.f : os * __expf(om - nm));
        m = nm;
    }
    if ((tid & 63) == 0) { sm[tid >> 6] = m; ss[tid >> 6] = s; }
    __syncthreads();
    const float M = fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3]));
    float S = 0.f;
    for (int w = 0; w < 4; ++w) S += ss[w] * __expf(sm[w] - M);
    const float inv = unit / S;
    const uint32_t t = targets[row];
    const float ic = softcap > 0.f ? 1.0f / softcap : 0.f;
    for (int i = tid * 8; i < ldd; i += 2048) {
        f16x8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int v = i + e;
            float d = 0.f;
            if (v < V) {
                const float z = l[v];
                d = __expf(z - M) * inv - (v == (int)t ? unit : 0.f);
                if (softcap > 0.f) {
                    const float tz = z * ic;
                    d *= 1.0f - tz * tz;
                }
            }
            o[e] = (f16)d;
        }
        *(f16x8*)(dl + frag_off(row, i, ldd)) = o;
    }
}

// Fragment-order transpose: dst [C][Rp] (fragment order, K = Rp) from src
// [R][C] (fragment order, K = C): dst(c, r) = src(src_row(r), c) for r < R,
// 0 for R <= r < Rp.  map 1 reads the W1|W3 16-row interleave of the SwiGLU
// weight as [W1 rows | W3 rows] (R = 2F).  64 x 64 tiles through LDS.
__device__ __forceinline__ int src_row(int r, int map, int R) {
    if (map == 1) {
        const int F = R / 2, w3 = r >= F, f = w3 ? r - F : r;
        return 32 * (f >> 4) + 16 * w3 + (f & 15);
    }
    return r;
}

// One transpose job; a launch runs one or two (blockIdx.z), so the backward's
// paired operand transposes take one launch instead of two.
struct TransposeJob {
    const f16* src;
    f16* dst;
    int R, C, Rp, map;
};

__global__ __launch_bounds__(256) void transpose_frag_kernel(TransposeJob j0, TransposeJob j1) {
    __shared__ f16 tile[64][64 + 2];
    const TransposeJob& jb = blockIdx.z ? j1 : j0;
    const f16* __restrict__ src = jb.src;
    f16* __restrict__ dst = jb.dst;
    const int R = jb.R, C = jb.C, Rp = jb.Rp, map = jb.map;
    const int c0 = blockIdx.x * 64, r0 = blockIdx.y * 64, tid = threadIdx.x;
    if (c0 >= C || r0 >= Rp) return;  // the grid covers the larger job (whole block)
    // load: 64 rows x 8 column groups of 8
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const int u = tid + 256 * p, rr = u >> 3, cg = (u & 7) * 8;
        const int r = r0 + rr, c = c0 + cg;
        f16x8 v = {};
        if (r < R && c < C) v = *(const f16x8*)(src + frag_off(src_row(r, map, R), c, C));
#pragma unroll
        for (int e = 0; e < 8; ++e) tile[rr][cg + e] = v[e];
    }
    __syncthreads();
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const int u = tid + 256 * p, cc = u >> 3, rg = (u & 7) * 8;
        const int c = c0 + cc, r = r0 + rg;
        if (c < C && r < Rp) {
            f16x8 v;
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = tile[rg + e][cc];
            *(f16x8*)(dst + frag_off(c, r, Rp)) = v;
        }
    }
}

// rmsnorm::backward_channel_first (cpu/rmsnorm.rs:185-240) on token-major
// rows: r = 1/sqrt(sum(x^2)/D + eps) recomputed from x; x_hat = x*r;
// dot = sum(dy*g*x_hat)/D; dx = r*(dy*g - x_hat*dot) (+ dres).  Writes dx
// (fp32, may alias dres), optionally hscale*dx as fp16 in fragment order,
// and this block's dgamma partial sum(dy*x_hat) over its rows.  dy is the sum
// of S split-K partials (split_stride floats apart), added in order.
// RB = 2 rows per block, one per 256-thread half, so both rows' loads (dres
// included) are in flight at once; the halves meet only at the barriers of
// the reductions and for the dgamma partial (second row's terms via LDS).
// NIT = D / 2048 rounded up: the feature groups of 8 per thread.
constexpr int RB = 2;
template <int S, int NIT>
__global__ __launch_bounds__(512) void rms_backward_kernel(const float* __restrict__ dy, size_t split_stride,
                                                           const float* __restrict__ x,
                                                           const float* __restrict__ gamma, const float* dres,
                                                           float* dx, f16* __restrict__ outh, float hscale,
                                                           float* __restrict__ dg_part, int M, int D, float eps) {
    __shared__ float red[2][4];
    __shared__ __attribute__((aligned(16))) float dgs[NIT * 2048];
    const int half = threadIdx.x >> 8, t = threadIdx.x & 255, w = t >> 6, lane = t & 63;
    const int row = blockIdx.x * RB + half;
    const bool live = row < M;
    // sum over this half's 4 waves; every thread of the half gets it
    auto half_sum = [&](float v) {
        v = wave_sum(v);
        __syncthreads();
        if (lane == 0) red[half][w] = v;
        __syncthreads();
        return (red[half][0] + red[half][1]) + (red[half][2] + red[half][3]);
    };
    const float* xr = x + (size_t)row * D;
    const float* dr = dy + (size_t)row * D;
    f32x4 gm[NIT][2], dgp[NIT][2], xv[NIT][2], dv[NIT][2], rv[NIT][2];
    float ss = 0.f;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int i = t * 8 + it * 2048;
        dgp[it][0] = dgp[it][1] = f32x4{};
        if (live && i < D) {
            f32x4 p[S][2];
#pragma unroll
            for (int sp = 0; sp < S; ++sp)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) p[sp][hh] = *(const f32x4*)(dr + sp * split_stride + i + 4 * hh);
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                xv[it][hh] = *(const f32x4*)(xr + i + 4 * hh);
                gm[it][hh] = *(const f32x4*)(gamma + i + 4 * hh);
                rv[it][hh] = dres ? *(const f32x4*)(dres + (size_t)row * D + i + 4 * hh) : f32x4{};
                dv[it][hh] = p[0][hh];
#pragma unroll
                for (int sp = 1; sp < S; ++sp) dv[it][hh] += p[sp][hh];
#pragma unroll
                for (int e = 0; e < 4; ++e) ss += xv[it][hh][e] * xv[it][hh][e];
            }
        }
    }
    ss = half_sum(ss);
    const float r = 1.0f / sqrtf(ss * (1.0f / (float)D) + eps);
    float dot = 0.f;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int i = t * 8 + it * 2048;
        if (live && i < D) {
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float xh = xv[it][hh][e] * r;
                    dot += dv[it][hh][e] * gm[it][hh][e] * xh;
                    dgp[it][hh][e] += dv[it][hh][e] * xh;
                }
        }
    }
    dot = half_sum(dot) * (1.0f / (float)D);
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int i = t * 8 + it * 2048;
        if (live && i < D) {
            f16x8 h;
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                f32x4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float xh = xv[it][hh][e] * r;
                    o[e] = r * (dv[it][hh][e] * gm[it][hh][e] - xh * dot) + rv[it][hh][e];
                    h[4 * hh + e] = (f16)(o[e] * hscale);
                }
                *(f32x4*)(dx + (size_t)row * D + i + 4 * hh) = o;
            }
            if (outh) *(f16x8*)(outh + frag_off(row, i, D)) = h;
        }
    }
    // dgamma partial of the block: first row's terms + second row's (zero
    // when the second row is past M)
    if (half == 1) {
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int i = t * 8 + it * 2048;
            if (i < D) {
                *(f32x4*)(dgs + i) = dgp[it][0];
                *(f32x4*)(dgs + i + 4) = dgp[it][1];
            }
        }
    }
    __syncthreads();
    if (half == 0) {
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int i = t * 8 + it * 2048;
            if (i < D) {
                *(f32x4*)(dg_part + (size_t)blockIdx.x * D + i) = dgp[it][0] + *(const f32x4*)(dgs + i);
                *(f32x4*)(dg_part + (size_t)blockIdx.x * D + i + 4) = dgp[it][1] + *(const f32x4*)(dgs + i + 4);
            }
        }
    }
}

// dgamma[d] += kappa * sum of the partials (deterministic: 16 fixed strided
// partial sums per column, then a fixed pairwise tree).  16 columns per
// block, so D/16 blocks keep enough loads in flight.
__global__ __launch_bounds__(256) void dgamma_reduce_kernel(const float* __restrict__ part, int nblk, int D,
                                                            float kappa, float* __restrict__ dgamma, int store) {
    __shared__ float red[16][17];
    const int c = threadIdx.x & 15, q = threadIdx.x >> 4, d = blockIdx.x * 16 + c;
    float s = 0.f;
    if (d < D) {
        // eight loads in flight per round, added in the same (ascending) order
        int b = q;
        for (; b + 7 * 16 < nblk; b += 8 * 16) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = part[(size_t)(b + 16 * u) * D + d];
#pragma unroll
            for (int u = 0; u < 8; ++u) s += v[u];
        }
        for (; b < nblk; b += 16) s += part[(size_t)b * D + d];
    }
    red[q][c] = s;
    __syncthreads();
    for (int h = 8; h > 0; h >>= 1) {
        if (q < h) red[q][c] += red[q + h][c];
        __syncthreads();
    }
    if (q == 0 && d < D) {
        const float v = kappa * red[0][c];
        dgamma[d] = store ? v : dgamma[d] + v;
    }
}

// embedding::backward_channel_first (cpu/embedding.rs:34-44): dembed[tok] +=
// kappa * dy[pos] for the positions of each distinct token in increasing
// order (one block per distinct token; idx/start a CSR built on the host).
__global__ __launch_bounds__(256) void embed_backward_kernel(const float* __restrict__ dy,
                                                             const uint32_t* __restrict__ utok,
                                                             const int* __restrict__ start,
                                                             const int* __restrict__ idx, float kappa,
                                                             float* __restrict__ dembed, int D) {
    const int u = blockIdx.x;
    float* row = dembed + (size_t)utok[u] * D;
    const int a = start[u], b = start[u + 1];
    for (int d = threadIdx.x; d < D; d += 256) {
        float v = row[d];
        for (int j = a; j < b; ++j) v += kappa * dy[(size_t)idx[j] * D + d];
        row[d] = v;
    }
}

}  // namespace

hipError_t launch_ce_backward(const float* logits, const uint32_t* targets, f16* dl, int rows, int V, int ldd,
                              float softcap, float unit, hipStream_t st) {
    if (V % 4 != 0 || ldd % 128 != 0 || ldd < V) return hipErrorInvalidValue;
    hipLaunchKernelGGL(ce_backward_kernel, dim3(rows), dim3(256), 0, st, logits, targets, dl, V, ldd, softcap, unit);
    return hipGetLastError();
}

hipError_t launch_transpose_frag(const f16* src, f16* dst, int R, int C, int Rp, int map, hipStream_t st) {
    if (C % 128 != 0 || Rp % 128 != 0 || Rp < R || (map == 1 && R % 32 != 0)) return hipErrorInvalidValue;
    const TransposeJob j{src, dst, R, C, Rp, map};
    hipLaunchKernelGGL(transpose_frag_kernel, dim3(C / 64, Rp / 64, 1), dim3(256), 0, st, j, j);
    return hipGetLastError();
}

hipError_t launch_transpose_frag2(const f16* src0, f16* dst0, int R0, int C0, const f16* src1, f16* dst1, int R1,
                                  int C1, int Rp, hipStream_t st) {
    if (C0 % 128 != 0 || C1 % 128 != 0 || Rp % 128 != 0 || Rp < R0 || Rp < R1) return hipErrorInvalidValue;
    const TransposeJob j0{src0, dst0, R0, C0, Rp, 0}, j1{src1, dst1, R1, C1, Rp, 0};
    hipLaunchKernelGGL(transpose_frag_kernel, dim3(std::max(C0, C1) / 64, Rp / 64, 2), dim3(256), 0, st, j0, j1);
    return hipGetLastError();
}

int rms_backward_blocks(int M) { return (M + RB - 1) / RB; }

hipError_t launch_rms_backward(const float* dy, int nsplit, size_t split_stride, const float* x,
                               const float* gamma, const float* dres, float* dx, f16* outh, float hscale,
                               float* dg_part, int M, int D, float eps, hipStream_t st) {
    if (D % 8 != 0 || D > 8192 || nsplit < 1 || nsplit > 8) return hipErrorInvalidValue;
#define RH_RB(S_)                                                                                             \
    case S_:                                                                                                  \
        if (D <= 4096)                                                                                        \
            hipLaunchKernelGGL((rms_backward_kernel<S_, 2>), dim3(rms_backward_blocks(M)), dim3(512), 0, st,   \
                               dy, split_stride, x, gamma, dres, dx, outh, hscale, dg_part, M, D, eps);       \
        else                                                                                                  \
            hipLaunchKernelGGL((rms_backward_kernel<S_, 4>), dim3(rms_backward_blocks(M)), dim3(512), 0, st,   \
                               dy, split_stride, x, gamma, dres, dx, outh, hscale, dg_part, M, D, eps);       \
        break
    switch (nsplit) {
        RH_RB(1); RH_RB(2); RH_RB(3); RH_RB(4); RH_RB(5); RH_RB(6); RH_RB(7); RH_RB(8);
    }
#undef RH_RB
    return hipGetLastError();
}

hipError_t launch_dgamma_reduce(const float* part, int nblk, int D, float kappa, float* dgamma, bool store,
                                hipStream_t st) {
    hipLaunchKernelGGL(dgamma_reduce_kernel, dim3((D + 15) / 16), dim3(256), 0, st, part, nblk, D, kappa, dgamma,
                       (int)store);
    return hipGetLastError();
}

hipError_t launch_embed_backward(const float* dy, const uint32_t* utok, const int* start, const int* idx, int nuniq,
                                 float kappa, float* dembed, int D, hipStream_t st) {
    if (nuniq <= 0) return hipSuccess;
    hipLaunchKernelGGL(embed_backward_kernel, dim3(nuniq), dim3(256), 0, st, dy, utok, start, idx, kappa, dembed, D);
    return hipGetLastError();
}

}  // namespace rh
