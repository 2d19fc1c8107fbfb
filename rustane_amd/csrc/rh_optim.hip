// rh_optim.hip -- the optimizer step: fused AdamW and the gradient norm.
//
// AdamW is step_fused (cpu/adam.rs:95-132; the reference's Metal shader,
// metal_adam.rs:16-40, computes the same): every element is read once (grad,
// m, v, fp32 master param) and written once (m, v, param) -- 28 bytes, an
// HBM-bound pass -- and the same pass writes the fp16 device copy the
// forward streams, in its fragment-order packing (transposed through LDS
// tiles where the packing transposes), so no second pass over the masters
// is needed.  The arithmetic follows the reference's operation order with
// FMA contraction off and IEEE division and square root, as rustc computes.
//
// The gradient norm is a per-tensor sum of squares: a fixed grid of blocks
// over fixed ranges, each reduced in a fixed tree, so the result is
// deterministic; the host adds the block partials in order.
#include <algorithm>

#include "rh_device.h"
#include "rh_kernels.h"

namespace rh {
namespace {

__device__ __forceinline__ float adam_elem(float p, float graw, float& m, float& v, const AdamArgs& a) {
#pragma clang fp contract(off)
    const float g = graw * a.gscale;
    const float mi = a.beta1 * m + a.omb1 * g;
    const float vi = a.beta2 * v + a.omb2 * g * g;
    m = mi;
    v = vi;
    const float m_hat = mi * a.bc1;
    const float v_hat = vi * a.bc2;
    const float update = m_hat / (sqrtf(v_hat) + a.eps);
    return p - a.lr * (update + a.wd * p);
}

// Elementwise over n (multiple of 4) with an optional row-packed fp16 copy
// (dst[frag_off(i / K, i % K, K)]).  grad null: zero gradients.
__global__ __launch_bounds__(256) void adam_rows_kernel(float* __restrict__ p, const float* __restrict__ g,
                                                        float* __restrict__ m, float* __restrict__ v, size_t n,
                                                        AdamArgs a, f16* __restrict__ dst, int K) {
    const size_t n4 = n / 4;
    for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < n4; t += (size_t)gridDim.x * blockDim.x) {
        const size_t i = 4 * t;
        f32x4 pv = *(const f32x4*)(p + i), mv = *(const f32x4*)(m + i), vv = *(const f32x4*)(v + i);
        const f32x4 gv = g ? *(const f32x4*)(g + i) : f32x4{};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float me = mv[e], ve = vv[e];
            pv[e] = adam_elem(pv[e], gv[e], me, ve, a);
            mv[e] = me;
            vv[e] = ve;
        }
        *(f32x4*)(p + i) = pv;
        *(f32x4*)(m + i) = mv;
        *(f32x4*)(v + i) = vv;
        if (dst) {
            const int r = (int)(i / K), k = (int)(i % K);  // K % 4 == 0: the 4 share a row
            *(f16x4*)(dst + frag_off(r, k, K)) = f16x4{(f16)pv[0], (f16)pv[1], (f16)pv[2], (f16)pv[3]};
        }
    }
}

__device__ __forceinline__ int packed_row(int c, int map, int row_off) {
    return map == 1 ? 32 * (c >> 4) + (c & 15) + row_off : c + row_off;
}

// A [R][C] tensor whose fp16 copy is transposed: element (r, c) goes to row
// packed_row(c), k = r, K = ldd.  32 x 32 tiles: the update reads and writes
// rows (coalesced), the fp16 copy is written from the LDS-transposed tile.
__global__ __launch_bounds__(256) void adam_transpose_kernel(float* __restrict__ p, const float* __restrict__ g,
                                                             float* __restrict__ m, float* __restrict__ v, int R,
                                                             int C, AdamArgs a, f16* __restrict__ dst, int ldd,
                                                             int map, int row_off) {
    __shared__ float tile[32][33];
    const int r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int y = ty; y < 32; y += 8) {
        const int r = r0 + y, c = c0 + tx;
        float np = 0.f;
        if (r < R && c < C) {
            const size_t i = (size_t)r * C + c;
            float mm = m[i], vv = v[i];
            np = adam_elem(p[i], g ? g[i] : 0.f, mm, vv, a);
            p[i] = np;
            m[i] = mm;
            v[i] = vv;
        }
        tile[y][tx] = np;
    }
    __syncthreads();
    for (int y = ty; y < 32; y += 8) {
        const int c = c0 + y, r = r0 + tx;
        if (c < C && r < R) dst[frag_off(packed_row(c, map, row_off), r, ldd)] = (f16)tile[tx][y];
    }
}

// Sum of squares of x[0..n): block b covers [b*chunk, (b+1)*chunk).
__global__ __launch_bounds__(256) void sumsq_kernel(const float* __restrict__ x, size_t n, size_t chunk,
                                                    float* __restrict__ part) {
    __shared__ float red[4];
    const size_t b0 = blockIdx.x * chunk, b1 = min(n, b0 + chunk);
    float s = 0.f;
    for (size_t i = b0 + threadIdx.x; i < b1; i += 256) s += x[i] * x[i];
    s = block_sum_256(s, red);
    if (threadIdx.x == 0) part[blockIdx.x] = s;
}

int grid_for(size_t n, int per) {
    const size_t g = (n + per - 1) / per;
    return (int)(g > 16384 ? 16384 : (g ? g : 1));
}

}  // namespace

hipError_t launch_adam_rows(float* p, const float* g, float* m, float* v, size_t n, const AdamArgs& a, f16* dst,
                            int K, hipStream_t st) {
    if (n % 4 != 0 || (dst && (K % 128 != 0 || n % K != 0))) return hipErrorInvalidValue;
    hipLaunchKernelGGL(adam_rows_kernel, dim3(grid_for(n / 4, 256)), dim3(256), 0, st, p, g, m, v, n, a, dst, K);
    return hipGetLastError();
}

hipError_t launch_adam_transpose(float* p, const float* g, float* m, float* v, int R, int C, const AdamArgs& a,
                                 f16* dst, int ldd, int map, int row_off, hipStream_t st) {
    if (!dst || ldd % 128 != 0) return hipErrorInvalidValue;
    const dim3 grid((C + 31) / 32, (R + 31) / 32);
    hipLaunchKernelGGL(adam_transpose_kernel, grid, dim3(256), 0, st, p, g, m, v, R, C, a, dst, ldd, map, row_off);
    return hipGetLastError();
}

int sumsq_blocks(size_t n) { return (int)std::min<size_t>(1024, (n + 4095) / 4096); }

hipError_t launch_sumsq(const float* x, size_t n, float* part, hipStream_t st) {
    const int nb = sumsq_blocks(n);
    const size_t chunk = (n + nb - 1) / nb;
    hipLaunchKernelGGL(sumsq_kernel, dim3(nb), dim3(256), 0, st, x, n, chunk, part);
    return hipGetLastError();
}

}  // namespace rh
