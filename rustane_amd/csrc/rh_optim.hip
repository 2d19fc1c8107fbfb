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
// Every fp32 stream is touched once per step, so loads and stores are
// nontemporal (35.6 against 36.7 - 38.3 ms per 7B update), as are the
// gradient norm's loads.
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
        f32x4 pv = ld_stream((const f32x4*)(p + i)), mv = ld_stream((const f32x4*)(m + i)),
              vv = ld_stream((const f32x4*)(v + i));
        const f32x4 gv = g ? ld_stream((const f32x4*)(g + i)) : f32x4{};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float me = mv[e], ve = vv[e];
            pv[e] = adam_elem(pv[e], gv[e], me, ve, a);
            mv[e] = me;
            vv[e] = ve;
        }
        __builtin_nontemporal_store(pv, (f32x4*)(p + i));
        __builtin_nontemporal_store(mv, (f32x4*)(m + i));
        __builtin_nontemporal_store(vv, (f32x4*)(v + i));
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
// packed_row(c), k = r, K = ldd.  64 x 64 tiles: the update reads and writes
// rows with 16-byte accesses (C % 4 == 0), the fp16 copy is written from the
// LDS-transposed tile as 16-byte runs of 8 consecutive k.
__global__ __launch_bounds__(256) void adam_transpose_kernel(float* __restrict__ p, const float* __restrict__ g,
                                                             float* __restrict__ m, float* __restrict__ v, int R,
                                                             int C, AdamArgs a, f16* __restrict__ dst, int ldd,
                                                             int map, int row_off) {
    __shared__ float tile[64][65];
    const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64, tid = threadIdx.x;
    const int cq = (tid & 15) * 4, ry = tid >> 4;  // 16 column quads x 16 rows per pass
#pragma unroll
    for (int pass = 0; pass < 4; ++pass) {
        const int rr = ry + 16 * pass, r = r0 + rr, c = c0 + cq;
        f32x4 np = {};
        if (r < R && c < C) {
            const size_t i = (size_t)r * C + c;
            f32x4 pv = ld_stream((const f32x4*)(p + i)), mv = ld_stream((const f32x4*)(m + i)),
                  vv = ld_stream((const f32x4*)(v + i));
            const f32x4 gv = g ? ld_stream((const f32x4*)(g + i)) : f32x4{};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float me = mv[e], ve = vv[e];
                pv[e] = adam_elem(pv[e], gv[e], me, ve, a);
                mv[e] = me;
                vv[e] = ve;
            }
            __builtin_nontemporal_store(pv, (f32x4*)(p + i));
            __builtin_nontemporal_store(mv, (f32x4*)(m + i));
            __builtin_nontemporal_store(vv, (f32x4*)(v + i));
            np = pv;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) tile[rr][cq + e] = np[e];
    }
    __syncthreads();
    // 64 columns x 8 runs of 8 rows: two 16-byte stores per thread
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
        const int u = tid + 256 * pass, cc = u >> 3, rg = (u & 7) * 8;
        const int c = c0 + cc, r = r0 + rg;
        if (c < C && r < R) {
            f16x8 o;
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = (f16)tile[rg + e][cc];
            *(f16x8*)(dst + frag_off(packed_row(c, map, row_off), r, ldd)) = o;
        }
    }
}

// Sum of squares of x[0..n) (n % 4 == 0): block b covers 16-byte groups
// [b*chunk, (b+1)*chunk), four independent accumulators per thread.
__global__ __launch_bounds__(256) void sumsq_kernel(const float* __restrict__ x, size_t n, size_t chunk,
                                                    float* __restrict__ part) {
    __shared__ float red[4];
    const size_t n4 = n / 4, b0 = blockIdx.x * chunk, b1 = min(n4, b0 + chunk);
    f32x4 s = {};
    for (size_t i = b0 + threadIdx.x; i < b1; i += 256) {
        const f32x4 v = ld_stream((const f32x4*)(x + 4 * i));
        s += v * v;
    }
    const float t = block_sum_256((s[0] + s[1]) + (s[2] + s[3]), red);
    if (threadIdx.x == 0) part[blockIdx.x] = t;
}

// One block: the sum of part[0..n) in double (each thread a strided run,
// then a fixed tree), written to *out.
__global__ __launch_bounds__(1024) void sum_parts_kernel(const float* __restrict__ part, size_t n,
                                                         double* __restrict__ out) {
    __shared__ double red[1024];
    double s = 0.0;
    for (size_t i = threadIdx.x; i < n; i += 1024) s += (double)part[i];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = 512; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) *out = red[0];
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
    // rows in runs of 8 (R % 8) and 16-byte column quads (C % 4)
    if (!dst || ldd % 128 != 0 || R % 8 != 0 || C % 4 != 0) return hipErrorInvalidValue;
    const dim3 grid((C + 63) / 64, (R + 63) / 64);
    hipLaunchKernelGGL(adam_transpose_kernel, grid, dim3(256), 0, st, p, g, m, v, R, C, a, dst, ldd, map, row_off);
    return hipGetLastError();
}

int sumsq_blocks(size_t n) { return (int)std::min<size_t>(2048, (n + 8191) / 8192); }

hipError_t launch_sum_parts(const float* part, size_t n, double* out, hipStream_t st) {
    if (n == 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(sum_parts_kernel, dim3(1), dim3(1024), 0, st, part, n, out);
    return hipGetLastError();
}

hipError_t launch_sumsq(const float* x, size_t n, float* part, hipStream_t st) {
    if (n % 4 != 0 || n == 0) return hipErrorInvalidValue;
    const int nb = sumsq_blocks(n);
    const size_t chunk = (n / 4 + nb - 1) / nb;
    hipLaunchKernelGGL(sumsq_kernel, dim3(nb), dim3(256), 0, st, x, n, chunk, part);
    return hipGetLastError();
}

}  // namespace rh
