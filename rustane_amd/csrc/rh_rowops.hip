// rh_rowops.hip -- bandwidth-bound row kernels of the forward and decode paths
// and the weight packing kernels.
//
//   embed      embedding::forward (cpu/embedding.rs:8-16), fp16 table -> fp32 rows
//   rmsnorm    rmsnorm::forward_channel_first (cpu/rmsnorm.rs:149-183):
//              r = 1/sqrt(sum(x^2) * (1/D) + eps), out = (x * r) * gamma  -> fp16
//   ce         cross_entropy::forward_backward_batch (cpu/cross_entropy.rs:58-96),
//              loss only: ln(sum exp(l - max)) - (l[t] - max), one block per row
//   mean       total / S per sequence (full_model.rs:987)
//   pack/unpack  reference orientation (layer.rs:52-63) <-> device [out, in] fp16
//              in fragment order (frag_off)
#include "rh_device.h"
#include "rh_kernels.h"

namespace rh {
namespace {

// E is the fragment-ordered [V, D] table (frag_off); 8 consecutive k of a row
// are 16 contiguous bytes.
__global__ void embed_kernel(const uint32_t* tok, const f16* E, float* x, int D, int V, int* err) {
    const int row = blockIdx.x;
    uint32_t t = tok[row];
    if (t >= (uint32_t)V) {
        if (threadIdx.x == 0) atomicAdd(err, 1);
        t = 0;
    }
    float* dst = x + (size_t)row * D;
    for (int i = threadIdx.x * 8; i < D; i += blockDim.x * 8) {
        const f16x8 v = *(const f16x8*)(E + frag_off((int)t, i, D));
        *(f32x4*)(dst + i) = f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
        *(f32x4*)(dst + i + 4) = f32x4{(float)v[4], (float)v[5], (float)v[6], (float)v[7]};
    }
}

// One block per row; NIT = ceil(D / 1024) groups of 4 features per thread.
// The row and gamma are loaded once, every load issued before the first use
// (one memory round trip instead of one per group and pass); each thread
// sums its groups in ascending feature order, as the fused GEMV norm does.
template <int NIT>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* x, const float* gamma, f16* out,
                                                      int D, float eps, int stride_rows,
                                                      int offset_rows) {
    __shared__ float red[4];
    const int row = blockIdx.x;
    const float* xr = x + ((size_t)row * stride_rows + offset_rows) * D;
    f32x4 v[NIT], gm[NIT];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int i = threadIdx.x * 4 + it * 1024;
        v[it] = i < D ? *(const f32x4*)(xr + i) : f32x4{};
        gm[it] = i < D ? *(const f32x4*)(gamma + i) : f32x4{};
    }
    float ss = 0.f;
#pragma unroll
    for (int it = 0; it < NIT; ++it)
        ss += v[it][0] * v[it][0] + v[it][1] * v[it][1] + v[it][2] * v[it][2] + v[it][3] * v[it][3];
    ss = block_sum_256(ss, red);
    const float r = 1.0f / sqrtf(ss * (1.0f / (float)D) + eps);
    f16* o = out + (size_t)row * D;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int i = threadIdx.x * 4 + it * 1024;
        if (i < D)
            *(f16x4*)(o + i) = f16x4{(f16)(v[it][0] * r * gm[it][0]), (f16)(v[it][1] * r * gm[it][1]),
                                     (f16)(v[it][2] * r * gm[it][2]), (f16)(v[it][3] * r * gm[it][3])};
    }
}

// RMSNorm into fragment order: one block per row (D <= 8192).  Each thread
// owns 8 consecutive columns per 2048-column pass and loads its whole share
// of the row before the first add (one memory round trip instead of one per
// pass and per sweep), sums in the split-K row kernel's order, then writes
// 16-byte fragment-order lane slots from the registers.
__global__ __launch_bounds__(256) void rmsnorm_frag_kernel(const float* x, const float* gamma, f16* out,
                                                           int D, float eps) {
    __shared__ float red[4];
    const int row = blockIdx.x;
    const float* xr = x + (size_t)row * D;
    f32x4 v[4][2];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int i = threadIdx.x * 8 + it * 2048;
        if (i < D) {
            v[it][0] = *(const f32x4*)(xr + i);
            v[it][1] = *(const f32x4*)(xr + i + 4);
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int i = threadIdx.x * 8 + it * 2048;
        if (i < D) {
#pragma unroll
            for (int e = 0; e < 4; ++e) ss += v[it][0][e] * v[it][0][e] + v[it][1][e] * v[it][1][e];
        }
    }
    ss = block_sum_256(ss, red);
    const float r = 1.0f / sqrtf(ss * (1.0f / (float)D) + eps);
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int i = threadIdx.x * 8 + it * 2048;
        if (i < D) {
            const f32x4 g0 = *(const f32x4*)(gamma + i), g1 = *(const f32x4*)(gamma + i + 4);
            f16x8 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                o[e] = (f16)(v[it][0][e] * r * g0[e]);
                o[e + 4] = (f16)(v[it][1][e] * r * g1[e]);
            }
            *(f16x8*)(out + frag_off(row, i, D)) = o;
        }
    }
}

// RMSNorm into fragment order for many rows: 8 rows per block (8 waves,
// wave w owns row r0 + w) so the block writes whole 128-byte lines of every
// fragment (8 rows x 16 bytes per k group) instead of one row's scattered
// 16-byte lane slots.  Pass 1: each wave loads its row once into registers
// (lane l owns columns 8l + 512p, every load issued before the first add),
// sums the squares, and writes the normalised fp16 row into LDS.  Pass 2:
// the block's half of the 16-row fragment block -- lane l of a wave covers
// fragment 2i + l/32, k group (l/8) % 4, row l % 8 -- from LDS.  (One row
// per block: 83.6 us for 8192 x 4096 at 7B batch 16, about 2.4 TB/s; reading
// the row twice from memory: 50 us.)
__global__ __launch_bounds__(512) void rmsnorm_frag8_kernel(const float* x, const float* gamma, f16* out, int M,
                                                            int D, float eps) {
    extern __shared__ __attribute__((aligned(16))) f16 srow[];  // [8][D]
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r0 = blockIdx.x * 8, row = r0 + w;
    if (row < M) {
        const float* xr = x + (size_t)row * D;
        f32x4 v[16][2];  // D <= 8192: 16 passes of 512 columns
#pragma unroll
        for (int p = 0; p < 16; ++p) {
            const int i = 8 * lane + 512 * p;
            if (i < D) {
                v[p][0] = *(const f32x4*)(xr + i);
                v[p][1] = *(const f32x4*)(xr + i + 4);
            }
        }
        float ss = 0.f;
#pragma unroll
        for (int p = 0; p < 16; ++p) {
            if (8 * lane + 512 * p < D) {
#pragma unroll
                for (int e = 0; e < 4; ++e) ss += v[p][0][e] * v[p][0][e] + v[p][1][e] * v[p][1][e];
            }
        }
        ss = wave_sum(ss);
        const float rs = 1.0f / sqrtf(ss * (1.0f / (float)D) + eps);
#pragma unroll
        for (int p = 0; p < 16; ++p) {
            const int i = 8 * lane + 512 * p;
            if (i < D) {
                const f32x4 g0 = *(const f32x4*)(gamma + i), g1 = *(const f32x4*)(gamma + i + 4);
                f16x8 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    o[e] = (f16)(v[p][0][e] * rs * g0[e]);
                    o[e + 4] = (f16)(v[p][1][e] * rs * g1[e]);
                }
                *(f16x8*)&srow[(size_t)w * D + i] = o;
            }
        }
    }
    __syncthreads();
    const int r = lane & 7, kq = (lane >> 3) & 3, half = lane >> 5;
    const int m = r0 + r;
    if (m >= M) return;
    const int nf = D / 32;
    for (int j = 2 * w + half; j < nf; j += 16) {
        const int k = 32 * j + 8 * kq;
        *(f16x8*)(out + frag_off(m, k, D)) = *(const f16x8*)&srow[(size_t)r * D + k];
    }
}

// Split-K reduction + residual + RMSNorm (x = xin + alpha * sum, xin may be
// x itself): one block per row; each thread
// owns 8 consecutive columns per 2048-column pass (up to 4 passes), keeps the
// updated values in registers between the sum of squares and the normalised
// 16-byte fragment-order writes.  S (the split count) is a template argument
// so every partial load of a pass is issued before the first add; partials
// are summed in split order.  (Nontemporal loads of the partials, which the
// split GEMM has just written, measured slower: 11.9 -> 14.2 us for W2.)
template <int S>
__global__ __launch_bounds__(256) void resid_norm_kernel(const float* xin, float* x, const float* part,
                                                         size_t split_stride,
                                                         float alpha, const float* gamma, float eps, f16* out,
                                                         int D) {
    __shared__ float red[4];
    const int row = blockIdx.x;
    float* xr = x + (size_t)row * D;
    const float* xir = xin + (size_t)row * D;
    const float* pr = part + (size_t)row * D;
    f32x4 v[4][2];
    float ss = 0.f;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int i = threadIdx.x * 8 + it * 2048;
        if (i < D) {
            f32x4 p0[S > 0 ? S : 1], p1[S > 0 ? S : 1];
#pragma unroll
            for (int sp = 0; sp < S; ++sp) {
                p0[sp] = *(const f32x4*)(pr + sp * split_stride + i);
                p1[sp] = *(const f32x4*)(pr + sp * split_stride + i + 4);
            }
            f32x4 x0 = *(const f32x4*)(xir + i), x1 = *(const f32x4*)(xir + i + 4);
            f32x4 a0 = {}, a1 = {};
#pragma unroll
            for (int sp = 0; sp < S; ++sp) {
                a0 += p0[sp];
                a1 += p1[sp];
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x0[e] = a0[e] * alpha + x0[e];
                x1[e] = a1[e] * alpha + x1[e];
                ss += x0[e] * x0[e] + x1[e] * x1[e];
            }
            *(f32x4*)(xr + i) = x0;
            *(f32x4*)(xr + i + 4) = x1;
            v[it][0] = x0;
            v[it][1] = x1;
        }
    }
    if (!gamma) return;  // uniform per launch
    ss = block_sum_256(ss, red);
    const float r = 1.0f / sqrtf(ss * (1.0f / (float)D) + eps);
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int i = threadIdx.x * 8 + it * 2048;
        if (i < D) {
            const f32x4 g0 = *(const f32x4*)(gamma + i), g1 = *(const f32x4*)(gamma + i + 4);
            f16x8 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                o[e] = (f16)(v[it][0][e] * r * g0[e]);
                o[e + 4] = (f16)(v[it][1][e] * r * g1[e]);
            }
            *(f16x8*)(out + frag_off(row, i, D)) = o;
        }
    }
}

__global__ __launch_bounds__(256) void ce_kernel(const float* logits, const uint32_t* targets,
                                                 float* loss, int V, int* err) {
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
    // combine (m, s) across the wave, then across the 4 waves
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float om = __shfl_xor(m, o, RH_WAVE), os = __shfl_xor(s, o, RH_WAVE);
        const float nm = fmaxf(m, om);
        s = (m == -INFINITY ? 0.f : s * __expf(m - nm)) + (om == -INFINITY ? 0.f : os * __expf(om - nm));
        m = nm;
    }
    if ((tid & 63) == 0) { sm[tid >> 6] = m; ss[tid >> 6] = s; }
    __syncthreads();
    if (tid == 0) {
        float M = fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3]));
        float S = 0.f;
        for (int w = 0; w < 4; ++w) S += ss[w] * __expf(sm[w] - M);
        uint32_t t = targets[row];
        if (t >= (uint32_t)V) { atomicAdd(err, 1); t = 0; }
        loss[row] = logf(S) - (l[t] - M);
    }
}

__global__ __launch_bounds__(256) void mean_kernel(const float* loss, float* mean, int S) {
    __shared__ float red[4];
    const int b = blockIdx.x;
    float s = 0.f;
    for (int i = threadIdx.x; i < S; i += 256) s += loss[(size_t)b * S + i];
    s = block_sum_256(s, red);
    if (threadIdx.x == 0) mean[b] = s / (float)S;
}

__global__ void set_state_kernel(int* state, int pos, int step) {
    if (threadIdx.x == 0) { state[0] = pos; state[1] = step; }
}
__global__ void fill_kernel(float* p, float v, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = v;
}

__device__ __forceinline__ int dst_row(int c, int map, int row_off) {
    return map == 1 ? 32 * (c >> 4) + (c & 15) + row_off : c + row_off;
}

// 32x32 tiles through LDS: src [R][C] (in x out) -> dst row dst_row(c), k = r,
// in fragment order with K = ldd.
__global__ void pack_transpose_kernel(const float* src, f16* dst, int R, int C, int ldd, int map,
                                      int row_off) {
    __shared__ float tile[32][33];
    const int r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 256 threads: 8 rows per pass
    for (int y = ty; y < 32; y += 8) {
        const int r = r0 + y, c = c0 + tx;
        tile[y][tx] = (r < R && c < C) ? src[(size_t)r * C + c] : 0.f;
    }
    __syncthreads();
    for (int y = ty; y < 32; y += 8) {
        const int c = c0 + y, r = r0 + tx;
        if (c < C && r < R) dst[frag_off(dst_row(c, map, row_off), r, ldd)] = (f16)tile[tx][y];
    }
}

__global__ void unpack_transpose_kernel(const f16* src, float* dst, int R, int C, int lds, int map,
                                        int row_off) {
    __shared__ float tile[32][33];
    const int r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int y = ty; y < 32; y += 8) {
        const int c = c0 + y, r = r0 + tx;
        tile[y][tx] = (c < C && r < R) ? (float)src[frag_off(dst_row(c, map, row_off), r, lds)] : 0.f;
    }
    __syncthreads();
    for (int y = ty; y < 32; y += 8) {
        const int r = r0 + y, c = c0 + tx;
        if (r < R && c < C) dst[(size_t)r * C + c] = tile[tx][y];
    }
}

// [R][K] fp32 rows (out x in) <-> fragment-ordered fp16.
__global__ void pack_rows_kernel(const float* s, f16* d, int R, int K) {
    const size_t n = (size_t)R * K;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        d[frag_off((int)(i / K), (int)(i % K), K)] = (f16)s[i];
}
__global__ void unpack_rows_kernel(const f16* s, float* d, int R, int K) {
    const size_t n = (size_t)R * K;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        d[i] = (float)s[frag_off((int)(i / K), (int)(i % K), K)];
}

__global__ void convert_f32_f16_kernel(const float* s, f16* d, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        d[i] = (f16)s[i];
}
__global__ void convert_f16_f32_kernel(const f16* s, float* d, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        d[i] = (float)s[i];
}

// Philox4x32-10 (Salmon et al., SC'11) with the published round constants.
__device__ __forceinline__ void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
    const uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint32_t hi0 = __umulhi(M0, c[0]), lo0 = M0 * c[0];
        const uint32_t hi1 = __umulhi(M1, c[2]), lo1 = M1 * c[2];
        const uint32_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
        c[0] = n0; c[1] = lo1; c[2] = n2; c[3] = lo0;
        k0 += W0; k1 += W1;
    }
}

// Element i of tensor `tid`: counter (i/4 pairs..) -> Box-Muller normals.
__global__ void init_normal_kernel(float* dst, size_t n, uint32_t seed_lo, uint32_t seed_hi,
                                   uint32_t tensor_id, float std) {
    const size_t npair = (n + 1) / 2;
    for (size_t p = blockIdx.x * (size_t)blockDim.x + threadIdx.x; p < npair;
         p += (size_t)gridDim.x * blockDim.x) {
        uint32_t c[4] = {(uint32_t)p, (uint32_t)(p >> 32), tensor_id, 0x52485354u};
        philox4x32_10(c, seed_lo, seed_hi);
        const float u1 = ((float)(c[0] >> 8) + 1.0f) * (1.0f / 16777216.0f);  // (0, 1]
        const float u2 = (float)(c[1] >> 8) * (1.0f / 16777216.0f);           // [0, 1)
        const float rad = sqrtf(-2.0f * logf(u1));
        const float th = 6.283185307179586f * u2;
        const size_t i = 2 * p;
        dst[i] = std * rad * cosf(th);
        if (i + 1 < n) dst[i + 1] = std * rad * sinf(th);
    }
}

inline int grid_for(size_t n, int per_block) {
    size_t g = (n + per_block - 1) / per_block;
    if (g > 65536) g = 65536;
    if (g < 1) g = 1;
    return (int)g;
}

}  // namespace

hipError_t launch_embed(const uint32_t* tok, const f16* E, float* x, int rows, int D, int V,
                        int* err, hipStream_t st) {
    hipLaunchKernelGGL(embed_kernel, dim3(rows), dim3(256), 0, st, tok, E, x, D, V, err);
    return hipGetLastError();
}
hipError_t launch_rmsnorm_strided(const float* x, const float* gamma, f16* out, int rows, int D,
                                  float eps, int stride_rows, int offset_rows, hipStream_t st) {
    if (D % 4 != 0 || D > 8192) return hipErrorInvalidValue;
#define RH_RMS(N_)                                                                                          \
    case N_:                                                                                                \
        hipLaunchKernelGGL(rmsnorm_kernel<N_>, dim3(rows), dim3(256), 0, st, x, gamma, out, D, eps, stride_rows, \
                           offset_rows);                                                                    \
        break
    switch ((D + 1023) / 1024) {
        RH_RMS(1); RH_RMS(2); RH_RMS(3); RH_RMS(4); RH_RMS(5); RH_RMS(6); RH_RMS(7); RH_RMS(8);
        default: return hipErrorInvalidValue;
    }
#undef RH_RMS
    return hipGetLastError();
}
hipError_t launch_rmsnorm(const float* x, const float* gamma, f16* out, int rows, int D, float eps,
                          hipStream_t st, bool frag) {
    if (frag) {
        if (D % 128 != 0 || D > 8192) return hipErrorInvalidValue;  // whole fragments; 4 passes of 8 columns
        if (rows >= 2048) {  // enough 8-row blocks to fill the chip
            hipLaunchKernelGGL(rmsnorm_frag8_kernel, dim3((rows + 7) / 8), dim3(512), (size_t)8 * D * sizeof(f16),
                               st, x, gamma, out, rows, D, eps);
            return hipGetLastError();
        }
        hipLaunchKernelGGL(rmsnorm_frag_kernel, dim3(rows), dim3(256), 0, st, x, gamma, out, D, eps);
        return hipGetLastError();
    }
    return launch_rmsnorm_strided(x, gamma, out, rows, D, eps, 1, 0, st);
}
hipError_t launch_resid_norm(const float* xin, float* x, const float* part, int S, size_t split_stride,
                             float alpha, const float* gamma, float eps, f16* out, int rows, int D,
                             hipStream_t st) {
    if (D % 8 != 0 || D > 8192 || S < 0 || S > 8 || (S > 0 && !part)) return hipErrorInvalidValue;
#define RH_RN(S_)                                                                                          \
    case S_:                                                                                               \
        hipLaunchKernelGGL(resid_norm_kernel<S_>, dim3(rows), dim3(256), 0, st, xin, x, part, split_stride, alpha, \
                           gamma, eps, out, D);                                                            \
        break
    switch (S) {
        RH_RN(0); RH_RN(1); RH_RN(2); RH_RN(3); RH_RN(4); RH_RN(5); RH_RN(6); RH_RN(7); RH_RN(8);
    }
#undef RH_RN
    return hipGetLastError();
}
hipError_t launch_cross_entropy(const float* logits, const uint32_t* targets, float* loss, int rows,
                                int V, int* err, hipStream_t st) {
    hipLaunchKernelGGL(ce_kernel, dim3(rows), dim3(256), 0, st, logits, targets, loss, V, err);
    return hipGetLastError();
}
hipError_t launch_mean_rows(const float* loss, float* mean, int B, int S, hipStream_t st) {
    hipLaunchKernelGGL(mean_kernel, dim3(B), dim3(256), 0, st, loss, mean, S);
    return hipGetLastError();
}
hipError_t launch_set_state(int* state, int pos, int step, hipStream_t st) {
    hipLaunchKernelGGL(set_state_kernel, dim3(1), dim3(64), 0, st, state, pos, step);
    return hipGetLastError();
}
hipError_t launch_fill_f32(float* p, float v, size_t n, hipStream_t st) {
    hipLaunchKernelGGL(fill_kernel, dim3(grid_for(n, 256)), dim3(256), 0, st, p, v, n);
    return hipGetLastError();
}
hipError_t launch_pack_transpose(const float* src, f16* dst, int R, int C, int ldd, int map,
                                 int row_off, hipStream_t st) {
    const dim3 grid((C + 31) / 32, (R + 31) / 32);
    hipLaunchKernelGGL(pack_transpose_kernel, grid, dim3(256), 0, st, src, dst, R, C, ldd, map, row_off);
    return hipGetLastError();
}
hipError_t launch_unpack_transpose(const f16* src, float* dst, int R, int C, int lds, int map,
                                   int row_off, hipStream_t st) {
    const dim3 grid((C + 31) / 32, (R + 31) / 32);
    hipLaunchKernelGGL(unpack_transpose_kernel, grid, dim3(256), 0, st, src, dst, R, C, lds, map, row_off);
    return hipGetLastError();
}
hipError_t launch_pack_rows(const float* src, f16* dst, int R, int K, hipStream_t st) {
    hipLaunchKernelGGL(pack_rows_kernel, dim3(grid_for((size_t)R * K, 256)), dim3(256), 0, st, src, dst, R, K);
    return hipGetLastError();
}
hipError_t launch_unpack_rows(const f16* src, float* dst, int R, int K, hipStream_t st) {
    hipLaunchKernelGGL(unpack_rows_kernel, dim3(grid_for((size_t)R * K, 256)), dim3(256), 0, st, src, dst, R, K);
    return hipGetLastError();
}
hipError_t launch_convert_f32_f16(const float* src, f16* dst, size_t n, hipStream_t st) {
    hipLaunchKernelGGL(convert_f32_f16_kernel, dim3(grid_for(n, 256)), dim3(256), 0, st, src, dst, n);
    return hipGetLastError();
}
hipError_t launch_convert_f16_f32(const f16* src, float* dst, size_t n, hipStream_t st) {
    hipLaunchKernelGGL(convert_f16_f32_kernel, dim3(grid_for(n, 256)), dim3(256), 0, st, src, dst, n);
    return hipGetLastError();
}
hipError_t launch_init_normal(float* dst, size_t n, uint64_t seed, uint32_t tensor_id, float std,
                              hipStream_t st) {
    hipLaunchKernelGGL(init_normal_kernel, dim3(grid_for((n + 1) / 2, 256)), dim3(256), 0, st, dst, n,
                       (uint32_t)seed, (uint32_t)(seed >> 32), tensor_id, std);
    return hipGetLastError();
}

}  // namespace rh
