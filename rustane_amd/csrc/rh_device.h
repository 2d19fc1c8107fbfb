// rh_device.h -- device types and helpers shared by the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define RH_WAVE 64

// 16x16x32 and 32x32x16 fp16 MFMA (gfx950).  For both, lane l holds 8
// consecutive-k elements of row (l % M) of A and of column (l % N) of B, in k
// group l / M; the output tile has column = l % N and rows
//   16x16: 4*(l/16) + v            (v = 0..3)
//   32x32: 8*(v/4) + 4*(l/32) + v%4 (v = 0..15).
__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Max / sum over the four lanes l, l ^ 16, l ^ 32, l ^ 48 of a wave (the
// lanes sharing l % 16), on gfx950's row-swap VALU ops instead of LDS-crossbar
// shuffles.  With a = b = v, v_permlane16_swap a, b leaves lane l holding
// (v[l & ~16], v[l | 16]) and v_permlane32_swap a, b (v[l & 31], v[(l & 31) +
// 32]) (checked on the device), so both lanes of a pair combine the same
// operands in the same order and all four lanes end with the same bits; the
// sum equals v + shfl_xor(v, 16), then + shfl_xor(., 32), bit for bit.  The
// swaps are written as inline assembly: the compiler's builtins for them fold
// a swap of two equal values to those values, which drops the data movement
// between rows.  The s_nop covers the VALU-write -> permlane-read hazard.
__device__ __forceinline__ void swap_rows16(float& a, float& b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap_halves32(float& a, float& b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ float xrow_max4(float v) {
    float a = v, b = v;
    swap_rows16(a, b);
    a = fmaxf(a, b);
    b = a;
    swap_halves32(a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float xrow_sum4(float v) {
    float a = v, b = v;
    swap_rows16(a, b);
    a = a + b;
    b = a;
    swap_halves32(a, b);
    return a + b;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, RH_WAVE);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, RH_WAVE));
    return v;
}

// Block-wide sum for blockDim.x == 256 (4 waves); every thread gets the result.
__device__ __forceinline__ float block_sum_256(float v, float* red /* [4] shared */) {
    v = wave_sum(v);
    const int w = threadIdx.x / RH_WAVE, l = threadIdx.x % RH_WAVE;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// Blocks are dispatched round-robin over the 8 XCDs (block b -> XCD b % 8),
// each with its own L2.  Remap so consecutive logical tiles land on the same
// XCD: tiles that share a weight panel then hit the same L2.
// Load of data streamed once per kernel (decode weights, the KV cache):
// nontemporal, so it does not displace reused lines.  A 4 GiB read sweep on
// MI355X streams 7.1 TB/s this way against 6.4 TB/s with plain loads.
template <class T>
__device__ __forceinline__ T ld_stream(const T* p) {
    return __builtin_nontemporal_load(p);
}

__device__ __forceinline__ int xcd_remap(int b, int total) {
    const int q = total / 8, r = total % 8;
    const int x = b % 8, k = b / 8;
    return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + k;
}

// Workgroup barrier ordering LDS only: the release fence waits for this
// wave's LDS accesses (lgkmcnt) but leaves global loads in flight, so
// register prefetches issued before the barrier keep overlapping it
// (__syncthreads would drain them with vmcnt(0)).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + __expf(-x)); }

// XOR swizzles of the 16-byte chunks of a 256-byte LDS row (an hd-128 fp16
// K / V / Q / dO row staged by DMA): chunk c of row k is stored at
// c ^ swz(k).  swz_k keeps the row-fragment reads of a 16x16x32 A operand
// (rows 8(r/4) + 4u + r%4, chunk 4kk + g) on distinct banks, swz_v the
// transposing reads (ds_read_b64_tr_b16) of keys 8g + 4h + r/4.
__device__ __forceinline__ int swz_k(int row) { return (row & 3) | (((row >> 3) & 3) << 2); }
__device__ __forceinline__ int swz_v(int row) { return ((row & 3) << 1) | (((row >> 3) & 1) << 3); }

// s_waitcnt vmcnt(n), other counters left at their maximum
template <int N>
__device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

typedef short s16x4 __attribute__((ext_vector_type(4)));

// Fragment order of a [N, K] fp16 weight (rows padded to a multiple of 16,
// K a multiple of 128): 16-row x 128-k chunks, each stored as four 1 KB
// fragments (k/32 % 4) of 64 lanes x 8 halves, lane = 16 * (k/8 % 4) + row % 16.
// One 16-byte-per-lane load then reads 1 KB contiguous, and the lane/k
// assignment is the 16x16x32 MFMA operand layout (k = 32u + 8g + e).
__host__ __device__ __forceinline__ size_t frag_off(int row, int k, int K) {
    const size_t chunk = (size_t)(row >> 4) * (size_t)(K >> 7) + (size_t)(k >> 7);
    return ((chunk * 4 + ((k >> 5) & 3)) * 64 + 16 * ((k >> 3) & 3) + (row & 15)) * 8 + (k & 7);
}
