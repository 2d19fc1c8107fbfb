// rh_attn_bwd.hip -- causal attention backward (the training pass).
//
// Semantics of the sdpaBwd1/sdpaBwd2 graphs (kernels/sdpa_bwd.rs:44-300):
// probabilities recomputed from q_rope, k_rope (scale 1/sqrt(hd), causal
// mask), dV = P^T dO, dP = dO V^T, dS = P * (dP - D) with D[q] = sum_k
// P dP = sum_d dO[q][d] O[q][d], dQ = scale dS K, dK = scale dS^T Q.  The
// reference materialises the S x S probabilities on the ANE; here they are
// recomputed tile by tile from the forward's per-query log-sum-exp, as in a
// flash-attention backward, and nothing S x S touches HBM.
//
// Two deterministic kernels (no atomics):
//   attn_bwd_dq_kernel    a block owns 64 queries of one (sequence, head), 4
//                         waves x 16 queries, and walks the key blocks up to
//                         the diagonal: S^T = K Q^T, dP^T = V dO^T, then
//                         dQ^T += K^T dS^T.  Every lane owns one query column
//                         (the forward kernel's arrangement), so the row
//                         statistics (lse, D) are lane scalars.
//   attn_bwd_dkdv_kernel  a block owns 64 keys, 4 waves x 16 keys, and walks
//                         the query blocks from the diagonal on: S = Q K^T,
//                         dP = dO V^T, then dV^T += dO^T P and dK^T += Q^T dS.
//                         Every lane owns one key column.
// The row permutation of the first MFMA's A operand (tile row r reads row
// 32c + 8(r/4) + 4u + r%4 of a 32-row chunk) makes the output tile's lane
// group g hold rows 32c + 8g + 0..7, which is exactly the k layout of the
// second MFMA's B operand, so P and dS go from accumulators to operands
// without data movement.  Operands needed transposed (K^T, Q^T, dO^T) are
// written transposed into LDS when the tile is staged.
#include "rh_device.h"
#include "rh_kernels.h"

namespace rh {
namespace {

typedef f16 f16x2 __attribute__((ext_vector_type(2)));

// Four consecutive dims d..d+3 (d % 4 == 0) of head h of token row `row`
// (sequence position pos) of the q (sec 0), k (1) or v (2) gradient, written
// as fp16 into the fragment-order operand [M][3D] of the dX GEMM; q and k
// first get the RoPE backward (rope_backward_inplace, layer.rs:7389-7407):
// the transposed rotation of the pairs (d, d+1), (d+2, d+3).
template <int HD>
__device__ __forceinline__ void store_dqkv4(f16* __restrict__ out, const float2* __restrict__ rope, int row,
                                            int pos, int sec, int D, int h, int d, f32x4 v) {
    if (sec < 2) {
        const float2 c0 = rope[(size_t)pos * (HD / 2) + d / 2], c1 = rope[(size_t)pos * (HD / 2) + d / 2 + 1];
        const float a0 = v[0], a1 = v[1], a2 = v[2], a3 = v[3];
        v[0] = c0.x * a0 + c0.y * a1;
        v[1] = -c0.y * a0 + c0.x * a1;
        v[2] = c1.x * a2 + c1.y * a3;
        v[3] = -c1.y * a2 + c1.x * a3;
    }
    *(f16x4*)(out + frag_off(row, sec * D + h * HD + d, 3 * D)) = f16x4{(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
}

// Stages rows r0..r0+63 (clamped to S - 1) of a [S][HD] fp16 matrix into
// LDS: row-major (ld HD + 8) when rm is set, and transposed [HD][64] (ld 72)
// when tr is set, two rows per 32-bit LDS store.
template <int HD>
__device__ __forceinline__ void stage_rows(const f16* __restrict__ src, int r0, int S, f16* rm, f16* tr) {
    constexpr int LD = HD + 8, LT = 64 + 8;
    const int tid = threadIdx.x;
    if (rm) {
#pragma unroll
        for (int p = 0; p < 64 * HD / 8 / 256; ++p) {
            const int c = tid + 256 * p, row = c / (HD / 8), col = (c % (HD / 8)) * 8;
            *(f16x8*)&rm[row * LD + col] = *(const f16x8*)(src + (size_t)min(r0 + row, S - 1) * HD + col);
        }
    }
    if (tr) {
#pragma unroll
        for (int p = 0; p < 32 * (HD / 8) / 256; ++p) {
            const int u = tid + 256 * p, rp = u & 31, col = (u >> 5) * 8;
            const f16x8 a = *(const f16x8*)(src + (size_t)min(r0 + 2 * rp, S - 1) * HD + col);
            const f16x8 b = *(const f16x8*)(src + (size_t)min(r0 + 2 * rp + 1, S - 1) * HD + col);
#pragma unroll
            for (int e = 0; e < 8; ++e) *(f16x2*)&tr[(col + e) * LT + 2 * rp] = f16x2{a[e], b[e]};
        }
    }
}

template <int HD>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(const f16* __restrict__ Q, const f16* __restrict__ K,
                                                          const f16* __restrict__ V, const f16* __restrict__ dO,
                                                          const float* __restrict__ lse,
                                                          const float* __restrict__ Drow, f16* __restrict__ dqkv,
                                                          const float2* __restrict__ rope,
                                                          int H, int S, float scale_log2, float scale) {
    constexpr int KB = 64, LD = HD + 8, LT = KB + 8, NKK = HD / 32, NHT = HD / 16;
    __shared__ __attribute__((aligned(16))) f16 sK[KB * LD];
    __shared__ __attribute__((aligned(16))) f16 sV[KB * LD];
    __shared__ __attribute__((aligned(16))) f16 sKt[HD * LT];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, r = lane & 15;
    const int nqt = (S + 63) / 64;
    // 1-D grid: one (sequence, head)'s tiles are consecutive logical tiles on
    // one XCD (xcd_remap), whose L2 then serves their shared K and V
    const int t = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    const int qt = nqt - 1 - t % nqt;  // longest rows first
    const int h = (t / nqt) % H, b = t / nqt / H;
    const int q0 = qt * 64, qi = q0 + w * 16 + r, qrow = min(qi, S - 1);
    const size_t bh = (size_t)b * H + h;
    const f16* Kb = K + bh * S * HD;
    const f16* Vb = V + bh * S * HD;
    f16x8 qf[NKK], df[NKK];
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
        qf[kk] = *(const f16x8*)(Q + (bh * S + qrow) * HD + 32 * kk + 8 * g);
        df[kk] = *(const f16x8*)(dO + (bh * S + qrow) * HD + 32 * kk + 8 * g);
    }
    const float L = lse[bh * S + qrow], Dq = Drow[bh * S + qrow];
    f32x4 acc[NHT];
#pragma unroll
    for (int j = 0; j < NHT; ++j) acc[j] = f32x4{};
    const int nkb = (min(S, q0 + 64) + KB - 1) / KB;
    for (int kb = 0; kb < nkb; ++kb) {
        const int k0 = kb * KB;
        __syncthreads();
        stage_rows<HD>(Kb, k0, S, sK, sKt);
        stage_rows<HD>(Vb, k0, S, sV, nullptr);
        __syncthreads();
        // S^T and dP^T: chunk c (32 keys) x half u; lane group g then holds
        // keys k0 + 32c + 8g + 4u + i in element [c][u][i].
        f32x4 sc[2][2], dp[2][2];
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                sc[c][u] = f32x4{};
                dp[c][u] = f32x4{};
                const int krow = 32 * c + 8 * (r >> 2) + 4 * u + (r & 3);
#pragma unroll
                for (int kk = 0; kk < NKK; ++kk) {
                    sc[c][u] = mfma16(*(const f16x8*)&sK[krow * LD + 32 * kk + 8 * g], qf[kk], sc[c][u]);
                    dp[c][u] = mfma16(*(const f16x8*)&sV[krow * LD + 32 * kk + 8 * g], df[kk], dp[c][u]);
                }
            }
        const int lim = qrow - k0 - 8 * g;  // key offsets above lim are masked (or past S)
        f16x8 dsf[2];
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const bool live = 32 * c + 4 * u + i <= lim;
                    const float p = live ? __builtin_amdgcn_exp2f(__builtin_fmaf(sc[c][u][i], scale_log2, -L)) : 0.f;
                    dsf[c][4 * u + i] = (f16)(p * (dp[c][u][i] - Dq));
                }
        // dQ^T[hd][q] += K^T[hd][keys] . dS^T[keys][q]
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int j = 0; j < NHT; ++j)
                acc[j] = mfma16(*(const f16x8*)&sKt[(16 * j + r) * LT + 32 * c + 8 * g], dsf[c], acc[j]);
    }
    if (qi < S) {
#pragma unroll
        for (int j = 0; j < NHT; ++j)
            store_dqkv4<HD>(dqkv, rope, b * S + qi, qi, 0, H * HD, h, 16 * j + 4 * g, acc[j] * scale);
    }
}

template <int HD>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_kernel(const f16* __restrict__ Q, const f16* __restrict__ K,
                                                            const f16* __restrict__ V, const f16* __restrict__ dO,
                                                            const float* __restrict__ lse,
                                                            const float* __restrict__ Drow,
                                                            f16* __restrict__ dqkv, const float2* __restrict__ rope,
                                                            int H, int S,
                                                            float scale_log2, float scale) {
    constexpr int QB = 64, LD = HD + 8, LT = QB + 8, NKK = HD / 32, NHT = HD / 16;
    __shared__ __attribute__((aligned(16))) f16 sQ[QB * LD];
    __shared__ __attribute__((aligned(16))) f16 sdO[QB * LD];
    __shared__ __attribute__((aligned(16))) f16 sQt[HD * LT];
    __shared__ __attribute__((aligned(16))) f16 sdOt[HD * LT];
    __shared__ float sL[QB], sD[QB];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, r = lane & 15;
    const int nkt = (S + 63) / 64;
    const int t = xcd_remap((int)blockIdx.x, (int)gridDim.x);  // a head's tiles share an XCD's L2
    const int kt = t % nkt;  // the first key blocks see the most queries: launched first
    const int h = (t / nkt) % H, b = t / nkt / H;
    const int k0 = kt * 64, ki = k0 + w * 16 + r, krow = min(ki, S - 1);
    const size_t bh = (size_t)b * H + h;
    const f16* Qb = Q + bh * S * HD;
    const f16* dOb = dO + bh * S * HD;
    f16x8 kf[NKK], vf[NKK];
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
        kf[kk] = *(const f16x8*)(K + (bh * S + krow) * HD + 32 * kk + 8 * g);
        vf[kk] = *(const f16x8*)(V + (bh * S + krow) * HD + 32 * kk + 8 * g);
    }
    f32x4 dk[NHT], dv[NHT];
#pragma unroll
    for (int j = 0; j < NHT; ++j) dk[j] = dv[j] = f32x4{};
    const int nqb = (S + QB - 1) / QB;
    for (int qb = kt; qb < nqb; ++qb) {
        const int q0 = qb * QB;
        __syncthreads();
        stage_rows<HD>(Qb, q0, S, sQ, sQt);
        stage_rows<HD>(dOb, q0, S, sdO, sdOt);
        if (tid < QB) {
            const int q = min(q0 + tid, S - 1);
            sL[tid] = lse[bh * S + q];
            sD[tid] = Drow[bh * S + q];
        }
        __syncthreads();
        // S and dP: chunk c (32 queries) x half u; lane group g then holds
        // queries q0 + 32c + 8g + 4u + i in element [c][u][i].
        f32x4 s[2][2], dp[2][2];
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                s[c][u] = f32x4{};
                dp[c][u] = f32x4{};
                const int qr = 32 * c + 8 * (r >> 2) + 4 * u + (r & 3);
#pragma unroll
                for (int kk = 0; kk < NKK; ++kk) {
                    s[c][u] = mfma16(*(const f16x8*)&sQ[qr * LD + 32 * kk + 8 * g], kf[kk], s[c][u]);
                    dp[c][u] = mfma16(*(const f16x8*)&sdO[qr * LD + 32 * kk + 8 * g], vf[kk], dp[c][u]);
                }
            }
        f16x8 pf[2], dsf[2];
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int qo = 32 * c + 8 * g + 4 * u + i, q = q0 + qo;
                    const bool live = q >= ki && q < S;
                    const float p = live ? __builtin_amdgcn_exp2f(__builtin_fmaf(s[c][u][i], scale_log2, -sL[qo])) : 0.f;
                    pf[c][4 * u + i] = (f16)p;
                    dsf[c][4 * u + i] = (f16)(p * (dp[c][u][i] - sD[qo]));
                }
        // dV^T[hd][key] += dO^T[hd][q] . P[q][key];  dK^T += Q^T . dS
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int j = 0; j < NHT; ++j) {
                dv[j] = mfma16(*(const f16x8*)&sdOt[(16 * j + r) * LT + 32 * c + 8 * g], pf[c], dv[j]);
                dk[j] = mfma16(*(const f16x8*)&sQt[(16 * j + r) * LT + 32 * c + 8 * g], dsf[c], dk[j]);
            }
    }
    if (ki < S) {
        const int D = H * HD;
#pragma unroll
        for (int j = 0; j < NHT; ++j) {
            store_dqkv4<HD>(dqkv, rope, b * S + ki, ki, 1, D, h, 16 * j + 4 * g, dk[j] * scale);
            store_dqkv4<HD>(dqkv, rope, b * S + ki, ki, 2, D, h, 16 * j + 4 * g, dv[j]);
        }
    }
}

// hd 128: the same two kernels with their operand tiles moved global -> LDS
// by DMA (global_load_lds_dwordx4, 16 bytes per lane at LDS base + 16 lane)
// through a two-stage pipeline, so the next tile's loads are in flight while
// this one is computed and no VGPRs or LDS stores stage them.  Tiles keep
// their natural [row][hd] order (256-byte rows) with the XOR chunk swizzles
// of the forward kernel: a tile read as row fragments (an A operand with
// rows = keys or queries) is stored with swz_k, one read transposed (K^T,
// Q^T, dO^T) with swz_v and read by ds_read_b64_tr_b16, so K (dq) and Q, dO
// (dk/dv) are moved twice, once per swizzle.  The MFMA operands and their
// order are those of the kernels above, so the results are identical.
//
// Wave w moves 1 KB units w, w + 4, w + 8, w + 12 of a 64-row tile (unit i
// holds rows 4i..4i+3; lane L row 4i + L/16 and stored chunk L%16).
__device__ __forceinline__ void dma_tile(const f16* __restrict__ base, int r0, int S, f16* dst, bool tr) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int i = w + 4 * t, row = 4 * i + (lane >> 4);
        const int sw = tr ? swz_v(row) : swz_k(row);
        const f16* src = base + (size_t)min(r0 + row, S - 1) * 128 + 8 * ((lane & 15) ^ sw);
        __builtin_amdgcn_global_load_lds((const void*)src, (__attribute__((address_space(3))) void*)(dst + i * 512),
                                         16, 0, 0);
    }
}

// Row fragment of a swz_k tile: 8 hd values 32kk + 8g .. +7 of row `row`.
__device__ __forceinline__ f16x8 tile_row(const f16* t, int row, int kk, int g) {
    return *(const f16x8*)&t[row * 128 + 8 * ((4 * kk + g) ^ swz_k(row))];
}

// Transposed fragment of a swz_v tile: element e = T[32c + 8g + e][16j + r]
// (rows of the tile as the k dimension), from two transposing reads.
__device__ __forceinline__ f16x8 tile_tr(const f16* t, int c, int j, int lane) {
    const int g = (lane >> 4) & 3, r = lane & 15, ch = 2 * j + ((lane & 3) >> 1);
    f16x8 out;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        const int row = 32 * c + 8 * g + 4 * hh + (r >> 2);
        const f16* a = &t[row * 128 + 8 * (ch ^ swz_v(row)) + 4 * (lane & 1)];
        const f16x4 v = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                      (__attribute__((address_space(3))) s16x4*)a));
#pragma unroll
        for (int e = 0; e < 4; ++e) out[4 * hh + e] = v[e];
    }
    return out;
}

__global__ __launch_bounds__(256) void attn_bwd_dq_dma_kernel(const f16* __restrict__ Q, const f16* __restrict__ K,
                                                              const f16* __restrict__ V, const f16* __restrict__ dO,
                                                              const float* __restrict__ lse,
                                                              const float* __restrict__ Drow,
                                                              f16* __restrict__ dqkv, const float2* __restrict__ rope,
                                                              int H, int S, float scale_log2, float scale) {
    constexpr int HD = 128, KB = 64, NKK = HD / 32, NHT = HD / 16, TILE = KB * HD;
    // one array per stage and role, so the compiler's wait-count tracking
    // tells a stage's reads from the DMA filling the other stage
    __shared__ __attribute__((aligned(1024))) f16 sK0[TILE], sV0[TILE], sKt0[TILE], sK1[TILE], sV1[TILE],
        sKt1[TILE];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, r = lane & 15;
    const int nqt = (S + 63) / 64;
    const int t = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    const int qt = nqt - 1 - t % nqt;  // longest rows first
    const int h = (t / nqt) % H, b = t / nqt / H;
    const int q0 = qt * 64, qi = q0 + w * 16 + r, qrow = min(qi, S - 1);
    const size_t bh = (size_t)b * H + h;
    const f16* Kb = K + bh * S * HD;
    const f16* Vb = V + bh * S * HD;
    f16x8 qf[NKK], df[NKK];
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
        qf[kk] = *(const f16x8*)(Q + (bh * S + qrow) * HD + 32 * kk + 8 * g);
        df[kk] = *(const f16x8*)(dO + (bh * S + qrow) * HD + 32 * kk + 8 * g);
    }
    const float L = lse[bh * S + qrow], Dq = Drow[bh * S + qrow];
    f32x4 acc[NHT];
#pragma unroll
    for (int j = 0; j < NHT; ++j) acc[j] = f32x4{};
    const int nkb = (min(S, q0 + 64) + KB - 1) / KB;
    auto issue = [&](int kb, auto ST) {
        constexpr int st = decltype(ST)::value;
        dma_tile(Kb, kb * KB, S, st ? sK1 : sK0, false);
        dma_tile(Vb, kb * KB, S, st ? sV1 : sV0, false);
        dma_tile(Kb, kb * KB, S, st ? sKt1 : sKt0, true);
    };
    auto step = [&](int kb, auto ST) {
        constexpr int cur = decltype(ST)::value;
        const int k0 = kb * KB;
        // this wave's DMAs of tile kb have landed (nothing else is in flight);
        // the barrier publishes every wave's and retires every wave's reads of
        // tile kb - 1, whose stage the next issue refills
        wait_vm<0>();
        lds_barrier();
        if (kb + 1 < nkb) issue(kb + 1, std::integral_constant<int, 1 - cur>{});
        const f16* sK = cur ? sK1 : sK0;
        const f16* sV = cur ? sV1 : sV0;
        const f16* sKt = cur ? sKt1 : sKt0;
        f32x4 sc[2][2], dp[2][2];
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                sc[c][u] = f32x4{};
                dp[c][u] = f32x4{};
                const int krow = 32 * c + 8 * (r >> 2) + 4 * u + (r & 3);
#pragma unroll
                for (int kk = 0; kk < NKK; ++kk) {
                    sc[c][u] = mfma16(tile_row(sK, krow, kk, g), qf[kk], sc[c][u]);
                    dp[c][u] = mfma16(tile_row(sV, krow, kk, g), df[kk], dp[c][u]);
                }
            }
        const int lim = qrow - k0 - 8 * g;  // key offsets above lim are masked (or past S)
        f16x8 dsf[2];
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const bool live = 32 * c + 4 * u + i <= lim;
                    const float p = live ? __builtin_amdgcn_exp2f(__builtin_fmaf(sc[c][u][i], scale_log2, -L)) : 0.f;
                    dsf[c][4 * u + i] = (f16)(p * (dp[c][u][i] - Dq));
                }
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int j = 0; j < NHT; ++j) acc[j] = mfma16(tile_tr(sKt, c, j, lane), dsf[c], acc[j]);
    };
    issue(0, std::integral_constant<int, 0>{});
    for (int kb0 = 0; kb0 < nkb; kb0 += 2) {
        step(kb0, std::integral_constant<int, 0>{});
        if (kb0 + 1 < nkb) step(kb0 + 1, std::integral_constant<int, 1>{});
    }
    if (qi < S) {
#pragma unroll
        for (int j = 0; j < NHT; ++j)
            store_dqkv4<HD>(dqkv, rope, b * S + qi, qi, 0, H * HD, h, 16 * j + 4 * g, acc[j] * scale);
    }
}

__global__ __launch_bounds__(256) void attn_bwd_dkdv_dma_kernel(const f16* __restrict__ Q,
                                                                const f16* __restrict__ K,
                                                                const f16* __restrict__ V,
                                                                const f16* __restrict__ dO,
                                                                const float* __restrict__ lse,
                                                                const float* __restrict__ Drow,
                                                                f16* __restrict__ dqkv, const float2* __restrict__ rope,
                                                            int H, int S,
                                                                float scale_log2, float scale) {
    constexpr int HD = 128, QB = 64, NKK = HD / 32, NHT = HD / 16, TILE = QB * HD;
    __shared__ __attribute__((aligned(1024))) f16 sQ0[TILE], sO0[TILE], sQt0[TILE], sOt0[TILE], sQ1[TILE],
        sO1[TILE], sQt1[TILE], sOt1[TILE];
    __shared__ __attribute__((aligned(256))) float sL0[QB], sD0[QB], sL1[QB], sD1[QB];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, r = lane & 15;
    const int nkt = (S + 63) / 64;
    const int t = xcd_remap((int)blockIdx.x, (int)gridDim.x);  // a head's tiles share an XCD's L2
    const int kt = t % nkt;  // the first key blocks see the most queries: launched first
    const int h = (t / nkt) % H, b = t / nkt / H;
    const int k0 = kt * 64, ki = k0 + w * 16 + r, krow = min(ki, S - 1);
    const size_t bh = (size_t)b * H + h;
    const f16* Qb = Q + bh * S * HD;
    const f16* dOb = dO + bh * S * HD;
    f16x8 kf[NKK], vf[NKK];
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
        kf[kk] = *(const f16x8*)(K + (bh * S + krow) * HD + 32 * kk + 8 * g);
        vf[kk] = *(const f16x8*)(V + (bh * S + krow) * HD + 32 * kk + 8 * g);
    }
    f32x4 dk[NHT], dv[NHT];
#pragma unroll
    for (int j = 0; j < NHT; ++j) dk[j] = dv[j] = f32x4{};
    const int nqb = (S + QB - 1) / QB;
    auto issue = [&](int qb, auto ST) {
        constexpr int st = decltype(ST)::value;
        const int q0 = qb * QB;
        dma_tile(Qb, q0, S, st ? sQ1 : sQ0, false);
        dma_tile(dOb, q0, S, st ? sO1 : sO0, false);
        dma_tile(Qb, q0, S, st ? sQt1 : sQt0, true);
        dma_tile(dOb, q0, S, st ? sOt1 : sOt0, true);
        // the 64 queries' lse and D, 4 bytes per lane (every wave writes the
        // same values, so each wave's DMA count stays the same)
        const size_t qv = bh * S + min(q0 + lane, S - 1);
        __builtin_amdgcn_global_load_lds((const void*)(lse + qv), (__attribute__((address_space(3))) void*)(st ? sL1 : sL0),
                                         4, 0, 0);
        __builtin_amdgcn_global_load_lds((const void*)(Drow + qv), (__attribute__((address_space(3))) void*)(st ? sD1 : sD0),
                                         4, 0, 0);
    };
    auto step = [&](int qb, auto ST) {
        constexpr int cur = decltype(ST)::value;
        const int q0 = qb * QB;
        wait_vm<0>();
        lds_barrier();
        if (qb + 1 < nqb) issue(qb + 1, std::integral_constant<int, 1 - cur>{});
        const f16* sQ = cur ? sQ1 : sQ0;
        const f16* sO = cur ? sO1 : sO0;
        const f16* sQt = cur ? sQt1 : sQt0;
        const f16* sOt = cur ? sOt1 : sOt0;
        const float* sL = cur ? sL1 : sL0;
        const float* sD = cur ? sD1 : sD0;
        f32x4 s[2][2], dp[2][2];
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                s[c][u] = f32x4{};
                dp[c][u] = f32x4{};
                const int qr = 32 * c + 8 * (r >> 2) + 4 * u + (r & 3);
#pragma unroll
                for (int kk = 0; kk < NKK; ++kk) {
                    s[c][u] = mfma16(tile_row(sQ, qr, kk, g), kf[kk], s[c][u]);
                    dp[c][u] = mfma16(tile_row(sO, qr, kk, g), vf[kk], dp[c][u]);
                }
            }
        f16x8 pf[2], dsf[2];
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int qo = 32 * c + 8 * g + 4 * u + i, q = q0 + qo;
                    const bool live = q >= ki && q < S;
                    const float p = live ? __builtin_amdgcn_exp2f(__builtin_fmaf(s[c][u][i], scale_log2, -sL[qo])) : 0.f;
                    pf[c][4 * u + i] = (f16)p;
                    dsf[c][4 * u + i] = (f16)(p * (dp[c][u][i] - sD[qo]));
                }
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int j = 0; j < NHT; ++j) {
                dv[j] = mfma16(tile_tr(sOt, c, j, lane), pf[c], dv[j]);
                dk[j] = mfma16(tile_tr(sQt, c, j, lane), dsf[c], dk[j]);
            }
    };
    issue(kt, std::integral_constant<int, 0>{});
    for (int qb0 = kt; qb0 < nqb; qb0 += 2) {
        step(qb0, std::integral_constant<int, 0>{});
        if (qb0 + 1 < nqb) step(qb0 + 1, std::integral_constant<int, 1>{});
    }
    if (ki < S) {
        const int D = H * HD;
#pragma unroll
        for (int j = 0; j < NHT; ++j) {
            store_dqkv4<HD>(dqkv, rope, b * S + ki, ki, 1, D, h, 16 * j + 4 * g, dk[j] * scale);
            store_dqkv4<HD>(dqkv, rope, b * S + ki, ki, 2, D, h, 16 * j + 4 * g, dv[j]);
        }
    }
}

// dO [M, H*hd] fp32 (token-major GEMM output, the sum of NS split-K
// partials split_stride floats apart, added in order) -> fp16 [B][H][S][hd],
// and D[b][h][s] = sum_d dO * O with O the forward's attention output
// (fragment order, 8 features of a row contiguous).  One thread per 8
// features, HD/8 neighbouring lanes per (token, head).
template <int NS, int HD>
__global__ __launch_bounds__(256) void attn_bwd_prep_kernel(const float* __restrict__ dOf, size_t split_stride,
                                                            const f16* __restrict__ O, f16* __restrict__ dOh,
                                                            float* __restrict__ Drow, int M, int H, int S) {
    constexpr int LPI = HD / 8;
    const int D = H * HD;
    const long long e = ((long long)blockIdx.x * 256 + threadIdx.x) * 8;
    // M * D is a multiple of HD, so a (token, head) group is all in or all out
    if (e >= (long long)M * D) return;
    const int m = (int)(e / D), c = (int)(e - (long long)m * D);
    const int h = c / HD, d = c - h * HD;
    f32x4 p[NS][2];
#pragma unroll
    for (int sp = 0; sp < NS; ++sp) {
        p[sp][0] = *(const f32x4*)(dOf + sp * split_stride + e);
        p[sp][1] = *(const f32x4*)(dOf + sp * split_stride + e + 4);
    }
    const f16x8 o = *(const f16x8*)(O + frag_off(m, c, D));
    f32x4 v0 = p[0][0], v1 = p[0][1];
#pragma unroll
    for (int sp = 1; sp < NS; ++sp) {
        v0 += p[sp][0];
        v1 += p[sp][1];
    }
    float acc = 0.f;
    f16x8 hv;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        acc += v0[q] * (float)o[q];
        hv[q] = (f16)v0[q];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        acc += v1[q] * (float)o[4 + q];
        hv[4 + q] = (f16)v1[q];
    }
#pragma unroll
    for (int off = LPI / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, RH_WAVE);
    const int b = m / S, s = m - b * S;
    const size_t row = ((size_t)b * H + h) * S + s;
    *(f16x8*)(dOh + row * HD + d) = hv;
    if (d == 0) Drow[row] = acc;
}

}  // namespace

hipError_t launch_attn_backward(const f16* q, const f16* k, const f16* v, const f16* o, const float* dOf,
                                int nsplit, size_t split_stride, const float* lse, f16* dOh, float* Drow,
                                f16* dqkv, const float2* rope, int B, int H, int S, int hd, hipStream_t st) {
    if ((hd != 128 && hd != 64) || nsplit < 1 || nsplit > 8) return hipErrorInvalidValue;
    const int M = B * S;
    const unsigned pgrid = (unsigned)(((long long)M * H * hd / 8 + 255) / 256);
#define RH_PREP(NS_)                                                                                               \
    case NS_:                                                                                                      \
        if (hd == 128)                                                                                             \
            hipLaunchKernelGGL((attn_bwd_prep_kernel<NS_, 128>), dim3(pgrid), dim3(256), 0, st, dOf, split_stride,  \
                               o, dOh, Drow, M, H, S);                                                             \
        else                                                                                                       \
            hipLaunchKernelGGL((attn_bwd_prep_kernel<NS_, 64>), dim3(pgrid), dim3(256), 0, st, dOf, split_stride,   \
                               o, dOh, Drow, M, H, S);                                                             \
        break
    switch (nsplit) {
        RH_PREP(1); RH_PREP(2); RH_PREP(3); RH_PREP(4); RH_PREP(5); RH_PREP(6); RH_PREP(7); RH_PREP(8);
    }
#undef RH_PREP
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const dim3 grid((S + 63) / 64 * H * B);
    const float scale = 1.0f / sqrtf((float)hd), sl2 = scale * 1.4426950408889634f;
    if (hd == 128) {
        hipLaunchKernelGGL(attn_bwd_dq_dma_kernel, grid, dim3(256), 0, st, q, k, v, dOh, lse, Drow, dqkv, rope, H, S, sl2,
                           scale);
        hipLaunchKernelGGL(attn_bwd_dkdv_dma_kernel, grid, dim3(256), 0, st, q, k, v, dOh, lse, Drow, dqkv, rope, H, S,
                           sl2, scale);
    } else {
        hipLaunchKernelGGL((attn_bwd_dq_kernel<64>), grid, dim3(256), 0, st, q, k, v, dOh, lse, Drow, dqkv, rope, H, S,
                           sl2, scale);
        hipLaunchKernelGGL((attn_bwd_dkdv_kernel<64>), grid, dim3(256), 0, st, q, k, v, dOh, lse, Drow, dqkv, rope, H, S,
                           sl2, scale);
    }
    return hipGetLastError();
}

}  // namespace rh
