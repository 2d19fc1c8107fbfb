// rh_gemm.hip -- prefill GEMMs on fp16 MFMA (gfx950) with fused epilogues.
//
// One kernel family serves every projection of the forward token loop
// (kernels/sdpa_fwd.rs:115-117 QKV, dyn_matmul.rs:15-75 Wo, ffn_fused.rs:80-160
// W1/W3/W2, full_model.rs:555-567 tied logits):
//     Y[m][n] = sum_k X[m][k] * W[n][k]
// X is the token-major fp16 activation [M, K] and W the weight repacked at
// upload to [N, K] ("out x in"); both are stored in fragment order (frag_off:
// 1 KB pieces of 16 rows x 32 k), so both stream along k in 1 KB pieces.  The
// MFMA computes the transposed tile (A = weight rows, B = token rows): each
// lane's accumulator then holds 4 consecutive output features of one token,
// which makes the RoPE pairs (2i, 2i+1) and 16-byte fp32 stores lane-local.
//
// Tile policy: DTile (below) -- both operands in fragment order in HBM, moved
// global -> LDS by DMA through a 4-stage (192x256: 5-stage) pipeline of 32-wide k slices,
// 32x32x16 MFMA (16x16x32 for the 8-wave tiles but 256x256) on fragments
// double-buffered in registers (256x256 keeps 32x32x16: its 16x16x32 form
// spills).  Instantiated as
// 256x256 (8 waves of 128x64, or 4 waves of 128x128 with AGPR accumulators),
// 256x128, 192x256, 192x128 and 128x128; a cost model picks one per shape.
// Out-of-range rows are clamped, not predicated (they only feed accumulator
// entries the epilogue never stores), so the loads are branch-free.  Tiles are
// remapped so blocks sharing a weight panel run on the same XCD (one L2).
//
// Stream-K: P blocks split the tiles x k-iterations space evenly.  A
// block whose range covers only part of a tile stores its fp32 partial; a
// second kernel sums each split tile's partials in block order
// (deterministic) and runs the epilogue.  Partials are each thread's own
// accumulator quads, so both MFMA forms use the same format (the long-K
// narrow outputs take the 8-wave 16x16x32 256x128 tile).  Blocks never communicate inside a
// kernel: on this multi-XCD part the per-XCD L2s are not coherent, and a
// device-scope fence costs an L2 writeback + invalidate.
#include <algorithm>
#include <type_traits>

#include <hip/hip_ext.h>

#include "rh_device.h"
#include "rh_kernels.h"

namespace rh {
namespace {

constexpr int SK_P = 256;  // stream-K blocks: one per CU

template <int TN, int TM>
struct Frag {
    f32x16 v[TN][TM];
};
// Accumulators of the 16x16x32 form: NA x NB tiles of 16 x 16.
template <int NA, int NB>
struct Frag16 {
    f32x4 v[NA][NB];
};

// ---------------------------------------------------------------------------
// Tile policy (DTile): operands go global -> LDS by DMA
// (global_load_lds_dwordx4: 16 bytes per lane land at LDS base + 16 * lane),
// so no registers stage them and NS = 4 stages of 32 k are in flight (5 for
// the 192x256 tile: its long-K and 5120-token shapes gain from the depth).  A
// stage holds BN/16 weight fragments and BM/16 activation fragments of 1 KB
// each; both operands are stored in fragment order in HBM (the activations by
// the kernels that produce them), so every DMA instruction reads 1 KB
// contiguous.  The 32x32x16 MFMA operand of lane 32h + r
// at k16-step s is then lane 16(2s + h) + r%16 of fragment r/16: 16 lanes read
// 256 contiguous bytes, conflict-free without padding.  One barrier per stage:
// each wave waits for its own DMA of the stage (an explicit vmcnt, since the
// stages behind it stay in flight), then the barrier publishes every wave's.
// The stages are separate LDS arrays so the compiler's own wait-count
// tracking can tell them apart and adds no drain of its own.
//
// M16 selects the MFMA shape.  false: 32x32x16 (a 32x32 output tile per
// instruction; operand lane 32h + r reads lane 16(2s + h) + r%16 of
// fragment r/16 at k16-step s).  true: 16x16x32, whose operand layout is the
// fragment itself (lane l: row l%16, k 8(l/16)..+7), so each operand is one
// 1 KB fragment read as is; same tile sizes, operand bytes and accumulator
// registers, a different output layout (epilogue16).
template <int WGN, int WGM, int TN, int TM, bool M16 = false, int NS_ = 4>
struct DTile {
    static_assert(NS_ == 4 || NS_ == 5, "4 or 5 stages");
    static constexpr bool kM16 = M16;
    static constexpr int NA = 2 * TN, NB = 2 * TM;  // 16-wide A / B tiles per wave (M16)
    static constexpr int BN = 32 * TN * WGN, BM = 32 * TM * WGM, NT = 64 * WGN * WGM;
    static constexpr int FTN = TN, FTM = TM, KI = 32, NS = NS_;
    static constexpr int NWF = BN / 16, NXF = BM / 16, NWAVE = WGN * WGM;
    // DMA instructions per wave per stage; when the fragments do not split
    // evenly, surplus slots repeat the last fragment (identical bytes to the
    // same LDS place), so every wave issues the same count and vmcnt stays exact.
    static constexpr int LPS = (NWF + NXF + NWAVE - 1) / NWAVE;
    static constexpr int SH = (NWF + NXF) * 512;     // halves per stage
    using Acc = std::conditional_t<M16, Frag16<NA, NB>, Frag<TN, TM>>;
    struct Smem {};
    __device__ static int nw(int n0) { return n0 + ((threadIdx.x >> 6) % WGN) * 32 * TN; }
    __device__ static int mw(int m0) { return m0 + ((threadIdx.x >> 6) / WGN) * 32 * TM; }
    // s_waitcnt with vmcnt <= n (expcnt, lgkmcnt left at their maximum)
    static constexpr int vm_wait(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
    // s_waitcnt with vmcnt <= n and lgkmcnt == 0: this wave's LDS reads are done
    static constexpr int vm_lgkm_wait(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4); }

    __device__ static void run(const GemmArgs& a, int n0, int m0, int kb, int ke, Acc& acc, Smem&) {
        __shared__ __attribute__((aligned(1024))) f16 st0[SH], st1[SH], st2[SH], st3[SH];
        // The fifth stage exists only in five-stage tiles, so the four-stage
        // ones keep their LDS size (two blocks per CU where they fit); there
        // buf(4) is never used and st4 merely names st3.
        f16* st4 = st3;
        if constexpr (NS > 4) {
            __shared__ __attribute__((aligned(1024))) f16 st4s[SH];
            st4 = st4s;
        }
        const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
        const int wn = wv % WGN, wm = wv / WGN;
        const int K = a.K;
        // this wave's DMA fragments: f = wv * LPS + q over [weight frags | activation frags]
        const f16* gp[LPS];
        int gstep[LPS], loff[LPS];
#pragma unroll
        for (int q = 0; q < LPS; ++q) {
            const int f = min(wv * LPS + q, NWF + NXF - 1);
            loff[q] = f * 512;
            if (f < NWF) {
                const int rb = min((n0 >> 4) + f, ((a.N + 15) >> 4) - 1);
                gp[q] = a.W + (size_t)rb * K * 16 + lane * 8;
                gstep[q] = 512;  // one 32-k fragment column of the 16-row block
            } else {
                const int rb = min((m0 >> 4) + f - NWF, ((a.M + 15) >> 4) - 1);
                gp[q] = a.X + (size_t)rb * K * 16 + lane * 8;
                gstep[q] = 512;
            }
        }
        const int r = lane & 31, h = lane >> 5;
        constexpr int AO = M16 ? NA : TN, BO = M16 ? NB : TM;
        int ao[AO], bo[BO];
        if constexpr (M16) {
#pragma unroll
            for (int i = 0; i < NA; ++i) ao[i] = (wn * NA + i) * 512 + 8 * lane;
#pragma unroll
            for (int j = 0; j < NB; ++j) bo[j] = (NWF + wm * NB + j) * 512 + 8 * lane;
        } else {
#pragma unroll
            for (int i = 0; i < TN; ++i)
                ao[i] = (((wn * 32 * TN + 32 * i) >> 4) + (r >> 4)) * 512 + 128 * h + 8 * (r & 15);
#pragma unroll
            for (int j = 0; j < TM; ++j)
                bo[j] = (NWF + ((wm * 32 * TM + 32 * j) >> 4) + (r >> 4)) * 512 + 128 * h + 8 * (r & 15);
        }
        auto buf = [&](int s) -> f16* { return s == 0 ? st0 : s == 1 ? st1 : s == 2 ? st2 : s == 3 ? st3 : st4; };
        auto issue = [&](int kt, f16* st) {
#pragma unroll
            for (int q = 0; q < LPS; ++q)
                __builtin_amdgcn_global_load_lds((const void*)(gp[q] + (size_t)kt * gstep[q]),
                                                 (__attribute__((address_space(3))) void*)(st + loff[q]), 16, 0, 0);
        };
        // fragments of one stage: 32x32: [k16 step][tile]; 16x16: [tile] (one k32)
        struct Frags32 { f16x8 a[2][TN], b[2][TM]; };
        struct Frags16 { f16x8 a[NA], b[NB]; };
        using Frags = std::conditional_t<M16, Frags16, Frags32>;
        // operand m of a stage, in the order the interleaved step reads them
        constexpr int NR = M16 ? NA + NB : 2 * (TN + TM);
        auto read1 = [&](const f16* st, Frags& f, int m) {
            if constexpr (M16) {
                if (m < NA) f.a[m] = *(const f16x8*)&st[ao[m]];
                else f.b[m - NA] = *(const f16x8*)&st[bo[m - NA]];
            } else {
                const int rks = m / (TN + TM), rr = m % (TN + TM);
                if (rr < TN) f.a[rks][rr] = *(const f16x8*)&st[ao[rr] + 256 * rks];
                else f.b[rks][rr - TN] = *(const f16x8*)&st[bo[rr - TN] + 256 * rks];
            }
        };
        auto readf = [&](const f16* st, Frags& f) {
#pragma unroll
            for (int m = 0; m < NR; ++m) read1(st, f, m);
        };
        // MFMA m of a stage
        constexpr int NM = M16 ? NA * NB : 2 * TN * TM;
        auto mfma1 = [&](const Frags& f, int m) {
            if constexpr (M16) {
                const int i = m / NB, j = m % NB;
                acc.v[i][j] = mfma16(f.a[i], f.b[j], acc.v[i][j]);
            } else {
                const int ks = m / (TN * TM), i = (m / TM) % TN, j = m % TM;
                acc.v[i][j] = mfma32(f.a[ks][i], f.b[ks][j], acc.v[i][j]);
            }
        };
        auto mfmas = [&](const Frags& f) {
#pragma unroll
            for (int m = 0; m < NM; ++m) mfma1(f, m);
        };
        if constexpr (M16) {
#pragma unroll
            for (int i = 0; i < NA; ++i)
#pragma unroll
                for (int j = 0; j < NB; ++j) acc.v[i][j] = f32x4{};
        } else {
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j) acc.v[i][j] = f32x16{};
        }
        // no wave may still read the stages from a previous call
        __builtin_amdgcn_s_waitcnt(vm_lgkm_wait(63));
        __builtin_amdgcn_s_barrier();
        const int n = ke - kb;
#pragma unroll
        for (int p = 0; p < NS - 1; ++p) issue(kb + min(p, n - 1), buf(p));
        // Stage t sits in buffer t % NS.  Step t: publish stage t+1, refill the
        // buffer stage t came from (its fragments are already in registers),
        // read stage t+1's fragments, then run stage t's MFMAs under those reads.
        Frags f0, f1;
        __builtin_amdgcn_s_waitcnt(vm_lgkm_wait((NS - 2) * LPS));
        __builtin_amdgcn_s_barrier();
        issue(kb + min(NS - 1, n - 1), buf(NS - 1));
        readf(buf(0), f0);
        // A full step, issued interleaved and pinned in that order: MFMA m,
        // then LDS read m, then DMA m.  With one or two waves per SIMD a
        // wave's in-order issue blocks whenever the vector-memory queue is
        // full; spreading the reads and DMAs between MFMAs keeps the matrix
        // pipe fed through those stalls (issued in bulk they idle it).
        auto step_il = [&](int t, Frags& cur, Frags& nxt, f16* refill, const f16* next) {
            __builtin_amdgcn_s_waitcnt(vm_lgkm_wait((NS - 2) * LPS));
            __builtin_amdgcn_s_barrier();
            const int kt = kb + min(t + NS, n - 1);
            constexpr int NG = NM > NR ? (NM > LPS ? NM : LPS) : (NR > LPS ? NR : LPS);
#pragma unroll
            for (int m = 0; m < NG; ++m) {
                if (m < NM) mfma1(cur, m);
                if (m < NR) read1(next, nxt, m);
                if (m < LPS)
                    __builtin_amdgcn_global_load_lds((const void*)(gp[m] + (size_t)kt * gstep[m]),
                                                     (__attribute__((address_space(3))) void*)(refill + loff[m]),
                                                     16, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        // Tail step (past the last stage: a harmless read of a stale buffer,
        // MFMAs skipped).
        auto step = [&](int t, Frags& cur, Frags& nxt, f16* refill, const f16* next) {
            __builtin_amdgcn_s_waitcnt(vm_lgkm_wait((NS - 2) * LPS));
            __builtin_amdgcn_s_barrier();
            issue(kb + min(t + NS, n - 1), refill);
            readf(next, nxt);
            if (t < n) mfmas(cur);
        };
        // Whole groups of NS steps run interleaved; the remainder runs one
        // more group of predicated steps.  Every step issues LPS DMAs, so the
        // vmcnt bookkeeping stays uniform.
        int t0 = 0;
        if constexpr (NS == 4) {
            for (; t0 + NS <= n; t0 += NS) {
                step_il(t0, f0, f1, buf(0), buf(1));
                step_il(t0 + 1, f1, f0, buf(1), buf(2));
                step_il(t0 + 2, f0, f1, buf(2), buf(3));
                step_il(t0 + 3, f1, f0, buf(3), buf(0));
            }
            if (t0 < n) {
                step(t0, f0, f1, buf(0), buf(1));
                step(t0 + 1, f1, f0, buf(1), buf(2));
                step(t0 + 2, f0, f1, buf(2), buf(3));
                step(t0 + 3, f1, f0, buf(3), buf(0));
            }
        } else {  // 5 stages: groups of 10 steps bring both the buffers and the fragment sets back around
            for (; t0 + 10 <= n; t0 += 10) {
                step_il(t0, f0, f1, buf(0), buf(1));
                step_il(t0 + 1, f1, f0, buf(1), buf(2));
                step_il(t0 + 2, f0, f1, buf(2), buf(3));
                step_il(t0 + 3, f1, f0, buf(3), buf(4));
                step_il(t0 + 4, f0, f1, buf(4), buf(0));
                step_il(t0 + 5, f1, f0, buf(0), buf(1));
                step_il(t0 + 6, f0, f1, buf(1), buf(2));
                step_il(t0 + 7, f1, f0, buf(2), buf(3));
                step_il(t0 + 8, f0, f1, buf(3), buf(4));
                step_il(t0 + 9, f1, f0, buf(4), buf(0));
            }
            if (t0 < n) {
                step(t0, f0, f1, buf(0), buf(1));
                step(t0 + 1, f1, f0, buf(1), buf(2));
                step(t0 + 2, f0, f1, buf(2), buf(3));
                step(t0 + 3, f1, f0, buf(3), buf(4));
                step(t0 + 4, f0, f1, buf(4), buf(0));
                step(t0 + 5, f1, f0, buf(0), buf(1));
                step(t0 + 6, f0, f1, buf(1), buf(2));
                step(t0 + 7, f1, f0, buf(2), buf(3));
                step(t0 + 8, f0, f1, buf(3), buf(4));
                step(t0 + 9, f1, f0, buf(4), buf(0));
            }
        }
        // the trailing (unused) stage loads must land before the LDS is reused
        __builtin_amdgcn_s_waitcnt(vm_wait(0));
    }
};

// SiLU-gate backward (layer.rs:7083-7104) of the gate gradient g = (v0..v3)
// of token m, features n..n+3, and the saved a1 = h1, a3 = h3 there:
// dh3 = g silu(h1), dh1 = g h3 silu'(h1), fp16 in fragment order [M][2N]
// (dh1 in columns 0..N-1, dh3 in N..2N-1).
__device__ __forceinline__ void silu_bwd4(const GemmArgs& a, int m, int n, float v0, float v1, float v2, float v3,
                                          f16x4 a1, f16x4 a3) {
    const float g[4] = {v0, v1, v2, v3};
    f16x4 o1, o3;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float h1 = (float)a1[e], h3 = (float)a3[e];
        const float sig = 1.0f / (1.0f + __expf(-h1));
        o3[e] = (f16)(g[e] * (h1 * sig));
        o1[e] = (f16)(g[e] * h3 * (sig * (1.0f + h1 * (1.0f - sig))));
    }
    *(f16x4*)(a.out_f16 + frag_off(m, n, 2 * a.ldo)) = o1;
    *(f16x4*)(a.out_f16 + frag_off(m, a.ldo + n, 2 * a.ldo)) = o3;
}

// Stores four consecutive output features n..n+3 of token m (every epilogue
// but SwiGLU, whose lanes hold W1 and W3 rows and store gate features).
template <int EPI>
__device__ __forceinline__ void store4(const GemmArgs& a, int m, int n, float v0, float v1, float v2, float v3) {
    if constexpr (EPI == EPI_F32) {
        if (a.alpha != 0.f) {  // optional output scale (0 = none)
            v0 *= a.alpha; v1 *= a.alpha; v2 *= a.alpha; v3 *= a.alpha;
        }
        if (a.softcap > 0.f) {
            const float c = a.softcap, ic = 1.0f / c;
            v0 = tanhf(v0 * ic) * c; v1 = tanhf(v1 * ic) * c;
            v2 = tanhf(v2 * ic) * c; v3 = tanhf(v3 * ic) * c;
        }
        f32x4* po = (f32x4*)(a.out_f32 + (size_t)m * a.ldo + n);
        if (a.nt_out) __builtin_nontemporal_store(f32x4{v0, v1, v2, v3}, po);
        else *po = f32x4{v0, v1, v2, v3};
    } else if constexpr (EPI == EPI_RESID) {
        const size_t o = (size_t)m * a.ldo + n;
        f32x4* px = (f32x4*)(a.out_f32 + o);
        f32x4 x = *(const f32x4*)((a.resid_in ? a.resid_in : a.out_f32) + o);
        x[0] = v0 * a.alpha + x[0]; x[1] = v1 * a.alpha + x[1];
        x[2] = v2 * a.alpha + x[2]; x[3] = v3 * a.alpha + x[3];
        if (a.nt_out) __builtin_nontemporal_store(x, px);
        else *px = x;
    } else if constexpr (EPI == EPI_QKV) {
        // no integer divisions by run-time values here but the per-row m / S
        // (hoisted out of the feature loop): n < 3D, hd a power of two
        const int sec = (n >= a.D) + (n >= 2 * a.D), c = n - sec * a.D;
        const int h = c >> __builtin_ctz(a.hd), d = c & (a.hd - 1);
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
    } else if constexpr (EPI == EPI_SILU_BWD) {
        const size_t o = (size_t)m * a.ldo + n, plane = (size_t)a.M * a.ldo;
        silu_bwd4(a, m, n, v0, v1, v2, v3, *(const f16x4*)(a.h13 + o), *(const f16x4*)(a.h13 + plane + o));
    }
}

// SwiGLU output of token m, gate features f..f+3 from h1 (W1 rows) and h3
// (the matching W3 rows); EPI_SWIGLU_SAVE also keeps h1, h3 for the backward.
template <int EPI>
__device__ __forceinline__ void store_swiglu(const GemmArgs& a, int m, int f, const float (&h1)[4],
                                             const float (&h3)[4]) {
    f16x4 g;
#pragma unroll
    for (int r = 0; r < 4; ++r) g[r] = (f16)(silu_f(h1[r]) * h3[r]);
    *(f16x4*)(a.out_f16 + frag_off(m, f, a.ldo)) = g;
    if constexpr (EPI == EPI_SWIGLU_SAVE) {
        // the pre-activations for the backward pass: h1 | h3 planes [M][F]
        const size_t o = (size_t)m * a.ldo + f, plane = (size_t)a.M * a.ldo;
        *(f16x4*)(a.h13 + o) = f16x4{(f16)h1[0], (f16)h1[1], (f16)h1[2], (f16)h1[3]};
        *(f16x4*)(a.h13 + plane + o) = f16x4{(f16)h3[0], (f16)h3[1], (f16)h3[2], (f16)h3[3]};
    }
}

// 32x32 tiles.  (nw, mw): the wave's first feature row and token.  Lane holds
// token m = mw + j*32 + lane%32 and, per q4, the four consecutive features
// n = nw + i*32 + 8*q4 + 4*(lane/32) + (0..3).
template <int TN, int TM, int EPI>
__device__ __forceinline__ void epilogue(const GemmArgs& a, int nw, int mw, const Frag<TN, TM>& acc) {
    const int lane = threadIdx.x & 63;
    const int N = a.N, M = a.M;
#pragma unroll
    for (int j = 0; j < TM; ++j) {
        const int m = mw + j * 32 + (lane & 31);
        if (m >= M) continue;
        if constexpr (EPI == EPI_SWIGLU || EPI == EPI_SWIGLU_SAVE) {
            // W1|W3 is interleaved in 16-row groups: rows 0..15 of 32-row tile T
            // are W1 rows of features 16T.., rows 16..31 the matching W3 rows,
            // and row r + 16 sits in the same lane as row r (accumulator + 8).
#pragma unroll
            for (int i = 0; i < TN; ++i) {
                const int T = (nw + i * 32) >> 5;
#pragma unroll
                for (int q4 = 0; q4 < 2; ++q4) {
                    const int f = 16 * T + 8 * q4 + 4 * (lane >> 5);
                    if (f >= a.ldo) continue;
                    float h1[4], h3[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        h1[r] = acc.v[i][j][4 * q4 + r];
                        h3[r] = acc.v[i][j][4 * q4 + 8 + r];
                    }
                    store_swiglu<EPI>(a, m, f, h1, h3);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const int n = nw + i * 32 + 8 * q4 + 4 * (lane >> 5);
                    if (n >= N) continue;
                    store4<EPI>(a, m, n, acc.v[i][j][4 * q4 + 0], acc.v[i][j][4 * q4 + 1], acc.v[i][j][4 * q4 + 2],
                                acc.v[i][j][4 * q4 + 3]);
                }
        }
    }
}

// 16x16 tiles: lane l holds token m = mw + 16j + l%16 and the four
// consecutive features n = nw + 16i + 4(l/16) + (0..3) of A tile i, B tile j.
template <int NA, int NB, int EPI>
__device__ __forceinline__ void epilogue(const GemmArgs& a, int nw, int mw, const Frag16<NA, NB>& acc) {
    const int lane = threadIdx.x & 63;
    const int N = a.N, M = a.M;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const int m = mw + 16 * j + (lane & 15);
        if (m >= M) continue;
        if constexpr (EPI == EPI_SWIGLU || EPI == EPI_SWIGLU_SAVE) {
            // A tiles 2p and 2p + 1 are the W1 rows of features 16T..16T+15 and
            // the matching W3 rows (T = (nw + 32p) / 32; nw is a multiple of 32)
#pragma unroll
            for (int p = 0; p < NA / 2; ++p) {
                const int f = 16 * ((nw + 32 * p) >> 5) + 4 * (lane >> 4);
                if (f >= a.ldo) continue;
                float h1[4], h3[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    h1[r] = acc.v[2 * p][j][r];
                    h3[r] = acc.v[2 * p + 1][j][r];
                }
                store_swiglu<EPI>(a, m, f, h1, h3);
            }
        } else {
#pragma unroll
            for (int i = 0; i < NA; ++i) {
                const int n = nw + 16 * i + 4 * (lane >> 4);
                if (n >= N) continue;
                store4<EPI>(a, m, n, acc.v[i][j][0], acc.v[i][j][1], acc.v[i][j][2], acc.v[i][j][3]);
            }
        }
    }
}

template <class Tl, int EPI>
__device__ __forceinline__ void run_epilogue(const GemmArgs& a, int nw, int mw, const typename Tl::Acc& acc) {
    if constexpr (Tl::kM16)
        epilogue<Tl::NA, Tl::NB, EPI>(a, nw, mw, acc);
    else
        epilogue<Tl::FTN, Tl::FTM, EPI>(a, nw, mw, acc);
}

// The accumulators of a thread as TN*TM*4 quads of 4 floats (the stream-K
// partial format; the same thread stores and reloads them).  32x32: quad
// (i*TM + j)*4 + q = acc.v[i][j][4q..4q+3]; 16x16: quad a*NB + b = acc.v[a][b].
template <int TN, int TM>
__device__ __forceinline__ f32x4 get_quad(const Frag<TN, TM>& f, int x) {
    const f32x16& v = f.v[x / (TM * 4)][(x / 4) % TM];
    const int e = 4 * (x % 4);
    return f32x4{v[e], v[e + 1], v[e + 2], v[e + 3]};
}
template <int TN, int TM>
__device__ __forceinline__ void set_quad(Frag<TN, TM>& f, int x, f32x4 q) {
    f32x16& v = f.v[x / (TM * 4)][(x / 4) % TM];
    const int e = 4 * (x % 4);
    v[e] = q[0]; v[e + 1] = q[1]; v[e + 2] = q[2]; v[e + 3] = q[3];
}
template <int NA, int NB>
__device__ __forceinline__ f32x4 get_quad(const Frag16<NA, NB>& f, int x) { return f.v[x / NB][x % NB]; }
template <int NA, int NB>
__device__ __forceinline__ void set_quad(Frag16<NA, NB>& f, int x, f32x4 q) { f.v[x / NB][x % NB] = q; }
// The quads of 32-row slice s of a wave's tile and the type holding them:
// 32x32: row tile s (TM tiles x 4 quads); 16x16: A tiles 2s, 2s+1 (2 x NB).
template <class Tl>
struct Slice {
    static constexpr int NQ = Tl::FTM * 4;
    using Acc = std::conditional_t<Tl::kM16, Frag16<2, Tl::NB>, Frag<1, Tl::FTM>>;
    __device__ static int quad_of(int s, int x) { return s * NQ + x; }  // both layouts: slice-major
};

// MODE: MODE_DP one block per tile; MODE_SK stream-K over P blocks (T =
// tiles x k-iterations); MODE_SPLIT P even k-splits per tile, each storing its
// fp32 partial [M][N] at sk_part + split * M * N.
enum { MODE_DP = 0, MODE_SK = 1, MODE_SPLIT = 2 };

template <class Tl, int EPI, int MODE>
__global__ __launch_bounds__(Tl::NT) void gemm_kernel(GemmArgs a, int P, long long T) {
    __shared__ __attribute__((aligned(16))) typename Tl::Smem sm;
    const int nbN = (a.N + Tl::BN - 1) / Tl::BN, nbM = (a.M + Tl::BM - 1) / Tl::BM;
    const int KT = a.K / Tl::KI;
    typename Tl::Acc acc;
    if constexpr (MODE == MODE_DP) {
        const int t = xcd_remap(blockIdx.x, nbN * nbM);
        // Consecutive tiles (run together on one XCD) walk groups of up to
        // 8 M-tiles x every N panel, M fastest: the 32 tiles an XCD runs at
        // a time then share 4 weight panels and 8 activation row blocks in
        // its L2, instead of one panel and 32 row blocks (7B batch 16: QKV
        // 785 -> 753 us, W2 870 -> 746 us, prefill 108.4 -> 101.5 ms).
        int nb, mb;
        if (nbM <= 8) {
            nb = t / nbM;
            mb = t - nb * nbM;
        } else {
            const int g = t / (8 * nbN), r = t - g * 8 * nbN, gm = min(8, nbM - g * 8);
            mb = g * 8 + r % gm;
            nb = r / gm;
        }
        if constexpr (EPI == EPI_SILU_BWD && Tl::kM16 && Tl::NA * Tl::NB <= 12) {
            // The saved h1, h3 of this lane's outputs are loaded before the k
            // loop, so they arrive under it instead of stalling the epilogue
            // (2 * NA * NB registers held through the loop: the larger tiles
            // would spill).
            const int nw = Tl::nw(nb * Tl::BN), mw = Tl::mw(mb * Tl::BM), lane = threadIdx.x & 63;
            const size_t plane = (size_t)a.M * a.ldo;
            f16x4 p1[Tl::NB][Tl::NA], p3[Tl::NB][Tl::NA];
#pragma unroll
            for (int j = 0; j < Tl::NB; ++j)
#pragma unroll
                for (int i = 0; i < Tl::NA; ++i) {
                    const int m = mw + 16 * j + (lane & 15), n = nw + 16 * i + 4 * (lane >> 4);
                    p1[j][i] = p3[j][i] = f16x4{};
                    if (m < a.M && n < a.N) {
                        const size_t o = (size_t)m * a.ldo + n;
                        p1[j][i] = *(const f16x4*)(a.h13 + o);
                        p3[j][i] = *(const f16x4*)(a.h13 + plane + o);
                    }
                }
            Tl::run(a, nb * Tl::BN, mb * Tl::BM, 0, KT, acc, sm);
#pragma unroll
            for (int j = 0; j < Tl::NB; ++j)
#pragma unroll
                for (int i = 0; i < Tl::NA; ++i) {
                    const int m = mw + 16 * j + (lane & 15), n = nw + 16 * i + 4 * (lane >> 4);
                    if (m < a.M && n < a.N)
                        silu_bwd4(a, m, n, acc.v[i][j][0], acc.v[i][j][1], acc.v[i][j][2], acc.v[i][j][3], p1[j][i],
                                  p3[j][i]);
                }
        } else {
            Tl::run(a, nb * Tl::BN, mb * Tl::BM, 0, KT, acc, sm);
            run_epilogue<Tl, EPI>(a, Tl::nw(nb * Tl::BN), Tl::mw(mb * Tl::BM), acc);
        }
    } else if constexpr (MODE == MODE_SPLIT) {
        // Blocks go round-robin to the 8 XCDs (block b on XCD b % 8).  When P
        // divides 8 and the tiles share out evenly, XCD x runs split x % P of
        // its 1/(8/P) of the tiles, panel by panel: each XCD's L2 then fetches
        // only its k-slice of the activation (which every tile reads) and
        // each weight slice once for all M-tiles of its panel.  Otherwise the
        // splits of one tile and the tiles of one weight panel share an XCD.
        const int tiles = nbN * nbM;
        int tile, sp;
        if (8 % P == 0 && tiles % (8 / P) == 0) {
            const int x = blockIdx.x & 7;
            sp = x % P;
            tile = (x / P) * (tiles / (8 / P)) + (blockIdx.x >> 3);
        } else {
            const int v = xcd_remap(blockIdx.x, tiles * P);
            tile = v / P;
            sp = v - tile * P;
        }
        const int nb = tile / nbM, mb = tile - nb * nbM;
        const int kb = (int)((long long)sp * KT / P), ke = (int)((long long)(sp + 1) * KT / P);
        Tl::run(a, nb * Tl::BN, mb * Tl::BM, kb, ke, acc, sm);
        GemmArgs b = a;
        b.out_f32 = a.sk_part + (size_t)sp * a.M * a.N;
        b.ldo = a.N;
        b.softcap = 0.f;
        b.alpha = 0.f;  // raw partials: the row kernel applies alpha once to their sum
        run_epilogue<Tl, EPI_F32>(b, Tl::nw(nb * Tl::BN), Tl::mw(mb * Tl::BM), acc);
    } else {
        constexpr int NT = Tl::NT;
        constexpr int NV = Tl::FTN * Tl::FTM * 4;  // f32x4 per thread per partial tile
        const int tid = threadIdx.x;
        const int lp = xcd_remap(blockIdx.x, P);
        const long long it0 = (long long)lp * T / P, it1 = (long long)(lp + 1) * T / P;
        long long it = it0;
        while (it < it1) {
            const int tile = (int)(it / KT);
            const int kb = (int)(it - (long long)tile * KT);
            const int ke = (int)((long long)KT < kb + (it1 - it) ? (long long)KT : kb + (it1 - it));
            const int nb = tile / nbM, mb = tile - nb * nbM;
            const int n0 = nb * Tl::BN, m0 = mb * Tl::BM;
            Tl::run(a, n0, m0, kb, ke, acc, sm);
            if (kb == 0 && ke == KT) {
                run_epilogue<Tl, EPI>(a, Tl::nw(n0), Tl::mw(m0), acc);
            } else {
                // A block's first segment goes to slot 0, its last to slot 1;
                // the fixup kernel merges them once this kernel has finished.
                const int slot = (it == it0) ? 0 : 1;
                f32x4* mine = (f32x4*)a.sk_part + ((size_t)(lp * 2 + slot) * NV) * NT + tid;
#pragma unroll
                for (int x = 0; x < NV; ++x) mine[(size_t)x * NT] = get_quad(acc, x);
            }
            it = (long long)tile * KT + ke;
        }
    }
}

// Stream-K fixup: one block per (tile, 32-row tile of every wave).  A tile covered
// by a single block was finished by gemm_kernel; for a split tile, sum the
// partials of its contributing blocks in block order (deterministic) and run
// the epilogue on the slice.
template <class Tl, int EPI>
__global__ __launch_bounds__(Tl::NT) void gemm_fixup_kernel(GemmArgs a, int P, long long T) {
    using Sl = Slice<Tl>;
    constexpr int NT = Tl::NT, NV = Tl::FTN * Tl::FTM * 4, NQ = Sl::NQ;
    const int nbM = (a.M + Tl::BM - 1) / Tl::BM;
    const int KT = a.K / Tl::KI;
    const int tile = blockIdx.x, i0 = blockIdx.y, tid = threadIdx.x;
    const long long tb = (long long)tile * KT, te = tb + KT;
    const int pf = (int)(((tb + 1) * P - 1) / T), pl = (int)((te * P - 1) / T);
    if (pf == pl) return;
    typename Sl::Acc acc;
#pragma unroll
    for (int x = 0; x < NQ; ++x) set_quad(acc, x, f32x4{});
    for (int c = pf; c <= pl; ++c) {
        // with fewer iterations than blocks some blocks own none and wrote nothing
        if ((long long)c * T / P == (long long)(c + 1) * T / P) continue;
        const int cslot = ((long long)c * T / P >= tb) ? 0 : 1;
        const f32x4* part = (const f32x4*)a.sk_part + ((size_t)(c * 2 + cslot) * NV) * NT + tid;
#pragma unroll
        for (int x = 0; x < NQ; ++x) set_quad(acc, x, get_quad(acc, x) + part[(size_t)Sl::quad_of(i0, x) * NT]);
    }
    const int nb = tile / nbM, mb = tile - nb * nbM;
    const int nw = Tl::nw(nb * Tl::BN) + 32 * i0, mw = Tl::mw(mb * Tl::BM);
    if constexpr (Tl::kM16)
        epilogue<2, Tl::NB, EPI>(a, nw, mw, acc);
    else
        epilogue<1, Tl::FTM, EPI>(a, nw, mw, acc);
}

template <class Tl, int EPI>
hipError_t launch_tile(const GemmArgs& a, bool sk, hipStream_t st) {
    const int nbN = (a.N + Tl::BN - 1) / Tl::BN, nbM = (a.M + Tl::BM - 1) / Tl::BM;
    const int tiles = nbN * nbM;
    const long long T = (long long)tiles * (a.K / Tl::KI);
    if (sk) {
        if (!a.sk_part || (size_t)SK_P * 2 * Tl::BN * Tl::BM > a.sk_part_floats) return hipErrorInvalidValue;
        if (a.prof_start && hipEventRecord(a.prof_start, st) != hipSuccess) return hipErrorInvalidValue;
        hipLaunchKernelGGL((gemm_kernel<Tl, EPI, MODE_SK>), dim3(SK_P), dim3(Tl::NT), 0, st, a, SK_P, T);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL((gemm_fixup_kernel<Tl, EPI>), dim3(tiles, Tl::FTN), dim3(Tl::NT), 0, st, a, SK_P, T);
        if (a.prof_stop && hipEventRecord(a.prof_stop, st) != hipSuccess) return hipErrorInvalidValue;
    } else if (a.prof_start) {
        hipExtLaunchKernelGGL((gemm_kernel<Tl, EPI, MODE_DP>), dim3(tiles), dim3(Tl::NT), 0, st, a.prof_start,
                              a.prof_stop, 0u, a, 1, T);
    } else {
        hipLaunchKernelGGL((gemm_kernel<Tl, EPI, MODE_DP>), dim3(tiles), dim3(Tl::NT), 0, st, a, 1, T);
    }
    return hipGetLastError();
}

// S-way split-K of a residual GEMM: partials only (the row kernel reduces).
template <class Tl>
hipError_t launch_split(const GemmArgs& a, int S, hipStream_t st) {
    const int tiles = ((a.N + Tl::BN - 1) / Tl::BN) * ((a.M + Tl::BM - 1) / Tl::BM);
    if (S < 1 || S > a.K / Tl::KI || !a.sk_part || (size_t)S * a.M * a.N > a.sk_part_floats)
        return hipErrorInvalidValue;
    if (a.prof_start && hipEventRecord(a.prof_start, st) != hipSuccess) return hipErrorInvalidValue;
    hipLaunchKernelGGL((gemm_kernel<Tl, EPI_F32, MODE_SPLIT>), dim3(tiles * S), dim3(Tl::NT), 0, st, a, S, 0LL);
    if (a.prof_stop && hipEventRecord(a.prof_stop, st) != hipSuccess) return hipErrorInvalidValue;
    return hipGetLastError();
}

// Weight-gradient GEMM (K = the token count, short; fp32 output, as large
// as the weights): persistent blocks of 8 compute waves running the 8-wave
// 16x16x32 128x128 DTile k loop and WG_SW store waves.  A tile's
// accumulators go to an LDS staging tile; the store waves write it out to
// HBM while the compute waves run the next tile, so the output stores
// overlap the MFMAs.  The compute waves issue no stores at all: on gfx950
// stores and the operand DMAs share one in-order vmcnt, so stores in the
// compute waves would make every later stage wait hold for them.
//
// Barriers: every wave of the block executes the same s_barrier sequence.
// Per tile the compute waves run Tl::run (2 + NS * ceil(KT / NS) barriers),
// then X (the store waves are done reading the staging tile), write the
// staging tile, then Y (published).  The store waves mirror that count,
// storing the previous tile in 16 rounds spread over the k loop's barriers,
// and the block's last tile after its Y.
//
// Tiles: block b runs on XCD b % 8 and takes every (gridDim / 8)-th tile of
// that XCD's contiguous share; tiles are numbered in groups of 8 M-tiles x all
// N panels (so 32 tiles in flight on an XCD span 4 panels x 8 M-tiles).
constexpr int WG_SW = 4;     // store waves
constexpr int WG_SP = 132;   // staging row pitch in floats (conflict-free b128 access)
template <class Tl, bool ACC>
__global__ __launch_bounds__(Tl::NT + 64 * WG_SW) void gemm_wgrad_kernel(GemmArgs a) {
    static_assert(Tl::kM16 && Tl::BN == 128 && Tl::BM == 128 && Tl::NWAVE == 8, "8-wave 128x128 tile");
    __shared__ __attribute__((aligned(16))) float stg[128 * WG_SP];
    typename Tl::Smem sm;
    const int nbN = (a.N + 127) / 128, nbM = (a.M + 127) / 128, T = nbN * nbM;
    const int KT = a.K / Tl::KI;
    const int xcd = blockIdx.x & 7, k = blockIdx.x >> 3, per = gridDim.x >> 3;
    const int t0 = (int)((long long)xcd * T / 8), t1 = (int)((long long)(xcd + 1) * T / 8);
    const int mine = (t1 - t0 > k) ? (t1 - t0 - k + per - 1) / per : 0;
    const int nbar = 2 + Tl::NS * ((KT + Tl::NS - 1) / Tl::NS);  // barriers of one Tl::run
    auto tile_at = [&](int i, int& n0, int& m0) {
        const int t = t0 + k + i * per;
        const int mg = t / (nbN * 8), rem = t - mg * nbN * 8, gsz = min(8, nbM - mg * 8);
        n0 = (rem / gsz) * 128;
        m0 = (mg * 8 + rem % gsz) * 128;
    };
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (wv < Tl::NWAVE) {
        typename Tl::Acc acc;
        for (int i = 0; i < mine; ++i) {
            int n0, m0;
            tile_at(i, n0, m0);
            Tl::run(a, n0, m0, 0, KT, acc, sm);
            __builtin_amdgcn_s_barrier();  // X
            const int nl = Tl::nw(n0) - n0, ml = Tl::mw(m0) - m0;
#pragma unroll
            for (int i2 = 0; i2 < Tl::NA; ++i2)
#pragma unroll
                for (int j = 0; j < Tl::NB; ++j)
                    *(f32x4*)&stg[(ml + 16 * j + (lane & 15)) * WG_SP + nl + 16 * i2 + 4 * (lane >> 4)] = acc.v[i2][j];
            lds_barrier();  // Y
        }
    } else {
        const int sw = wv - Tl::NWAVE;
        int pn0 = 0, pm0 = 0;  // the staged tile
        // round r: rows 2 (4r + sw) + lane / 32 of the staged tile, 4 columns per lane
        auto store_round = [&](int r) {
            const int ml = 2 * (WG_SW * r + sw) + (lane >> 5), nl = 4 * (lane & 31);
            const int m = pm0 + ml, n = pn0 + nl;
            if (m < a.M && n < a.N) {
                f32x4 v = *(const f32x4*)&stg[ml * WG_SP + nl];
                float* po = a.out_f32 + (size_t)m * a.ldo + n;
                if constexpr (ACC) {
                    f32x4 x = *(const f32x4*)po;
                    x[0] = v[0] * a.alpha + x[0]; x[1] = v[1] * a.alpha + x[1];
                    x[2] = v[2] * a.alpha + x[2]; x[3] = v[3] * a.alpha + x[3];
                    v = x;
                } else if (a.alpha != 0.f) {
                    v[0] *= a.alpha; v[1] *= a.alpha; v[2] *= a.alpha; v[3] *= a.alpha;
                }
                // the gradients are read only by the optimizer: streaming stores
                // keep them from evicting the other stream's operands
                __builtin_nontemporal_store(v, (f32x4*)po);
            }
        };
        constexpr int NR = 128 / (2 * WG_SW);  // rounds per tile
        for (int i = 0; i < mine; ++i) {
            for (int bar = 0; bar < nbar; ++bar) {
                __builtin_amdgcn_s_barrier();
                if (i > 0)
                    for (int r = bar * NR / nbar; r < (bar + 1) * NR / nbar; ++r) store_round(r);
            }
            __builtin_amdgcn_s_waitcnt(Tl::vm_lgkm_wait(63));  // staging reads done before X
            __builtin_amdgcn_s_barrier();  // X
            __builtin_amdgcn_s_barrier();  // Y
            tile_at(i, pn0, pm0);
        }
        if (mine > 0)
            for (int r = 0; r < NR; ++r) store_round(r);
    }
}

template <int EPI>
hipError_t launch_epi(const GemmArgs& a, hipStream_t st) {
    int cfg = a.force_cfg;
    if (cfg == GCFG_AUTO) {
        // Data-parallel tiles: estimated time = rounds of one block per CU x
        // tile FLOPs / that tile's per-CU rate.  The rates are fitted to MI355X
        // timings of every tile on 27 GEMM shapes of the 7B forward and
        // training step (M 512 - 8192, random fp16 operands; the picks land
        // within 0.5% of the per-shape best in total); the estimate trades wave
        // quantization (e.g. 172 vs 230 tiles at M = 512) against per-tile
        // efficiency.  Narrow outputs (Wo) and long K (W2) use stream-K
        // instead, when every block gets at least two 32-wide k-iterations.
        struct Cand { int cfg, bn, bm; float rate; };
        constexpr Cand dp[] = {{GCFG_D8_256x256, 256, 256, 4.4f}, {GCFG_D8_192x256, 192, 256, 4.35f},
                               {GCFG_D8_256x128, 256, 128, 3.6f}, {GCFG_D8_192x128, 192, 128, 3.7f},
                               {GCFG_D8_128x128, 128, 128, 3.0f}};
        const long long KT = a.K / 32;
        const int t256x128 = ((a.N + 255) / 256) * ((a.M + 127) / 128);
        const int t128 = ((a.N + 127) / 128) * ((a.M + 127) / 128);
        const bool sk_ok = a.sk_part && (size_t)SK_P * 2 * 256 * 256 <= a.sk_part_floats;
        if (sk_ok && a.K >= 8192 && t256x128 < 160 && t256x128 * KT >= 2 * SK_P) {
            cfg = GCFG_D8_256x128_SK;
        } else if (sk_ok && t128 < 160 && t128 * KT >= 2 * SK_P && KT * (SK_P - t128) >= 28 * SK_P) {
            // stream-K saves the idle CUs' share of one tile's k loop (about
            // 0.36 us per 32-k step) but pays a fix-up launch (about 9 us): at
            // 600M, M = 512, QKV (144 tiles, K 1536) one round of whole tiles is
            // faster (15.3 + 8.5 us stream-K + fix-up against one 17.5 us round)
            cfg = GCFG_D8_128x128_SK;
        } else {
            float best = 3.0e38f;
            for (const Cand& c : dp) {
                const long long tiles = (long long)((a.N + c.bn - 1) / c.bn) * ((a.M + c.bm - 1) / c.bm);
                const float t = (float)((tiles + SK_P - 1) / SK_P) * (float)c.bn * (float)c.bm / c.rate;
                if (t < best) { best = t; cfg = c.cfg; }
            }
        }
    }
    // The 8-wave 192x256, 192x128, 256x128 and 128x128 tiles run the
    // 16x16x32 form: at M = 512 (7B) W1|W3 takes 84.5 us as 8-wave 16x16x32
    // 192x256, against 87.8 as a 4-wave 16x16x32 tile and 91.4 as 8-wave
    // 32x32x16; QKV 60.4 us as 8-wave 16x16x32 192x128 against 64.7 as 4-wave
    // 32x32x16; the 8-wave 256x128 and 128x128 tiles are 0-12% and 1-6%
    // faster in that form than their 32x32x16 twins on every shape timed.  The
    // 4-wave 192x128 tile stays 32x32x16: the weight-gradient GEMMs need its
    // two blocks per CU, which the 16x16x32 form's extra registers would
    // cost; the 8-wave 256x256 tile spills in that form.
    switch (cfg) {
        case GCFG_D8_256x256: return launch_tile<DTile<2, 4, 4, 2>, EPI>(a, false, st);
        case GCFG_D8_256x256_SK: return launch_tile<DTile<2, 4, 4, 2>, EPI>(a, true, st);
        case GCFG_D4_128x128: return launch_tile<DTile<2, 2, 2, 2>, EPI>(a, false, st);
        case GCFG_D4_128x128_SK: return launch_tile<DTile<2, 2, 2, 2>, EPI>(a, true, st);
        case GCFG_D8_256x128: return launch_tile<DTile<4, 2, 2, 2, true>, EPI>(a, false, st);
        case GCFG_D8_256x128_SK: return launch_tile<DTile<4, 2, 2, 2, true>, EPI>(a, true, st);
        case GCFG_D4_256x256: return launch_tile<DTile<2, 2, 4, 4>, EPI>(a, false, st);
        case GCFG_D4_256x256_SK: return launch_tile<DTile<2, 2, 4, 4>, EPI>(a, true, st);
        case GCFG_D4_256x128: return launch_tile<DTile<2, 2, 4, 2>, EPI>(a, false, st);
        case GCFG_D4_256x128_SK: return launch_tile<DTile<2, 2, 4, 2>, EPI>(a, true, st);
        case GCFG_D4_192x128: return launch_tile<DTile<2, 2, 3, 2>, EPI>(a, false, st);
        case GCFG_D8_192x128: return launch_tile<DTile<2, 4, 3, 1, true>, EPI>(a, false, st);
        case GCFG_D8_192x128_SK: return launch_tile<DTile<2, 4, 3, 1, true>, EPI>(a, true, st);
        case GCFG_D8_128x128: return launch_tile<DTile<2, 4, 2, 1, true>, EPI>(a, false, st);
        case GCFG_D8_128x128_SK: return launch_tile<DTile<2, 4, 2, 1, true>, EPI>(a, true, st);
        case GCFG_D4_192x128_SK: return launch_tile<DTile<2, 2, 3, 2>, EPI>(a, true, st);
        case GCFG_D8_192x256: return launch_tile<DTile<2, 4, 3, 2, true, 5>, EPI>(a, false, st);
        case GCFG_D8_192x256_SK: return launch_tile<DTile<2, 4, 3, 2, true, 5>, EPI>(a, true, st);
        case GCFG_D4_192x256: return launch_tile<DTile<2, 2, 3, 4>, EPI>(a, false, st);
        case GCFG_D4_192x256_SK: return launch_tile<DTile<2, 2, 3, 4>, EPI>(a, true, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace

size_t gemm_sk_part_floats() { return (size_t)SK_P * 2 * 256 * 256; }

hipError_t launch_gemm_wgrad(const GemmArgs& a, bool accumulate, hipStream_t st) {
    if (a.K % 128 != 0 || a.N % 4 != 0 || a.M <= 0 || a.N <= 0 || a.ldo < a.N || !a.out_f32)
        return hipErrorInvalidValue;
    using Tl = DTile<2, 4, 2, 1, true>;
    if (accumulate)
        hipLaunchKernelGGL((gemm_wgrad_kernel<Tl, true>), dim3(SK_P), dim3(Tl::NT + 64 * WG_SW), 0, st, a);
    else
        hipLaunchKernelGGL((gemm_wgrad_kernel<Tl, false>), dim3(SK_P), dim3(Tl::NT + 64 * WG_SW), 0, st, a);
    return hipGetLastError();
}

namespace {

// Split K when the output has too few tiles to fill the CUs: S splits per
// tile, at most 8 and at least 8 k-iterations each, within the workspace;
// 1 = no split.
int split_count(const GemmArgs& a) {
    const int bn = a.K >= 8192 ? 256 : 128, bm = 128;
    const int tiles = ((a.N + bn - 1) / bn) * ((a.M + bm - 1) / bm);
    int S = 1;
    if (a.force_cfg == GCFG_AUTO && a.sk_part && tiles < 160) {
        S = std::min(std::min(SK_P / tiles, 8), a.K / 32 / 8);
        while (S > 1 && (size_t)S * a.M * a.N > a.sk_part_floats) --S;
    }
    return S;
}

// K >= 8192 (W2): 256x128 tiles as 8 waves of 16x16x32 (50.3 vs 52.9 us as 4
// waves of 32x32x16 at 7B, M = 512); otherwise 128x128 (the two forms measure
// the same there)
hipError_t launch_split_any(const GemmArgs& a, int S, hipStream_t st) {
    return a.K >= 8192 ? launch_split<DTile<4, 2, 2, 2, true>>(a, S, st) : launch_split<DTile<2, 2, 2, 2>>(a, S, st);
}

}  // namespace

hipError_t launch_gemm_partials(const GemmArgs& a, int* nsplit, hipStream_t st) {
    *nsplit = 0;
    if (a.K % 128 != 0 || a.N % 8 != 0 || a.M <= 0) return hipErrorInvalidValue;
    const int S = split_count(a);
    if (S < 2) return hipSuccess;
    const hipError_t e = launch_split_any(a, S, st);
    if (e == hipSuccess) *nsplit = S;
    return e;
}

hipError_t launch_gemm_resid_norm(const GemmArgs& a, const float* gamma, float eps, f16* xn, hipStream_t st) {
    if (a.K % 128 != 0 || a.N % 8 != 0 || a.N > 8192 || a.M <= 0 || a.ldo != a.N) return hipErrorInvalidValue;
    const int S = split_count(a);
    if (S >= 2) {
        const hipError_t e = launch_split_any(a, S, st);
        if (e != hipSuccess) return e;
        return launch_resid_norm(a.resid_in ? a.resid_in : a.out_f32, a.out_f32, a.sk_part, S, (size_t)a.M * a.N,
                                 a.alpha, gamma, eps, xn, a.M, a.N, st);
    }
    const hipError_t e = launch_epi<EPI_RESID>(a, st);
    if (e != hipSuccess || !gamma) return e;
    return launch_rmsnorm(a.out_f32, gamma, xn, a.M, a.N, eps, st, true);
}

hipError_t launch_gemm(int epi, const GemmArgs& a, hipStream_t st) {
    if (a.K % 128 != 0 || a.N % 4 != 0 || a.M <= 0) return hipErrorInvalidValue;
    switch (epi) {
        case EPI_F32: return launch_epi<EPI_F32>(a, st);
        case EPI_RESID: return launch_epi<EPI_RESID>(a, st);
        case EPI_SWIGLU:
            if (a.N % 32 != 0) return hipErrorInvalidValue;
            return launch_epi<EPI_SWIGLU>(a, st);
        case EPI_QKV:
            if (a.hd <= 0 || (a.hd & (a.hd - 1)) != 0 || a.N != 3 * a.D || a.S <= 0) return hipErrorInvalidValue;
            return launch_epi<EPI_QKV>(a, st);
        case EPI_SWIGLU_SAVE:
            if (a.N % 32 != 0 || !a.h13) return hipErrorInvalidValue;
            return launch_epi<EPI_SWIGLU_SAVE>(a, st);
        case EPI_SILU_BWD:
            if (a.N % 128 != 0 || a.ldo != a.N || !a.h13 || !a.out_f16) return hipErrorInvalidValue;
            return launch_epi<EPI_SILU_BWD>(a, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace rh
