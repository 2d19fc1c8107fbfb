// rh_attn.hip -- causal attention for the forward (prefill) and decode paths.
//
// Semantics follow the sdpaFwd graph (kernels/sdpa_fwd.rs:62-287): scores =
// (q_rope . k_rope) * 1/sqrt(hd), keys after the query masked out (the
// reference adds -65504, whose exp is exactly 0 after the row max is
// subtracted), row softmax, P.V.  Q/K are RoPE'd by the QKV GEMM epilogue.
//
// Prefill: flash-style online softmax.  A block owns 64 queries of one
// (sequence, head), 4 waves x 16 queries, and walks 64-key blocks up to the
// causal limit with K and V resident in LDS (head dim 128: moved by DMA into
// swizzled [key][hd] tiles, V^T fragments by the transposing LDS read; head
// dim 64: staged through registers, V stored transposed).  The MFMAs compute the
// transposed problem (S^T = K Q^T, O^T = V^T P^T) so that every lane owns one
// query column throughout: the softmax row statistics, the rescaling of O and
// the fp16 P operand all stay lane-local, and the row reductions are two
// xor-shuffles over the 4 lane groups that share a query.
//
// Decode: split-context.  One block per (sequence, head, 128-position chunk)
// scores its chunk with 16-byte K loads (hd/8 lanes per position) and keeps
// (max, sum, P.V) partials; a small kernel merges them.  The position is read
// from device memory so the step can be replayed as a graph.
#include <type_traits>

#include "rh_device.h"
#include "rh_kernels.h"

namespace rh {
namespace {

constexpr float LOG2E = 1.4426950408889634f;

template <int HD, int PF>
__global__ __launch_bounds__(256) void attn_prefill_kernel(const f16* __restrict__ Q,
                                                           const f16* __restrict__ Kc,
                                                           const f16* __restrict__ Vc,
                                                           f16* __restrict__ out, float* __restrict__ lse,
                                                           int H, int S, int ctx, float scale_log2) {
    constexpr int KB = 64;             // keys per block
    constexpr int LDK = HD + 8;        // padded K row (halfs)
    constexpr int LDV = KB + 8;        // padded V^T row (halfs)
    constexpr int NKK = HD / 32;       // 32-wide k steps for Q.K
    constexpr int NHT = HD / 16;       // 16-row hd tiles of O^T
    __shared__ __attribute__((aligned(16))) f16 sK[KB * LDK];
    __shared__ __attribute__((aligned(16))) f16 sVt[HD * LDV];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4;
    const int nqt = (S + 63) / 64;
    const int qt = nqt - 1 - (int)blockIdx.x;  // longest rows first
    const int h = blockIdx.y, b = blockIdx.z;
    const int q0 = qt * 64;
    const int qi = q0 + w * 16 + (lane & 15);  // this lane's query
    const size_t bh = (size_t)b * H + h;
    const f16* Kb = Kc + bh * ctx * HD;
    const f16* Vb = Vc + bh * ctx * HD;

    f16x8 qf[NKK];
    {
        const f16x8 z = {};
        const f16* qp = Q + (bh * S + (qi < S ? qi : 0)) * HD + 8 * g;
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) qf[kk] = qi < S ? *(const f16x8*)(qp + kk * 32) : z;
    }
    f32x4 o[NHT];
#pragma unroll
    for (int j = 0; j < NHT; ++j) o[j] = f32x4{};
    float m_run = -INFINITY, l_run = 0.f;

    const int kend = min(S, q0 + 64);
    const int nkb = (kend + KB - 1) / KB;
    // K/V of key block kb + PF are loaded into register set kb % PF while
    // block kb is computed; set kb % PF goes to LDS at the top of iteration
    // kb.  The LDS-only barriers leave those loads in flight, so each has PF
    // iterations of compute to land.
    constexpr int KL = KB * HD / 8 / 256;           // 16-byte K loads per thread
    constexpr int VL = (KB / 2) * (HD / 8) / 256;   // key pairs per thread
    f16x8 rk[PF][KL], rva[PF][VL], rvb[PF][VL];
    // Keys past the sequence read the last row instead (branch-free): their
    // scores are masked to -inf, so they add p = 0 times a finite V row.
    auto gload = [&](int k0, int set) {
#pragma unroll
        for (int p = 0; p < KL; ++p) {
            const int c = tid + 256 * p, row = c / (HD / 8), col = (c % (HD / 8)) * 8;
            const int key = min(k0 + row, S - 1);
            rk[set][p] = *(const f16x8*)(Kb + (size_t)key * HD + col);
        }
#pragma unroll
        for (int p = 0; p < VL; ++p) {
            const int u = tid + 256 * p, kp = u & 31, col = (u >> 5) * 8;
            const int key0 = min(k0 + 2 * kp, S - 1), key1 = min(k0 + 2 * kp + 1, S - 1);
            rva[set][p] = *(const f16x8*)(Vb + (size_t)key0 * HD + col);
            rvb[set][p] = *(const f16x8*)(Vb + (size_t)key1 * HD + col);
        }
    };
#pragma unroll
    for (int u = 0; u < PF; ++u)
        if (u < nkb) gload(u * KB, u);
    for (int base = 0; base < nkb; base += PF) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
        const int kb = base + u;
        if (kb >= nkb) break;  // uniform
        const int k0 = kb * KB;
        lds_barrier();
        // K block -> sK[key][hd]
#pragma unroll
        for (int p = 0; p < KL; ++p) {
            const int c = tid + 256 * p, row = c / (HD / 8), col = (c % (HD / 8)) * 8;
            *(f16x8*)&sK[row * LDK + col] = rk[u][p];
        }
        // V block -> sVt[hd][key], two keys per 32-bit LDS store
#pragma unroll
        for (int p = 0; p < VL; ++p) {
            const int v = tid + 256 * p, kp = v & 31, col = (v >> 5) * 8;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                typedef f16 f16x2 __attribute__((ext_vector_type(2)));
                *(f16x2*)&sVt[(col + e) * LDV + 2 * kp] = f16x2{rva[u][p][e], rvb[u][p][e]};
            }
        }
        lds_barrier();
        if (kb + PF < nkb) gload(k0 + PF * KB, u);

        // S^T tiles: chunk c (32 keys) x half u; tile row r -> key
        // 32c + 8(r/4) + 4u + r%4, so lane group g holds keys 32c + 8g + (0..7).
        // All K fragments are read before the MFMAs and all V fragments
        // before the softmax, so the LDS latency is paid once per block
        // (read-one-use-one would serialise it under every MFMA).
        f16x8 kf[2][2][NKK];
        {
            const int r = lane & 15;
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int krow = 32 * c + 8 * (r >> 2) + 4 * u + (r & 3);
#pragma unroll
                    for (int kk = 0; kk < NKK; ++kk)
                        kf[c][u][kk] = *(const f16x8*)&sK[krow * LDK + kk * 32 + 8 * g];
                }
        }
        __builtin_amdgcn_sched_barrier(0);
        f32x4 sc[2][2];
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int u = 0; u < 2; ++u) sc[c][u] = f32x4{};
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk)
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int u = 0; u < 2; ++u) sc[c][u] = mfma16(kf[c][u][kk], qf[kk], sc[c][u]);
        __builtin_amdgcn_sched_barrier(0);
        f16x8 vf[2][NHT];
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int j = 0; j < NHT; ++j)
                vf[c][j] = *(const f16x8*)&sVt[(16 * j + (lane & 15)) * LDV + 32 * c + 8 * g];
        __builtin_amdgcn_sched_barrier(0);
        // Online softmax in the log2 domain on raw scores: the 1/sqrt(hd)
        // scale rides in the exponent's fma.  The running max only moves when
        // a row's block max exceeds it by more than 8 (log2 units); exp2 of
        // (score - stale max) then stays <= 256, as exact in the fp16 P operand
        // as values <= 1, and the O rescale (32 multiplies) is skipped for the
        // whole wave in the common case.  Only the block holding the diagonal
        // (or the sequence end) runs the mask: key offsets within the block
        // above lim are out.
        const int lim = min(qi, S - 1) - k0 - 8 * g;
        auto block_max = [&](auto diag) {
            float mx = -INFINITY;
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if constexpr (decltype(diag)::value)
                            if (32 * c + 4 * u + i > lim) sc[c][u][i] = -INFINITY;
                        mx = fmaxf(mx, sc[c][u][i]);
                    }
            return mx;
        };
        float mloc = (k0 + KB > q0 || k0 + KB > S) ? block_max(std::true_type{}) : block_max(std::false_type{});
        mloc = xrow_max4(mloc);
        mloc *= scale_log2;
        if (__any(mloc > m_run + 8.0f)) {
            const float m_new = fmaxf(m_run, mloc);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int j = 0; j < NHT; ++j) o[j] *= alpha;
            m_run = m_new;
        }
        float psum = 0.f;
        f16x8 pf[2];
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[c][u][i], scale_log2, -m_run));
                    psum += p;
                    pf[c][4 * u + i] = (f16)p;
                }
        l_run += psum;
        // O^T[hd][q] += V^T[hd][keys] . P^T[keys][q]
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int j = 0; j < NHT; ++j) o[j] = mfma16(vf[c][j], pf[c], o[j]);
    }
    }
    const float lt = xrow_sum4(l_run);
    if (qi < S) {
        // Log-sum-exp of the scaled scores in the log2 domain, for the
        // backward pass: P[q][k] = exp2(score * scale_log2 - lse[q]).
        if (lse && g == 0) lse[bh * S + qi] = m_run + log2f(lt);
        // token-major [B*S][H*HD] in fragment order (the Wo GEMM's operand layout)
        const float inv = 1.0f / lt;
        const int row = b * S + qi;
#pragma unroll
        for (int j = 0; j < NHT; ++j)
            *(f16x4*)(out + frag_off(row, h * HD + 16 * j + 4 * g, H * HD)) =
                f16x4{(f16)(o[j][0] * inv), (f16)(o[j][1] * inv), (f16)(o[j][2] * inv), (f16)(o[j][3] * inv)};
    }
}

// Prefill attention for head dim 128 with K and V moved global -> LDS by DMA
// (global_load_lds_dwordx4) through an NS-stage pipeline, so no VGPRs or LDS
// store instructions stage them and NS - 1 key blocks are in flight while
// one is computed.  The math, the MFMA arrangement (S^T = K Q^T, O^T = V^T P^T,
// one query column per lane) and the lazy rescale are those of
// attn_prefill_kernel; what changes is how the operands reach the MFMAs:
//   * K and V sit in LDS in their natural [key][hd] order (256 B rows), as the
//     DMA writes 1 KB per instruction (4 rows).  16-byte chunks are XOR
//     swizzled per row by permuting each lane's global address, so the
//     fragment reads below hit distinct banks: K chunk c of row k is stored at
//     c ^ swz_k(k), V chunk c at c ^ swz_v(k).
//   * V^T fragments come from the gfx950 transposing LDS read
//     ds_read_b64_tr_b16: within each 16-lane group, result element e of lane
//     m is element m % 4 of the 8 bytes read by lane 4e + m / 4.  Lane l of
//     group g therefore reads hd 16j + 4(l % 4) .. +3 of key 32c + 8g + 4h +
//     (l % 16) / 4, and gets V[32c + 8g + 4h + e][16j + l % 16] for e = 0..3:
//     two reads (h = 0, 1) make the 8-key k slice of the O^T MFMA's A operand.

// NG = 2: two groups of 4 waves share the block's 64 queries and split its
// key blocks (group G takes blocks G, G + 2, ...), each through its own half
// of every stage's LDS arrays; the groups step in lockstep under the block's
// barrier (a group without a block in the last step only joins the barrier)
// and group 1 hands its (m, l, o) to group 0 through LDS at the end.  This
// halves the serial key-block chain of the heavy (late) query tiles, which
// sets the kernel time when there are few (sequence, head) pairs.
template <int NS, int NG>
__global__ __launch_bounds__(256 * NG) void attn_prefill_dma_kernel(const f16* __restrict__ Q,
                                                                    const f16* __restrict__ Kc,
                                                                    const f16* __restrict__ Vc,
                                                                    f16* __restrict__ out, float* __restrict__ lse,
                                                                    int H, int S, int ctx, float scale_log2) {
    constexpr int HD = 128, KB = 64, NKK = HD / 32, NHT = HD / 16;
    constexpr int TILE = KB * HD;  // halves of one K or V block (16 KB)
    static_assert(NS == 2 || NS == 3, "2 or 3 stages");
    static_assert(NG == 1 || (NG == 2 && NS == 2), "two groups run the 2-stage pipeline");
    // One LDS array per stage, operand and group, each addressed from its
    // start: the compiler's wait-count pass then knows a stage's reads do not
    // alias the DMA filling another stage.  (With one array it drains every
    // DMA before the first read; with a group's stages at an offset inside a
    // shared array it drains the DMA just issued for the next key block
    // before each transposing V read.)
    __shared__ __attribute__((aligned(1024))) f16 sK0[TILE], sV0[TILE], sK1[TILE], sV1[TILE], sK2[TILE], sV2[TILE];
    f16 *gK0 = sK0, *gV0 = sV0, *gK1 = sK1, *gV1 = sV1;  // group 1's stages (NG == 2)
    if constexpr (NG == 2) {
        __shared__ __attribute__((aligned(1024))) f16 tK0[TILE], tV0[TILE], tK1[TILE], tV1[TILE];
        gK0 = tK0; gV0 = tV0; gK1 = tK1; gV1 = tV1;
    }

    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, r = lane & 15;
    // wave within its group, group (scalar, so the group's branches are uniform)
    const int w = __builtin_amdgcn_readfirstlane((tid >> 6) & 3);
    const int grp = NG == 1 ? 0 : __builtin_amdgcn_readfirstlane(tid >> 8);
    const int nqt = (S + 63) / 64;
    // 1-D grid: the query tiles of one (sequence, head) are consecutive
    // logical tiles, which xcd_remap puts on one XCD, so that XCD's L2 serves
    // their shared K and V (measured 13.1 -> 11.5 us at 7B, B 1, S 512; 144 ->
    // 98 us at B 16); within a head the longest rows come first
    const int t = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    const int bhi = t / nqt, qt = nqt - 1 - t % nqt;
    const int h = bhi % H, b = bhi / H;
    const int q0 = qt * 64;
    const int qi = q0 + w * 16 + r;
    const size_t bh = (size_t)b * H + h;
    const f16* Kb = Kc + bh * ctx * HD;
    const f16* Vb = Vc + bh * ctx * HD;

    f16x8 qf[NKK];
    {
        const f16x8 z = {};
        const f16* qp = Q + (bh * S + (qi < S ? qi : 0)) * HD + 8 * g;
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) qf[kk] = qi < S ? *(const f16x8*)(qp + kk * 32) : z;
    }
    f32x4 o[NHT];
#pragma unroll
    for (int j = 0; j < NHT; ++j) o[j] = f32x4{};
    float m_run = -INFINITY, l_run = 0.f;

    const int kend = min(S, q0 + 64);
    const int nkb = (kend + KB - 1) / KB;
    // The group's k loop, instantiated per group so that every stage buffer
    // it names is a compile-time choice of array.
    auto group_loop = [&](auto G) {
        constexpr int GI = decltype(G)::value;
        auto kbuf = [&](auto I) -> f16* {
            if constexpr (decltype(I)::value == 0) return GI ? gK0 : sK0;
            else if constexpr (decltype(I)::value == 1) return GI ? gK1 : sK1;
            else return sK2;
        };
        auto vbuf = [&](auto I) -> f16* {
            if constexpr (decltype(I)::value == 0) return GI ? gV0 : sV0;
            else if constexpr (decltype(I)::value == 1) return GI ? gV1 : sV1;
            else return sV2;
        };
        // Wave w moves 1 KB units w, w + 4, w + 8, w + 12 of the K block and of the
        // V block (8 DMA instructions per stage); unit i holds rows 4i..4i+3, lane L
        // row 4i + L/16 and stored chunk L%16.  Keys past the sequence read the
        // last row (masked below).
        auto issue = [&](int kb, auto ST) {
            const int k0 = kb * KB;
            f16* dk = kbuf(ST);
            f16* dv = vbuf(ST);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int i = w + 4 * t, row = 4 * i + (lane >> 4);
                const size_t key = (size_t)min(k0 + row, S - 1);
                __builtin_amdgcn_global_load_lds((const void*)(Kb + key * HD + 8 * ((lane & 15) ^ swz_k(row))),
                                                 (__attribute__((address_space(3))) void*)(dk + i * 512), 16, 0, 0);
                __builtin_amdgcn_global_load_lds((const void*)(Vb + key * HD + 8 * ((lane & 15) ^ swz_v(row))),
                                                 (__attribute__((address_space(3))) void*)(dv + i * 512), 16, 0, 0);
            }
        };
        if (GI < nkb) issue(GI, std::integral_constant<int, 0>{});  // nkb >= 1
        if constexpr (NS == 3)
            if (nkb > 1) issue(1, std::integral_constant<int, 1>{});

        // one key block on stage ST (a compile-time buffer choice); with two
        // groups, kb is this group's block (kb >= nkb: a barrier-only step)
        auto step = [&](int kb, auto ST) {
            constexpr int cur = decltype(ST)::value;
            const int k0 = kb * KB;
            // this wave's 8 DMAs of stage kb have landed when at most 8 per stage
            // issued after it are outstanding; the barrier publishes every wave's
            // and retires every wave's reads of stage kb - 1, whose buffer the
            // next issue refills
            const int ahead = min(NS - 2, nkb - 1 - kb);
            if (ahead >= 2) wait_vm<16>();
            else if (ahead == 1) wait_vm<8>();
            else wait_vm<0>();
            lds_barrier();
            if (kb + NG * (NS - 1) < nkb) issue(kb + NG * (NS - 1), std::integral_constant<int, (cur + NS - 1) % NS>{});
            if (NG > 1 && kb >= nkb) return;  // group-uniform
            const f16* sK = kbuf(ST);
            const f16* sV = vbuf(ST);

            f16x8 kf[2][2][NKK];
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int krow = 32 * c + 8 * (r >> 2) + 4 * u + (r & 3);
#pragma unroll
                    for (int kk = 0; kk < NKK; ++kk)
                        kf[c][u][kk] = *(const f16x8*)&sK[krow * HD + 8 * ((4 * kk + g) ^ swz_k(krow))];
                }
            __builtin_amdgcn_sched_barrier(0);
            f32x4 sc[2][2];
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int u = 0; u < 2; ++u) sc[c][u] = f32x4{};
#pragma unroll
            for (int kk = 0; kk < NKK; ++kk)
#pragma unroll
                for (int c = 0; c < 2; ++c)
#pragma unroll
                    for (int u = 0; u < 2; ++u) sc[c][u] = mfma16(kf[c][u][kk], qf[kk], sc[c][u]);
            __builtin_amdgcn_sched_barrier(0);
            f16x8 vf[2][NHT];
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int j = 0; j < NHT; ++j) {
                    const int ch = 2 * j + ((lane & 3) >> 1);
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        const int key = 32 * c + 8 * g + 4 * hh + (r >> 2);
                        const f16* a = &sV[key * HD + 8 * (ch ^ swz_v(key)) + 4 * (lane & 1)];
                        const s16x4 t = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                            (__attribute__((address_space(3))) s16x4*)a);
                        const f16x4 tv = __builtin_bit_cast(f16x4, t);
#pragma unroll
                        for (int e = 0; e < 4; ++e) vf[c][j][4 * hh + e] = tv[e];
                    }
                }
            __builtin_amdgcn_sched_barrier(0);
            const int lim = min(qi, S - 1) - k0 - 8 * g;
            auto block_max = [&](auto diag) {
                float mx = -INFINITY;
#pragma unroll
                for (int c = 0; c < 2; ++c)
#pragma unroll
                    for (int u = 0; u < 2; ++u)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            if constexpr (decltype(diag)::value)
                                if (32 * c + 4 * u + i > lim) sc[c][u][i] = -INFINITY;
                            mx = fmaxf(mx, sc[c][u][i]);
                        }
                return mx;
            };
            float mloc = (k0 + KB > q0 || k0 + KB > S) ? block_max(std::true_type{}) : block_max(std::false_type{});
            mloc = xrow_max4(mloc);
            mloc *= scale_log2;
            if (__any(mloc > m_run + 8.0f)) {
                const float m_new = fmaxf(m_run, mloc);
                const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
                l_run *= alpha;
#pragma unroll
                for (int j = 0; j < NHT; ++j) o[j] *= alpha;
                m_run = m_new;
            }
            float psum = 0.f;
            f16x8 pf[2];
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[c][u][i], scale_log2, -m_run));
                        psum += p;
                        pf[c][4 * u + i] = (f16)p;
                    }
            l_run += psum;
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int j = 0; j < NHT; ++j) o[j] = mfma16(vf[c][j], pf[c], o[j]);
        };
        if constexpr (NG == 1) {
            for (int kb0 = 0; kb0 < nkb; kb0 += NS) {
                step(kb0, std::integral_constant<int, 0>{});
                if (kb0 + 1 < nkb) step(kb0 + 1, std::integral_constant<int, 1>{});
                if constexpr (NS == 3)
                    if (kb0 + 2 < nkb) step(kb0 + 2, std::integral_constant<int, 2>{});
            }
        } else {
            // both groups take ceil(nkb / 2) steps (block-uniform count)
            const int nst = (nkb + 1) / 2;
            for (int s0 = 0; s0 < nst; s0 += 2) {
                step(2 * s0 + GI, std::integral_constant<int, 0>{});
                if (s0 + 1 < nst) step(2 * (s0 + 1) + GI, std::integral_constant<int, 1>{});
            }
        }
    };
    if constexpr (NG == 1) {
        group_loop(std::integral_constant<int, 0>{});
    } else {
        if (grp == 0) group_loop(std::integral_constant<int, 0>{});
        else group_loop(std::integral_constant<int, 1>{});
        // group 1 hands (m, l, o) to group 0 through the (now idle) stage buffers
        lds_barrier();
        // o of hd tiles 0..3 in sK0, 4..7 in sK1: [4 waves][16 values][64 lanes]
        auto xo = [&](int j, int e) -> float& {
            return ((float*)(j < NHT / 2 ? sK0 : sK1))[(w * 16 + 4 * (j % (NHT / 2)) + e) * 64 + lane];
        };
        float* xm = (float*)sV0;  // [4 waves][2][64 lanes]
        if (grp == 1) {
#pragma unroll
            for (int j = 0; j < NHT; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) xo(j, e) = o[j][e];
            xm[(w * 2) * 64 + lane] = m_run;
            xm[(w * 2 + 1) * 64 + lane] = l_run;
        }
        lds_barrier();
        if (grp == 1) return;
        const float m1 = xm[(w * 2) * 64 + lane], l1 = xm[(w * 2 + 1) * 64 + lane];
        const float mm = fmaxf(m_run, m1);
        const float c0 = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - mm);
        const float c1 = m1 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - mm);
        l_run = l_run * c0 + l1 * c1;
#pragma unroll
        for (int j = 0; j < NHT; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) o[j][e] = o[j][e] * c0 + xo(j, e) * c1;
        m_run = mm;
    }
    const float lt = xrow_sum4(l_run);
    if (qi < S) {
        if (lse && g == 0) lse[bh * S + qi] = m_run + log2f(lt);
        const float inv = 1.0f / lt;
        const int row = b * S + qi;
#pragma unroll
        for (int j = 0; j < NHT; ++j)
            *(f16x4*)(out + frag_off(row, h * HD + 16 * j + 4 * g, H * HD)) =
                f16x4{(f16)(o[j][0] * inv), (f16)(o[j][1] * inv), (f16)(o[j][2] * inv), (f16)(o[j][3] * inv)};
    }
}

// Sum over the N (8 or 16) consecutive lanes of a DPP row, in every one of
// them: quad pairs, quad halves, then the mirrored halves of 8 and of 16.
// Each step adds a lane's value to its partner's, so partners hold equal sums
// (addition commutes) and the N lanes end bitwise equal.  DPP moves stay in
// the VALU; __shfl_xor goes through the LDS crossbar (ds_bpermute).
#define RH_DPP_STEP(v, ctrl) \
    ((v) + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (v)), (ctrl), 0xF, 0xF, true)))
template <int N>
__device__ __forceinline__ float row_sum_dpp(float v) {
    static_assert(N == 8 || N == 16, "8 or 16 lanes");
    v = RH_DPP_STEP(v, 0xB1);   // quad_perm [1, 0, 3, 2]
    v = RH_DPP_STEP(v, 0x4E);   // quad_perm [2, 3, 0, 1]
    v = RH_DPP_STEP(v, 0x141);  // row_half_mirror: lane i <-> 7 - i within 8
    if constexpr (N == 16) v = RH_DPP_STEP(v, 0x140);  // row_mirror: lane i <-> 15 - i
    return v;
}
#undef RH_DPP_STEP

// Decode attention: one block per (chunk, head, sequence), 4 waves.  A chunk
// covers `per` consecutive positions (0: ceil(positions / chunks), computed
// on the device from the current position), split evenly over the 4 waves.
// Small batches split the context into many short chunks so the grid fills
// the chip and every load of a block is in flight at once; large batches
// give each (head, sequence) one block, which then writes the fp16 output
// itself (no partials, no merge).  Lane = LPP * slot + j: j owns dims
// 8j..8j+7 of one position (16-byte K/V loads), so a wave covers
// SL = 64 / LPP positions per load instruction and STEP = SL * NP positions
// per iteration.  K and V are streamed with nontemporal loads, double-
// buffered in registers over iterations: the next iteration's loads are in
// flight while the current one computes.  Each lane slot keeps an online-
// softmax state (m, l, o); slots merge with shuffles and the 4 waves through
// LDS once at the end.  Positions past the wave's range read a clamped
// (valid) row and are masked; a chunk past the current position stores an
// empty partial (m = -inf, l = 0, o = 0).
// Offset of element (token b, column c) of a decode output with C columns:
// row-major, or fragment order (frag) for the decode GEMV's x_frag input.
__device__ __forceinline__ size_t dec_out_off(int b, int c, int C, int frag) {
    return frag ? frag_off(b, c, C) : (size_t)b * C + c;
}

template <int HD, int NP>
__global__ __launch_bounds__(256) void attn_decode_kernel(const f16* __restrict__ Q,
                                                          const f16* __restrict__ Kc,
                                                          const f16* __restrict__ Vc,
                                                          const int* __restrict__ pos,
                                                          float* part_m, float* part_l,
                                                          float* part_o, f16* out, int H, int ctx,
                                                          int per_fixed, float scale, int out_frag) {
    constexpr int LPP = HD / 8, SL = 64 / LPP, STEP = SL * NP;
    __shared__ float sm_[4], sl_[4];
    __shared__ float so_[4][HD];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int j = lane % LPP, slot = lane / LPP;
    const int chunk = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int nch = gridDim.x;
    const int nctx = min(*pos + 1, ctx);  // a position past the cache attends over the whole cache
    const int per = per_fixed > 0 ? per_fixed : (nctx + nch - 1) / nch;
    const int t0 = min(chunk * per, nctx), t1 = min(nctx, t0 + per);
    const size_t bh = (size_t)b * H + h;
    if (t0 >= t1) {  // chunk past the current position (only with fixed chunks, nch > 1)
        const size_t pidx = bh * nch + chunk;
        if (tid == 0) { part_m[pidx] = -INFINITY; part_l[pidx] = 0.f; }
        if (tid < HD) part_o[pidx * HD + tid] = 0.f;
        return;
    }
    const int wper = (t1 - t0 + 3) / 4;
    const int w0 = min(t0 + w * wper, t1), w1 = min(t1, w0 + wper);
    const f16x8 qv = *(const f16x8*)(Q + bh * HD + 8 * j);
    const f16* Kb = Kc + bh * ctx * HD + 8 * j;
    const f16* Vb = Vc + bh * ctx * HD + 8 * j;
    // iterations of this wave (wave-uniform); an empty range loads row 0
    const int niter = (w1 - w0 + STEP - 1) / STEP;
    const int last = w1 > w0 ? w1 - 1 : 0;
    float m = -INFINITY, l = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    f16x8 ka[NP], va[NP], kb[NP], vb[NP];
    auto load = [&](int it, f16x8 (&kr)[NP], f16x8 (&vr)[NP]) {
        const int tb = w0 + it * STEP + slot;
#pragma unroll
        for (int i = 0; i < NP; ++i) kr[i] = ld_stream((const f16x8*)(Kb + (size_t)min(tb + i * SL, last) * HD));
#pragma unroll
        for (int i = 0; i < NP; ++i) vr[i] = ld_stream((const f16x8*)(Vb + (size_t)min(tb + i * SL, last) * HD));
    };
    auto step = [&](int it, const f16x8 (&kr)[NP], const f16x8 (&vr)[NP]) {
        const int tb = w0 + it * STEP + slot;
        float sc[NP];
        float mloc = -INFINITY;
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            float d = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) d += (float)qv[e] * (float)kr[i][e];
            d = row_sum_dpp<LPP>(d);
            sc[i] = tb + i * SL < w1 ? d * scale : -INFINITY;
            mloc = fmaxf(mloc, sc[i]);
        }
        const float mn = fmaxf(m, mloc);
        if (mn == -INFINITY) return;  // nothing live in this slot yet
        const float c = m == -INFINITY ? 0.f : __expf(m - mn);
        l *= c;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] *= c;
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const float p = sc[i] == -INFINITY ? 0.f : __expf(sc[i] - mn);
            l += p;
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] += p * (float)vr[i][e];
        }
        m = mn;
    };
    load(0, ka, va);
    if (niter <= 1) {  // wave-uniform: a short range needs no second buffer
        step(0, ka, va);
    } else {
        for (int it = 0; it < niter; it += 2) {
            load(it + 1, kb, vb);
            step(it, ka, va);
            load(it + 2, ka, va);
            step(it + 1, kb, vb);
        }
    }
    // merge the SL slots of the wave (lanes with equal j): each step combines
    // lane pairs (l, l ^ off) as (lower lane, upper lane), so both lanes of a
    // pair compute the same expression; off 16 and 32 move their operands with
    // the row-swap VALU ops, smaller offsets with shuffles
#pragma unroll
    for (int off = LPP; off < 64; off <<= 1) {
        float mp[2], lp[2], op[8][2];
        auto pair = [&](float v, float (&pr)[2]) {
            if (off == 16 || off == 32) {
                pr[0] = v; pr[1] = v;
                if (off == 16) swap_rows16(pr[0], pr[1]);
                else swap_halves32(pr[0], pr[1]);
            } else {
                const float x = __shfl_xor(v, off, RH_WAVE);
                const bool lo = (lane & off) == 0;
                pr[0] = lo ? v : x;
                pr[1] = lo ? x : v;
            }
        };
        pair(m, mp);
        pair(l, lp);
#pragma unroll
        for (int e = 0; e < 8; ++e) pair(o[e], op[e]);
        const float nm = fmaxf(mp[0], mp[1]);
        const float ca = mp[0] == -INFINITY ? 0.f : __expf(mp[0] - nm);
        const float cb = mp[1] == -INFINITY ? 0.f : __expf(mp[1] - nm);
        l = lp[0] * ca + lp[1] * cb;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = op[e][0] * ca + op[e][1] * cb;
        m = nm;
    }
    if (slot == 0) {
        if (j == 0) { sm_[w] = m; sl_[w] = l; }
#pragma unroll
        for (int e = 0; e < 8; ++e) so_[w][8 * j + e] = o[e];
    }
    __syncthreads();
    if (tid < HD) {
        const float M = fmaxf(fmaxf(sm_[0], sm_[1]), fmaxf(sm_[2], sm_[3]));
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float c = sm_[v] == -INFINITY ? 0.f : __expf(sm_[v] - M);
            L += sl_[v] * c;
            O += so_[v][tid] * c;
        }
        if (nch == 1) {
            out[dec_out_off(b, h * HD + tid, H * HD, out_frag)] = (f16)(O / L);
        } else {
            const size_t pidx = bh * nch + chunk;
            part_o[pidx * HD + tid] = O;
            if (tid == 0) { part_m[pidx] = M; part_l[pidx] = L; }
        }
    }
}

// Merges the chunk partials of one (head, sequence), MAXCH chunks per round:
// all loads of a round are issued before the first use, so the block pays
// one round trip per MAXCH partials (written by blocks on other XCDs);
// empty chunks carry m = -inf, l = 0, o = 0.
template <int MAXCH>
__global__ void attn_merge_kernel(const float* part_m, const float* part_l, const float* part_o,
                                  f16* out, int H, int HD, int nch, int out_frag) {
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    const size_t bh = (size_t)b * H + h;
    const float* pm = part_m + bh * nch;
    const float* pl = part_l + bh * nch;
    const float* po = part_o + bh * nch * HD + d;
    float M = -INFINITY, l = 0.f, o = 0.f;
    for (int c0 = 0; c0 < nch; c0 += MAXCH) {
        float mv[MAXCH], lv[MAXCH], ov[MAXCH];
#pragma unroll
        for (int c = 0; c < MAXCH; ++c) {
            const int cc = min(c0 + c, nch - 1);
            mv[c] = pm[cc];
            lv[c] = pl[cc];
            ov[c] = po[(size_t)cc * HD];
        }
        float Mn = M;
#pragma unroll
        for (int c = 0; c < MAXCH; ++c) Mn = c0 + c < nch ? fmaxf(Mn, mv[c]) : Mn;
        if (Mn == -INFINITY) continue;  // nothing live yet
        const float r = M == -INFINITY ? 0.f : __expf(M - Mn);
        l *= r;
        o *= r;
#pragma unroll
        for (int c = 0; c < MAXCH; ++c) {
            const float wgt = (c0 + c >= nch || mv[c] == -INFINITY) ? 0.f : __expf(mv[c] - Mn);
            l += lv[c] * wgt;
            o += ov[c] * wgt;
        }
        M = Mn;
    }
    out[dec_out_off(b, h * HD + d, H * HD, out_frag)] = (f16)(o / l);
}

}  // namespace

// Two key-splitting wave groups per block while the grid is at most about
// two blocks per CU, where the heaviest query tile's serial chain sets the
// time; one group (two blocks per CU) once the grid is larger.
int attn_prefill_groups(int B, int H, int S) {
    return (long long)B * H * ((S + 63) / 64) <= 512 ? 2 : 1;
}

hipError_t launch_attn_prefill(const f16* q, const f16* k, const f16* v, f16* out, int B, int H,
                               int S, int hd, int ctx, hipStream_t st, float* lse) {
    const dim3 grid((S + 63) / 64, H, B);
    const float sl2 = (1.0f / sqrtf((float)hd)) * LOG2E;
    constexpr int PF = 1;  // deeper register prefetch measured no faster
    // hd 128: DMA pipeline with 2 stages (64 KB of LDS, two blocks per CU; 3
    // stages measured slower at every shape for the lost occupancy)
    if (hd == 128 && attn_prefill_groups(B, H, S) == 2)
        hipLaunchKernelGGL((attn_prefill_dma_kernel<2, 2>), dim3((S + 63) / 64 * H * B), dim3(512), 0, st, q, k, v,
                           out, lse, H, S, ctx, sl2);
    else if (hd == 128)
        hipLaunchKernelGGL((attn_prefill_dma_kernel<2, 1>), dim3((S + 63) / 64 * H * B), dim3(256), 0, st, q, k, v,
                           out, lse, H, S, ctx, sl2);
    else if (hd == 64)
        hipLaunchKernelGGL((attn_prefill_kernel<64, PF>), grid, dim3(256), 0, st, q, k, v, out, lse, H, S, ctx, sl2);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

// Small batches: chunks of ATTN_DEC_CHUNK positions over the whole cache
// (ceil(ctx / ATTN_DEC_CHUNK) blocks per (head, sequence), those past the
// current position exit at once).  Once B * H blocks fill the chip: one
// chunk per (head, sequence).  Measured at 7B, ctx 2176: B 1 7.3 us +
// 3.5 us merge (128-position chunks; 8 or 16 whole-context chunks took
// 9.2 - 9.6 us), B 16 86 us (one chunk) vs 91 (128-position chunks).
int attn_decode_chunks(int B, int H, int ctx) {
    return B * H >= 256 ? 1 : (ctx + ATTN_DEC_CHUNK - 1) / ATTN_DEC_CHUNK;
}

hipError_t launch_attn_decode(const f16* q, const f16* k, const f16* v, const int* pos,
                              float* part_m, float* part_l, float* part_o, f16* out, int B, int H,
                              int hd, int ctx, hipStream_t st, int nch, bool out_frag) {
    if (B < 1 || H < 1 || ctx < 1) return hipErrorInvalidValue;
    if (out_frag && (B > 16 || (H * hd) % 128 != 0)) return hipErrorInvalidValue;
    const int of = out_frag ? 1 : 0;
    int per = 0;  // whole context split over nch chunks (forced nch: tuning)
    if (nch <= 0) {
        nch = attn_decode_chunks(B, H, ctx);
        if (nch > 1) per = ATTN_DEC_CHUNK;
    }
    const dim3 grid(nch, H, B);
    const float scale = 1.0f / sqrtf((float)hd);
    if (hd == 128)
        hipLaunchKernelGGL((attn_decode_kernel<128, 8>), grid, dim3(256), 0, st, q, k, v, pos, part_m, part_l,
                           part_o, out, H, ctx, per, scale, of);
    else if (hd == 64)
        hipLaunchKernelGGL((attn_decode_kernel<64, 4>), grid, dim3(256), 0, st, q, k, v, pos, part_m, part_l,
                           part_o, out, H, ctx, per, scale, of);
    else
        return hipErrorInvalidValue;
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || nch == 1) return e;
    // one round of loads covers contexts up to 32 * ATTN_DEC_CHUNK positions
    hipLaunchKernelGGL((attn_merge_kernel<32>), dim3(H, B), dim3(hd), 0, st, part_m, part_l, part_o, out, H, hd,
                       nch, of);
    return hipGetLastError();
}

}  // namespace rh
