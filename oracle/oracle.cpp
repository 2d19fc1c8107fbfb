// oracle.cpp -- CPU fp32 restatement of rustane's forward token loop.
//
// TEST INFRASTRUCTURE ONLY: the parity checker for the HIP path and the timed
// CPU baseline.  Nothing in the product (rustane_amd/, include/) links or loads
// this file.  See oracle.h for the per-function parity pins.
//
// Reference files restated here (whiskeypolitik/rustane, crates/engine/src/):
//   cpu/vdsp.rs:150-402       vDSP/cblas contracts -> portable loops below
//   cpu/embedding.rs:8-16     embedding::forward
//   cpu/rmsnorm.rs:10-40,149-183  rmsnorm::forward, forward_channel_first
//   cpu/silu.rs:37-46         silu::silu_gate
//   cpu/cross_entropy.rs:13-96    cross_entropy::forward, forward_backward_batch
//   kernels/sdpa_fwd.rs:24-247    rope_table, causal_mask, RoPE permutation, SDPA
//   kernels/ffn_fused.rs:22-160   SwiGLU FFN + DeepNet residual
//   layer.rs:4409-4624        layer::forward orchestration (alpha = 1/sqrt(2L))
//   layer.rs:1556-1567        random_vec LCG
//   full_model.rs:915-991,1603-1660  forward / forward_losses
//   full_model.rs:592-702     backward_ws (CE grad, tied-embedding grads, final norm)
//   layer.rs:7037-7407        layer::backward_into, accumulate_dw, rope_backward_inplace
//   cpu/rmsnorm.rs:185-240    rmsnorm::backward_channel_first
//   cpu/embedding.rs:34-44    embedding::backward_channel_first
//   kernels/sdpa_bwd.rs:44-300    sdpa backward graphs (probs, dP, dS, dQ, dK, dV)
//   cpu/adam.rs:95-132        AdamW step_fused;  full_model.rs:903-913 learning_rate
#include "oracle.h"

#include <cmath>
#include <cstring>
#include <vector>
#include <algorithm>
#ifdef _OPENMP
#include <omp.h>
#include <immintrin.h>
#endif

namespace {

typedef float v8 __attribute__((vector_size(32)));

inline v8 ld8(const float* p) { v8 v; std::memcpy(&v, p, sizeof(v)); return v; }
inline void st8(float* p, v8 v) { std::memcpy(p, &v, sizeof(v)); }
inline v8 bc8(float x) { return v8{x, x, x, x, x, x, x, x}; }
inline float hsum8(v8 v) {
    return ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
}

// Rounds p[0..n) through fp16 in place (round to nearest even, F16C): the
// operand precision of an fp16 device path (orc_config.fp16_operands).
void round_f16(float* p, size_t n) {
    const size_t n8 = n & ~size_t(7);
#pragma omp parallel for schedule(static) if (n > 65536)
    for (size_t i = 0; i < n8; i += 8)
        _mm256_storeu_ps(p + i, _mm256_cvtph_ps(_mm256_cvtps_ph(_mm256_loadu_ps(p + i), _MM_FROUND_TO_NEAREST_INT)));
    for (size_t i = n8; i < n; ++i) p[i] = _cvtsh_ss(_cvtss_sh(p[i], _MM_FROUND_TO_NEAREST_INT));
}
inline float r16(float x) { return _cvtsh_ss(_cvtss_sh(x, _MM_FROUND_TO_NEAREST_INT)); }

// C[M,N] += A[M,K] * B[K,N]   (all row-major with leading dims)
void gemm_nn(size_t M, size_t N, size_t K, const float* A, size_t lda, const float* B,
             size_t ldb, float* C, size_t ldc) {
    const size_t MB = 64, NB = 256, KB = 256;
    const size_t mblocks = (M + MB - 1) / MB, nblocks = (N + NB - 1) / NB;
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (size_t ib = 0; ib < mblocks; ++ib) {
        for (size_t jb = 0; jb < nblocks; ++jb) {
            const size_t i0 = ib * MB, i1 = std::min(M, i0 + MB);
            const size_t j0 = jb * NB, j1 = std::min(N, j0 + NB);
            for (size_t k0 = 0; k0 < K; k0 += KB) {
                const size_t k1 = std::min(K, k0 + KB);
                size_t i = i0;
                for (; i + 4 <= i1; i += 4) {
                    size_t j = j0;
                    for (; j + 16 <= j1; j += 16) {
                        v8 c00 = bc8(0), c01 = bc8(0), c10 = bc8(0), c11 = bc8(0);
                        v8 c20 = bc8(0), c21 = bc8(0), c30 = bc8(0), c31 = bc8(0);
                        for (size_t k = k0; k < k1; ++k) {
                            const v8 b0 = ld8(B + k * ldb + j), b1 = ld8(B + k * ldb + j + 8);
                            const v8 a0 = bc8(A[(i + 0) * lda + k]), a1 = bc8(A[(i + 1) * lda + k]);
                            const v8 a2 = bc8(A[(i + 2) * lda + k]), a3 = bc8(A[(i + 3) * lda + k]);
                            c00 += a0 * b0; c01 += a0 * b1; c10 += a1 * b0; c11 += a1 * b1;
                            c20 += a2 * b0; c21 += a2 * b1; c30 += a3 * b0; c31 += a3 * b1;
                        }
                        float* c0 = C + (i + 0) * ldc + j; float* c1 = C + (i + 1) * ldc + j;
                        float* c2 = C + (i + 2) * ldc + j; float* c3 = C + (i + 3) * ldc + j;
                        st8(c0, ld8(c0) + c00); st8(c0 + 8, ld8(c0 + 8) + c01);
                        st8(c1, ld8(c1) + c10); st8(c1 + 8, ld8(c1 + 8) + c11);
                        st8(c2, ld8(c2) + c20); st8(c2 + 8, ld8(c2 + 8) + c21);
                        st8(c3, ld8(c3) + c30); st8(c3 + 8, ld8(c3 + 8) + c31);
                    }
                    for (; j < j1; ++j)
                        for (size_t r = 0; r < 4; ++r) {
                            float s = 0.f;
                            for (size_t k = k0; k < k1; ++k) s += A[(i + r) * lda + k] * B[k * ldb + j];
                            C[(i + r) * ldc + j] += s;
                        }
                }
                for (; i < i1; ++i)
                    for (size_t k = k0; k < k1; ++k) {
                        const float a = A[i * lda + k];
                        for (size_t j = j0; j < j1; ++j) C[i * ldc + j] += a * B[k * ldb + j];
                    }
            }
        }
    }
}

// C[M,N] += A[M,K] * B[N,K]^T   (dot-product form; cblas NoTrans x Trans, beta = 1)
void gemm_nt(size_t M, size_t N, size_t K, const float* A, size_t lda, const float* B,
             size_t ldb, float* C, size_t ldc) {
    const size_t MB = 32, NB = 128;
    const size_t mblocks = (M + MB - 1) / MB, nblocks = (N + NB - 1) / NB;
    const size_t K8 = K & ~size_t(7);
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (size_t ib = 0; ib < mblocks; ++ib) {
        for (size_t jb = 0; jb < nblocks; ++jb) {
            const size_t i0 = ib * MB, i1 = std::min(M, i0 + MB);
            const size_t j0 = jb * NB, j1 = std::min(N, j0 + NB);
            for (size_t i = i0; i < i1; i += 4) {
                const size_t ri = std::min<size_t>(4, i1 - i);
                for (size_t j = j0; j < j1; j += 4) {
                    const size_t rj = std::min<size_t>(4, j1 - j);
                    if (ri == 4 && rj == 4) {
                        v8 acc[4][4];
                        for (int a = 0; a < 4; ++a)
                            for (int b = 0; b < 4; ++b) acc[a][b] = bc8(0);
                        for (size_t k = 0; k < K8; k += 8) {
                            v8 av[4], bv[4];
                            for (int a = 0; a < 4; ++a) av[a] = ld8(A + (i + a) * lda + k);
                            for (int b = 0; b < 4; ++b) bv[b] = ld8(B + (j + b) * ldb + k);
                            for (int a = 0; a < 4; ++a)
                                for (int b = 0; b < 4; ++b) acc[a][b] += av[a] * bv[b];
                        }
                        for (int a = 0; a < 4; ++a)
                            for (int b = 0; b < 4; ++b) {
                                float s = hsum8(acc[a][b]);
                                for (size_t k = K8; k < K; ++k)
                                    s += A[(i + a) * lda + k] * B[(j + b) * ldb + k];
                                C[(i + a) * ldc + j + b] += s;
                            }
                    } else {
                        for (size_t a = 0; a < ri; ++a)
                            for (size_t b = 0; b < rj; ++b) {
                                v8 acc = bc8(0);
                                for (size_t k = 0; k < K8; k += 8)
                                    acc += ld8(A + (i + a) * lda + k) * ld8(B + (j + b) * ldb + k);
                                float s = hsum8(acc);
                                for (size_t k = K8; k < K; ++k)
                                    s += A[(i + a) * lda + k] * B[(j + b) * ldb + k];
                                C[(i + a) * ldc + j + b] += s;
                            }
                    }
                }
            }
        }
    }
}

// Token-major RMSNorm with the channel-first arithmetic of
// rmsnorm::forward_channel_first (cpu/rmsnorm.rs:149-183): sum of squares in
// channel order, rms_inv = 1/sqrt(sum * (1/dim) + eps), out = (x * rms_inv) * g.
void rmsnorm_rows(const float* x, const float* g, float* out, float* rms_inv, size_t rows,
                  size_t dim, float eps) {
    const float inv_dim = 1.0f / (float)dim;
#pragma omp parallel for schedule(static)
    for (size_t s = 0; s < rows; ++s) {
        const float* xr = x + s * dim;
        float acc = 0.f;
        for (size_t d = 0; d < dim; ++d) acc += xr[d] * xr[d];
        const float r = 1.0f / std::sqrt(acc * inv_dim + eps);
        if (rms_inv) rms_inv[s] = r;
        float* o = out + s * dim;
        for (size_t d = 0; d < dim; ++d) o[d] = xr[d] * r * g[d];
    }
}

inline float sigmoid_ref(float x) { return 1.0f / (1.0f + std::exp(-x)); }

// theta = p / base^(2i/hd) in fp32 (kernels/sdpa_fwd.rs:24-39).
inline float rope_theta(size_t p, size_t i, size_t hd, float base) {
    return (float)p / std::pow(base, 2.0f * (float)i / (float)hd);
}

// Activations one layer keeps for its backward pass (the ForwardCache of
// layer.rs:79-126), token-major [n, *].
struct LayerCache {
    std::vector<float> x, xn, rms1, q, k, v, attn, x2, x2n, rms2, h1, h3, gate;
};

// Where one row's K/V go and which keys it attends to: row t is at absolute
// position pos and appends its k, v to kc/vc ([ctx, D] token-major caches) at
// pos; its attention runs over keys 0..pos of the same caches.
struct RowSlot {
    float* kc;
    float* vc;
    size_t pos;
};

// One layer over n token-major rows, row t described by slots[t].  Rows of
// one sequence share its caches (the forward and prefill: positions
// p0..p0+n-1); rows of different sequences each have their own (a batched
// decode step).  Attention over keys 0..pos is the additive -65504 causal
// mask of kernels/sdpa_fwd.rs:41-51 applied to keys 0..p0+n-1: a masked key
// contributes exp(-65504 + s - max) = 0 exactly in fp32 and never holds the
// max, so leaving it out changes no bit of the result.
void layer_rows_slots(const orc_config* cfg, const float* const* lw, float* x, size_t n,
                      const RowSlot* slots, LayerCache* cache = nullptr, bool multi_token = true) {
    const int32_t m16 = cfg->fp16_operands;
    const bool p16 = (m16 & ORC_F16_P) && multi_token;  // P.V on fp16 probabilities (prefill passes)
    const size_t D = cfg->dim, F = cfg->hidden, H = cfg->heads, hd = cfg->head_dim;
    const float alpha = 1.0f / std::sqrt(2.0f * (float)cfg->nlayers);   // layer.rs:4640
    const float scale = 1.0f / std::sqrt((float)hd);                    // sdpa_fwd.rs:70
    const float* wq = lw[0]; const float* wk = lw[1]; const float* wv = lw[2];
    const float* wo = lw[3]; const float* w1 = lw[4]; const float* w3 = lw[5];
    const float* w2 = lw[6]; const float* g1 = lw[7]; const float* g2 = lw[8];

    std::vector<float> xn(n * D), q(n * D, 0.f), k(n * D, 0.f), v(n * D, 0.f), rms1(n);
    if (cache) cache->x.assign(x, x + n * D);
    rmsnorm_rows(x, g1, xn.data(), rms1.data(), n, D, cfg->rms_eps);
    if (m16 & ORC_F16_XN) round_f16(xn.data(), n * D);
    // Q/K/V = xn^T W  (sdpa_fwd.rs:115-117)
    gemm_nn(n, D, D, xn.data(), D, wq, D, q.data(), D);
    gemm_nn(n, D, D, xn.data(), D, wk, D, k.data(), D);
    gemm_nn(n, D, D, xn.data(), D, wv, D, v.data(), D);
    // Interleaved RoPE through the permutation matrix of sdpa_fwd.rs:53-60:
    // rot[2i] = -x[2i+1], rot[2i+1] = x[2i]; x' = x*cos + rot*sin.
#pragma omp parallel for schedule(static)
    for (size_t t = 0; t < n; ++t) {
        const size_t p = slots[t].pos;
        for (size_t h = 0; h < H; ++h)
            for (size_t i = 0; i < hd / 2; ++i) {
                const float th = rope_theta(p, i, hd, cfg->rope_base);
                const float c = std::cos(th), s = std::sin(th);
                float* qr = &q[t * D + h * hd + 2 * i];
                float* kr = &k[t * D + h * hd + 2 * i];
                const float q0 = qr[0], q1 = qr[1], k0 = kr[0], k1 = kr[1];
                qr[0] = q0 * c + (-q1) * s; qr[1] = q1 * c + q0 * s;
                kr[0] = k0 * c + (-k1) * s; kr[1] = k1 * c + k0 * s;
            }
    }
    if (m16 & ORC_F16_Q) round_f16(q.data(), n * D);
    if (m16 & ORC_F16_K) round_f16(k.data(), n * D);
    if (m16 & ORC_F16_V) round_f16(v.data(), n * D);
    for (size_t t = 0; t < n; ++t) {
        std::memcpy(slots[t].kc + slots[t].pos * D, &k[t * D], D * sizeof(float));
        std::memcpy(slots[t].vc + slots[t].pos * D, &v[t * D], D * sizeof(float));
    }
    size_t nk_max = 0;
    for (size_t t = 0; t < n; ++t) nk_max = std::max(nk_max, slots[t].pos + 1);
    std::vector<float> attn(n * D, 0.f);
#pragma omp parallel
    {
        std::vector<float> sc(nk_max);
#pragma omp for collapse(2) schedule(dynamic)
        for (size_t h = 0; h < H; ++h)
            for (size_t t = 0; t < n; ++t) {
                const size_t nk = slots[t].pos + 1;
                const float* kc = slots[t].kc;
                const float* vc = slots[t].vc;
                const float* qr = &q[t * D + h * hd];
                float mx = -INFINITY;
                for (size_t t2 = 0; t2 < nk; ++t2) {
                    const float* kr = kc + t2 * D + h * hd;
                    float d = 0.f;
                    for (size_t i = 0; i < hd; ++i) d += qr[i] * kr[i];
                    const float s = d * scale;
                    sc[t2] = s;
                    mx = std::max(mx, s);
                }
                float sum = 0.f;
                for (size_t t2 = 0; t2 < nk; ++t2) { sc[t2] = std::exp(sc[t2] - mx); sum += sc[t2]; }
                const float inv = 1.0f / sum;
                float* o = &attn[t * D + h * hd];
                if (p16) {
                    // unnormalised fp16 probabilities into P.V, then / sum
                    for (size_t t2 = 0; t2 < nk; ++t2) {
                        const float p = r16(sc[t2]);
                        if (p == 0.f) continue;
                        const float* vr = vc + t2 * D + h * hd;
                        for (size_t i = 0; i < hd; ++i) o[i] += p * vr[i];
                    }
                    for (size_t i = 0; i < hd; ++i) o[i] *= inv;
                    continue;
                }
                for (size_t t2 = 0; t2 < nk; ++t2) {
                    const float p = sc[t2] * inv;
                    if (p == 0.f) continue;
                    const float* vr = vc + t2 * D + h * hd;
                    for (size_t i = 0; i < hd; ++i) o[i] += p * vr[i];
                }
            }
    }
    if (m16 & ORC_F16_ATTN) round_f16(attn.data(), n * D);
    // o = attn^T Wo, x2 = o*alpha + x  (dyn_matmul.rs:15-75, vdsp::vsma)
    std::vector<float> o(n * D, 0.f);
    gemm_nn(n, D, D, attn.data(), D, wo, D, o.data(), D);
    for (size_t i = 0; i < n * D; ++i) x[i] = o[i] * alpha + x[i];
    if (cache) {
        cache->xn = xn; cache->rms1 = rms1; cache->q = q; cache->k = k; cache->v = v;
        cache->attn = attn; cache->x2.assign(x, x + n * D);
    }
    // FFN (ffn_fused.rs:22-160): h1 = x2n W1, h3 = x2n W3, gate = silu(h1)*h3,
    // f = gate W2^T, x_next = f*alpha + x2.
    std::vector<float> x2n(n * D), h1(n * F, 0.f), h3(n * F, 0.f), rms2(n);
    rmsnorm_rows(x, g2, x2n.data(), rms2.data(), n, D, cfg->rms_eps);
    if (m16 & ORC_F16_XN2) round_f16(x2n.data(), n * D);
    gemm_nn(n, F, D, x2n.data(), D, w1, F, h1.data(), F);
    gemm_nn(n, F, D, x2n.data(), D, w3, F, h3.data(), F);
    if (cache) { cache->x2n = x2n; cache->rms2 = rms2; cache->h1 = h1; cache->h3 = h3; }
    orc_silu_gate(h1.data(), h3.data(), h1.data(), n * F);
    if (m16 & ORC_F16_GATE) round_f16(h1.data(), n * F);
    if (cache) cache->gate = h1;
    std::vector<float> f(n * D, 0.f);
    gemm_nt(n, D, F, h1.data(), F, w2, F, f.data(), D);
    for (size_t i = 0; i < n * D; ++i) x[i] = f[i] * alpha + x[i];
}

// One layer over n rows of one sequence at absolute positions p0..p0+n-1,
// its K/V cache kc/vc.
void layer_rows(const orc_config* cfg, const float* const* lw, float* x, size_t n, size_t p0,
                float* kc, float* vc, LayerCache* cache = nullptr) {
    std::vector<RowSlot> slots(n);
    for (size_t t = 0; t < n; ++t) slots[t] = RowSlot{kc, vc, p0 + t};
    layer_rows_slots(cfg, lw, x, n, slots.data(), cache, n > 1);
}

// Final RMSNorm -> tied logits (logits.fill(0); sgemm_at) -> softcap
// (full_model.rs:542-576).  xf: [n, D] token-major, logits [n, V].
void tail_logits(const orc_config* cfg, const orc_weights* w, const float* x, size_t n,
                 float* logits) {
    const size_t D = cfg->dim, V = cfg->vocab;
    std::vector<float> xf(n * D);
    rmsnorm_rows(x, w->gamma_final, xf.data(), nullptr, n, D, cfg->rms_eps);
    if (cfg->fp16_operands & ORC_F16_XF) round_f16(xf.data(), n * D);
    std::fill(logits, logits + n * V, 0.f);
    gemm_nt(n, V, D, xf.data(), D, w->embed, D, logits, V);
    if (cfg->softcap > 0.f) {
        const float c = cfg->softcap, ic = 1.0f / c;
        for (size_t i = 0; i < n * V; ++i) logits[i] = std::tanh(logits[i] * ic) * c;
    }
}

// C[M,N] += A[K,M]^T B[K,N] (accumulate_dw -> vdsp::sgemm_at, layer.rs:7368-7370,
// with token-major operands): transposed copies, then the dot-product kernel.
void gemm_tn(size_t M, size_t N, size_t K, const float* A, size_t lda, const float* B, size_t ldb,
             float* C, size_t ldc) {
    std::vector<float> at(M * K), bt(N * K);
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < M; ++i)
        for (size_t k = 0; k < K; ++k) at[i * K + k] = A[k * lda + i];
#pragma omp parallel for schedule(static)
    for (size_t j = 0; j < N; ++j)
        for (size_t k = 0; k < K; ++k) bt[j * K + k] = B[k * ldb + j];
    gemm_nt(M, N, K, at.data(), K, bt.data(), K, C, ldc);
}

// rmsnorm::backward_channel_first (cpu/rmsnorm.rs:185-240) on token-major
// rows, same arithmetic: x_hat = x * r; dgamma[d] += sum_s dy * x_hat (in
// position order); dot[s] = (sum_d (dy * g) * x_hat, channel order) / dim;
// dx = r * (dy * g - x_hat * dot).
void rmsnorm_bwd_rows(const float* dy, const float* x, const float* g, const float* rms_inv, float* dx,
                      float* dgamma, size_t rows, size_t dim) {
    const float inv_dim = 1.0f / (float)dim;
    std::vector<float> dot(rows);
#pragma omp parallel for schedule(static)
    for (size_t s = 0; s < rows; ++s) {
        float acc = 0.f;
        for (size_t d = 0; d < dim; ++d) acc += dy[s * dim + d] * g[d] * (x[s * dim + d] * rms_inv[s]);
        dot[s] = acc * inv_dim;
    }
#pragma omp parallel for schedule(static)
    for (size_t d = 0; d < dim; ++d) {
        float acc = 0.f;
        for (size_t s = 0; s < rows; ++s) acc += dy[s * dim + d] * (x[s * dim + d] * rms_inv[s]);
        dgamma[d] += acc;
    }
#pragma omp parallel for schedule(static)
    for (size_t s = 0; s < rows; ++s)
        for (size_t d = 0; d < dim; ++d) {
            const float xh = x[s * dim + d] * rms_inv[s];
            dx[s * dim + d] = rms_inv[s] * (dy[s * dim + d] * g[d] - xh * dot[s]);
        }
}

// SiLU-gate backward loop of layer::backward_into (layer.rs:7083-7104):
// sig = 1/(1 + exp(-h1)); dh3 = dg * h1 * sig; dh1 = dg * h3 * sig * (1 + h1 * (1 - sig)).
void silu_gate_bwd(const float* dg, const float* h1, const float* h3, float* dh1, float* dh3, size_t n) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) {
        const float sig = 1.0f / (1.0f + std::exp(-h1[i]));
        const float silu_val = h1[i] * sig;
        const float deriv = sig * (1.0f + h1[i] * (1.0f - sig));
        dh3[i] = dg[i] * silu_val;
        dh1[i] = dg[i] * h3[i] * deriv;
    }
}

// sdpa_bwd graphs (kernels/sdpa_bwd.rs:44-300) over token-major q, k, v, da
// [n, D] (q, k after RoPE): probabilities recomputed as in the forward (scale
// 1/sqrt(hd), additive -65504 causal mask, softmax); dV = P^T dA; dP = dA V^T;
// dS = P * (dP - rowsum(P * dP)) * scale; dQ = dS K; dK = dS^T Q.  Keys above
// the query have P = exp(-65504 + ...) = 0 exactly, so they are skipped.
void sdpa_bwd_rows(const orc_config* cfg, size_t n, const float* q, const float* k, const float* v,
                   const float* da, float* dq, float* dk, float* dv) {
    const size_t D = cfg->dim, H = cfg->heads, hd = cfg->head_dim;
    const float scale = 1.0f / std::sqrt((float)hd);
    std::fill(dq, dq + n * D, 0.f);
    std::fill(dk, dk + n * D, 0.f);
    std::fill(dv, dv + n * D, 0.f);
#pragma omp parallel for schedule(dynamic)
    for (size_t h = 0; h < H; ++h) {
        std::vector<float> p(n), dp(n);
        for (size_t t = 0; t < n; ++t) {
            const float* qr = q + t * D + h * hd;
            const float* ar = da + t * D + h * hd;
            float mx = -INFINITY;
            for (size_t t2 = 0; t2 <= t; ++t2) {
                const float* kr = k + t2 * D + h * hd;
                float d = 0.f;
                for (size_t i = 0; i < hd; ++i) d += qr[i] * kr[i];
                p[t2] = d * scale;
                mx = std::max(mx, p[t2]);
            }
            float sum = 0.f;
            for (size_t t2 = 0; t2 <= t; ++t2) { p[t2] = std::exp(p[t2] - mx); sum += p[t2]; }
            const float inv = 1.0f / sum;
            float pdp = 0.f;
            for (size_t t2 = 0; t2 <= t; ++t2) {
                p[t2] *= inv;
                const float* vr = v + t2 * D + h * hd;
                float d = 0.f;
                for (size_t i = 0; i < hd; ++i) d += ar[i] * vr[i];
                dp[t2] = d;
                pdp += p[t2] * d;
            }
            float* dqr = dq + t * D + h * hd;
            for (size_t t2 = 0; t2 <= t; ++t2) {
                const float ds = p[t2] * (dp[t2] - pdp) * scale;
                const float* kr = k + t2 * D + h * hd;
                float* dkr = dk + t2 * D + h * hd;
                float* dvr = dv + t2 * D + h * hd;
                for (size_t i = 0; i < hd; ++i) {
                    dqr[i] += ds * kr[i];
                    dkr[i] += ds * qr[i];
                    dvr[i] += p[t2] * ar[i];
                }
            }
        }
    }
}

// rope_backward_inplace (layer.rs:7389-7407): the inverse rotation,
// d[2i] = c*d0 + s*d1, d[2i+1] = -s*d0 + c*d1, rows at positions 0..n-1.
void rope_bwd_rows(const orc_config* cfg, float* dx, size_t n) {
    const size_t D = cfg->dim, H = cfg->heads, hd = cfg->head_dim;
#pragma omp parallel for schedule(static)
    for (size_t t = 0; t < n; ++t)
        for (size_t h = 0; h < H; ++h)
            for (size_t i = 0; i < hd / 2; ++i) {
                const float th = rope_theta(t, i, hd, cfg->rope_base);
                const float c = std::cos(th), sn = std::sin(th);
                float* r = dx + t * D + h * hd + 2 * i;
                const float d0 = r[0], d1 = r[1];
                r[0] = c * d0 + sn * d1;
                r[1] = -sn * d0 + c * d1;
            }
}

// layer::backward_into (layer.rs:7037-7366) for one sequence, token-major:
// dy [n, D] -> dx_out [n, D]; gradients accumulate into lg[9] (RSTK order).
void layer_backward_rows(const orc_config* cfg, const float* const* lw, const LayerCache& c,
                         const float* dy, float* const* lg, float* dx_out, size_t n) {
    const size_t D = cfg->dim, F = cfg->hidden;
    const float alpha = 1.0f / std::sqrt(2.0f * (float)cfg->nlayers);  // layer.rs:7054
    const float* wq = lw[0]; const float* wk = lw[1]; const float* wv = lw[2];
    const float* wo = lw[3]; const float* w1 = lw[4]; const float* w3 = lw[5];
    const float* w2 = lw[6]; const float* g1 = lw[7]; const float* g2 = lw[8];
    // 1-3: dffn = alpha dy; dsilu = dffn W2 (W2 [D, F] out x in); SiLU-gate backward
    std::vector<float> dffn(n * D), dg(n * F, 0.f), dh1(n * F), dh3(n * F);
    for (size_t i = 0; i < n * D; ++i) dffn[i] = dy[i] * alpha;
    gemm_nn(n, F, D, dffn.data(), D, w2, F, dg.data(), F);
    silu_gate_bwd(dg.data(), c.h1.data(), c.h3.data(), dh1.data(), dh3.data(), n * F);
    // 4-5: dx_ffn = dh1 W1^T + dh3 W3^T; dW3 += x2n^T dh3
    std::vector<float> dxf(n * D, 0.f);
    gemm_nt(n, D, F, dh1.data(), F, w1, F, dxf.data(), D);
    gemm_nt(n, D, F, dh3.data(), F, w3, F, dxf.data(), D);
    gemm_tn(D, F, n, c.x2n.data(), D, dh3.data(), F, lg[5], F);
    // 6: RMSNorm2 backward, dx2 += dy
    std::vector<float> dx2(n * D);
    rmsnorm_bwd_rows(dxf.data(), c.x2.data(), g2, c.rms2.data(), dx2.data(), lg[8], n, D);
    for (size_t i = 0; i < n * D; ++i) dx2[i] = dx2[i] + dy[i];
    // 7: da = (alpha dx2) Wo^T (Wo [q_dim, D] in x out)
    std::vector<float> dx2s(n * D), da(n * D, 0.f);
    for (size_t i = 0; i < n * D; ++i) dx2s[i] = dx2[i] * alpha;
    gemm_nt(n, D, D, dx2s.data(), D, wo, D, da.data(), D);
    // 9: dWo += attn^T dx2s; dW2 += dffn^T gate
    gemm_tn(D, D, n, c.attn.data(), D, dx2s.data(), D, lg[3], D);
    gemm_tn(D, F, n, dffn.data(), D, c.gate.data(), F, lg[6], F);
    // 10: attention backward; dW1 += x2n^T dh1
    std::vector<float> dq(n * D), dk(n * D), dv(n * D);
    sdpa_bwd_rows(cfg, n, c.q.data(), c.k.data(), c.v.data(), da.data(), dq.data(), dk.data(), dv.data());
    gemm_tn(D, F, n, c.x2n.data(), D, dh1.data(), F, lg[4], F);
    // 11: RoPE backward on dq, dk
    rope_bwd_rows(cfg, dq.data(), n);
    rope_bwd_rows(cfg, dk.data(), n);
    // 13: dx_attn = dq Wq^T; dx_kv = dk Wk^T + dv Wv^T; dWq/dWk/dWv += xn^T d{q,k,v}
    std::vector<float> dxa(n * D, 0.f), dxkv(n * D, 0.f);
    gemm_nt(n, D, D, dq.data(), D, wq, D, dxa.data(), D);
    gemm_nt(n, D, D, dk.data(), D, wk, D, dxkv.data(), D);
    gemm_nt(n, D, D, dv.data(), D, wv, D, dxkv.data(), D);
    gemm_tn(D, D, n, c.xn.data(), D, dq.data(), D, lg[0], D);
    gemm_tn(D, D, n, c.xn.data(), D, dk.data(), D, lg[1], D);
    gemm_tn(D, D, n, c.xn.data(), D, dv.data(), D, lg[2], D);
    // 15-16: RMSNorm1 backward of the merged input gradient; dx = dx_rms1 + dx2
    std::vector<float> dxm(n * D), dxr(n * D);
    for (size_t i = 0; i < n * D; ++i) dxm[i] = dxa[i] + dxkv[i];
    rmsnorm_bwd_rows(dxm.data(), c.x.data(), g1, c.rms1.data(), dxr.data(), lg[7], n, D);
    for (size_t i = 0; i < n * D; ++i) dx_out[i] = dxr[i] + dx2[i];
}

}  // namespace

struct orc_kv {
    int max_ctx, pos, nlayers;
    size_t dim;
    std::vector<std::vector<float>> k, v;  // per layer [max_ctx, D]
};

extern "C" {

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

// vDSP_vsma: out = a*s + b  (cpu/vdsp.rs:217-231)
void orc_vsma(const float* a, float s, const float* b, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = a[i] * s + b[i];
}
// vDSP_vsub: out = b - a  (cpu/vdsp.rs:183-197, KAT vsub_order :427-434)
void orc_vsub(const float* a, const float* b, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = b[i] - a[i];
}
// vDSP_mtrans: a is [m, n] -> c is [n, m]  (cpu/vdsp.rs:295-311; a_cols == n, c_cols == m)
void orc_mtrans(const float* a, size_t a_cols, float* c, size_t c_cols, size_t m, size_t n) {
    if (a_cols != n || c_cols != m) return;
    for (size_t i = 0; i < m; ++i)
        for (size_t j = 0; j < n; ++j) c[j * m + i] = a[i * n + j];
}
// cblas_sgemm(RowMajor, NoTrans, Trans, alpha 1, beta 1): C += A B^T  (cpu/vdsp.rs:351-376)
void orc_sgemm_at(const float* a, size_t m, size_t k, const float* b, size_t n, float* c) {
    gemm_nt(m, n, k, a, k, b, k, c, n);
}

// random_vec (layer.rs:1556-1567, full_model.rs:1473-1484): wrapping u64 LCG,
// seed = 42 + n, r = ((s >> 32) as f32 / u32::MAX as f32) * 2 - 1, x = r * scale.
void orc_random_vec(float* out, size_t n, float scale) {
    uint64_t s = 42u + (uint64_t)n;
    const float umax = (float)4294967295u;
    for (size_t i = 0; i < n; ++i) {
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        const float r = ((float)(uint32_t)(s >> 32) / umax) * 2.0f - 1.0f;
        out[i] = r * scale;
    }
}

// embedding::forward (cpu/embedding.rs:8-16): out[s] = table[ids[s]], [S, D].
void orc_embedding_forward(const float* table, size_t dim, const uint32_t* ids, size_t seq,
                           float* out) {
    for (size_t s = 0; s < seq; ++s)
        std::memcpy(out + s * dim, table + (size_t)ids[s] * dim, dim * sizeof(float));
}

// rmsnorm::forward (cpu/rmsnorm.rs:15-40): mean_sq = sve(x*x)/dim.
float orc_rmsnorm_forward(const float* x, const float* gamma, float* out, size_t dim, float eps) {
    float acc = 0.f;
    for (size_t d = 0; d < dim; ++d) acc += x[d] * x[d];
    const float mean_sq = acc / (float)dim;
    const float r = 1.0f / std::sqrt(mean_sq + eps);
    for (size_t d = 0; d < dim; ++d) out[d] = (x[d] * r) * gamma[d];
    return r;
}

// rmsnorm::forward_channel_first (cpu/rmsnorm.rs:149-183), x/out [dim, seq].
void orc_rmsnorm_forward_channel_first(const float* x, const float* gamma, float* out,
                                       float* rms_inv, size_t dim, size_t seq, float eps) {
    for (size_t s = 0; s < seq; ++s) rms_inv[s] = 0.f;
    for (size_t d = 0; d < dim; ++d)
        for (size_t s = 0; s < seq; ++s) rms_inv[s] += x[d * seq + s] * x[d * seq + s];
    const float inv_dim = 1.0f / (float)dim;
    for (size_t s = 0; s < seq; ++s) rms_inv[s] = 1.0f / std::sqrt(rms_inv[s] * inv_dim + eps);
    for (size_t d = 0; d < dim; ++d)
        for (size_t s = 0; s < seq; ++s) out[d * seq + s] = x[d * seq + s] * rms_inv[s] * gamma[d];
}

// silu::silu_gate (cpu/silu.rs:37-46): out = gate * sigmoid(gate) * up.
void orc_silu_gate(const float* gate, const float* up, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const float sig = sigmoid_ref(gate[i]);
        out[i] = gate[i] * sig * up[i];
    }
}

// cross_entropy::forward (cpu/cross_entropy.rs:13-38).
float orc_cross_entropy_forward(const float* logits, size_t vocab, uint32_t target, float* log_sm) {
    float mx = -INFINITY;
    for (size_t i = 0; i < vocab; ++i) mx = std::max(mx, logits[i]);
    float sum = 0.f;
    for (size_t i = 0; i < vocab; ++i) sum += std::exp(logits[i] - mx);
    const float lse = std::log(sum);
    if (log_sm)
        for (size_t i = 0; i < vocab; ++i) log_sm[i] = (logits[i] - mx) - lse;
    return -((logits[target] - mx) - lse);
}

// cross_entropy::forward_backward_batch (cpu/cross_entropy.rs:58-96): returns the
// total loss (not averaged); dlogits = (softmax - onehot) * inv_seq.
float orc_cross_entropy_forward_backward_batch(const float* logits, const uint32_t* targets,
                                               size_t seq, size_t vocab, float* dlogits,
                                               float inv_seq) {
    float total = 0.f;
    std::vector<float> ex(vocab);
    for (size_t s = 0; s < seq; ++s) {
        const float* l = logits + s * vocab;
        float mx = -INFINITY;
        for (size_t i = 0; i < vocab; ++i) mx = std::max(mx, l[i]);
        float sum = 0.f;
        for (size_t i = 0; i < vocab; ++i) { ex[i] = std::exp(l[i] - mx); sum += ex[i]; }
        const uint32_t t = targets[s];
        total -= (l[t] - mx) - std::log(sum);
        if (dlogits) {
            float* d = dlogits + s * vocab;
            const float is = 1.0f / sum;
            for (size_t i = 0; i < vocab; ++i) d[i] = ex[i] * is;
            d[t] -= 1.0f;
        }
    }
    if (dlogits)
        for (size_t i = 0; i < seq * vocab; ++i) dlogits[i] *= inv_seq;
    return total;
}

// rope_table (kernels/sdpa_fwd.rs:24-39): cos/sin [seq, hd], pairs duplicated.
void orc_rope_table(size_t seq, size_t hd, float base, float* cos_buf, float* sin_buf) {
    for (size_t p = 0; p < seq; ++p)
        for (size_t i = 0; i < hd / 2; ++i) {
            const float th = rope_theta(p, i, hd, base);
            const float c = std::cos(th), s = std::sin(th);
            cos_buf[p * hd + 2 * i] = c; cos_buf[p * hd + 2 * i + 1] = c;
            sin_buf[p * hd + 2 * i] = s; sin_buf[p * hd + 2 * i + 1] = s;
        }
}

// sdpa_fwd graph (kernels/sdpa_fwd.rs:62-287), channel-first in and out.
void orc_sdpa_fwd(const orc_config* cfg, size_t seq, const float* xnorm, const float* wq,
                  const float* wk, const float* wv, float* attn_out, float* q_rope,
                  float* k_rope, float* v) {
    const size_t D = cfg->dim, H = cfg->heads, hd = cfg->head_dim;
    const float scale = 1.0f / std::sqrt((float)hd);
    std::vector<float> xt(seq * D), q(seq * D, 0.f), k(seq * D, 0.f), vv(seq * D, 0.f);
    orc_mtrans(xnorm, seq, xt.data(), D, D, seq);
    gemm_nn(seq, D, D, xt.data(), D, wq, D, q.data(), D);
    gemm_nn(seq, D, D, xt.data(), D, wk, D, k.data(), D);
    gemm_nn(seq, D, D, xt.data(), D, wv, D, vv.data(), D);
    std::vector<float> cb(seq * hd), sb(seq * hd);
    orc_rope_table(seq, hd, cfg->rope_base, cb.data(), sb.data());
    for (size_t t = 0; t < seq; ++t)
        for (size_t h = 0; h < H; ++h)
            for (size_t i = 0; i < hd; i += 2) {
                const size_t c0 = t * D + h * hd + i;
                const float q0 = q[c0], q1 = q[c0 + 1], k0 = k[c0], k1 = k[c0 + 1];
                q[c0] = q0 * cb[t * hd + i] + (-q1) * sb[t * hd + i];
                q[c0 + 1] = q1 * cb[t * hd + i + 1] + q0 * sb[t * hd + i + 1];
                k[c0] = k0 * cb[t * hd + i] + (-k1) * sb[t * hd + i];
                k[c0 + 1] = k1 * cb[t * hd + i + 1] + k0 * sb[t * hd + i + 1];
            }
    std::vector<float> at(seq * D, 0.f);
    std::vector<float> sc(seq);
    for (size_t h = 0; h < H; ++h)
        for (size_t t = 0; t < seq; ++t) {
            float mx = -INFINITY;
            for (size_t t2 = 0; t2 < seq; ++t2) {
                float d = 0.f;
                for (size_t i = 0; i < hd; ++i) d += q[t * D + h * hd + i] * k[t2 * D + h * hd + i];
                float s = d * scale + (t2 > t ? -65504.0f : 0.0f);
                sc[t2] = s;
                mx = std::max(mx, s);
            }
            float sum = 0.f;
            for (size_t t2 = 0; t2 < seq; ++t2) { sc[t2] = std::exp(sc[t2] - mx); sum += sc[t2]; }
            for (size_t t2 = 0; t2 < seq; ++t2) {
                const float p = sc[t2] / sum;
                for (size_t i = 0; i < hd; ++i) at[t * D + h * hd + i] += p * vv[t2 * D + h * hd + i];
            }
        }
    orc_mtrans(at.data(), D, attn_out, seq, seq, D);
    if (q_rope) orc_mtrans(q.data(), D, q_rope, seq, seq, D);
    if (k_rope) orc_mtrans(k.data(), D, k_rope, seq, seq, D);
    if (v) orc_mtrans(vv.data(), D, v, seq, seq, D);
}

// layer::forward (layer.rs:4409-4624), channel-first x [D, S] -> x_next [D, S].
void orc_layer_forward(const orc_config* cfg, size_t seq, const float* const* lw, const float* x,
                       float* x_next) {
    const size_t D = cfg->dim;
    std::vector<float> xt(seq * D), kc(seq * D), vc(seq * D);
    orc_mtrans(x, seq, xt.data(), D, D, seq);
    layer_rows(cfg, lw, xt.data(), seq, 0, kc.data(), vc.data());
    orc_mtrans(xt.data(), D, x_next, seq, seq, D);
}

int orc_forward(const orc_config* cfg, const orc_weights* w, const uint32_t* tokens,
                const uint32_t* targets, int batch, int seq, float* logits_out,
                float* token_losses_out, float* mean_loss_out) {
    if (!cfg || !w || !tokens || batch <= 0 || seq <= 0) return -1;
    const size_t D = cfg->dim, V = cfg->vocab, S = seq;
    for (size_t i = 0; i < (size_t)batch * S; ++i)
        if (tokens[i] >= V || (targets && targets[i] >= V)) return -2;
    std::vector<float> x(S * D), kc(S * D), vc(S * D), logits(S * V);
    for (int b = 0; b < batch; ++b) {
        const uint32_t* tk = tokens + (size_t)b * S;
        orc_embedding_forward(w->embed, D, tk, S, x.data());
        for (int l = 0; l < cfg->nlayers; ++l)
            layer_rows(cfg, w->layers + 9 * l, x.data(), S, 0, kc.data(), vc.data());
        tail_logits(cfg, w, x.data(), S, logits.data());
        if (logits_out) std::memcpy(logits_out + (size_t)b * S * V, logits.data(), S * V * sizeof(float));
        if (targets) {
            const uint32_t* tg = targets + (size_t)b * S;
            float total = 0.f;
            std::vector<float> per(S);
#pragma omp parallel for schedule(static)
            for (size_t s = 0; s < S; ++s)
                per[s] = orc_cross_entropy_forward_backward_batch(logits.data() + s * V, tg + s, 1, V,
                                                                  nullptr, 1.0f);
            for (size_t s = 0; s < S; ++s) total += per[s];
            if (token_losses_out) std::memcpy(token_losses_out + (size_t)b * S, per.data(), S * sizeof(float));
            if (mean_loss_out) mean_loss_out[b] = total / (float)S;
        }
    }
    return 0;
}

// full_model::forward + backward_ws (full_model.rs:915-991, 592-702) for
// `batch` independent sequences; every gradient accumulates (+=).
int orc_forward_backward(const orc_config* cfg, const orc_weights* w, const uint32_t* tokens,
                         const uint32_t* targets, int batch, int seq, float loss_scale,
                         const orc_grads* g, float* mean_loss_out) {
    if (!cfg || !w || !g || !tokens || !targets || batch <= 0 || seq <= 0) return -1;
    const size_t D = cfg->dim, V = cfg->vocab, S = seq;
    const int L = cfg->nlayers;
    for (size_t i = 0; i < (size_t)batch * S; ++i)
        if (tokens[i] >= V || targets[i] >= V) return -2;
    std::vector<float> x(S * D), kc(S * D), vc(S * D), xf(S * D), rmsf(S), logits(S * V), t(S * V);
    std::vector<float> dl(S * V), dxf(S * D), dy(S * D), dxo(S * D);
    std::vector<LayerCache> caches(L);
    for (int b = 0; b < batch; ++b) {
        const uint32_t* tk = tokens + (size_t)b * S;
        const uint32_t* tg = targets + (size_t)b * S;
        orc_embedding_forward(w->embed, D, tk, S, x.data());
        for (int l = 0; l < L; ++l)
            layer_rows(cfg, w->layers + 9 * l, x.data(), S, 0, kc.data(), vc.data(), &caches[l]);
        // finalize_logits_and_loss (full_model.rs:283-329); t = tanh(z / c) when softcapped
        rmsnorm_rows(x.data(), w->gamma_final, xf.data(), rmsf.data(), S, D, cfg->rms_eps);
        std::fill(logits.begin(), logits.end(), 0.f);
        gemm_nt(S, V, D, xf.data(), D, w->embed, D, logits.data(), V);
        const bool cap = cfg->softcap > 0.f;
        if (cap) {
            const float c = cfg->softcap, ic = 1.0f / c;
            for (size_t i = 0; i < S * V; ++i) { t[i] = std::tanh(logits[i] * ic); logits[i] = t[i] * c; }
        }
        std::vector<float> per(S);
#pragma omp parallel for schedule(static)
        for (size_t s = 0; s < S; ++s)
            per[s] = orc_cross_entropy_forward_backward_batch(logits.data() + s * V, tg + s, 1, V,
                                                              dl.data() + s * V, 1.0f / (float)S);
        float total = 0.f;
        for (size_t s = 0; s < S; ++s) total += per[s];
        if (mean_loss_out) mean_loss_out[b] = total / (float)S;
        // backward_ws steps 1-2: dl = dlogits * loss_scale (* (1 - t^2) when softcapped)
        for (size_t i = 0; i < S * V; ++i)
            dl[i] = cap ? dl[i] * loss_scale * (1.0f - t[i] * t[i]) : dl[i] * loss_scale;
        // 3a: dx_final = dl E; 3b: dembed += dl^T x_final
        std::fill(dxf.begin(), dxf.end(), 0.f);
        gemm_nn(S, D, V, dl.data(), V, w->embed, D, dxf.data(), D);
        gemm_tn(V, D, S, dl.data(), V, xf.data(), D, g->dembed, D);
        // 4: final RMSNorm backward (x_prenorm = x after the last layer)
        rmsnorm_bwd_rows(dxf.data(), x.data(), w->gamma_final, rmsf.data(), dy.data(), g->dgamma_final, S, D);
        // 5: layers in reverse
        for (int l = L - 1; l >= 0; --l) {
            layer_backward_rows(cfg, w->layers + 9 * l, caches[l], dy.data(), g->layers + 9 * l, dxo.data(), S);
            std::swap(dy, dxo);
        }
        // 6: embedding::backward_channel_first (cpu/embedding.rs:34-44), positions in order
        for (size_t s = 0; s < S; ++s)
            for (size_t d = 0; d < D; ++d) g->dembed[(size_t)tk[s] * D + d] += dy[s * D + d];
    }
    return 0;
}

void orc_rmsnorm_backward_channel_first(const float* dy, const float* x, const float* gamma,
                                        const float* rms_inv, float* dx, float* dgamma, size_t dim,
                                        size_t seq) {
    // channel-first [dim, seq] in and out, through the token-major routine
    std::vector<float> dyt(seq * dim), xt(seq * dim), dxt(seq * dim);
    orc_mtrans(dy, seq, dyt.data(), dim, dim, seq);
    orc_mtrans(x, seq, xt.data(), dim, dim, seq);
    rmsnorm_bwd_rows(dyt.data(), xt.data(), gamma, rms_inv, dxt.data(), dgamma, seq, dim);
    orc_mtrans(dxt.data(), dim, dx, seq, seq, dim);
}

void orc_silu_gate_backward(const float* dgate, const float* h1, const float* h3, float* dh1,
                            float* dh3, size_t n) {
    silu_gate_bwd(dgate, h1, h3, dh1, dh3, n);
}

void orc_sdpa_backward(const orc_config* cfg, size_t seq, const float* q, const float* k,
                       const float* v, const float* da, float* dq, float* dk, float* dv) {
    sdpa_bwd_rows(cfg, seq, q, k, v, da, dq, dk, dv);
}

void orc_rope_backward(const orc_config* cfg, float* dx, size_t seq) { rope_bwd_rows(cfg, dx, seq); }

float orc_powi(float b, uint32_t t) {
    float r = 1.0f, x = b;
    for (uint32_t e = t; e; e >>= 1) {
        if (e & 1u) r *= x;
        x *= x;
    }
    return r;
}

// step_fused (cpu/adam.rs:95-132), one element at a time in the reference's
// operation order (the library is built with -ffp-contract=off, like rustc).
void orc_adam_step_fused(float* param, const float* grad, float* m, float* v, size_t n, uint32_t t, float lr,
                         float beta1, float beta2, float eps, float weight_decay, float grad_scale) {
    const float bc1 = 1.0f / (1.0f - orc_powi(beta1, t));
    const float bc2 = 1.0f / (1.0f - orc_powi(beta2, t));
    const float omb1 = 1.0f - beta1, omb2 = 1.0f - beta2;
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) {
        const float g = (grad ? grad[i] : 0.0f) * grad_scale;
        const float mi = beta1 * m[i] + omb1 * g;
        const float vi = beta2 * v[i] + omb2 * g * g;
        m[i] = mi;
        v[i] = vi;
        const float m_hat = mi * bc1;
        const float v_hat = vi * bc2;
        const float update = m_hat / (std::sqrt(v_hat) + eps);
        param[i] -= lr * (update + weight_decay * param[i]);
    }
}

float orc_svesq(const float* x, size_t n) {
    float s = 0.f;
    for (size_t i = 0; i < n; ++i) s += x[i] * x[i];
    return s;
}

// learning_rate (full_model.rs:903-913).
float orc_learning_rate(uint32_t step, float max_lr, float min_lr_frac, uint32_t warmup_steps,
                        uint32_t total_steps) {
    if (step < warmup_steps) return max_lr * (float)(step + 1) / (float)warmup_steps;
    const float decay = (float)(step - warmup_steps) / (float)(total_steps - warmup_steps);
    const float min_lr = max_lr * min_lr_frac;
    return min_lr + 0.5f * (1.0f + std::cos(3.14159265358979323846f * decay)) * (max_lr - min_lr);
}

orc_kv* orc_kv_create(const orc_config* cfg, int max_ctx) {
    if (!cfg || max_ctx <= 0) return nullptr;
    orc_kv* kv = new orc_kv;
    kv->max_ctx = max_ctx; kv->pos = 0; kv->nlayers = cfg->nlayers; kv->dim = cfg->dim;
    kv->k.assign(cfg->nlayers, std::vector<float>((size_t)max_ctx * cfg->dim, 0.f));
    kv->v.assign(cfg->nlayers, std::vector<float>((size_t)max_ctx * cfg->dim, 0.f));
    return kv;
}
void orc_kv_destroy(orc_kv* kv) { delete kv; }
int orc_kv_pos(const orc_kv* kv) { return kv ? kv->pos : -1; }

static int run_rows(const orc_config* cfg, const orc_weights* w, orc_kv* kv, const uint32_t* tokens,
                    int n, float* last_logits) {
    const size_t D = cfg->dim, V = cfg->vocab;
    if (kv->pos + n > kv->max_ctx) return -3;
    for (int i = 0; i < n; ++i) if (tokens[i] >= V) return -2;
    std::vector<float> x((size_t)n * D);
    orc_embedding_forward(w->embed, D, tokens, n, x.data());
    for (int l = 0; l < cfg->nlayers; ++l)
        layer_rows(cfg, w->layers + 9 * l, x.data(), n, kv->pos, kv->k[l].data(), kv->v[l].data());
    kv->pos += n;
    if (last_logits) tail_logits(cfg, w, x.data() + (size_t)(n - 1) * D, 1, last_logits);
    return 0;
}

int orc_prefill(const orc_config* cfg, const orc_weights* w, orc_kv* kv, const uint32_t* tokens,
                int len, float* last_logits) {
    if (!cfg || !w || !kv || !tokens || len <= 0) return -1;
    kv->pos = 0;
    return run_rows(cfg, w, kv, tokens, len, last_logits);
}

int orc_decode_step(const orc_config* cfg, const orc_weights* w, orc_kv* kv, uint32_t token,
                    float* logits_out) {
    if (!cfg || !w || !kv) return -1;
    std::vector<float> lg(cfg->vocab);
    float* out = logits_out ? logits_out : lg.data();
    const int rc = run_rows(cfg, w, kv, &token, 1, out);
    if (rc) return rc;
    int best = 0;
    for (int i = 1; i < cfg->vocab; ++i) if (out[i] > out[best]) best = i;
    return best;
}


// B independent sequences, each with its own cache, run through the layers
// as one set of rows (the GEMMs see all of them at once; attention stays per
// sequence): rows r = b*n + t of sequence b at position kvs[b]->pos + t.
static int run_rows_batch(const orc_config* cfg, const orc_weights* w, orc_kv* const* kvs, int B,
                          const uint32_t* tokens, int n, float* last_logits) {
    const size_t D = cfg->dim, V = cfg->vocab;
    for (int b = 0; b < B; ++b)
        if (!kvs[b] || kvs[b]->pos + n > kvs[b]->max_ctx || kvs[b]->nlayers != cfg->nlayers) return -3;
    const size_t rows = (size_t)B * n;
    for (size_t i = 0; i < rows; ++i) if (tokens[i] >= V) return -2;
    std::vector<float> x(rows * D);
    orc_embedding_forward(w->embed, D, tokens, rows, x.data());
    std::vector<RowSlot> slots(rows);
    for (int l = 0; l < cfg->nlayers; ++l) {
        for (int b = 0; b < B; ++b)
            for (int t = 0; t < n; ++t)
                slots[(size_t)b * n + t] = RowSlot{kvs[b]->k[l].data(), kvs[b]->v[l].data(),
                                                   (size_t)(kvs[b]->pos + t)};
        layer_rows_slots(cfg, w->layers + 9 * l, x.data(), rows, slots.data(), nullptr, n > 1);
    }
    for (int b = 0; b < B; ++b) kvs[b]->pos += n;
    if (last_logits) {
        std::vector<float> xl((size_t)B * D);
        for (int b = 0; b < B; ++b)
            std::memcpy(&xl[(size_t)b * D], &x[((size_t)b * n + n - 1) * D], D * sizeof(float));
        tail_logits(cfg, w, xl.data(), B, last_logits);
    }
    return 0;
}

int orc_prefill_batch(const orc_config* cfg, const orc_weights* w, orc_kv* const* kvs, int B,
                      const uint32_t* tokens, int len, float* last_logits) {
    if (!cfg || !w || !kvs || !tokens || B <= 0 || len <= 0) return -1;
    for (int b = 0; b < B; ++b)
        if (kvs[b]) kvs[b]->pos = 0;
    return run_rows_batch(cfg, w, kvs, B, tokens, len, last_logits);
}

int orc_decode_step_batch(const orc_config* cfg, const orc_weights* w, orc_kv* const* kvs, int B,
                          const uint32_t* tokens, float* logits_out, int32_t* argmax_out) {
    if (!cfg || !w || !kvs || !tokens || !logits_out || B <= 0) return -1;
    const int rc = run_rows_batch(cfg, w, kvs, B, tokens, 1, logits_out);
    if (rc) return rc;
    if (argmax_out)
        for (int b = 0; b < B; ++b) {
            const float* r = logits_out + (size_t)b * cfg->vocab;
            int best = 0;
            for (int i = 1; i < cfg->vocab; ++i) if (r[i] > r[best]) best = i;
            argmax_out[b] = best;
        }
    return 0;
}

}  // extern "C"
