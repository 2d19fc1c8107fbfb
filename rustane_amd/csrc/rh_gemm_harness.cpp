// rh_gemm_harness.cpp -- test harness over the prefill GEMM family.
//
// Runs one launch_gemm / launch_gemm_resid_norm on host buffers with a forced
// tile configuration, so parity tests can sweep every configuration (data
// parallel, stream-K, split-K, the 16x16x32 tile) and epilogue on ragged
// shapes that the shape heuristic would not pick.  Not part of the library's
// interface (include/rustane_hip.h): it is linked into its own
// librustane_gemm_harness.so, which only the tests load.
//
// Host operands are fp16 bit patterns already in fragment order (frag_off),
// W with ceil(N/16)*16 rows and X with ceil(M/16)*16 rows of K halves.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <vector>

#include "rh_kernels.h"

namespace {

struct Dev {
    std::vector<void*> ptrs;
    ~Dev() {
        for (void* p : ptrs) (void)hipFree(p);
    }
    template <class T>
    T* alloc(size_t elems) {
        void* p = nullptr;
        if (hipMalloc(&p, elems * sizeof(T) + 256) != hipSuccess) return nullptr;
        ptrs.push_back(p);
        return (T*)p;
    }
};

int up16(int x) { return (x + 15) / 16 * 16; }

}  // namespace

extern "C" {

// epi: 0 fp32 store (alpha scale when nonzero, softcap when > 0), 1 residual
// (io_f32 += alpha * acc), 2 SwiGLU (out_f16 = gate [M][N/2] in fragment
// order), 3 QKV + RoPE (q16 [B][H][S][hd], k16 / v16 [B][H][ctx][hd], rope
// [ctx][hd/2] cos/sin pairs; M = B*S, N = 3*H*hd, positions pos0 .. pos0+S-1),
// 4 SwiGLU + saved pre-activations (h13 = [2][M][N/2] row-major), 5 SiLU-gate
// backward (h13 = [2][M][N] input, out_f16 = dh1 | dh3 [M][2N] in fragment
// order).  cfg is a GemmCfg value (0 = the shape heuristic).  Returns 0 or a
// hipError_t / -1.
int rhh_gemm(int epi, int cfg, const uint16_t* wf, const uint16_t* xf, int M, int N, int K, float alpha,
             float softcap, float* io_f32, uint16_t* out_f16, uint16_t* h13, int B, int S, int H, int hd, int ctx,
             int pos0, const float* rope, uint16_t* q16, uint16_t* k16, uint16_t* v16) {
    if (M <= 0 || N <= 0 || K <= 0 || !wf || !xf) return -1;
    Dev d;
    const size_t wn = (size_t)up16(N) * K, xn = (size_t)up16(M) * K;
    f16* W = d.alloc<f16>(wn);
    f16* X = d.alloc<f16>(xn);
    const size_t skf = rh::gemm_sk_part_floats();
    float* sk = d.alloc<float>(skf);
    if (!W || !X || !sk) return -1;
    if (hipMemcpy(W, wf, wn * 2, hipMemcpyHostToDevice) != hipSuccess) return -1;
    if (hipMemcpy(X, xf, xn * 2, hipMemcpyHostToDevice) != hipSuccess) return -1;
    rh::GemmArgs a{};
    a.W = W; a.X = X; a.M = M; a.N = N; a.K = K;
    a.alpha = alpha; a.softcap = softcap;
    a.sk_part = sk; a.sk_part_floats = skf;
    a.force_cfg = cfg;
    float* of = nullptr;
    f16 *o16 = nullptr, *hh = nullptr, *dq = nullptr, *dk = nullptr, *dv = nullptr;
    size_t o16n = 0, qn = 0, kvn = 0;
    if (epi == rh::EPI_F32 || epi == rh::EPI_RESID) {
        if (!io_f32) return -1;
        of = d.alloc<float>((size_t)M * N);
        if (!of) return -1;
        if (hipMemcpy(of, io_f32, (size_t)M * N * 4, hipMemcpyHostToDevice) != hipSuccess) return -1;
        a.out_f32 = of; a.ldo = N;
    } else if (epi == rh::EPI_SWIGLU || epi == rh::EPI_SWIGLU_SAVE) {
        if (!out_f16 || N % 2) return -1;
        a.ldo = N / 2;
        o16n = (size_t)up16(M) * a.ldo;
        o16 = d.alloc<f16>(o16n);
        if (!o16 || hipMemset(o16, 0, o16n * 2) != hipSuccess) return -1;
        a.out_f16 = o16;
        if (epi == rh::EPI_SWIGLU_SAVE) {
            if (!h13) return -1;
            hh = d.alloc<f16>((size_t)2 * M * a.ldo);
            if (!hh) return -1;
            a.h13 = hh;
        }
    } else if (epi == rh::EPI_SILU_BWD) {
        if (!out_f16 || !h13) return -1;
        a.ldo = N;
        o16n = (size_t)up16(M) * 2 * N;
        o16 = d.alloc<f16>(o16n);
        f16* hin = d.alloc<f16>((size_t)2 * M * N);
        if (!o16 || !hin || hipMemset(o16, 0, o16n * 2) != hipSuccess) return -1;
        if (hipMemcpy(hin, h13, (size_t)2 * M * N * 2, hipMemcpyHostToDevice) != hipSuccess) return -1;
        a.out_f16 = o16;
        a.h13 = hin;
    } else if (epi == rh::EPI_QKV) {
        if (!rope || !q16 || !k16 || !v16 || B * S != M || N != 3 * H * hd || pos0 + S > ctx) return -1;
        qn = (size_t)B * H * S * hd;
        kvn = (size_t)B * H * ctx * hd;
        dq = d.alloc<f16>(qn); dk = d.alloc<f16>(kvn); dv = d.alloc<f16>(kvn);
        float2* dr = d.alloc<float2>((size_t)ctx * hd / 2);
        if (!dq || !dk || !dv || !dr) return -1;
        if (hipMemset(dq, 0, qn * 2) != hipSuccess || hipMemset(dk, 0, kvn * 2) != hipSuccess ||
            hipMemset(dv, 0, kvn * 2) != hipSuccess)
            return -1;
        if (hipMemcpy(dr, rope, (size_t)ctx * hd * 4, hipMemcpyHostToDevice) != hipSuccess) return -1;
        a.q = dq; a.kc = dk; a.vc = dv; a.rope = dr;
        a.S = S; a.D = H * hd; a.H = H; a.hd = hd; a.ctx = ctx; a.pos0 = pos0;
    } else {
        return -1;
    }
    hipError_t e = rh::launch_gemm(epi, a, nullptr);
    if (e != hipSuccess) return (int)e;
    if ((e = hipDeviceSynchronize()) != hipSuccess) return (int)e;
    if (of && hipMemcpy(io_f32, of, (size_t)M * N * 4, hipMemcpyDeviceToHost) != hipSuccess) return -1;
    if (o16 && hipMemcpy(out_f16, o16, o16n * 2, hipMemcpyDeviceToHost) != hipSuccess) return -1;
    if (hh && hipMemcpy(h13, hh, (size_t)2 * M * a.ldo * 2, hipMemcpyDeviceToHost) != hipSuccess) return -1;
    if (dq) {
        if (hipMemcpy(q16, dq, qn * 2, hipMemcpyDeviceToHost) != hipSuccess ||
            hipMemcpy(k16, dk, kvn * 2, hipMemcpyDeviceToHost) != hipSuccess ||
            hipMemcpy(v16, dv, kvn * 2, hipMemcpyDeviceToHost) != hipSuccess)
            return -1;
    }
    return 0;
}

// Residual GEMM + RMSNorm as the forward runs it after Wo and W2: x += alpha *
// (X W^T), then xn = RMSNorm(x) * gamma in fragment order ([ceil(M/16)*16][N]
// halves).  With xin set the residual is read from there (out of place, as
// the training forward runs it) and x only written.  cfg 0 takes the split-K
// path when the output has few tiles.
int rhh_gemm_resid_norm(int cfg, const uint16_t* wf, const uint16_t* xf, int M, int N, int K, float alpha,
                        const float* xin, float* x, const float* gamma, float eps, uint16_t* xn_out) {
    if (M <= 0 || N <= 0 || K <= 0 || !wf || !xf || !x || !gamma || !xn_out) return -1;
    Dev d;
    const size_t wn = (size_t)up16(N) * K, xn = (size_t)up16(M) * K, on = (size_t)up16(M) * N;
    f16* W = d.alloc<f16>(wn);
    f16* X = d.alloc<f16>(xn);
    float* dx = d.alloc<float>((size_t)M * N);
    float* dxin = xin ? d.alloc<float>((size_t)M * N) : nullptr;
    float* dg = d.alloc<float>(N);
    f16* dxn = d.alloc<f16>(on);
    const size_t skf = rh::gemm_sk_part_floats();
    float* sk = d.alloc<float>(skf);
    if (!W || !X || !dx || !dg || !dxn || !sk || (xin && !dxin)) return -1;
    if (hipMemcpy(W, wf, wn * 2, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(X, xf, xn * 2, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(dx, x, (size_t)M * N * 4, hipMemcpyHostToDevice) != hipSuccess ||
        (xin && hipMemcpy(dxin, xin, (size_t)M * N * 4, hipMemcpyHostToDevice) != hipSuccess) ||
        hipMemcpy(dg, gamma, (size_t)N * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemset(dxn, 0, on * 2) != hipSuccess)
        return -1;
    rh::GemmArgs a{};
    a.W = W; a.X = X; a.M = M; a.N = N; a.K = K;
    a.resid_in = dxin; a.out_f32 = dx; a.ldo = N; a.alpha = alpha;
    a.sk_part = sk; a.sk_part_floats = skf;
    a.force_cfg = cfg;
    hipError_t e = rh::launch_gemm_resid_norm(a, dg, eps, dxn, nullptr);
    if (e != hipSuccess) return (int)e;
    if ((e = hipDeviceSynchronize()) != hipSuccess) return (int)e;
    if (hipMemcpy(x, dx, (size_t)M * N * 4, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(xn_out, dxn, on * 2, hipMemcpyDeviceToHost) != hipSuccess)
        return -1;
    return 0;
}

// Weight-gradient GEMM (launch_gemm_wgrad): io_f32 [M][N] = alpha * (X W^T)
// (alpha 0: unscaled), or io_f32 += alpha * (X W^T) when accumulate.
int rhh_gemm_wgrad(const uint16_t* wf, const uint16_t* xf, int M, int N, int K, float alpha, int accumulate,
                   float* io_f32) {
    if (M <= 0 || N <= 0 || K <= 0 || !wf || !xf || !io_f32) return -1;
    Dev d;
    const size_t wn = (size_t)up16(N) * K, xn = (size_t)up16(M) * K;
    f16* W = d.alloc<f16>(wn);
    f16* X = d.alloc<f16>(xn);
    float* of = d.alloc<float>((size_t)M * N);
    if (!W || !X || !of) return -1;
    if (hipMemcpy(W, wf, wn * 2, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(X, xf, xn * 2, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(of, io_f32, (size_t)M * N * 4, hipMemcpyHostToDevice) != hipSuccess)
        return -1;
    rh::GemmArgs a{};
    a.W = W; a.X = X; a.M = M; a.N = N; a.K = K;
    a.out_f32 = of; a.ldo = N; a.alpha = alpha;
    hipError_t e = rh::launch_gemm_wgrad(a, accumulate != 0, nullptr);
    if (e != hipSuccess) return (int)e;
    if ((e = hipDeviceSynchronize()) != hipSuccess) return (int)e;
    if (hipMemcpy(io_f32, of, (size_t)M * N * 4, hipMemcpyDeviceToHost) != hipSuccess) return -1;
    return 0;
}

}  // extern "C"
