"""GPU parity of every prefill GEMM tile configuration and epilogue.

The forward only reaches the tile configurations its shape heuristic picks
for the model widths under test.  Through the GEMM test harness
(rustane_amd/librustane_gemm_harness.so) each configuration -- one block per
tile (including the 16x16x32 8-wave tiles), stream-K with its fix-up kernel,
split-K with the summing residual + RMSNorm row kernel -- runs every epilogue
on ragged shapes (M, N not multiples of any tile) and is checked against a
float64 numpy product of the same fp16 operands:
    Y[m][n] = sum_k X[m][k] W[n][k]
The epilogue references restate crates/engine/src/kernels/sdpa_fwd.rs:115-117
(QKV + RoPE into q and the K/V cache), kernels/ffn_fused.rs:80-160 (SwiGLU on
interleaved W1|W3 rows) and the residual update x += alpha * Y followed by
RMSNorm (cpu/rmsnorm.rs:149-183).
Tolerances: fp32 outputs 1e-5 of max|Y| (fp32 accumulation of K <= 8192
products), fp16 outputs 2e-3 of the output's max (one fp16 rounding).
"""
import ctypes
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(os.path.dirname(HERE), "rustane_amd", "librustane_gemm_harness.so")

EPI_F32, EPI_RESID, EPI_SWIGLU, EPI_QKV, EPI_SWIGLU_SAVE, EPI_SILU_BWD = 0, 1, 2, 3, 4, 5
# GemmCfg values (rh_kernels.h): one block per tile, and their stream-K twins
DP = {"D8_256x256": 6, "D4_128x128": 8, "D8_256x128": 10, "D4_256x256": 12, "D4_256x128": 14,
      "D4_192x128": 16, "D8_192x256": 18, "D4_192x256": 20, "D8_192x128": 24, "D8_128x128": 26}
SK = {k + "_SK": v + 1 for k, v in DP.items()}
CFGS = {"auto": 0, **DP, **SK}


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built (python -m rustane_amd.build)")
    h = ctypes.CDLL(LIB)
    f, i, p = ctypes.c_float, ctypes.c_int, ctypes.c_void_p
    h.rhh_gemm.argtypes = [i, i, p, p, i, i, i, f, f, p, p, p, i, i, i, i, i, i, p, p, p, p]
    h.rhh_gemm.restype = i
    h.rhh_gemm_resid_norm.argtypes = [i, p, p, i, i, i, f, p, p, p, f, p]
    h.rhh_gemm_resid_norm.restype = i
    h.rhh_gemm_wgrad.argtypes = [p, p, i, i, i, f, i, p]
    h.rhh_gemm_wgrad.restype = i
    return h


def up16(x):
    return (x + 15) // 16 * 16


def frag_index(R, K):
    """Flat fragment-order offset of every (row, k) of an [R][K] array (frag_off)."""
    rows = np.arange(R, dtype=np.int64)[:, None]
    ks = np.arange(K, dtype=np.int64)[None, :]
    chunk = (rows >> 4) * (K >> 7) + (ks >> 7)
    return ((chunk * 4 + ((ks >> 5) & 3)) * 64 + 16 * ((ks >> 3) & 3) + (rows & 15)) * 8 + (ks & 7)


def frag_pack(a):
    """[R][K] fp16 -> fragment order, rows zero-padded to a multiple of 16."""
    R, K = a.shape
    pad = np.zeros((up16(R), K), np.float16)
    pad[:R] = a
    out = np.empty(pad.size, np.float16)
    out[frag_index(up16(R), K).ravel()] = pad.ravel()
    return out


def frag_unpack(buf, R, K):
    return buf[frag_index(R, K)]


def operands(seed, M, N, K):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float16)
    w = rng.standard_normal((N, K)).astype(np.float16)
    y = x.astype(np.float64) @ w.astype(np.float64).T
    return x, w, y


def ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def run(lib, epi, cfg, x, w, alpha=0.0, softcap=0.0, io=None, out16=None, h13=None, qkv=None):
    M, K = x.shape
    N = w.shape[0]
    xf, wf = frag_pack(x), frag_pack(w)
    B = S = H = hd = ctx = pos0 = 0
    rope = q = k = v = None
    if qkv is not None:
        B, S, H, hd, ctx, pos0, rope, q, k, v = qkv
    rc = lib.rhh_gemm(epi, cfg, ptr(wf), ptr(xf), M, N, K, alpha, softcap, ptr(io), ptr(out16), ptr(h13),
                      B, S, H, hd, ctx, pos0, ptr(rope), ptr(q), ptr(k), ptr(v))
    assert rc == 0, f"rhh_gemm epi {epi} cfg {cfg}: error {rc}"


def close(got, want, rel, what):
    scale = float(np.abs(want).max())
    err = float(np.abs(got.astype(np.float64) - want).max())
    assert err <= rel * scale, f"{what}: max error {err:.3e} > {rel:g} x {scale:.3e}"


def silu(x):
    return x / (1.0 + np.exp(-x))


@pytest.mark.parametrize("name", list(CFGS))
def test_fp32_store_scale_softcap(lib, name):
    x, w, y = operands(1, 300, 1000, 384)
    out = np.zeros((300, 1000), np.float32)
    run(lib, EPI_F32, CFGS[name], x, w, io=out)
    close(out, y, 1e-5, f"{name} store")
    out2 = np.zeros_like(out)
    run(lib, EPI_F32, CFGS[name], x, w, alpha=0.5, softcap=15.0, io=out2)
    close(out2, 15.0 * np.tanh(0.5 * y / 15.0), 1e-5, f"{name} alpha+softcap")


@pytest.mark.parametrize("K", [128, 640, 1152])
@pytest.mark.parametrize("name", ["D8_192x256", "D8_192x256_SK", "D8_256x128", "D8_128x128"])
def test_k_step_counts(lib, name, K):
    """k loops of 4, 20 and 36 steps: the five-stage tile (192x256) runs
    groups of 10 steps and a predicated remainder, the four-stage ones
    groups of 4, so these cover a remainder only, whole groups only, and
    both."""
    x, w, y = operands(11, 200, 700, K)
    out = np.zeros((200, 700), np.float32)
    run(lib, EPI_F32, CFGS[name], x, w, io=out)
    close(out, y, 1e-5, f"{name} K {K}")


@pytest.mark.parametrize("name", list(CFGS))
def test_residual(lib, name):
    x, w, y = operands(2, 300, 1000, 384)
    x0 = np.random.default_rng(3).standard_normal((300, 1000)).astype(np.float32)
    io = x0.copy()
    run(lib, EPI_RESID, CFGS[name], x, w, alpha=0.125, io=io)
    close(io, x0.astype(np.float64) + 0.125 * y, 1e-5, f"{name} residual")


def swiglu_ref(y):
    """Gate features of interleaved W1|W3 rows: 32-row group T holds W1 rows
    16T..16T+15, then the matching W3 rows."""
    M, N = y.shape
    F = N // 2
    f = np.arange(F)
    r1 = 32 * (f // 16) + f % 16
    h1, h3 = y[:, r1], y[:, r1 + 16]
    return silu(h1) * h3, h1, h3


@pytest.mark.parametrize("name", list(CFGS))
def test_swiglu_and_saved_preactivations(lib, name):
    M, F, K = 300, 640, 384
    x, w, y = operands(4, M, 2 * F, K)
    g_ref, h1, h3 = swiglu_ref(y)
    out16 = np.zeros(up16(M) * F, np.float16)
    run(lib, EPI_SWIGLU, CFGS[name], x, w, out16=out16)
    close(frag_unpack(out16, M, F), g_ref, 2e-3, f"{name} swiglu")
    out16[:] = 0
    h13 = np.zeros(2 * M * F, np.float16)
    run(lib, EPI_SWIGLU_SAVE, CFGS[name], x, w, out16=out16, h13=h13)
    close(frag_unpack(out16, M, F), g_ref, 2e-3, f"{name} swiglu_save gate")
    close(h13[:M * F].reshape(M, F), h1, 2e-3, f"{name} saved h1")
    close(h13[M * F:].reshape(M, F), h3, 2e-3, f"{name} saved h3")


@pytest.mark.parametrize("name", list(CFGS))
def test_silu_gate_backward(lib, name):
    """The gate gradient g = X W^T with the SiLU-gate backward in the
    epilogue (crates/engine/src/layer.rs:7083-7104, cpu/silu.rs:68-90):
    dh3 = g silu(h1), dh1 = g h3 silu'(h1), written as [dh1 | dh3] in
    fragment order."""
    M, F, K = 300, 640, 384
    x, w, g = operands(9, M, F, K)
    rng = np.random.default_rng(10)
    h13 = (rng.standard_normal(2 * M * F) * 2).astype(np.float16)
    out16 = np.zeros(up16(M) * 2 * F, np.float16)
    run(lib, EPI_SILU_BWD, CFGS[name], x, w, out16=out16, h13=h13)
    h1 = h13[:M * F].reshape(M, F).astype(np.float64)
    h3 = h13[M * F:].reshape(M, F).astype(np.float64)
    sig = 1.0 / (1.0 + np.exp(-h1))
    dh = frag_unpack(out16, M, 2 * F)
    close(dh[:, :F], g * h3 * sig * (1.0 + h1 * (1.0 - sig)), 2e-3, f"{name} dh1")
    close(dh[:, F:], g * h1 * sig, 2e-3, f"{name} dh3")


@pytest.mark.parametrize("name", ["auto", "D4_192x128", "D8_192x128", "D8_192x256", "D8_256x256", "D4_128x128_SK"])
def test_qkv_rope_scatter(lib, name):
    B, S, H, hd, ctx, pos0, K = 2, 150, 2, 128, 200, 10, 384
    D = H * hd
    x, w, y = operands(5, B * S, 3 * D, K)
    rng = np.random.default_rng(6)
    ang = rng.uniform(-np.pi, np.pi, (ctx, hd // 2))
    rope = np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)
    q = np.zeros((B, H, S, hd), np.float16)
    k = np.zeros((B, H, ctx, hd), np.float16)
    v = np.zeros((B, H, ctx, hd), np.float16)
    run(lib, EPI_QKV, CFGS[name], x, w, qkv=(B, S, H, hd, ctx, pos0, rope, q, k, v))
    y = y.reshape(B, S, 3, H, hd)
    cs = rope[pos0:pos0 + S].astype(np.float64)  # [S][hd/2][2]

    def rot(t):  # t [B][S][H][hd]: pairs (2i, 2i+1) rotated by the position's (cos, sin)
        e, o = t[..., 0::2], t[..., 1::2]
        c, s = cs[None, :, None, :, 0], cs[None, :, None, :, 1]
        out = np.empty_like(t)
        out[..., 0::2] = e * c - o * s
        out[..., 1::2] = o * c + e * s
        return out

    q_ref = rot(y[:, :, 0]).transpose(0, 2, 1, 3)
    k_ref = rot(y[:, :, 1]).transpose(0, 2, 1, 3)
    v_ref = y[:, :, 2].transpose(0, 2, 1, 3)
    close(q, q_ref, 2e-3, f"{name} q")
    close(k[:, :, pos0:pos0 + S], k_ref, 2e-3, f"{name} k cache")
    close(v[:, :, pos0:pos0 + S], v_ref, 2e-3, f"{name} v cache")
    # positions outside pos0 .. pos0+S-1 are untouched
    assert not k[:, :, :pos0].any() and not k[:, :, pos0 + S:].any()
    assert not v[:, :, :pos0].any() and not v[:, :, pos0 + S:].any()


@pytest.mark.parametrize("out_of_place", [False, True])
@pytest.mark.parametrize("cfg,K,M", [(0, 1024, 300), (0, 8192, 300), (16, 1024, 300), (9, 1024, 300),
                                     (16, 1024, 2100)])
def test_residual_then_rmsnorm(lib, cfg, K, M, out_of_place):
    """cfg 0 at these shapes takes split-K (K 1024: 128x128 tiles, K 8192:
    256x128) with the summing row kernel; 16 / 9 are one block per tile and
    stream-K followed by the plain RMSNorm kernel (one row per block; from
    2048 rows on, 8 rows per block -- M 2100 ends in a partial block).  Out
    of place the residual is read from its own buffer and the output buffer
    starts as garbage."""
    N, eps, alpha = 1024, 1e-5, 0.25
    x, w, y = operands(7, M, N, K)
    rng = np.random.default_rng(8)
    x0 = rng.standard_normal((M, N)).astype(np.float32)
    gamma = rng.uniform(0.5, 1.5, N).astype(np.float32)
    xf, wf = frag_pack(x), frag_pack(w)
    xin = x0.copy() if out_of_place else None
    io = np.full_like(x0, np.nan) if out_of_place else x0.copy()
    xn = np.zeros(up16(M) * N, np.float16)
    rc = lib.rhh_gemm_resid_norm(cfg, ptr(wf), ptr(xf), M, N, K, alpha, ptr(xin), ptr(io), ptr(gamma), eps,
                                 ptr(xn))
    assert rc == 0, f"rhh_gemm_resid_norm cfg {cfg}: error {rc}"
    x1 = x0.astype(np.float64) + alpha * y
    close(io, x1, 1e-5, "residual")
    xn_ref = x1 / np.sqrt((x1 * x1).mean(1, keepdims=True) + eps) * gamma
    close(frag_unpack(xn, M, N), xn_ref, 2e-3, "rmsnorm output")


# Weight-gradient GEMM (persistent blocks, store waves draining an LDS-staged
# tile): few tiles (XCDs without a tile), ragged edges, more tiles than blocks
# (several per block), K from 128 to 2048 (the token count), store with and
# without a scale and accumulate.
@pytest.mark.parametrize("M,N,K", [(100, 60, 128), (300, 1000, 384), (1100, 2060, 512), (4096, 1100, 640),
                                   (640, 384, 2048)])
def test_weight_gradient_gemm(lib, M, N, K):
    x, w, y = operands(11, M, N, K)
    xf, wf = frag_pack(x), frag_pack(w)
    out = np.full((M, N), np.nan, np.float32)  # every element must be written
    assert lib.rhh_gemm_wgrad(ptr(wf), ptr(xf), M, N, K, 0.0, 0, ptr(out)) == 0
    close(out, y, 1e-5, "store")
    out = np.zeros((M, N), np.float32)
    assert lib.rhh_gemm_wgrad(ptr(wf), ptr(xf), M, N, K, 0.25, 0, ptr(out)) == 0
    close(out, 0.25 * y, 1e-5, "scaled store")
    x0 = np.random.default_rng(12).standard_normal((M, N)).astype(np.float32)
    io = x0.copy()
    assert lib.rhh_gemm_wgrad(ptr(wf), ptr(xf), M, N, K, 0.5, 1, ptr(io)) == 0
    close(io, x0.astype(np.float64) + 0.5 * y, 1e-5, "accumulate")
