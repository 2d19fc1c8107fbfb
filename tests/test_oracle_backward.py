"""Pins the oracle's backward pass (test infrastructure) against independent
mathematics: float64 autograd of a torch restatement of the forward (built
from library routines -- RMSNorm by formula, RoPE as a complex rotation, torch
SDPA, silu, cross_entropy), the reference's numerical-gradient KATs
(cpu/rmsnorm.rs:278-316, cpu/silu.rs:68-90), and algebraic properties
(accumulation, loss-scale linearity, RoPE backward inverting the rotation)."""
import ctypes
import math

import numpy as np
import pytest

from rustane_amd.engine import ModelWeights

from helpers import oracle_cfg, oracle_weights, random_gammas, small_cfg, tokens_uniform


def torch_grads64(cfg, w, tok, tgt, softcap=0.0, loss_scale=1.0):
    """loss_scale x d(mean CE)/d(params) per sequence, summed over the batch,
    by float64 autograd.  Returns (embed, gamma_final, [[9 per layer]], losses)."""
    import torch
    import torch.nn.functional as Fn
    T = lambda a: torch.tensor(np.asarray(a, np.float64), requires_grad=True)
    E, gf = T(w.embed), T(w.gamma_final)
    layers = [[T(t) for t in lw.tensors()] for lw in w.layers]
    H, hd, L = cfg.heads, cfg.hd, cfg.nlayers
    a = 1.0 / math.sqrt(2 * L)

    def rms(y, g):
        return y / torch.sqrt((y ** 2).mean(-1, keepdim=True) + 1e-5) * g

    def rope(x):  # [S, H, hd], pairs (2i, 2i+1) rotated by p / 1e4^(2i/hd)
        S = x.shape[0]
        th = torch.arange(S, dtype=torch.float64)[:, None, None] / \
            1e4 ** (2 * torch.arange(hd // 2, dtype=torch.float64)[None, None, :] / hd)
        c, s = torch.cos(th), torch.sin(th)
        x0, x1 = x[..., 0::2], x[..., 1::2]
        return torch.stack([x0 * c - x1 * s, x1 * c + x0 * s], -1).reshape(x.shape)

    losses = []
    total = 0
    for b in range(tok.shape[0]):
        ids = torch.from_numpy(tok[b].astype(np.int64))
        S = ids.shape[0]
        x = E[ids]
        for wq, wk, wv, wo, w1, w3, w2, g1, g2 in layers:
            xn = rms(x, g1)
            q = rope((xn @ wq).reshape(S, H, hd)).transpose(0, 1)
            k = rope((xn @ wk).reshape(S, H, hd)).transpose(0, 1)
            v = (xn @ wv).reshape(S, H, hd).transpose(0, 1)
            att = Fn.scaled_dot_product_attention(q, k, v, is_causal=True).transpose(0, 1).reshape(S, -1)
            x = x + a * (att @ wo)
            h = rms(x, g2)
            x = x + a * ((Fn.silu(h @ w1) * (h @ w3)) @ w2.T)
        logits = rms(x, gf) @ E.T
        if softcap > 0:
            logits = softcap * torch.tanh(logits / softcap)
        loss = Fn.cross_entropy(logits, torch.from_numpy(tgt[b].astype(np.int64)))
        losses.append(float(loss.detach()))
        total = total + loss * loss_scale
    total.backward()
    g = lambda t: t.grad.numpy()
    return g(E), g(gf), [[g(t) for t in lw] for lw in layers], np.array(losses)


NAMES = ["wq", "wk", "wv", "wo", "w1", "w3", "w2", "gamma1", "gamma2"]


def assert_grads_close(og, ref, rel=3e-4):
    pairs = [("embed", og.embed, ref[0]), ("gamma_final", og.gamma_final, ref[1])]
    for l, (a, b) in enumerate(zip(og.layers, ref[2])):
        pairs += [(f"layer{l}.{n}", x, y) for n, x, y in zip(NAMES, a, b)]
    for name, got, want in pairs:
        scale = np.abs(want).max()
        assert scale > 0, name
        err = np.abs(got - want).max() / scale
        assert err <= rel, f"{name}: max err {err:.2e} of max |g| {scale:.2e}"


def _setup(seed, softcap=0.0, batch=1, seq=13):
    cfg = small_cfg(dim=64, hidden=128, heads=2, hd=32, nlayers=2, vocab=96, seq=seq)
    w = random_gammas(ModelWeights.normal(cfg, seed=seed, std=0.15, fp16_round=False), seed + 1)
    tok, tgt = tokens_uniform(seed + 2, cfg.vocab, batch, seq)
    return cfg, w, tok, tgt


@pytest.mark.parametrize("softcap,loss_scale,batch", [(0.0, 1.0, 1), (2.0, 256.0, 2)])
def test_forward_backward_matches_float64_autograd(orc, softcap, loss_scale, batch):
    cfg, w, tok, tgt = _setup(41, softcap, batch)
    g, ml = orc.forward_backward(oracle_cfg(orc, cfg, softcap), oracle_weights(orc, w), tok, tgt,
                                 loss_scale=loss_scale)
    ref = torch_grads64(cfg, w, tok, tgt, softcap, loss_scale)
    np.testing.assert_allclose(ml, ref[3], rtol=1e-5)
    assert_grads_close(g, ref)


def test_gradients_accumulate_and_scale_linearly(orc):
    cfg, w, tok, tgt = _setup(43)
    oc, ow = oracle_cfg(orc, cfg), oracle_weights(orc, w)
    g1, _ = orc.forward_backward(oc, ow, tok, tgt)
    g2, _ = orc.forward_backward(oc, ow, tok, tgt)
    orc.forward_backward(oc, ow, tok, tgt, grads=g2)          # += a second pass
    g3, _ = orc.forward_backward(oc, ow, tok, tgt, loss_scale=8.0)
    flat = lambda g: [g.embed, g.gamma_final] + [t for lw in g.layers for t in lw]
    for a, b, c in zip(flat(g1), flat(g2), flat(g3)):
        np.testing.assert_allclose(b, 2 * a, rtol=1e-5, atol=1e-7 * np.abs(a).max())
        np.testing.assert_allclose(c, 8 * a, rtol=1e-5, atol=1e-7 * np.abs(a).max())
    assert all(np.abs(t).max() > 0 for t in flat(g1))   # every weight group gets a gradient


def test_rmsnorm_backward_numerical_kat(orc):  # cpu/rmsnorm.rs:278-316
    x = np.array([1.0, -2.0, 3.0, -0.5], np.float32).reshape(4, 1)
    gamma = np.array([1.0, 0.5, 2.0, 1.5], np.float32)
    dy = np.ones((4, 1), np.float32)
    out = np.zeros_like(x)
    rinv = np.zeros(1, np.float32)
    orc.lib().orc_rmsnorm_forward_channel_first(orc.fp(x), orc.fp(gamma), orc.fp(out), orc.fp(rinv), 4, 1,
                                                ctypes.c_float(1e-5))
    dx = np.zeros_like(x)
    dg = np.zeros(4, np.float32)
    orc.lib().orc_rmsnorm_backward_channel_first(orc.fp(dy), orc.fp(x), orc.fp(gamma), orc.fp(rinv),
                                                 orc.fp(dx), orc.fp(dg), 4, 1)
    eps = 1e-4
    for i in range(4):
        num = []
        for sgn in (1, -1):
            xp = x.astype(np.float64).copy()
            xp[i] += sgn * eps
            num.append((xp[:, 0] / np.sqrt((xp[:, 0] ** 2).mean() + 1e-5) * gamma).sum())
        assert abs(dx[i, 0] - (num[0] - num[1]) / (2 * eps)) < 1e-2
    # dgamma = dy * x_hat
    np.testing.assert_allclose(dg, x[:, 0] * rinv[0], rtol=1e-6)


def test_silu_backward_numerical_kat(orc):  # cpu/silu.rs:68-90
    x = np.array([-1.0, 0.0, 0.5, 2.0], np.float32)
    one = np.ones(4, np.float32)
    dh1, dh3 = np.zeros(4, np.float32), np.zeros(4, np.float32)
    orc.lib().orc_silu_gate_backward(orc.fp(one), orc.fp(x), orc.fp(one), orc.fp(dh1), orc.fp(dh3), 4)
    silu = lambda v: v / (1 + np.exp(-v))
    eps = 1e-4
    for i in range(4):
        num = (silu(np.float64(x[i]) + eps) - silu(np.float64(x[i]) - eps)) / (2 * eps)
        assert abs(dh1[i] - num) < 1e-3
    np.testing.assert_allclose(dh3, silu(x.astype(np.float64)), rtol=1e-6)


def test_sdpa_backward_matches_autograd(orc):
    import torch
    rng = np.random.default_rng(47)
    S, H, hd = 19, 2, 16
    D = H * hd
    cfg = orc.make_config(D, 64, H, 1, 32, head_dim=hd)
    q, k, v, da = (rng.standard_normal((S, D), dtype=np.float32) for _ in range(4))
    outs = [np.zeros((S, D), np.float32) for _ in range(3)]
    orc.lib().orc_sdpa_backward(ctypes.byref(cfg), S, *[orc.fp(t) for t in (q, k, v, da)],
                                *[orc.fp(o) for o in outs])
    T = lambda a: torch.tensor(a.astype(np.float64).reshape(S, H, hd).transpose(1, 0, 2), requires_grad=True)
    tq, tk, tv = T(q), T(k), T(v)
    o = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=True)
    o.backward(torch.from_numpy(da.astype(np.float64).reshape(S, H, hd).transpose(1, 0, 2).copy()))
    for got, t in zip(outs, (tq, tk, tv)):
        want = t.grad.numpy().transpose(1, 0, 2).reshape(S, D)
        np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4 * np.abs(want).max())


def test_rope_backward_inverts_rotation(orc):
    from test_oracle_kats import rope_complex
    rng = np.random.default_rng(48)
    S, H, hd = 23, 3, 16
    cfg = orc.make_config(H * hd, 64, H, 1, 32, head_dim=hd)
    x = rng.standard_normal((S, H, hd))
    r = np.ascontiguousarray(rope_complex(x).reshape(S, H * hd), dtype=np.float32)
    orc.lib().orc_rope_backward(ctypes.byref(cfg), orc.fp(r), S)
    np.testing.assert_allclose(r.reshape(S, H, hd), x, rtol=1e-4, atol=1e-4)
