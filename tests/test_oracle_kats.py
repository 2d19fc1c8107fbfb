"""Pins the CPU oracle (test infrastructure) against the reference's own
known-answer tests and against independent mathematics.

KATs are the reference's unit tests (crates/engine/src/cpu/*.rs #[cfg(test)]);
RoPE is checked against the complex-exponential closed form, attention against
torch's scaled_dot_product_attention in float64, the layer against a float64
restatement built from those library routines, and the decode cache against
the full forward (causality)."""
import ctypes
import math

import numpy as np
import pytest

from rustane_amd.engine import ModelConfig, ModelWeights, random_vec

from helpers import oracle_cfg, oracle_weights, small_cfg, tokens_uniform


def f32(*v):
    return np.array(v, np.float32)


# ---------------------------------------------------------------- vDSP contracts
def test_vsma_kat(orc):  # vdsp.rs:476-483
    a, b, out = f32(1, 2, 3), f32(10, 20, 30), np.zeros(3, np.float32)
    orc.lib().orc_vsma(orc.fp(a), 2.0, orc.fp(b), orc.fp(out), 3)
    assert out.tolist() == [12.0, 24.0, 36.0]


def test_vsub_order_kat(orc):  # vdsp.rs:427-434: out = b - a
    a, b, out = f32(1, 2, 3), f32(10, 20, 30), np.zeros(3, np.float32)
    orc.lib().orc_vsub(orc.fp(a), orc.fp(b), orc.fp(out), 3)
    assert out.tolist() == [9.0, 18.0, 27.0]


def test_mtrans(orc):
    a = np.arange(6, dtype=np.float32).reshape(2, 3)
    c = np.zeros((3, 2), np.float32)
    orc.lib().orc_mtrans(orc.fp(a), 3, orc.fp(c), 2, 2, 3)
    np.testing.assert_array_equal(c, a.T)


def test_sgemm_at_accumulates(orc):  # vdsp.rs:351-376: beta = 1
    rng = np.random.default_rng(0)
    a = rng.standard_normal((37, 19), dtype=np.float32)
    b = rng.standard_normal((23, 19), dtype=np.float32)
    c = np.ones((37, 23), np.float32)
    orc.lib().orc_sgemm_at(orc.fp(a), 37, 19, orc.fp(b), 23, orc.fp(c))
    np.testing.assert_allclose(c, 1.0 + a.astype(np.float64) @ b.T.astype(np.float64), rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------- cpu ops
def test_embedding_kats(orc):  # embedding.rs:53-62, :85-93
    table = f32(1, 2, 3, 4, 5, 6)
    ids = np.array([2, 0, 1], np.uint32)
    out = np.zeros(6, np.float32)
    orc.lib().orc_embedding_forward(orc.fp(table), 2, orc.up(ids), 3, orc.fp(out))
    assert out.tolist() == [5, 6, 1, 2, 3, 4]
    table = f32(10, 20, 30, 40)
    out = np.zeros(4, np.float32)
    orc.lib().orc_embedding_forward(orc.fp(table), 2, orc.up(np.array([0, 1], np.uint32)), 2, orc.fp(out))
    assert out.tolist() == table.tolist()


def test_rmsnorm_kats(orc):  # rmsnorm.rs:244-277
    L = orc.lib()
    x, g, out = f32(3, 4), f32(1, 1), np.zeros(2, np.float32)
    r = L.orc_rmsnorm_forward(orc.fp(x), orc.fp(g), orc.fp(out), 2, 1e-5)
    er = math.sqrt(12.5 + 1e-5)
    assert abs(r - 1 / er) < 1e-5 and abs(out[0] - 3 / er) < 1e-5 and abs(out[1] - 4 / er) < 1e-5
    x, g, out = f32(1, 2, 3, 4), f32(0.5, 0.5, 0.5, 0.5), np.zeros(4, np.float32)
    r = L.orc_rmsnorm_forward(orc.fp(x), orc.fp(g), orc.fp(out), 4, 1e-5)
    er = 1 / math.sqrt(7.5 + 1e-5)
    assert abs(r - er) < 1e-5
    np.testing.assert_allclose(out, x * er * 0.5, atol=1e-5)


def test_rmsnorm_channel_first_matches_rows(orc):  # rmsnorm.rs:320-369
    dim, seq = 4, 3
    gamma = f32(1.5, 0.5, 2.0, 0.8)
    x_cf = np.array([((i * 17 + 3) % 100) * 0.01 - 0.5 for i in range(dim * seq)], np.float32)
    out = np.zeros_like(x_cf)
    ri = np.zeros(seq, np.float32)
    orc.lib().orc_rmsnorm_forward_channel_first(orc.fp(x_cf), orc.fp(gamma), orc.fp(out), orc.fp(ri),
                                                dim, seq, 1e-5)
    xt = x_cf.reshape(dim, seq).T.astype(np.float64)
    r64 = 1 / np.sqrt((xt ** 2).mean(1) + 1e-5)
    np.testing.assert_allclose(ri, r64, rtol=1e-5)
    np.testing.assert_allclose(out.reshape(dim, seq).T, xt * r64[:, None] * gamma, atol=1e-5)


def test_silu_gate_kats(orc):  # silu.rs:53-70, :98-109
    L = orc.lib()
    g, u, out = f32(0.0, 2.0), f32(1.0, 1.0), np.zeros(2, np.float32)
    L.orc_silu_gate(orc.fp(g), orc.fp(u), orc.fp(out), 2)
    assert abs(out[0]) < 1e-6
    assert abs(out[1] - 2.0 / (1 + math.exp(-2.0))) < 1e-6
    g, u, out = f32(1, 2), f32(3, 4), np.zeros(2, np.float32)
    L.orc_silu_gate(orc.fp(g), orc.fp(u), orc.fp(out), 2)
    import torch
    want = torch.nn.functional.silu(torch.tensor([1.0, 2.0], dtype=torch.float64)).numpy() * [3, 4]
    np.testing.assert_allclose(out, want, rtol=1e-6)


def _ce(orc, logits, target):
    logits = np.ascontiguousarray(logits, np.float32)
    lsm = np.zeros_like(logits)
    loss = orc.lib().orc_cross_entropy_forward(orc.fp(logits), len(logits), target, orc.fp(lsm))
    return loss, lsm


def test_cross_entropy_kats(orc):  # cross_entropy.rs:102-155
    loss, _ = _ce(orc, [1, 2, 3, 4], 3)
    assert 0 < loss < 2.0
    lo, _ = _ce(orc, [1, 1, 1, 1], 3)
    hi, _ = _ce(orc, [0, 0, 0, 10], 3)
    assert hi < lo
    _, lsm = _ce(orc, [1, 2, 3], 1)
    d = np.exp(lsm)
    d[1] -= 1
    assert abs(d.sum()) < 1e-5
    logits = f32(2.0, -1.0, 0.5, 1.5)
    _, lsm = _ce(orc, logits, 2)
    grad = np.exp(lsm)
    grad[2] -= 1
    for i in range(4):
        p, m = logits.copy(), logits.copy()
        p[i] += 1e-4
        m[i] -= 1e-4
        num = (_ce(orc, p, 2)[0] - _ce(orc, m, 2)[0]) / 2e-4
        assert abs(grad[i] - num) < 5e-3


def test_cross_entropy_batch_is_logsumexp(orc):
    from scipy.special import logsumexp
    rng = np.random.default_rng(1)
    S, V = 7, 301
    logits = (rng.standard_normal((S, V)) * 3).astype(np.float32)
    tg = rng.integers(0, V, S).astype(np.uint32)
    dl = np.zeros_like(logits)
    total = orc.lib().orc_cross_entropy_forward_backward_batch(orc.fp(logits), orc.up(tg), S, V,
                                                               orc.fp(dl), 1.0 / S)
    want = sum(logsumexp(logits[s].astype(np.float64)) - logits[s, tg[s]] for s in range(S))
    assert abs(total - want) < 1e-4
    np.testing.assert_allclose(dl.sum(1), 0, atol=1e-6)


# ---------------------------------------------------------------- init
@pytest.mark.parametrize("n,scale", [(1, 1.0), (4095, 0.5), (4097, 0.005), (512 * 1408, 1 / math.sqrt(1408))])
def test_lcg_bit_exact(orc, n, scale):
    a = random_vec(n, scale)
    b = np.empty(n, np.float32)
    orc.lib().orc_random_vec(orc.fp(b), n, float(np.float32(scale)))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_lcg_first_value():
    # s1 = (42 + 1) * A + C mod 2^64; r = (s1 >> 32) / u32::MAX * 2 - 1
    s1 = (43 * 6364136223846793005 + 1442695040888963407) % 2 ** 64
    r = np.float32(np.float32(s1 >> 32) / np.float32(4294967295.0)) * np.float32(2) - np.float32(1)
    assert random_vec(1, 1.0)[0] == np.float32(r)


# ---------------------------------------------------------------- RoPE / attention
def test_rope_table_complex_form(orc):
    seq, hd = 37, 16
    c = np.zeros((seq, hd), np.float32)
    s = np.zeros((seq, hd), np.float32)
    orc.lib().orc_rope_table(seq, hd, 1e4, orc.fp(c), orc.fp(s))
    p = np.arange(seq)[:, None]
    i = np.arange(hd // 2)[None, :]
    z = np.exp(1j * p / 10000.0 ** (2 * i / hd))
    np.testing.assert_allclose(c[:, 0::2], z.real, atol=2e-5 * seq)
    np.testing.assert_allclose(c[:, 1::2], z.real, atol=2e-5 * seq)
    np.testing.assert_allclose(s[:, 0::2], z.imag, atol=2e-5 * seq)
    assert np.all(c[0] == 1) and np.all(s[0] == 0)


def rope_complex(x, base=1e4):
    """x [S, H, hd] float64; interleaved pairs as complex numbers times e^{i p theta_i}."""
    S, H, hd = x.shape
    z = x[..., 0::2] + 1j * x[..., 1::2]
    th = np.arange(S)[:, None, None] / base ** (2 * np.arange(hd // 2)[None, None, :] / hd)
    r = z * np.exp(1j * th)
    out = np.empty_like(x)
    out[..., 0::2], out[..., 1::2] = r.real, r.imag
    return out


def attn_reference64(xn, wq, wk, wv, H):
    """xn [S, D] float64 -> attention output [S, D] via torch SDPA (causal)."""
    import torch
    S, D = xn.shape
    hd = D // H
    q = rope_complex((xn @ wq).reshape(S, H, hd))
    k = rope_complex((xn @ wk).reshape(S, H, hd))
    v = (xn @ wv).reshape(S, H, hd)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a.transpose(1, 0, 2)))
    o = torch.nn.functional.scaled_dot_product_attention(t(q), t(k), t(v), is_causal=True)
    return o.numpy().transpose(1, 0, 2).reshape(S, D), q, k, v


def test_sdpa_matches_library_attention(orc):
    rng = np.random.default_rng(3)
    D, H, S = 64, 4, 29
    cfg = orc.make_config(D, 128, H, 1, 64, head_dim=D // H)
    xn = rng.standard_normal((D, S), dtype=np.float32)
    wq, wk, wv = (rng.standard_normal((D, D), dtype=np.float32) * 0.2 for _ in range(3))
    outs = [np.zeros((D, S), np.float32) for _ in range(4)]
    orc.lib().orc_sdpa_fwd(ctypes.byref(cfg), S, orc.fp(xn), orc.fp(wq), orc.fp(wk), orc.fp(wv),
                           *[orc.fp(o) for o in outs])
    ref, q, k, v = attn_reference64(xn.T.astype(np.float64), wq.astype(np.float64),
                                    wk.astype(np.float64), wv.astype(np.float64), H)
    np.testing.assert_allclose(outs[0].T, ref, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(outs[1].T, q.reshape(S, D), rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(outs[2].T, k.reshape(S, D), rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(outs[3].T, v.reshape(S, D), rtol=1e-4, atol=1e-4)
    # position 0 attends only to itself: attn_out[:, 0] = v[:, 0]
    np.testing.assert_allclose(outs[0][:, 0], outs[3][:, 0], rtol=1e-6, atol=1e-6)
    # RoPE is a rotation: per-head norms of q are preserved
    qn = (xn.T.astype(np.float64) @ wq).reshape(S, H, D // H)
    np.testing.assert_allclose(np.linalg.norm(outs[1].T.reshape(S, H, -1), axis=-1),
                               np.linalg.norm(qn, axis=-1), rtol=1e-4)


def layer_reference64(x, lw, H, L):
    """One layer in float64 from library routines; x [S, D] token-major."""
    import torch
    wq, wk, wv, wo, w1, w3, w2, g1, g2 = [np.asarray(t, np.float64) for t in lw]
    a = 1 / math.sqrt(2 * L)
    rms = lambda y, g: y / np.sqrt((y ** 2).mean(-1, keepdims=True) + 1e-5) * g
    att, *_ = attn_reference64(rms(x, g1), wq, wk, wv, H)
    x2 = x + a * (att @ wo)
    h = rms(x2, g2)
    gate = torch.nn.functional.silu(torch.from_numpy(h @ w1)).numpy() * (h @ w3)
    return x2 + a * (gate @ w2.T)


def test_layer_forward_matches_float64_restatement(orc):
    cfg = small_cfg(dim=128, hidden=256, heads=2, hd=64, nlayers=3, vocab=64, seq=23)
    w = ModelWeights.normal(cfg, seed=21, std=0.08, fp16_round=False)
    lw = w.layers[1].tensors()
    rng = np.random.default_rng(22)
    x = rng.standard_normal((cfg.dim, cfg.seq), dtype=np.float32)
    out = np.zeros_like(x)
    ptrs = (ctypes.POINTER(ctypes.c_float) * 9)(*[orc.fp(np.ascontiguousarray(t)) for t in lw])
    oc = oracle_cfg(orc, cfg)
    orc.lib().orc_layer_forward(ctypes.byref(oc), cfg.seq, ptrs, orc.fp(x), orc.fp(out))
    want = layer_reference64(x.T.astype(np.float64), lw, cfg.heads, cfg.nlayers)
    np.testing.assert_allclose(out.T, want, rtol=1e-4, atol=1e-4)


def test_model_forward_matches_float64(orc):
    cfg = small_cfg(dim=128, hidden=256, heads=2, hd=64, nlayers=2, vocab=96, seq=17)
    w = ModelWeights.normal(cfg, seed=23, std=0.08, fp16_round=False)
    tok, tgt = tokens_uniform(24, cfg.vocab, 1, cfg.seq)
    lg, tl, ml = orc.forward(oracle_cfg(orc, cfg), oracle_weights(orc, w), tok, tgt)
    x = w.embed[tok[0]].astype(np.float64)
    for lw in w.layers:
        x = layer_reference64(x, lw.tensors(), cfg.heads, cfg.nlayers)
    xf = x / np.sqrt((x ** 2).mean(-1, keepdims=True) + 1e-5)
    logits = xf @ w.embed.T.astype(np.float64)
    from scipy.special import logsumexp
    losses = logsumexp(logits, axis=1) - logits[np.arange(cfg.seq), tgt[0]]
    np.testing.assert_allclose(lg[0], logits, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(tl[0], losses, rtol=1e-4, atol=1e-4)
    assert abs(ml[0] - losses.mean()) < 1e-4


def test_softcap_closed_form(orc):
    cfg = small_cfg(dim=128, hidden=256, heads=2, hd=64, nlayers=1, vocab=64, seq=9)
    w = ModelWeights.normal(cfg, seed=25, std=0.3, fp16_round=False)
    tok, tgt = tokens_uniform(26, cfg.vocab, 1, cfg.seq)
    lg0, _, _ = orc.forward(oracle_cfg(orc, cfg), oracle_weights(orc, w), tok, tgt)
    lg1, _, _ = orc.forward(oracle_cfg(orc, cfg, softcap=2.0), oracle_weights(orc, w), tok, tgt)
    np.testing.assert_allclose(lg1, 2.0 * np.tanh(lg0 / 2.0), rtol=1e-5, atol=1e-5)


def test_causality(orc):
    cfg = small_cfg(dim=128, hidden=256, heads=2, hd=64, nlayers=2, vocab=64, seq=16)
    w = ModelWeights.normal(cfg, seed=27, std=0.08, fp16_round=False)
    tok, tgt = tokens_uniform(28, cfg.vocab, 1, cfg.seq)
    lg0, _, _ = orc.forward(oracle_cfg(orc, cfg), oracle_weights(orc, w), tok, tgt)
    tok2 = tok.copy()
    tok2[0, 9] = (tok2[0, 9] + 1) % cfg.vocab
    lg1, _, _ = orc.forward(oracle_cfg(orc, cfg), oracle_weights(orc, w), tok2, tgt)
    np.testing.assert_array_equal(lg0[0, :9], lg1[0, :9])
    assert np.abs(lg0[0, 9:] - lg1[0, 9:]).max() > 0


def test_batch_equals_independent_sequences(orc):
    cfg = small_cfg(dim=128, hidden=256, heads=2, hd=64, nlayers=1, vocab=64, seq=11)
    w = ModelWeights.normal(cfg, seed=29, std=0.08, fp16_round=False)
    tok, tgt = tokens_uniform(30, cfg.vocab, 3, cfg.seq)
    lg, tl, ml = orc.forward(oracle_cfg(orc, cfg), oracle_weights(orc, w), tok, tgt)
    for b in range(3):
        l1, t1, m1 = orc.forward(oracle_cfg(orc, cfg), oracle_weights(orc, w), tok[b], tgt[b])
        np.testing.assert_array_equal(lg[b], l1[0])
        assert ml[b] == m1[0]


def test_decode_cache_matches_forward(orc):
    cfg = small_cfg(dim=128, hidden=256, heads=2, hd=64, nlayers=2, vocab=80, seq=24)
    w = ModelWeights.normal(cfg, seed=31, std=0.08, fp16_round=False)
    tok, tgt = tokens_uniform(32, cfg.vocab, 1, cfg.seq)
    oc, ow = oracle_cfg(orc, cfg), oracle_weights(orc, w)
    lg, _, _ = orc.forward(oc, ow, tok, tgt)
    kv = orc.KV(oc, 64)
    last = kv.prefill(ow, tok[0, :10])
    np.testing.assert_allclose(last, lg[0, 9], rtol=1e-5, atol=1e-5)
    for p in range(10, cfg.seq):
        best, step = kv.step(ow, tok[0, p])
        np.testing.assert_allclose(step, lg[0, p], rtol=1e-5, atol=1e-5)
        assert best == int(np.argmax(lg[0, p]))
    assert kv.pos == cfg.seq


def test_batched_decode_equals_separate_sequences(orc):
    """orc_prefill_batch / orc_decode_step_batch over 3 sequences (prompts of
    equal length, different tokens) against each sequence's own forward: the
    last prefill position and every teacher-forced step equal the forward's
    logits at that position, and a batch of 1 equals orc_decode_step."""
    cfg = small_cfg(dim=128, hidden=256, heads=2, hd=64, nlayers=2, vocab=80, seq=20)
    w = ModelWeights.normal(cfg, seed=34, std=0.08, fp16_round=False)
    tok, tgt = tokens_uniform(35, cfg.vocab, 3, cfg.seq)
    oc, ow = oracle_cfg(orc, cfg), oracle_weights(orc, w)
    lg, _, _ = orc.forward(oc, ow, tok, tgt)
    kb = orc.KVBatch(oc, 3, 32)
    last = kb.prefill(ow, tok[:, :8])
    np.testing.assert_allclose(last, lg[:, 7], rtol=1e-5, atol=1e-5)
    for p in range(8, cfg.seq):
        best, step = kb.step(ow, tok[:, p])
        np.testing.assert_allclose(step, lg[:, p], rtol=1e-5, atol=1e-5)
        np.testing.assert_array_equal(best, np.argmax(lg[:, p], axis=1))
    assert kb.pos == [cfg.seq] * 3
    # batch of 1 == the single-sequence path, bit for bit
    k1, kb1 = orc.KV(oc, 32), orc.KVBatch(oc, 1, 32)
    np.testing.assert_array_equal(k1.prefill(ow, tok[1, :8]), kb1.prefill(ow, tok[1:2, :8])[0])
    b1, s1 = k1.step(ow, tok[1, 8])
    bb, sb = kb1.step(ow, tok[1:2, 8])
    np.testing.assert_array_equal(s1, sb[0])
    assert b1 == bb[0]


def test_oracle_rejects_bad_tokens(orc):
    cfg = small_cfg(dim=128, hidden=256, heads=2, hd=64, nlayers=1, vocab=64, seq=4)
    w = ModelWeights.normal(cfg, seed=33, fp16_round=False)
    tok = np.array([[1, 2, 64, 3]], np.uint32)
    with pytest.raises(ValueError):
        orc.forward(oracle_cfg(orc, cfg), oracle_weights(orc, w), tok, tok)


ROUND_POINTS = ("xn", "q", "k", "v", "p", "attn", "xn2", "gate", "xf")


def forward_fp16_operands_np(w, tok, H, L, points, p_rows):
    """Float64 restatement of the forward with fp16 rounding (numpy's
    round-to-nearest-even) at the named points; 'p' rounds the unnormalised
    probabilities of the rows in p_rows (the row sums stay unrounded)."""
    f16 = lambda a: a.astype(np.float16).astype(np.float64)
    r = lambda name, a: f16(a) if name in points else a
    rms = lambda y, g: y / np.sqrt((y ** 2).mean(-1, keepdims=True) + 1e-5) * g
    x = w.embed[tok].astype(np.float64)
    S, D = x.shape
    hd = D // H
    al = 1 / math.sqrt(2 * L)
    mask = np.triu(np.full((S, S), -np.inf), 1)
    for lw in w.layers:
        wq, wk, wv, wo, w1, w3, w2, g1, g2 = [np.asarray(t, np.float64) for t in lw.tensors()]
        xn = r("xn", rms(x, g1))
        q = r("q", rope_complex((xn @ wq).reshape(S, H, hd)))
        k = r("k", rope_complex((xn @ wk).reshape(S, H, hd)))
        v = r("v", (xn @ wv).reshape(S, H, hd))
        o = np.empty((S, H, hd))
        for h in range(H):
            s = q[:, h] @ k[:, h].T / math.sqrt(hd) + mask
            p = np.exp(s - s.max(-1, keepdims=True))
            l = p.sum(-1, keepdims=True)
            if "p" in points:
                p[p_rows] = f16(p[p_rows])
            o[:, h] = p @ v[:, h] / l
        x = x + al * (r("attn", o.reshape(S, D)) @ wo)
        xn2 = r("xn2", rms(x, g2))
        h1 = xn2 @ w1
        x = x + al * (r("gate", h1 / (1 + np.exp(-h1)) * (xn2 @ w3)) @ w2.T)
    return r("xf", rms(x, w.gamma_final.astype(np.float64))) @ w.embed.T.astype(np.float64)


def test_fp16_operand_mode_matches_rounding_restatement(orc):
    """Each rounding point of the oracle's fp16-operand mode, alone, against
    the float64 restatement rounding at the same point: their difference is
    a small fraction of that point's own effect on the logits (RMS ratio
    <= 0.25; rounding at another place, e.g. q before RoPE or the gate before
    the SiLU product, gives a ratio near 1).  Rounded chains cannot agree bit
    for bit -- the two compute each pre-rounding value in a different order,
    and every later rounding turns that tiny difference into an ulp -- so the
    points are checked one at a time.  Decode steps keep P in fp32: with only
    the probability point set, a step equals the fp32 oracle's step."""
    cfg = small_cfg(dim=128, hidden=256, heads=2, hd=64, nlayers=2, vocab=96, seq=40)
    w = ModelWeights.normal(cfg, seed=37, std=0.08)
    tok, tgt = tokens_uniform(38, cfg.vocab, 1, cfg.seq)
    ow = oracle_weights(orc, w)
    S = cfg.seq
    rms = lambda a: float(np.sqrt((np.asarray(a, np.float64) ** 2).mean()))
    lg32, _, _ = orc.forward(oracle_cfg(orc, cfg), ow, tok, tgt)
    ref32 = forward_fp16_operands_np(w, tok[0], cfg.heads, cfg.nlayers, [], np.arange(S))
    assert np.abs(lg32[0] - ref32).max() < 1e-4

    def cfg16(bits):
        return orc.make_config(cfg.dim, cfg.hidden, cfg.heads, cfg.nlayers, cfg.vocab, head_dim=cfg.hd,
                               fp16_operands=bits)

    for pt in ROUND_POINTS:
        lg, _, _ = orc.forward(cfg16(orc.F16_POINTS[pt]), ow, tok, tgt)
        ref = forward_fp16_operands_np(w, tok[0], cfg.heads, cfg.nlayers, [pt], np.arange(S))
        effect, match = rms(lg[0] - lg32[0]), rms(lg[0] - ref)
        assert effect > 5e-5, (pt, effect)
        assert match <= 0.25 * effect, (pt, match, effect)
    # all points: the effect is the sum of the parts (no point cancels another)
    lg_all, _, _ = orc.forward(cfg16(True), ow, tok, tgt)
    ref_all = forward_fp16_operands_np(w, tok[0], cfg.heads, cfg.nlayers, ROUND_POINTS, np.arange(S))
    assert rms(lg_all[0] - lg32[0]) == pytest.approx(rms(ref_all - ref32), rel=0.3)
    # decode steps keep the probabilities in fp32: from a one-token prefill
    # (P = 1 exactly, nothing to round) every step equals the fp32 oracle's
    kvp, kv32 = orc.KV(cfg16(orc.F16_POINTS["p"]), S + 1), orc.KV(oracle_cfg(orc, cfg), S + 1)
    kvp.prefill(ow, tok[0, :1])
    kv32.prefill(ow, tok[0, :1])
    for t in tok[0, 1:12]:
        np.testing.assert_array_equal(kvp.step(ow, int(t))[1], kv32.step(ow, int(t))[1])
