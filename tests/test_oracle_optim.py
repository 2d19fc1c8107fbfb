"""Pins the oracle's optimizer (test infrastructure): the reference's Adam
unit tests (cpu/adam.rs:138-190), AdamW against an independent float64
restatement, the learning-rate schedule's end points (full_model.rs:903-913),
the global gradient norm against numpy, and the clip rule of
train_step_with_options (full_model.rs:1573-1600)."""
import numpy as np
import pytest

# AdamConfig::default (cpu/adam.rs:20-30)
LR, B1, B2, EPS, WD = 1e-3, 0.9, 0.999, 1e-8, 0.01


def test_adam_moves_toward_minimum(orc):  # adam.rs:138-156
    p = np.full(4, 5.0, np.float32)
    g = np.ones(4, np.float32)
    m, v = np.zeros(4, np.float32), np.zeros(4, np.float32)
    before = p.sum()
    for t in range(1, 11):
        orc.adam_step_fused(p, g, m, v, t, LR, B1, B2, EPS, WD, 1.0)
    assert p.sum() < before


def test_adam_zero_grad_only_weight_decay(orc):  # adam.rs:158-172
    p = np.ones(2, np.float32)
    m, v = np.zeros(2, np.float32), np.zeros(2, np.float32)
    orc.adam_step_fused(p, np.zeros(2, np.float32), m, v, 1, LR, B1, B2, EPS, 0.1, 1.0)
    assert p[0] < 1.0
    np.testing.assert_allclose(p, 1.0 - LR * 0.1, rtol=1e-7)  # update = 0/(0 + eps) = 0


def test_adam_momentum_accumulates(orc):  # adam.rs:174-190
    p = np.zeros(2, np.float32)
    m, v = np.zeros(2, np.float32), np.zeros(2, np.float32)
    orc.adam_step_fused(p, np.ones(2, np.float32), m, v, 1, LR, B1, B2, EPS, 0.0, 1.0)
    assert abs(m[0] - 0.1) < 1e-6 and abs(v[0] - 0.001) < 1e-6
    np.testing.assert_allclose(p, -LR, rtol=1e-6)  # first step: |update| = 1


def test_adamw_matches_float64_restatement(orc):
    rng = np.random.default_rng(5)
    n, lr, b1, b2, eps, wd, gs = 1000, 3e-3, 0.9, 0.95, 1e-8, 0.1, 0.25
    p = rng.standard_normal(n).astype(np.float32)
    m, v = np.zeros(n, np.float32), np.zeros(n, np.float32)
    P, M, V = p.astype(np.float64), np.zeros(n), np.zeros(n)
    for t in range(1, 6):
        g = rng.standard_normal(n).astype(np.float32)
        orc.adam_step_fused(p, g, m, v, t, lr, b1, b2, eps, wd, gs)
        G = g.astype(np.float64) * gs
        M = b1 * M + (1 - b1) * G
        V = b2 * V + (1 - b2) * G * G
        upd = (M / (1 - b1 ** t)) / (np.sqrt(V / (1 - b2 ** t)) + eps)
        P = P - lr * (upd + wd * P)
    np.testing.assert_allclose(p, P, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(m, M, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(v, V, rtol=1e-5, atol=1e-9)


def test_powi_matches_pow(orc):
    for b in (0.9, 0.95, 0.999):
        bf = float(np.float32(b))  # the fp32 base the function receives
        for t in (1, 2, 7, 100, 1000):
            want = bf ** t
            # fp32 squarings: relative error grows with t; fp32 underflows below 1.2e-38
            assert abs(orc.lib().orc_powi(b, t) - want) <= 1.2e-7 * t * want + 1.2e-38


def test_learning_rate_schedule(orc):
    tc = orc.TrainConfig(max_lr=3e-4, min_lr_frac=0.1, warmup_steps=100, total_steps=10000)
    assert orc.learning_rate(0, tc) == pytest.approx(3e-6, rel=1e-6)
    assert orc.learning_rate(99, tc) == pytest.approx(3e-4, rel=1e-6)
    assert orc.learning_rate(100, tc) == pytest.approx(3e-4, rel=1e-6)     # cos(0) = 1
    assert orc.learning_rate(5050, tc) == pytest.approx(0.55 * 3e-4, rel=1e-5)  # cos(pi/2) = 0
    assert orc.learning_rate(10000, tc) == pytest.approx(3e-5, rel=1e-5)   # cos(pi) = -1


def _weights(orc, seed):
    from rustane_amd.engine import ModelWeights
    from helpers import oracle_weights, small_cfg
    cfg = small_cfg(dim=64, hidden=128, heads=2, hd=32, nlayers=3, vocab=96, seq=8)
    return cfg, oracle_weights(orc, ModelWeights.normal(cfg, seed=seed, std=0.1, fp16_round=False))


def test_grad_norm_matches_numpy(orc):
    cfg, w = _weights(orc, 6)
    g = orc.Grads(w)
    rng = np.random.default_rng(7)
    for a in [g.embed, g.gamma_final] + [t for lw in g.layers for t in lw]:
        a[...] = rng.standard_normal(a.shape).astype(np.float32)
    flat = np.concatenate([a.ravel().astype(np.float64) for a in
                           [g.embed, g.gamma_final] + [t for lw in g.layers for t in lw]])
    assert orc.grad_norm(g) == pytest.approx(float(np.sqrt((flat ** 2).sum())), rel=1e-5)


@pytest.mark.parametrize("big", [False, True])
def test_train_update_clip_rule_and_groups(orc, big):
    """combined scale = clip/raw when raw*gsc > clip, else gsc; embed at
    lr*embed_lr_scale without decay, matrices at lr*matrix_lr_scale with
    decay, gammas at lr without decay."""
    cfg, w = _weights(orc, 8)
    g = orc.Grads(w)
    rng = np.random.default_rng(9)
    scale = 1e4 if big else 1e-2
    for a in [g.embed, g.gamma_final] + [t for lw in g.layers for t in lw]:
        a[...] = (rng.standard_normal(a.shape) * scale).astype(np.float32)
    tc = orc.TrainConfig(accum_steps=2, loss_scale=256.0, grad_clip=1.0, warmup_steps=10, total_steps=100)
    before = [w.embed.copy(), w.layers[0][0].copy(), w.layers[0][7].copy()]
    o = orc.OptState(w)
    scaled, combined, lr = orc.train_update(w, g, o, 0, tc)  # step 0 -> t = 1
    raw = orc.grad_norm(g)
    gsc = 1.0 / (2 * 256.0)
    assert scaled == pytest.approx(raw * gsc, rel=1e-6)
    assert combined == pytest.approx(1.0 / raw if big else gsc, rel=1e-6)
    assert lr == pytest.approx(3e-4 * 1 / 10, rel=1e-6)
    # first Adam step in closed form: m_hat = g, v_hat = g^2, so the update
    # is g / (|g| + eps) with g = grad * combined scale
    for b, after, glr, wd, grad in [(before[0], w.embed, lr * 5.0, 0.0, g.embed),
                                    (before[1], w.layers[0][0], lr * 0.05, 0.1, g.layers[0][0]),
                                    (before[2], w.layers[0][7], lr, 0.0, g.layers[0][7])]:
        gg = grad.astype(np.float64) * combined
        want = b - glr * (gg / (np.abs(gg) + 1e-8) + wd * b)
        np.testing.assert_allclose(after, want, rtol=1e-4, atol=glr * 1e-4)
