"""GPU parity of the optimizer and the training step (full_model.rs:1123-1600).

* The fused AdamW kernels against the oracle's step_fused on identical
  inputs (the GPU's own gradients and pre-update weights): bit-exact fp32
  masters, both operations in the reference's order without FMA contraction.
  The fp16 device copy the same pass writes must equal the masters rounded
  (checked through a forward of a second context loaded from the masters).
* The gradient norm against numpy.
* rh_train_step end to end against the oracle's restatement of
  train_step_with_options: same microbatch positions, losses, clip decision
  and update (to the fp16 gradient tolerance), determinism, and the
  reference's training property checks (phase4_pretraining_checks.rs:95-170:
  every weight group moves; an overfit run lowers the loss)."""
import numpy as np
import pytest

from rustane_amd import hip_bridge as hb
from rustane_amd.engine import ModelWeights

from helpers import LOSS_RTOL, oracle_cfg, oracle_weights, random_gammas, small_cfg, tokens_uniform

pytestmark = pytest.mark.gpu


def _cfg():
    return small_cfg(dim=256, hidden=512, heads=2, hd=128, nlayers=2, vocab=1024, seq=64)


def _load(c, w):
    c.load_weights(w.embed, w.gamma_final, [lw.tensors() for lw in w.layers])


def _flat(e, g, layers):
    return [e, g] + [t for lw in layers for t in lw]


def test_adamw_kernels_bit_exact_and_fp16_copy(orc):
    cfg = _cfg()
    w = random_gammas(ModelWeights.normal(cfg, seed=101, std=0.05), 102)
    tok, tgt = tokens_uniform(103, cfg.vocab, 2, cfg.seq)
    tc = hb.train_config(weight_decay=0.1, matrix_lr_scale=0.05, embed_lr_scale=5.0)
    otc = orc.TrainConfig(beta1=tc.beta1, beta2=tc.beta2, eps=tc.eps, weight_decay=tc.weight_decay,
                          matrix_lr_scale=tc.matrix_lr_scale, embed_lr_scale=tc.embed_lr_scale)
    print("[case] AdamW kernels vs oracle step_fused, 2 steps", flush=True)
    with hb.Context(cfg.to_rh(), 0, 2, 0) as c:
        _load(c, w)
        e0, g0, l0 = c.read_weights()
        ow = orc.Weights(e0, g0, l0)
        opt = orc.OptState(ow)
        for t, lr, gs in [(1, 1e-3, 1.0 / 512), (2, 7e-4, 1.0 / 300)]:
            c.zero_grads()
            c.forward_backward(tok, tgt, loss_scale=256.0)
            ge, gg, gl = c.read_grads()
            og = orc.Grads(ow)
            for dst, src in zip(_flat(og.embed, og.gamma_final, og.layers), _flat(ge, gg, gl)):
                dst[...] = src
            c.update_weights(t, lr, tc, gs)
            orc.update_weights(ow, og, opt, t, lr, otc, gs)
            e1, g1, l1 = c.read_weights()
            for got, want in zip(_flat(e1, g1, l1), _flat(ow.embed, ow.gamma_final, ow.layers)):
                np.testing.assert_array_equal(got, want)
        # the fp16 copy written by the same pass == the masters rounded to fp16
        out = c.forward(tok, tgt)
    with hb.Context(cfg.to_rh(), 0, 2, 0) as c2:
        c2.load_weights(e1, g1, l1)
        out2 = c2.forward(tok, tgt)
    np.testing.assert_array_equal(out.logits, out2.logits)


def test_grad_norm_matches_numpy():
    cfg = _cfg()
    w = ModelWeights.normal(cfg, seed=104, std=0.05)
    tok, tgt = tokens_uniform(105, cfg.vocab, 1, cfg.seq)
    print("[case] grad norm", flush=True)
    with hb.Context(cfg.to_rh(), 0, 1, 0) as c:
        _load(c, w)
        c.forward_backward(tok, tgt, loss_scale=4.0)
        n = c.grad_norm()
        g = c.read_grads()
        c.zero_grads()
        assert c.grad_norm() == 0.0
    want = np.sqrt(sum(float((t.astype(np.float64) ** 2).sum()) for t in _flat(*g)))
    assert n == pytest.approx(want, rel=1e-5)


def _token_file(path, n, vocab, seed):
    rng = np.random.default_rng(seed)
    rng.integers(0, vocab, size=n).astype("<u2").tofile(path)
    return np.fromfile(path, "<u2").astype(np.uint32)


def oracle_train_step(orc, ocfg, ow, og_unused, opt, data, step, otc, seq):
    """train_step_with_options (full_model.rs:1510-1600) over the oracle."""
    g = orc.Grads(ow)
    max_pos = len(data) - seq - 1
    total = np.float32(0.0)
    for micro in range(otc.accum_steps):
        pos = (step * 7919 + micro * 104729) % max_pos
        tok, tgt = data[pos:pos + seq][None], data[pos + 1:pos + seq + 1][None]
        _, ml = orc.forward_backward(ocfg, ow, np.ascontiguousarray(tok), np.ascontiguousarray(tgt), grads=g,
                                     loss_scale=otc.loss_scale)
        total = np.float32(total + np.float32(ml[0]))
    scaled, combined, lr = orc.train_update(ow, g, opt, step, otc)
    return float(total / np.float32(otc.accum_steps)), scaled


@pytest.mark.parametrize("clip", [1.0, 1e-4])
def test_train_step_matches_oracle(orc, tmp_path, clip):
    """accum_steps 3 with max_batch 2 (one batch of 2, one of 1), two steps;
    clip 1e-4 forces the clipped branch."""
    cfg = _cfg()
    w = random_gammas(ModelWeights.normal(cfg, seed=106, std=0.05), 107)
    data = _token_file(str(tmp_path / "train.bin"), 5000, cfg.vocab, 108)
    kw = dict(max_lr=1e-3, warmup_steps=2, total_steps=10, accum_steps=3, loss_scale=256.0, grad_clip=clip)
    tc = hb.train_config(**kw)
    otc = orc.TrainConfig(**kw)
    ow = oracle_weights(orc, w)
    opt = orc.OptState(ow)
    print(f"[case] train_step vs oracle, clip {clip}", flush=True)
    td = hb.TokenData(str(tmp_path / "train.bin"))
    with hb.Context(cfg.to_rh(), 0, 2, 0) as c:
        _load(c, w)
        e0, _, l0 = c.read_weights()
        for step in range(2):
            loss, norm = c.train_step(td, step, tc)
            oloss, onorm = oracle_train_step(orc, oracle_cfg(orc, cfg), ow, None, opt, data, step, otc, cfg.seq)
            print(f"[result] step {step}: loss {loss:.6f} vs {oloss:.6f}, norm {norm:.5g} vs {onorm:.5g}",
                  flush=True)
            assert loss == pytest.approx(oloss, rel=LOSS_RTOL)
            assert norm == pytest.approx(onorm, rel=2e-2)
            assert (norm > clip) == (onorm > clip)
        e1, g1, l1 = c.read_weights()
    td.close()
    # Adam's early updates are about lr * sign(gradient): an update of the
    # GPU and of the oracle agree wherever the gradient signs agree; compare
    # the update vectors of every tensor by cosine and their mean difference.
    for name, got, want, before, lr_g in [("embed", e1, ow.embed, e0, 5e-3)] + \
            [(f"l{l}.{j}", l1[l][j], ow.layers[l][j], l0[l][j], 1e-3 * (0.05 if j < 7 else 1))
             for l in range(cfg.nlayers) for j in range(9)]:
        du, dw = (got - before).ravel().astype(np.float64), (want - before).ravel().astype(np.float64)
        cs = du @ dw / (np.linalg.norm(du) * np.linalg.norm(dw) + 1e-300)
        assert cs >= 0.98, f"{name}: update cosine {cs:.4f}"
        assert np.abs(du - dw).mean() <= 0.1 * lr_g * 2, name


def test_train_step_deterministic_moves_all_weights_and_overfits(tmp_path):
    """Two runs from the same weights give identical results; every weight
    group moves (phase4_pretraining_checks.rs:95-170); 30 steps on a short
    repeated sequence lower the loss (an overfit check, :309-380)."""
    cfg = _cfg()
    w = ModelWeights.normal(cfg, seed=109, std=0.05)
    # a 70-token corpus: every window is the same few tokens, easy to memorise
    rng = np.random.default_rng(110)
    base = rng.integers(0, cfg.vocab, size=8)
    np.tile(base, 9).astype("<u2")[:70].tofile(str(tmp_path / "rep.bin"))
    td = hb.TokenData(str(tmp_path / "rep.bin"))
    tc = hb.train_config(max_lr=3e-3, warmup_steps=1, total_steps=40, accum_steps=2, weight_decay=0.0,
                         matrix_lr_scale=1.0, embed_lr_scale=1.0, loss_scale=1.0)
    print("[case] train_step determinism / overfit", flush=True)
    runs = []
    for _ in range(2):
        with hb.Context(cfg.to_rh(), 0, 2, 0) as c:
            _load(c, w)
            before = c.read_weights()
            losses = [c.train_step(td, s, tc)[0] for s in range(30)]
            runs.append((losses, c.read_weights(), before))
    td.close()
    (l1, w1, b1), (l2, w2, _) = runs
    assert l1 == l2
    for a, b in zip(_flat(*w1), _flat(*w2)):
        np.testing.assert_array_equal(a, b)
    for a, b in zip(_flat(*w1), _flat(*b1)):
        assert np.abs(a - b).max() > 0
    print(f"[result] overfit loss {l1[0]:.4f} -> {l1[-1]:.4f}", flush=True)
    assert l1[-1] < 0.7 * l1[0]
