"""GPU parity of the training pass (forward + backward): every gradient of the
HIP path vs the CPU oracle's backward (itself pinned by float64 autograd and
the reference's numerical-gradient KATs).

Weights are N(0, std) rounded through fp16 with non-unit gammas (both sides
see identical parameters).  The GPU runs the GEMMs on fp16 operands with fp32
accumulation, so the bar is a tolerance: per gradient tensor, cosine >= 0.999
and max |error| <= 3e-2 x max |gradient| (the reference's own backward checks
are looser: phase4_pretraining_checks.rs compares ANE and CPU gradients by
cosine > 0.9).  Losses agree to 1e-3 relative.

The two-call form (rh_forward_train -> ForwardResult, then rh_backward, as
full_model::forward / full_model::backward) gives the fused call's gradients
bit for bit."""
import numpy as np
import pytest

from rustane_amd import hip_bridge as hb
from rustane_amd.engine import ModelWeights, cfg_600m, cfg_7b, tiny_config

from helpers import LOSS_RTOL, cosine, oracle_cfg, oracle_weights, random_gammas, small_cfg, tokens_uniform

pytestmark = pytest.mark.gpu

NAMES = ["wq", "wk", "wv", "wo", "w1", "w3", "w2", "gamma1", "gamma2"]
GRAD_REL = 3e-2
GRAD_COS = 0.999


def _pairs(gpu, ref):
    ge, gg, gl = gpu
    out = [("embed", ge, ref.embed), ("gamma_final", gg, ref.gamma_final)]
    for l, (a, b) in enumerate(zip(gl, ref.layers)):
        out += [(f"layer{l}.{n}", x, y) for n, x, y in zip(NAMES, a, b)]
    return out


def _check_grads(gpu, ref, rel=GRAD_REL, cos=GRAD_COS):
    worst = 0.0
    for name, got, want in _pairs(gpu, ref):
        assert np.isfinite(got).all(), name
        scale = float(np.abs(want).max())
        err = float(np.abs(got - want).max()) / scale
        cs = cosine(got, want)
        worst = max(worst, err)
        assert err <= rel and cs >= cos, f"{name}: max err {err:.2e} of {scale:.2e}, cosine {cs:.6f}"
    return worst


def _run(orc, cfg, w, tok, tgt, softcap=0.0, loss_scale=1.0, calls=1):
    B, S = tok.shape
    print(f"[case] backward dim={cfg.dim} F={cfg.hidden} L={cfg.nlayers} V={cfg.vocab} hd={cfg.hd} "
          f"B={B} S={S} softcap={softcap} loss_scale={loss_scale}", flush=True)
    with hb.Context(cfg.to_rh(softcap), 0, B, 0) as c:
        c.load_weights(w.embed, w.gamma_final, [lw.tensors() for lw in w.layers])
        for _ in range(calls):
            ml = c.forward_backward(tok, tgt, loss_scale)
        g = c.read_grads()
    ow = oracle_weights(orc, w)
    og = None
    for _ in range(calls):
        og, oml = orc.forward_backward(oracle_cfg(orc, cfg, softcap), ow, tok, tgt, grads=og,
                                       loss_scale=loss_scale)
    np.testing.assert_allclose(ml, oml, rtol=LOSS_RTOL)
    worst = _check_grads(g, og)
    print(f"[result] worst max-err ratio {worst:.3e}", flush=True)
    return g, og


def test_backward_small_matches_oracle(orc):
    cfg = small_cfg(dim=256, hidden=512, heads=2, hd=128, nlayers=2, vocab=1024, seq=64)
    w = random_gammas(ModelWeights.normal(cfg, seed=81, std=0.05), 82)
    tok, tgt = tokens_uniform(83, cfg.vocab, 1, cfg.seq)
    _run(orc, cfg, w, tok, tgt)


def test_backward_batch_ragged_softcap_loss_scale(orc):
    """B=3, S=100 (not a multiple of the 64-token attention blocks or of
    128), V=1000 (padded to 1024 inside), softcap 30, loss_scale 256."""
    cfg = small_cfg(dim=256, hidden=768, heads=2, hd=128, nlayers=2, vocab=1000, seq=100)
    w = random_gammas(ModelWeights.normal(cfg, seed=84, std=0.05), 85)
    tok, tgt = tokens_uniform(86, cfg.vocab, 3, cfg.seq)
    _run(orc, cfg, w, tok, tgt, softcap=30.0, loss_scale=256.0)


def test_backward_tiny_config_hd64(orc):
    """Tiny Llama-style decoder: 512/1408/8L/8h(hd 64)/V8192/S256."""
    cfg = tiny_config()
    w = random_gammas(ModelWeights.normal(cfg, seed=87, std=0.05), 88)
    tok, tgt = tokens_uniform(89, cfg.vocab, 1, cfg.seq)
    _run(orc, cfg, w, tok, tgt)


def test_backward_accumulates_and_is_deterministic(orc):
    """Two calls add up (the reference's ModelGrads accumulate); a repeated
    pass from zeroed gradients is bit-identical."""
    cfg = small_cfg(dim=256, hidden=512, heads=2, hd=128, nlayers=2, vocab=1024, seq=64)
    w = ModelWeights.normal(cfg, seed=90, std=0.05)
    tok, tgt = tokens_uniform(91, cfg.vocab, 2, cfg.seq)
    print("[case] backward accumulation / determinism", flush=True)
    with hb.Context(cfg.to_rh(), 0, 2, 0) as c:
        c.load_weights(w.embed, w.gamma_final, [lw.tensors() for lw in w.layers])
        c.forward_backward(tok, tgt)
        one = c.read_grads()
        c.forward_backward(tok, tgt)
        two = c.read_grads()
        c.zero_grads()
        c.forward_backward(tok, tgt)
        again = c.read_grads()
    flat = lambda g: [g[0], g[1]] + [t for lw in g[2] for t in lw]
    for a, b, r in zip(flat(one), flat(two), flat(again)):
        np.testing.assert_array_equal(a, r)
        np.testing.assert_allclose(b, 2 * a, rtol=1e-5, atol=1e-6 * np.abs(a).max())
    assert all(np.abs(t).max() > 0 for t in flat(one))  # every weight group gets a gradient


def test_backward_workspace_growth_between_calls(orc):
    """B 1, then B 2 (the activation caches, operand copies and activation
    gradients are reallocated while the weight-gradient stream exists), then
    B 1 again: the accumulated gradients equal the oracle's three calls."""
    cfg = small_cfg(dim=256, hidden=512, heads=2, hd=128, nlayers=2, vocab=1024, seq=64)
    w = random_gammas(ModelWeights.normal(cfg, seed=93, std=0.05), 94)
    t1, g1 = tokens_uniform(95, cfg.vocab, 1, cfg.seq)
    t2, g2 = tokens_uniform(96, cfg.vocab, 2, cfg.seq)
    print("[case] backward workspace growth B1 -> B2 -> B1", flush=True)
    with hb.Context(cfg.to_rh(), 0, 2, 0) as c:
        c.load_weights(w.embed, w.gamma_final, [lw.tensors() for lw in w.layers])
        for tok, tgt in ((t1, g1), (t2, g2), (t1, g1)):
            c.forward_backward(tok, tgt)
        got = c.read_grads()
    ow, oc, og = oracle_weights(orc, w), oracle_cfg(orc, cfg), None
    for tok, tgt in ((t1, g1), (t2, g2), (t1, g1)):
        og, _ = orc.forward_backward(oc, ow, tok, tgt, grads=og)
    _check_grads(got, og)


def test_backward_weights_reload_rebuilds_transposed_copies(orc):
    """New weights after a backward must be seen by the next backward (the
    data-gradient GEMMs read transposed copies built per weight version)."""
    cfg = small_cfg(dim=256, hidden=512, heads=2, hd=128, nlayers=1, vocab=1024, seq=64)
    w1 = ModelWeights.normal(cfg, seed=92, std=0.05)
    w2 = random_gammas(ModelWeights.normal(cfg, seed=93, std=0.05), 94)
    tok, tgt = tokens_uniform(95, cfg.vocab, 1, cfg.seq)
    print("[case] backward after a weight reload", flush=True)
    with hb.Context(cfg.to_rh(), 0, 1, 0) as c:
        c.load_weights(w1.embed, w1.gamma_final, [lw.tensors() for lw in w1.layers])
        c.forward_backward(tok, tgt)
        c.zero_grads()
        c.load_weights(w2.embed, w2.gamma_final, [lw.tensors() for lw in w2.layers])
        c.forward_backward(tok, tgt)
        g = c.read_grads()
    og, _ = orc.forward_backward(oracle_cfg(orc, cfg), oracle_weights(orc, w2), tok, tgt)
    _check_grads(g, og)


@pytest.mark.parametrize("name", ["600m", "7b"])
def test_backward_model_widths_match_oracle(orc, name):
    """The real GEMM/attention shapes (seq 512, vocab 32000) with the depth
    cut to two layers; weights N(0, 0.02) generated on the device."""
    cfg = {"600m": cfg_600m, "7b": cfg_7b}[name]()
    cfg.nlayers = 2
    tok, tgt = tokens_uniform(96, cfg.vocab, 1, cfg.seq)
    print(f"[case] backward {name} width dim={cfg.dim} F={cfg.hidden} L=2 S={cfg.seq}", flush=True)
    with hb.Context(cfg.to_rh(), 0, 1, 0) as c:
        c.init_normal(seed=97, std=0.02)
        ml = c.forward_backward(tok, tgt)
        g = c.read_grads()
        embed, gf, layers = c.read_weights()
    og, oml = orc.forward_backward(oracle_cfg(orc, cfg), orc.Weights(embed, gf, layers), tok, tgt)
    np.testing.assert_allclose(ml, oml, rtol=LOSS_RTOL)
    worst = _check_grads(g, og)
    print(f"[result] {name}: worst max-err ratio {worst:.3e}", flush=True)


@pytest.mark.parametrize("softcap", [0.0, 30.0])
def test_forward_then_backward_equals_fused_call(softcap):
    """full_model::forward -> ForwardResult, full_model::backward(&fwd)
    (crates/engine/tests/phase4_training.rs:61-72) against rh_forward_backward:
    losses, gradients and, after a second backward of the same forward, the
    accumulated gradients are bit-identical; the returned norm is
    rh_grad_norm's."""
    cfg = small_cfg(dim=256, hidden=512, heads=2, hd=128, nlayers=2, vocab=1000, seq=64)
    w = random_gammas(ModelWeights.normal(cfg, seed=231, std=0.05), seed=232)
    tok, tgt = tokens_uniform(233, cfg.vocab, 2, cfg.seq)
    print(f"[case] forward_train + backward vs forward_backward, softcap {softcap}", flush=True)
    with hb.Context(cfg.to_rh(softcap), 0, 2, 0) as c:
        c.load_weights(w.embed, w.gamma_final, [lw.tensors() for lw in w.layers])
        ml_fused = c.forward_backward(tok, tgt, 256.0)
        g1 = c.read_grads()
        n1 = c.grad_norm()
        c.forward_backward(tok, tgt, 256.0)
        g2 = c.read_grads()
    with hb.Context(cfg.to_rh(), 0, 2, 0) as c:  # the context's own softcap stays 0
        c.load_weights(w.embed, w.gamma_final, [lw.tensors() for lw in w.layers])
        fwd, ml = c.forward_train(tok, tgt, softcap=softcap)
        np.testing.assert_array_equal(ml, ml_fused)
        n = c.backward(fwd, tok, softcap=softcap, loss_scale=256.0)
        assert n == n1
        for (name, a, _), (_, b, _) in zip(_pairs(c.read_grads(), _Ref(g1)), _pairs(g1, _Ref(g1))):
            np.testing.assert_array_equal(a, b, err_msg=name)
        c.backward(fwd, softcap=softcap, loss_scale=256.0)
        for (name, a, _), (_, b, _) in zip(_pairs(c.read_grads(), _Ref(g2)), _pairs(g2, _Ref(g2))):
            np.testing.assert_array_equal(a, b, err_msg=name)
        fwd.close()


def test_backward_refuses_stale_or_mismatched_forward():
    cfg = small_cfg(dim=256, hidden=512, heads=2, hd=128, nlayers=1, vocab=512, seq=32)
    w = ModelWeights.normal(cfg, seed=234, std=0.05)
    tok, tgt = tokens_uniform(235, cfg.vocab, 1, cfg.seq)
    print("[case] stale and mismatched forward results", flush=True)
    with hb.Context(cfg.to_rh(), 0, 1, 64) as c:
        c.load_weights(w.embed, w.gamma_final, [lw.tensors() for lw in w.layers])
        fwd, _ = c.forward_train(tok, tgt)
        other = tok.copy()
        other[0, 3] = (other[0, 3] + 1) % cfg.vocab
        for kw, code in [(dict(tokens=other), hb.RH_EINVAL), (dict(softcap=5.0), hb.RH_EINVAL)]:
            with pytest.raises(hb.HipBridgeError) as e:
                c.backward(fwd, **kw)
            assert e.value.code == code
        c.backward(fwd, want_norm=False)  # still valid after the refused calls
        for run in (lambda: c.forward(tok, tgt), lambda: c.prefill(tok[:, :10]),
                    lambda: c.forward_train(tok, tgt)[0].close()):
            fwd.close()
            fwd, _ = c.forward_train(tok, tgt)
            run()
            with pytest.raises(hb.HipBridgeError) as e:
                c.backward(fwd)
            assert e.value.code == hb.RH_ESTATE
        fwd.close()


class _Ref:
    """Adapts a read_grads() triple to _pairs' second argument."""

    def __init__(self, g):
        self.embed, self.gamma_final, self.layers = g
