"""GPU parity of the greedy decode path (KV cache + GEMV + split-context
attention + argmax) against the CPU oracle.

Contract (no reference implementation exists; crates/metal-decode/src/lib.rs:1-8
only plans it): decode logits at position p equal the forward's logits at p,
and greedy token ids equal the oracle's.  Where the oracle's top-2 margin is
within the fp16 tolerance the argmax is a near-tie; the test then requires
the GPU's pick to be within tolerance of the oracle max and stops comparing
the free-running sequences there (they legitimately diverge)."""
import numpy as np
import pytest

from rustane_amd import hip_bridge as hb
from rustane_amd.engine import ModelConfig, ModelWeights

from helpers import LOGIT_ATOL, oracle_cfg, oracle_weights, random_gammas, small_cfg, tokens_uniform

pytestmark = pytest.mark.gpu


def _ctx(cfg, w, max_batch, max_ctx):
    print(f"[case] decode ctx dim={cfg.dim} L={cfg.nlayers} hd={cfg.hd} B={max_batch} ctx={max_ctx}",
          flush=True)
    c = hb.Context(cfg.to_rh(), 0, max_batch, max_ctx)
    c.load_weights(w.embed, w.gamma_final, [lw.tensors() for lw in w.layers])
    return c


def _margin(lg):
    s = np.sort(lg)
    return float(s[-1] - s[-2])


def test_prefill_and_teacher_forced_steps_match_forward(orc):
    cfg = small_cfg(seq=48)
    w = ModelWeights.normal(cfg, seed=41)
    tok, tgt = tokens_uniform(42, cfg.vocab, 2, cfg.seq)
    lg, _, _ = orc.forward(oracle_cfg(orc, cfg), oracle_weights(orc, w), tok, tgt)
    p0 = 20
    with _ctx(cfg, w, 2, 64) as c:
        nxt, last = c.prefill(tok[:, :p0], want_logits=True)
        assert np.abs(last - lg[:, p0 - 1]).max() <= LOGIT_ATOL
        for b in range(2):
            if _margin(lg[b, p0 - 1]) > 2 * LOGIT_ATOL:
                assert nxt[b] == np.argmax(lg[b, p0 - 1])
        worst = 0.0
        for p in range(p0, cfg.seq):
            out, dl = c.decode_step(tok[:, p], want_logits=True)
            worst = max(worst, float(np.abs(dl - lg[:, p]).max()))
            for b in range(2):
                if _margin(lg[b, p]) > 2 * LOGIT_ATOL:
                    assert out[b] == np.argmax(lg[b, p]), (p, b)
        assert c.pos == cfg.seq
    print(f"[result] worst decode logit error {worst:.3e}", flush=True)
    assert worst <= LOGIT_ATOL


def _oracle_greedy(orc, cfg, w, prompt, nsteps):
    kv = orc.KV(oracle_cfg(orc, cfg), len(prompt) + nsteps + 1)
    ow = oracle_weights(orc, w)
    lg = kv.prefill(ow, prompt)
    toks, logits = [int(np.argmax(lg))], [lg]
    for _ in range(nsteps):
        best, lg = kv.step(ow, toks[-1])
        toks.append(best)
        logits.append(lg)
    return toks, logits


@pytest.mark.parametrize("graphs", [True, False])
def test_greedy_decode_matches_oracle(orc, graphs):
    cfg = small_cfg(dim=256, hidden=512, heads=2, hd=128, nlayers=2, vocab=512, seq=40)
    w = ModelWeights.normal(cfg, seed=43, std=0.05)
    prompt, _ = tokens_uniform(44, cfg.vocab, 1, 40)
    nsteps = 32
    otoks, ologits = _oracle_greedy(orc, cfg, w, prompt[0], nsteps)
    with _ctx(cfg, w, 1, 128) as c:
        c.set_graphs(graphs)
        nxt, _ = c.prefill(prompt)
        gtoks = [int(nxt[0])] + [int(t) for t in c.decode(nxt, nsteps)[:, 0]]
    compared = 0
    for i, (g, o) in enumerate(zip(gtoks, otoks)):
        lg = ologits[i]
        if g != o:
            assert _margin(lg) <= 2 * LOGIT_ATOL and lg[o] - lg[g] <= 2 * LOGIT_ATOL, (i, g, o)
            break
        compared += 1
    print(f"[result] greedy: {compared} of {len(otoks)} tokens identical (graphs={graphs})", flush=True)
    assert compared >= 16


def test_graph_and_eager_decode_identical():
    cfg = small_cfg(seq=16)
    w = ModelWeights.normal(cfg, seed=45)
    prompt, _ = tokens_uniform(46, cfg.vocab, 3, 16)
    outs = []
    for graphs in (False, True):
        with _ctx(cfg, w, 3, 64) as c:
            c.set_graphs(graphs)
            nxt, _ = c.prefill(prompt)
            seq = c.decode(nxt, 12)
            more, lgs = c.decode_step(seq[-1], want_logits=True)
            outs.append((seq, more, lgs))
    np.testing.assert_array_equal(outs[0][0], outs[1][0])
    np.testing.assert_array_equal(outs[0][1], outs[1][1])
    np.testing.assert_array_equal(outs[0][2], outs[1][2])


def test_decode_batch16_long_context_hd128(orc):
    """16 sequences, hd 128, a 300-token prompt (two decode-attention chunks)."""
    cfg = small_cfg(dim=256, hidden=512, heads=2, hd=128, nlayers=2, vocab=512, seq=306)
    w = ModelWeights.normal(cfg, seed=47)
    tok, tgt = tokens_uniform(48, cfg.vocab, 16, cfg.seq)
    lg, _, _ = orc.forward(oracle_cfg(orc, cfg), oracle_weights(orc, w), tok, tgt)
    with _ctx(cfg, w, 16, 320) as c:
        _, last = c.prefill(tok[:, :300], want_logits=True)
        assert np.abs(last - lg[:, 299]).max() <= LOGIT_ATOL
        for p in range(300, 306):
            _, dl = c.decode_step(tok[:, p], want_logits=True)
            err = float(np.abs(dl - lg[:, p]).max())
            assert err <= LOGIT_ATOL, (p, err)


@pytest.mark.parametrize("dim,batch", [(256, 2), (2048, 9), (2048, 16)])
def test_decode_nonunit_gammas(orc, dim, batch):
    """Random gammas through the decode norms: at dim 256 the RMSNorm is fused
    into the GEMV (the normalised rows fit in LDS); at dim 2048 x 9 or 16 rows
    the first norm of a step is a row kernel and the others come from the
    residual GEMVs (x * gamma and sums of squares) with 1/rms applied by the
    next GEMV (9: seven padded token rows in the MFMA tiles)."""
    cfg = small_cfg(dim=dim, hidden=1024, heads=dim // 128, hd=128, nlayers=2, vocab=1024, seq=40)
    w = random_gammas(ModelWeights.normal(cfg, seed=53), seed=54)
    tok, tgt = tokens_uniform(55, cfg.vocab, batch, cfg.seq)
    lg, _, _ = orc.forward(oracle_cfg(orc, cfg), oracle_weights(orc, w), tok, tgt)
    with _ctx(cfg, w, batch, 64) as c:
        _, last = c.prefill(tok[:, :32], want_logits=True)
        assert np.abs(last - lg[:, 31]).max() <= LOGIT_ATOL
        for p in range(32, 40):
            _, dl = c.decode_step(tok[:, p], want_logits=True)
            err = float(np.abs(dl - lg[:, p]).max())
            assert err <= LOGIT_ATOL, (p, err)


def test_decode_large_residual_matches_forward(orc):
    """Residual entries up to 3e4 (an embedding U(-3e4, 3e4), fp16-exact)
    times gammas up to 6 (|x * gamma| past fp16's 65504) at 16 sequences of
    dim 2048, where the residual GEMVs hand the next GEMV fp16(x * gamma)
    scaled by a power of two and the sums of squares: decode logits equal the
    forward's at every position (relative to the logits' scale, which the
    tied embedding sets near 1e6)."""
    cfg = small_cfg(dim=2048, hidden=1024, heads=16, hd=128, nlayers=2, vocab=1024, seq=40)
    w = ModelWeights.normal(cfg, seed=56)
    rng = np.random.default_rng(57)
    w.embed = rng.uniform(-3e4, 3e4, w.embed.shape).astype(np.float16).astype(np.float32)
    D = cfg.dim
    for lw in w.layers:
        lw.gamma1 = rng.uniform(2.0, 6.0, D).astype(np.float32)
        lw.gamma2 = rng.uniform(2.0, 6.0, D).astype(np.float32)
    w.gamma_final = rng.uniform(0.5, 1.5, D).astype(np.float32)
    batch = 16
    tok, tgt = tokens_uniform(58, cfg.vocab, batch, cfg.seq)
    print("[case] decode with |x * gamma| beyond fp16, dim 2048, batch 16", flush=True)
    with _ctx(cfg, w, batch, 64) as c:
        out = c.forward(tok, tgt)
        lg = out.logits
        scale = float(np.abs(lg).max())
        assert np.isfinite(lg).all() and scale > 1e5
        nxt, last = c.prefill(tok[:, :32], want_logits=True)
        assert np.abs(last - lg[:, 31]).max() <= 2e-3 * scale
        for p in range(32, 40):
            nxt, dl = c.decode_step(tok[:, p], want_logits=True)
            assert np.isfinite(dl).all(), p
            err = float(np.abs(dl - lg[:, p]).max()) / scale
            print(f"[result] position {p}: max|dlogit| / max|logit| {err:.2e}", flush=True)
            assert err <= 2e-3, (p, err)


@pytest.mark.parametrize("batch", [1, 12])
def test_decode_tiny_config_hd64(orc, batch):
    """hd 64; at 12 sequences the attention output and the gate reach the Wo
    and W2 GEMVs in 16-row fragment order (the merge kernel writes it)."""
    from rustane_amd.engine import tiny_config
    cfg = tiny_config()
    cfg.seq = 72
    w = ModelWeights.normal(cfg, seed=49)
    tok, tgt = tokens_uniform(50, cfg.vocab, batch, cfg.seq)
    lg, _, _ = orc.forward(oracle_cfg(orc, cfg), oracle_weights(orc, w), tok, tgt)
    with _ctx(cfg, w, batch, 80) as c:
        c.prefill(tok[:, :64])
        for p in range(64, 72):
            _, dl = c.decode_step(tok[:, p], want_logits=True)
            assert np.abs(dl - lg[:, p]).max() <= LOGIT_ATOL


def test_decode_state_errors():
    cfg = small_cfg(seq=8)
    w = ModelWeights.normal(cfg, seed=51)
    with _ctx(cfg, w, 1, 10) as c:
        with pytest.raises(hb.HipBridgeError) as e:
            c.decode_step(np.array([1], np.uint32))
        assert e.value.code == hb.RH_ESTATE
        with pytest.raises(hb.HipBridgeError) as e:
            c.prefill(np.zeros((1, 11), np.uint32))
        assert e.value.code == hb.RH_ERANGE
        nxt, _ = c.prefill(np.arange(8, dtype=np.uint32)[None])
        c.decode(nxt, 2)
        with pytest.raises(hb.HipBridgeError) as e:
            c.decode_step(nxt)  # cache full at 10
        assert e.value.code == hb.RH_ERANGE
    with hb.Context(cfg.to_rh(), 0, 1, 0) as c:
        with pytest.raises(hb.HipBridgeError) as e:
            c.prefill(np.zeros((1, 4), np.uint32))
        assert e.value.code == hb.RH_ESTATE
