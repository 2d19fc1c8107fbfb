"""GPU checks of the boundary's state rules, through the C-ABI.

* Weights changed in place are seen by the next forward of the engine
  mirror (the reference re-stages weights on every call, layer.rs:4670-4705;
  a cached upload is only kept for weights that carry a version).
* fp32 weights loaded into a context come back exactly, and training resumes
  from them: a checkpoint saved after optimizer steps and loaded into a
  fresh context reads back the trained fp32 values bit for bit.
* A RoPE table regrown by a long forward does not leave the captured decode
  graph reading the old table.
* rh_train_step leaves the context's own softcap as it was.
* Decode calls whose batch differs from the prefill batch are refused.
* Forward graphs evicted from the per-shape cache while earlier replays are
  still queued leave every result intact.
"""
import numpy as np
import pytest

from rustane_amd import engine as eng
from rustane_amd import hip_bridge as hb
from rustane_amd.engine import ModelWeights

from helpers import LOGIT_ATOL, oracle_cfg, oracle_weights, random_gammas, small_cfg, tokens_uniform

pytestmark = pytest.mark.gpu


def _load(c, w):
    c.load_weights(w.embed, w.gamma_final, [lw.tensors() for lw in w.layers])


def test_in_place_weight_change_is_seen(orc):
    cfg = small_cfg(seq=32)
    w = ModelWeights.normal(cfg, seed=201, std=0.05)
    tok, tgt = tokens_uniform(202, cfg.vocab, 1, cfg.seq)
    print("[case] engine forward after an in-place weight change", flush=True)
    k = eng.CompiledKernels.compile(cfg)
    try:
        a = eng.forward(cfg, k, w, tok[0], tgt[0])
        w.layers[1].w2 *= np.float32(3.0)       # in place, no bump: still seen
        w.gamma_final[:] = np.float32(0.5)
        b = eng.forward(cfg, k, w, tok[0], tgt[0])
        lg, _, ml = orc.forward(oracle_cfg(orc, cfg), oracle_weights(orc, w), tok, tgt)
        err = float(np.abs(b.logits - lg[0]).max())
        print(f"[result] loss before {a.loss:.6f}, after {b.loss:.6f} (oracle {ml[0]:.6f}), "
              f"max|dlogit| {err:.3e}", flush=True)
        assert err <= LOGIT_ATOL
        assert abs(b.loss - a.loss) > 1e-3
        # with a version the upload is cached until bump()
        w.bump()
        c = eng.forward(cfg, k, w, tok[0], tgt[0])
        w.layers[0].wq *= np.float32(0.0)
        w.bump()
        d = eng.forward(cfg, k, w, tok[0], tgt[0])
        lg2, _, _ = orc.forward(oracle_cfg(orc, cfg), oracle_weights(orc, w), tok, tgt)
        assert float(np.abs(c.logits - b.logits).max()) == 0.0
        assert float(np.abs(d.logits - lg2[0]).max()) <= LOGIT_ATOL
    finally:
        k.close()


def test_fp32_load_and_trained_checkpoint_round_trip_exactly(tmp_path):
    cfg = small_cfg(dim=256, hidden=512, heads=2, hd=128, nlayers=2, vocab=1024, seq=64)
    w = random_gammas(ModelWeights.normal(cfg, seed=203, std=0.05, fp16_round=False), seed=204)
    assert not np.array_equal(w.embed, w.embed.astype(np.float16).astype(np.float32))
    tok, tgt = tokens_uniform(205, cfg.vocab, 2, cfg.seq)
    tc = hb.train_config(max_lr=1e-3, warmup_steps=1, total_steps=10)
    p = str(tmp_path / "trained.bin")
    print("[case] fp32 masters: load, train two steps, save, reload", flush=True)
    with hb.Context(cfg.to_rh(), 0, 2, 0) as c:
        c.set_fp32_masters(True)
        _load(c, w)
        e, gf, layers = c.read_weights()
        np.testing.assert_array_equal(e, w.embed)
        for lw, got in zip(w.layers, layers):
            for x, y in zip(lw.tensors(), got):
                np.testing.assert_array_equal(x, y)
        for t in (1, 2):
            c.zero_grads()
            c.forward_backward(tok, tgt, loss_scale=256.0)
            c.update_weights(t, 1e-3, tc, 1.0 / 512)
        trained = c.read_weights()
        c.save_checkpoint(p, 2)
    with hb.Context(cfg.to_rh(), 0, 2, 0) as c2:
        c2.set_fp32_masters(True)
        assert c2.load_checkpoint(p) == 2
        back = c2.read_weights()
    for x, y in zip([trained[0], trained[1]] + [t for lw in trained[2] for t in lw],
                    [back[0], back[1]] + [t for lw in back[2] for t in lw]):
        np.testing.assert_array_equal(x, y)
    # the trained masters are not fp16 values: the round trip kept fp32
    assert not np.array_equal(back[0], back[0].astype(np.float16).astype(np.float32))


def test_update_after_fp32_load_starts_from_exact_masters(orc):
    """One AdamW step on a context loaded with fp32 weights equals the
    oracle's step_fused on those exact fp32 weights (bit for bit)."""
    cfg = small_cfg(dim=256, hidden=512, heads=2, hd=128, nlayers=1, vocab=512, seq=32)
    w = ModelWeights.normal(cfg, seed=206, std=0.05, fp16_round=False)
    tok, tgt = tokens_uniform(207, cfg.vocab, 1, cfg.seq)
    tc = hb.train_config()
    otc = orc.TrainConfig()
    with hb.Context(cfg.to_rh(), 0, 1, 0) as c:
        c.set_fp32_masters(True)
        _load(c, w)
        c.forward_backward(tok, tgt, loss_scale=256.0)
        ge, gg, gl = c.read_grads()
        c.update_weights(1, 3e-4, tc, 1.0 / 256)
        e1, g1, l1 = c.read_weights()
    ow = oracle_weights(orc, w)
    og = orc.Grads(ow)
    for dst, src in zip([og.embed, og.gamma_final] + [t for lw in og.layers for t in lw],
                        [ge, gg] + [t for lw in gl for t in lw]):
        dst[...] = src
    orc.update_weights(ow, og, orc.OptState(ow), 1, 3e-4, otc, 1.0 / 256)
    for got, want in zip([e1, g1] + [t for lw in l1 for t in lw],
                         [ow.embed, ow.gamma_final] + [t for lw in ow.layers for t in lw]):
        np.testing.assert_array_equal(got, want)


def test_fp32_masters_are_opt_in():
    """Without rh_set_fp32_masters an fp32 load keeps only the fp16 device
    weights (read back widened); with it the load is exact; dropping them
    returns to fp16 reads; once an optimizer state exists they cannot be
    dropped."""
    cfg = small_cfg(dim=256, hidden=512, heads=2, hd=128, nlayers=1, vocab=512, seq=32)
    w = ModelWeights.normal(cfg, seed=211, std=0.05, fp16_round=False)
    r16 = lambda a: a.astype(np.float16).astype(np.float32)
    tok, tgt = tokens_uniform(212, cfg.vocab, 1, cfg.seq)
    print("[case] fp32 masters opt-in", flush=True)
    with hb.Context(cfg.to_rh(), 0, 1, 0) as c:
        _load(c, w)
        e, _, layers = c.read_weights()
        np.testing.assert_array_equal(e, r16(w.embed))
        np.testing.assert_array_equal(layers[0][6], r16(w.layers[0].w2))
        c.set_fp32_masters(True)
        e, _, _ = c.read_weights()  # the masters start as the fp16 weights widened
        np.testing.assert_array_equal(e, r16(w.embed))
        _load(c, w)
        e, _, layers = c.read_weights()
        np.testing.assert_array_equal(e, w.embed)
        np.testing.assert_array_equal(layers[0][4], w.layers[0].w1)
        c.set_fp32_masters(False)
        e, _, _ = c.read_weights()
        np.testing.assert_array_equal(e, r16(w.embed))
        c.set_fp32_masters(True)
        _load(c, w)
        c.forward_backward(tok, tgt, loss_scale=256.0)
        c.update_weights(1, 1e-3, hb.train_config(), 1.0 / 256)
        with pytest.raises(hb.HipBridgeError) as ex:
            c.set_fp32_masters(False)
        assert ex.value.code == hb.RH_ESTATE


def test_decode_graph_survives_rope_regrowth(orc):
    """decode (graph) -> forward longer than every earlier table (the RoPE
    table is reallocated) -> decode again, against the same calls with
    graphs off."""
    cfg = small_cfg(dim=256, hidden=512, heads=2, hd=128, nlayers=2, vocab=512, seq=32)
    w = ModelWeights.normal(cfg, seed=208, std=0.05)
    prompt, _ = tokens_uniform(209, cfg.vocab, 1, 20)
    long_tok, long_tgt = tokens_uniform(210, cfg.vocab, 1, 200)
    outs = []
    for graphs in (True, False):
        print(f"[case] rope regrowth, graphs={graphs}", flush=True)
        with hb.Context(cfg.to_rh(), 0, 1, 64) as c:
            _load(c, w)
            c.set_graphs(graphs)
            nxt, _ = c.prefill(prompt)
            t1, l1 = c.decode_step(nxt, want_logits=True)
            c.forward(long_tok, long_tgt)         # seq 200 > max(cfg.seq, max_ctx): table regrown
            t2, l2 = c.decode_step(t1, want_logits=True)
            outs.append((t1, l1, t2, l2))
    for a, b in zip(outs[0], outs[1]):
        np.testing.assert_array_equal(a, b)


def test_train_step_keeps_context_softcap(tmp_path, orc):
    cfg = small_cfg(seq=32)
    w = ModelWeights.normal(cfg, seed=211, std=0.05)
    path = str(tmp_path / "tok.bin")
    np.random.default_rng(212).integers(0, cfg.vocab, size=400).astype("<u2").tofile(path)
    tok, tgt = tokens_uniform(213, cfg.vocab, 1, cfg.seq)
    with hb.Context(cfg.to_rh(), 0, 1, 0) as c:
        _load(c, w)
        before = c.forward(tok, tgt)
        c.train_step(hb.TokenData(path), 0, hb.train_config(softcap=15.0, accum_steps=1, max_lr=0.0))
        after = c.forward(tok, tgt)   # max_lr 0: weights unchanged, softcap still 0
    np.testing.assert_array_equal(before.logits, after.logits)


def test_decode_refuses_other_batch():
    cfg = small_cfg(seq=16)
    w = ModelWeights.normal(cfg, seed=214)
    with hb.Context(cfg.to_rh(), 0, 4, 64) as c:
        _load(c, w)
        c.prefill(np.ones((3, 8), np.uint32))
        for call in (lambda: c.decode_step(np.ones(2, np.uint32)), lambda: c.decode(np.ones(4, np.uint32), 2)):
            with pytest.raises(hb.HipBridgeError) as e:
                call()
            assert e.value.code == hb.RH_EINVAL
        assert c.pos == 8
        out, _ = c.decode_step(np.ones(3, np.uint32))
        assert out.shape == (3,) and c.pos == 9


def test_forward_graph_eviction_with_replays_in_flight():
    """More (batch, seq) shapes than the forward-graph cache holds, enqueued
    back to back with rh_forward_dev (no synchronisation between calls): each
    new shape evicts the oldest graph while earlier replays may still be
    queued.  Every call's per-token losses must equal the synchronous
    host-pointer forward of the same tokens."""
    from rustane_amd import hip_rt
    cfg = small_cfg(seq=96)
    w = ModelWeights.normal(cfg, seed=71)
    shapes = [(1, 96)] + [(1 + i % 2, 40 + 4 * i) for i in range(10)] * 2
    print(f"[case] forward graph eviction: {len(shapes)} async forwards over 10 shapes", flush=True)
    with hb.Context(cfg.to_rh(), 0, 2, 0) as c:
        _load(c, w)
        keep, want = [], []
        for k, (B, S) in enumerate(shapes):
            tok, tgt = tokens_uniform(500 + k, cfg.vocab, B, S)
            want.append(c.forward(tok, tgt, want_logits=False).token_losses)
            keep.append((hip_rt.DeviceArray.from_numpy(tok), hip_rt.DeviceArray.from_numpy(tgt),
                         hip_rt.DeviceArray((B, S), np.float32)))
        for (B, S), (dt, dg, dl) in zip(shapes, keep):
            c.forward_dev(dt.ptr, dg.ptr, B, S, None, dl.ptr, None)
        c.sync()
        for k, (_, _, dl) in enumerate(keep):
            assert np.array_equal(dl.numpy(), want[k]), k
