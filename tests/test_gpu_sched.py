"""Request scheduler (multistream::ForwardScheduler, multistream.rs:54-161)
through the C-ABI: batched forward requests against the oracle's
per-request losses, FIFO batching by shape, batched generation equal to
one-at-a-time generation, and per-request errors."""
import numpy as np
import pytest

from rustane_amd import hip_bridge as hb
from rustane_amd.engine import ModelWeights

from helpers import LOSS_RTOL, oracle_cfg, oracle_weights, small_cfg

pytestmark = pytest.mark.gpu


def _ctx(cfg, w, max_batch, max_ctx=0):
    print(f"[case] scheduler ctx max_batch={max_batch} max_ctx={max_ctx}", flush=True)
    c = hb.Context(cfg.to_rh(), 0, max_batch, max_ctx)
    c.load_weights(w.embed, w.gamma_final, [lw.tensors() for lw in w.layers])
    return c


def test_forward_requests_batched_match_oracle(orc):
    cfg = small_cfg(dim=256, hidden=512, heads=2, hd=128, nlayers=2, vocab=1024, seq=64)
    w = ModelWeights.normal(cfg, seed=91)
    rng = np.random.default_rng(92)
    reqs = []
    for i in range(7):
        S = 64 if i % 3 else 40  # two shapes interleaved: batches never mix lengths
        t = rng.integers(0, cfg.vocab, size=S + 1).astype(np.uint32)
        reqs.append((100 + i, t[:-1], t[1:]))
    with _ctx(cfg, w, 4) as c, hb.Scheduler(c, max_batch=4, max_wait_us=200000) as s:
        res = s.run_batch(reqs[::-1])  # submitted out of id order
    assert [r.request_id for r in res] == [100 + i for i in range(7)]
    ocfg, ow = oracle_cfg(orc, cfg), oracle_weights(orc, w)
    for (rid, tok, tgt), r in zip(reqs, res):
        assert r.status == hb.RH_OK, r.message
        _, _, ml = orc.forward(ocfg, ow, tok[None], tgt[None])
        assert r.loss == pytest.approx(float(ml[0]), rel=LOSS_RTOL)
        assert r.total_ms >= r.service_ms > 0 and r.queue_wait_ms >= 0
    print(f"[result] batches {[r.batch for r in res]}", flush=True)
    assert max(r.batch for r in res) > 1
    assert all(1 <= r.batch <= 4 for r in res)


def test_generate_batched_equals_one_at_a_time():
    cfg = small_cfg(dim=256, hidden=512, heads=2, hd=128, nlayers=2, vocab=512, seq=32)
    w = ModelWeights.normal(cfg, seed=93, std=0.05)
    rng = np.random.default_rng(94)
    prompts = [rng.integers(0, cfg.vocab, size=20).astype(np.uint32) for _ in range(3)]
    reqs = [(i, p, None, 8) for i, p in enumerate(prompts)]
    with _ctx(cfg, w, 3, 64) as c:
        with hb.Scheduler(c, max_batch=3, max_wait_us=200000) as s:
            batched = s.run_batch(reqs)
        with hb.Scheduler(c, max_batch=1) as s:
            single = s.run_batch(reqs)
    assert [r.batch for r in single] == [1, 1, 1]
    print(f"[result] generate batches {[r.batch for r in batched]}", flush=True)
    for a, b in zip(batched, single):
        assert a.status == b.status == hb.RH_OK
        np.testing.assert_array_equal(a.tokens, b.tokens)


def test_request_errors():
    cfg = small_cfg(seq=16)
    w = ModelWeights.normal(cfg, seed=95)
    good = np.arange(17, dtype=np.uint32) % cfg.vocab
    bad = good.copy()
    bad[3] = cfg.vocab  # out of range
    with _ctx(cfg, w, 2, 32) as c, hb.Scheduler(c, max_batch=1) as s:
        res = s.run_batch([(1, good[:-1], good[1:]), (2, bad[:-1], bad[1:]), (3, good[:-1], good[1:])])
        assert [r.status for r in res] == [hb.RH_OK, hb.RH_ERANGE, hb.RH_OK]
        assert res[1].message
        assert res[0].loss == res[2].loss
        with pytest.raises(hb.HipBridgeError) as e:  # prompt + steps beyond the KV cache
            s.run_batch([(4, np.zeros(30, np.uint32), None, 8)])
        assert e.value.code == hb.RH_ERANGE


def test_request_error_fails_alone_in_a_batch():
    """With max_batch 4 the bad request is queued among good ones of the same
    shape; it fails alone and the others are batched and succeed."""
    cfg = small_cfg(seq=16)
    w = ModelWeights.normal(cfg, seed=96)
    good = np.arange(17, dtype=np.uint32) % cfg.vocab
    bad_tok, bad_tgt = good.copy(), good.copy()
    bad_tok[5] = cfg.vocab + 7
    bad_tgt[9] = cfg.vocab
    reqs = [(1, good[:-1], good[1:]), (2, bad_tok[:-1], good[1:]), (3, good[:-1], good[1:]),
            (4, good[:-1], bad_tgt[1:]), (5, good[:-1], good[1:])]
    prompt_bad = good[:10].copy()
    prompt_bad[2] = cfg.vocab
    with _ctx(cfg, w, 4, 64) as c, hb.Scheduler(c, max_batch=4, max_wait_us=200000) as s:
        res = s.run_batch(reqs)
        gen = s.run_batch([(6, good[:10], None, 4), (7, prompt_bad, None, 4), (8, good[:10], None, 4)])
    print(f"[result] statuses {[r.status for r in res]}, batches {[r.batch for r in res]}", flush=True)
    assert [r.status for r in res] == [hb.RH_OK, hb.RH_ERANGE, hb.RH_OK, hb.RH_ERANGE, hb.RH_OK]
    assert "token" in res[1].message and "target" in res[3].message
    assert res[1].batch == res[3].batch == 1
    assert max(res[i].batch for i in (0, 2, 4)) > 1
    assert res[0].loss == res[2].loss == res[4].loss
    assert [r.status for r in gen] == [hb.RH_OK, hb.RH_ERANGE, hb.RH_OK]
    np.testing.assert_array_equal(gen[0].tokens, gen[2].tokens)
