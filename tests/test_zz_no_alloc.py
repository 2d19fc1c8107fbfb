"""rh_decode_step_noalloc against rh_decode_step, through the C-ABI.

Two contexts hold the same weights and the same prefilled KV cache; one
steps with rh_decode_step (host buffers, the context's own decode buffers,
graph replay), the other with rh_decode_step_noalloc (device buffers, the
library's fixed scratch array, eager launches).  Greedy ids must be equal and
logits within the fp16 bar.  Two calls in a row: batch 12 at dim 2048 (the
first RMSNorm of a step as a row kernel, the others from the residual GEMVs,
and the GEMV inputs in 16-row fragment order), then a fresh prefill at batch
2 (the norm fused into the GEMVs, row-major inputs), so the second call runs
on scratch the first one left behind.

The step is also captured into a HIP graph on the context stream and
replayed: each replay reads and advances the context's device-side
position, so the replays continue the greedy sequence rh_decode_step makes,
and the host-side calls after them (rh_decode_pos, rh_decode_step) pick the
position up from the device.  Replays past a full cache write nothing and
are reported by rh_sync.  Contexts on one GPU hold separate scratch slots.
"""
import numpy as np
import pytest

from rustane_amd import hip_bridge as hb
from rustane_amd import hip_rt
from rustane_amd.engine import ModelConfig, ModelWeights

from helpers import LOGIT_ATOL, random_gammas, tokens_uniform

pytestmark = pytest.mark.gpu


def _noalloc_step(c, tok, want_logits=True):
    tok = np.ascontiguousarray(tok, np.uint32).reshape(-1)
    B = tok.size
    din = hip_rt.DeviceArray.from_numpy(tok)
    dout = hip_rt.DeviceArray((B,), np.uint32)
    dlog = hip_rt.DeviceArray((B, c.cfg.vocab), np.float32) if want_logits else None
    c.decode_step_noalloc(B, din.ptr, dout.ptr, dlog.ptr if dlog else None)
    c.sync()
    return dout.numpy(), (dlog.numpy() if dlog else None)


def test_noalloc_step_matches_decode_step():
    cfg = ModelConfig(2048, 1024, 16, 16, 128, 64, 2, 1000)
    w = random_gammas(ModelWeights.normal(cfg, seed=91, std=0.05), seed=92)
    tensors = [lw.tensors() for lw in w.layers]
    ref = hb.Context(cfg.to_rh(), 0, 12, 256)
    noa = hb.Context(cfg.to_rh(), 0, 12, 256)
    try:
        for c in (ref, noa):
            c.load_weights(w.embed, w.gamma_final, tensors)
        for call, (B, P) in enumerate([(12, 140), (2, 37)]):
            print(f"[case] noalloc call {call}: batch {B}, prompt {P}", flush=True)
            prompt, _ = tokens_uniform(93 + call, cfg.vocab, B, P)
            n_ref, _ = ref.prefill(prompt)
            n_noa, _ = noa.prefill(prompt)
            np.testing.assert_array_equal(n_ref, n_noa)
            tok = n_ref
            for step in range(3):
                want = step != 1  # the middle step lets the logits go to the scratch array
                o_ref, l_ref = ref.decode_step(tok, want_logits=True)
                o_noa, l_noa = _noalloc_step(noa, tok, want_logits=want)
                np.testing.assert_array_equal(o_ref, o_noa)
                if want:
                    err = float(np.abs(l_ref - l_noa).max())
                    print(f"[result] call {call} step {step}: max|dlogit| {err:.3e} "
                          f"(bit-identical: {bool(np.array_equal(l_ref, l_noa))})", flush=True)
                    assert err <= LOGIT_ATOL
                tok = o_ref
            assert ref.pos == noa.pos == P + 3
    finally:
        ref.close()
        noa.close()


def test_noalloc_argument_and_state_errors():
    cfg = ModelConfig(256, 512, 2, 2, 128, 32, 1, 512)
    with hb.Context(cfg.to_rh(), 0, 4, 64) as c:
        tok = hip_rt.DeviceArray.from_numpy(np.zeros(2, np.uint32))
        out = hip_rt.DeviceArray((2,), np.uint32)
        with pytest.raises(hb.HipBridgeError) as e:
            c.decode_step_noalloc(2, tok.ptr, out.ptr, None)
        assert e.value.code == hb.RH_ESTATE
        c.prefill(np.ones((2, 5), np.uint32))
        with pytest.raises(hb.HipBridgeError) as e:
            c.decode_step_noalloc(1, tok.ptr, out.ptr, None)
        assert e.value.code == hb.RH_EINVAL
        with pytest.raises(hb.HipBridgeError) as e:
            c.decode_step_noalloc(2, None, out.ptr, None)
        assert e.value.code == hb.RH_EINVAL
        assert c.pos == 5


def test_noalloc_rejects_scratch_beyond_its_maximum():
    """A 2^20-token vocabulary at batch 16 needs 64 MiB for the logits alone;
    with the caller's logits buffer the same call fits."""
    cfg = ModelConfig(128, 128, 1, 1, 128, 16, 1, 1 << 20)
    with hb.Context(cfg.to_rh(), 0, 16, 64) as c:
        tok = hip_rt.DeviceArray.from_numpy(np.zeros(16, np.uint32))
        out = hip_rt.DeviceArray((16,), np.uint32)
        with pytest.raises(hb.HipBridgeError) as e:
            c.decode_step_noalloc(16, tok.ptr, out.ptr, None)
        assert e.value.code == hb.RH_ERANGE
        assert "scratch" in str(e.value)
        lg = hip_rt.DeviceArray((16, cfg.vocab), np.float32)
        with pytest.raises(hb.HipBridgeError) as e:  # fits: fails on state, not size
            c.decode_step_noalloc(16, tok.ptr, out.ptr, lg.ptr)
        assert e.value.code == hb.RH_ESTATE


def _weights(cfg, seed):
    w = random_gammas(ModelWeights.normal(cfg, seed=seed, std=0.05), seed=seed + 1)
    return w, [lw.tensors() for lw in w.layers]


@pytest.mark.parametrize("B", [1, 6, 12])
def test_captured_noalloc_step_replays_advance(B):
    """A graph of one allocation-free step with in_tok == out_tok, replayed
    n times with eager work and synchronisations in between, equals n eager
    rh_decode_step calls of another context; rh_decode_step continues after
    the replays at the right position."""
    cfg = ModelConfig(512, 1024, 4, 4, 128, 64, 2, 1000)
    w, tensors = _weights(cfg, 95)
    P, n = 50, 5
    prompt, _ = tokens_uniform(97 + B, cfg.vocab, B, P)
    print(f"[case] captured noalloc step, batch {B}, prompt {P}, {n} replays", flush=True)
    ref = hb.Context(cfg.to_rh(), 0, B, 128)
    noa = hb.Context(cfg.to_rh(), 0, B, 128)
    try:
        for c in (ref, noa):
            c.load_weights(w.embed, w.gamma_final, tensors)
        tok, _ = ref.prefill(prompt)
        n_noa, _ = noa.prefill(prompt)
        np.testing.assert_array_equal(tok, n_noa)
        dtok = hip_rt.DeviceArray.from_numpy(tok)
        dlog = hip_rt.DeviceArray((B, cfg.vocab), np.float32)
        g = hip_rt.Graph(noa.stream, lambda: noa.decode_step_noalloc(B, dtok.ptr, dtok.ptr, dlog.ptr))
        try:
            for r in range(n):
                g.launch()
                noa.sync()
                got_tok, got_log = dtok.numpy(), dlog.numpy()
                tok, want_log = ref.decode_step(tok, want_logits=True)
                np.testing.assert_array_equal(got_tok, tok)
                err = float(np.abs(got_log - want_log).max())
                print(f"[result] replay {r}: max|dlogit| {err:.3e}", flush=True)
                assert err <= LOGIT_ATOL
                assert noa.pos == P + r + 1  # re-read from the device
        finally:
            g.close()
        # an eager host-side step continues from the device's position
        t_noa, l_noa = noa.decode_step(tok, want_logits=True)
        t_ref, l_ref = ref.decode_step(tok, want_logits=True)
        np.testing.assert_array_equal(t_noa, t_ref)
        assert float(np.abs(l_noa - l_ref).max()) <= LOGIT_ATOL
        assert noa.pos == ref.pos == P + n + 1
    finally:
        ref.close()
        noa.close()


def test_captured_noalloc_replays_past_the_cache_are_reported():
    """Replays beyond max_ctx write nothing to the cache (the position stays
    at max_ctx) and rh_sync reports RH_ERANGE; the context is usable after a
    new prefill."""
    cfg = ModelConfig(256, 512, 2, 2, 128, 32, 1, 512)
    w, tensors = _weights(cfg, 96)
    M = 40
    with hb.Context(cfg.to_rh(), 0, 1, M) as c:
        c.load_weights(w.embed, w.gamma_final, tensors)
        print(f"[case] noalloc replays past a {M}-position cache", flush=True)
        tok, _ = c.prefill(np.arange(M - 2, dtype=np.uint32)[None])
        dtok = hip_rt.DeviceArray.from_numpy(tok)
        g = hip_rt.Graph(c.stream, lambda: c.decode_step_noalloc(1, dtok.ptr, dtok.ptr, None))
        try:
            g.launch()
            g.launch()
            c.sync()
            assert c.pos == M
            g.launch()
            with pytest.raises(hb.HipBridgeError) as e:
                c.sync()
            assert e.value.code == hb.RH_ERANGE and "KV cache" in str(e.value)
            assert c.pos == M
        finally:
            g.close()
        with pytest.raises(hb.HipBridgeError) as e:
            c.decode_step(tok)
        assert e.value.code == hb.RH_ERANGE
        nxt, _ = c.prefill(np.arange(5, dtype=np.uint32)[None])
        c.decode_step(nxt)
        assert c.pos == 6


def test_noalloc_scratch_slots_per_context():
    """Four contexts on one GPU step with their own scratch slots, interleaved,
    each matching a context that steps alone; a fifth is refused until one
    of the four is destroyed."""
    cfg = ModelConfig(256, 512, 2, 2, 128, 32, 1, 512)
    w, tensors = _weights(cfg, 98)
    prompts = [tokens_uniform(99 + i, cfg.vocab, 1, 20 + i)[0] for i in range(5)]
    print("[case] noalloc scratch slots: 4 interleaved contexts, a fifth refused", flush=True)
    ctxs = [hb.Context(cfg.to_rh(), 0, 1, 64) for _ in range(5)]
    ref = hb.Context(cfg.to_rh(), 0, 1, 64)
    try:
        for c in ctxs + [ref]:
            c.load_weights(w.embed, w.gamma_final, tensors)
        toks = [c.prefill(p)[0] for c, p in zip(ctxs, prompts)]
        dts = [hip_rt.DeviceArray.from_numpy(t) for t in toks]
        for step in range(3):
            for i in range(4):
                ctxs[i].decode_step_noalloc(1, dts[i].ptr, dts[i].ptr, None)
        for c in ctxs[:4]:
            c.sync()
        with pytest.raises(hb.HipBridgeError) as e:
            ctxs[4].decode_step_noalloc(1, dts[4].ptr, dts[4].ptr, None)
        assert e.value.code == hb.RH_ERANGE and "slot" in str(e.value)
        for i in range(4):
            t, _ = ref.prefill(prompts[i])
            for step in range(3):
                t, _ = ref.decode_step(t)
            np.testing.assert_array_equal(dts[i].numpy(), t)
        ctxs[0].close()
        ctxs[4].decode_step_noalloc(1, dts[4].ptr, dts[4].ptr, None)
        ctxs[4].sync()
        t, _ = ref.prefill(prompts[4])
        t, _ = ref.decode_step(t)
        np.testing.assert_array_equal(dts[4].numpy(), t)
    finally:
        for c in ctxs + [ref]:
            c.close()
