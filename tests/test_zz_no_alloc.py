"""rh_decode_step_noalloc against rh_decode_step, through the C-ABI.

Two contexts hold the same weights and the same prefilled KV cache; one
steps with rh_decode_step (host buffers, the context's own decode buffers,
graph replay), the other with rh_decode_step_noalloc (device buffers, the
library's fixed scratch array, eager launches).  Greedy ids must be equal and
logits within the fp16 bar.  Two calls in a row: batch 8 (the RMSNorm row
kernel path), then a fresh prefill at batch 2 (the norm fused into the
GEMVs), so the second call runs on scratch the first one left behind.
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
    cfg = ModelConfig(512, 1024, 4, 4, 128, 64, 2, 1000)
    w = random_gammas(ModelWeights.normal(cfg, seed=91, std=0.05), seed=92)
    tensors = [lw.tensors() for lw in w.layers]
    ref = hb.Context(cfg.to_rh(), 0, 8, 256)
    noa = hb.Context(cfg.to_rh(), 0, 8, 256)
    try:
        for c in (ref, noa):
            c.load_weights(w.embed, w.gamma_final, tensors)
        for call, (B, P) in enumerate([(8, 140), (2, 37)]):
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
