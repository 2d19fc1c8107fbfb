"""Host-side engine logic (CPU): model presets, parameter counts and the work
conventions the benchmark's roofline fractions are computed from."""
from __future__ import annotations

import numpy as np
import pytest

from rustane_amd import engine as E


def test_benchmark_shapes():
    c = E.cfg_7b()
    assert (c.dim, c.hidden, c.nlayers, c.heads, c.hd, c.vocab, c.seq) == (4096, 11008, 32, 32, 128, 32000, 512)
    c = E.cfg_600m()
    assert (c.dim, c.hidden, c.nlayers, c.heads, c.hd, c.vocab) == (1536, 4096, 20, 12, 128, 32000)
    c = E.cfg_5b_deep()
    assert (c.dim, c.hidden, c.nlayers, c.heads, c.hd, c.vocab) == (2560, 6912, 60, 20, 128, 32000)
    c = E.tiny_config()
    assert (c.dim, c.hidden, c.nlayers, c.heads, c.hd, c.vocab, c.seq) == (512, 1408, 8, 8, 64, 8192, 256)


@pytest.mark.parametrize("make,gflop", [(E.cfg_7b, 6834.50), (E.cfg_600m, 646.29),
                                        (E.cfg_5b_deep, 5036.68), (E.tiny_config, 15.84)])
def test_prefill_flops(make, gflop):
    """GEMM 2*S*L*(4D^2 + 3DF) + causal attention 2*D*S*(S+1)*L + logits 2*S*D*V."""
    fl = E.prefill_flops(make())
    assert fl["total"] / 1e9 == pytest.approx(gflop, abs=0.006)
    assert fl["total"] == fl["gemm"] + fl["attn"] + fl["logits"]
    assert E.prefill_flops(make(), batch=4)["total"] == 4 * fl["total"]


def test_prefill_flops_7b_parts():
    fl = E.prefill_flops(E.cfg_7b())
    assert fl["gemm"] / 1e9 == pytest.approx(6631.43, abs=0.006)
    assert fl["attn"] / 1e9 == pytest.approx(68.85, abs=0.006)
    assert fl["logits"] / 1e9 == pytest.approx(134.22, abs=0.006)
    # one W1|W3 launch: 2 * S * (2F) * D
    assert fl["w13_per_launch"] == 2 * 512 * 2 * 11008 * 4096


def test_decode_bytes_7b():
    """13.214 GB of fp16 weights per step plus, per sequence, the K/V read at
    the mean context of a 2048 -> 2303 run and the K/V append."""
    c = E.cfg_7b()
    b1 = E.decode_bytes(c, 2048 + 255 / 2.0, 1)
    assert b1["weights"] / 1e9 == pytest.approx(13.214, abs=5e-4)
    assert b1["total"] / 1e9 == pytest.approx(14.355, abs=5e-4)
    b16 = E.decode_bytes(c, 2048 + 255 / 2.0, 16)
    assert b16["total"] / 1e9 == pytest.approx(31.472, abs=5e-4)


def test_param_count_7b():
    """model.rs:109-114: L(4D^2 + 3DF) + VD + D(2L + 1)."""
    c = E.ModelConfig.custom(4096, 11008, 32, 32, 512)
    assert c.param_count() == 6_509_826_048


def test_reference_init_structure():
    """LayerWeights::random (layer.rs:1509-1524): same-size tensors are
    identical (seed 42 + n), Wo = W2 = 0, gammas 1, embed scale 0.005."""
    cfg = E.ModelConfig(256, 512, 4, 4, 64, 32, 2, 1024)
    w = E.ModelWeights.random(cfg)
    l0, l1 = w.layers
    np.testing.assert_array_equal(l0.wq, l0.wk)
    np.testing.assert_array_equal(l0.wq, l0.wv)
    np.testing.assert_array_equal(l0.w1, l0.w3)
    np.testing.assert_array_equal(l0.wq, l1.wq)
    assert not l0.wo.any() and not l0.w2.any()
    assert (l0.gamma1 == 1).all() and (w.gamma_final == 1).all()
    assert np.abs(w.embed).max() <= 0.005
    assert np.abs(l0.wq).max() <= 1 / np.sqrt(256) + 1e-7
    assert np.abs(l0.w1).max() <= 1 / np.sqrt(512) + 1e-7


def test_normal_weights_are_fp16_exact():
    cfg = E.ModelConfig(256, 512, 4, 4, 64, 32, 1, 1024)
    w = E.ModelWeights.normal(cfg, seed=3)
    for t in [w.embed] + w.layers[0].tensors()[:7]:
        np.testing.assert_array_equal(t, t.astype(np.float16).astype(np.float32))
    assert 0.018 < float(w.embed.std()) < 0.022


def test_forward_checks_shapes_without_a_device():
    """Host-side argument checks fire before any library call."""
    cfg = E.ModelConfig(256, 512, 4, 4, 64, 32, 1, 1024)
    with pytest.raises(ValueError):
        E._check(cfg, np.zeros(31, np.uint32), np.zeros(31, np.uint32))
    with pytest.raises(ValueError):
        E._check(cfg, np.zeros(32, np.uint32), np.zeros(16, np.uint32))
