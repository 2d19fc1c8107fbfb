"""The oracle against the reference's published forward losses (CPU).

With the reference init (ModelWeights::random, full_model.rs:132-141) every
layer is an identity map: Wo = W2 = 0 (layer.rs:1516,1519) and the residual
adds alpha * 0.  The published losses therefore depend only on the LCG
embedding (scale 0.005), the final RMSNorm (eps 1e-5), the tied logits and the
mean cross-entropy, for tokens (i*31+7) % 8192 and targets shifted by one
(tests/bench_fwd_only_scale.rs:110-115).  One layer is run so the residual
path is on the checked route; the loss does not depend on the layer count,
hidden size or head count, which the published ladder itself shows
(7B and 10B share dim 4096 and loss 9.322805; 13B and 20B share 10.287367).

Fixture: tests/golden/reference_losses.json (extract_reference_losses.py),
values from results/forward_utilization/scale_ladder.json (6 d.p.),
results/2026-03-18_1830_param-sweep.md (loss0, 3 d.p.) and README.md:58.
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

from rustane_amd.engine import ModelConfig, ModelWeights

from helpers import oracle_cfg, oracle_weights, reference_tokens

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = json.load(open(os.path.join(HERE, "golden", "reference_losses.json")))
ENTRIES = FIXTURE["entries"]
# one oracle run per (dim, seq): the loss depends on nothing else
GROUPS = sorted({(e["dim"], e["seq"]) for e in ENTRIES})
_cache: dict = {}


def _oracle_loss(orc, dim: int, seq: int) -> float:
    if (dim, seq) not in _cache:
        cfg = ModelConfig.custom(dim, 256, dim // 128, 1, seq)
        w = ModelWeights.random(cfg)
        tok, tgt = reference_tokens(cfg.vocab, seq)
        _, _, mean = orc.forward(oracle_cfg(orc, cfg), oracle_weights(orc, w), tok[None],
                                 tgt[None], want_logits=False)
        _cache[(dim, seq)] = float(mean[0])
    return _cache[(dim, seq)]


@pytest.mark.parametrize("dim,seq", GROUPS, ids=[f"d{d}_s{s}" for d, s in GROUPS])
def test_published_losses(orc, dim, seq):
    loss = _oracle_loss(orc, dim, seq)
    for e in (e for e in ENTRIES if e["dim"] == dim and e["seq"] == seq):
        # half a unit in the last published place, plus fp32 summation-order slack
        tol = 0.5 * 10.0 ** -e["decimals"] + 3e-6
        assert abs(loss - e["loss"]) <= tol, (e["name"], e["source"], loss, e["loss"])


def test_golden_is_sensitive_to_the_tail(orc):
    """Plausible slips in the tail move the loss far outside the golden
    tolerance: targets that are not shifted, or a final gamma that is ignored."""
    dim, seq = 2048, 512
    cfg = ModelConfig.custom(dim, 256, dim // 128, 1, seq)
    w = ModelWeights.random(cfg)
    tok, tgt = reference_tokens(cfg.vocab, seq)
    base = _oracle_loss(orc, dim, seq)
    ocfg = oracle_cfg(orc, cfg)
    _, _, mean = orc.forward(ocfg, oracle_weights(orc, w), tok[None], tok[None], want_logits=False)
    assert abs(float(mean[0]) - base) > 1e-2  # targets not shifted
    w.gamma_final = np.full(dim, 1.1, np.float32)
    _, _, mean = orc.forward(ocfg, oracle_weights(orc, w), tok[None], tgt[None], want_logits=False)
    assert abs(float(mean[0]) - base) > 1e-4  # gamma ignored or mis-scaled


def test_param_counts_match_published(orc):
    """ModelConfig.param_count (model.rs:109-114) against the params_b the
    reference records for each probe."""
    for e in ENTRIES:
        if "params_b" not in e:
            continue
        cfg = ModelConfig.custom(e["dim"], e["hidden"], e["heads"], e["nlayers"], e["seq"])
        assert cfg.param_count() == round(e["params_b"] * 1e9), e["name"]
