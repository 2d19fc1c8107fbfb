"""Shared helpers for the parity tests: seeded inputs, oracle runs, tolerances."""
from __future__ import annotations

import numpy as np

from rustane_amd.engine import ModelConfig, ModelWeights

# The reference's own bar for equivalent forwards
# (crates/engine/tests/test_combined_forward_correctness.rs:13-14).
LOGIT_ATOL = 2e-2
LOSS_RTOL = 1e-3


def oracle_cfg(orc, cfg: ModelConfig, softcap: float = 0.0):
    return orc.make_config(cfg.dim, cfg.hidden, cfg.heads, cfg.nlayers, cfg.vocab,
                           head_dim=cfg.hd, softcap=softcap)


def oracle_weights(orc, w: ModelWeights):
    return orc.Weights(w.embed, w.gamma_final, [lw.tensors() for lw in w.layers])


def tokens_uniform(seed: int, vocab: int, batch: int, seq: int):
    """S + 1 uniform ids per sequence; inputs [0..S), targets [1..S+1)."""
    rng = np.random.default_rng(seed)
    t = rng.integers(0, vocab, size=(batch, seq + 1), dtype=np.int64).astype(np.uint32)
    return np.ascontiguousarray(t[:, :-1]), np.ascontiguousarray(t[:, 1:])


def reference_tokens(vocab: int, seq: int):
    """(i*31 + 7) % vocab (tests/bench_fwd_only_scale.rs:110-115)."""
    tok = np.array([(i * 31 + 7) % vocab for i in range(seq)], np.uint32)
    tgt = np.array([(i * 31 + 7) % vocab for i in range(1, seq + 1)], np.uint32)
    return tok, tgt


def small_cfg(dim=256, hidden=512, heads=4, hd=64, nlayers=2, vocab=1024, seq=64):
    return ModelConfig(dim, hidden, heads, heads, hd, seq, nlayers, vocab)


def random_gammas(w: ModelWeights, seed: int):
    """Replaces every RMSNorm gamma (both per layer and the final one) with a
    distinct U(0.5, 1.5) vector, so a kernel that drops a gamma or applies the
    wrong one fails parity."""
    rng = np.random.default_rng(seed)
    D = w.gamma_final.shape[0]
    for lw in w.layers:
        lw.gamma1 = rng.uniform(0.5, 1.5, D).astype(np.float32)
        lw.gamma2 = rng.uniform(0.5, 1.5, D).astype(np.float32)
    w.gamma_final = rng.uniform(0.5, 1.5, D).astype(np.float32)
    return w


def rstk_bytes(cfg: ModelConfig, w: ModelWeights, step: int) -> bytes:
    """An RSTK v1 checkpoint built from the format definition
    (bin/train.rs:238-275): 28-byte little-endian header, then every tensor
    as little-endian fp32 in upload order."""
    import struct
    parts = [struct.pack("<4s6I", b"RSTK", 1, step, cfg.dim, cfg.nlayers, cfg.vocab, cfg.seq),
             np.ascontiguousarray(w.embed, "<f4").tobytes(), np.ascontiguousarray(w.gamma_final, "<f4").tobytes()]
    for lw in w.layers:
        parts += [np.ascontiguousarray(t, "<f4").tobytes() for t in lw.tensors()]
    return b"".join(parts)


def cosine(a, b):
    a = a.ravel().astype(np.float64)
    b = b.ravel().astype(np.float64)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))
