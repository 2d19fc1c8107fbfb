"""Which fp16 rounding point drives the full-depth drift of an fp16-operand
forward?  (CPU only; run by hand, not collected by pytest.)

Runs the oracle forward on one set of N(0, 0.02) weights rounded to fp16
(the values an fp16 device path holds) and seeded uniform tokens, in fp32,
with every rounding point of its fp16-operand mode (oracle.h ORC_F16_*), with
each point alone, and with all points but one, and prints each run's logit
deviation from the fp32 run (RMS and max-abs).  The results bound the full-
depth parity tests (tests/test_gpu_fullsize.py): at 7B width, 32 layers, no
single point dominates; the per-point RMS deviations add in quadrature to
the all-points one.

    python tests/fp16_drift_by_point.py [nlayers]     # 7B width; 32 by default

At 32 layers the weights take 26 GB of host memory and each forward about a
minute on 8 cores.
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, HERE)

import oracle as orc  # noqa: E402
from helpers import tokens_uniform  # noqa: E402
from rustane_amd.engine import cfg_7b  # noqa: E402


def main():
    L = int(sys.argv[1]) if len(sys.argv) > 1 else 32
    cfg = cfg_7b()
    cfg.nlayers = L
    D, F, V = cfg.dim, cfg.hidden, cfg.vocab
    rng = np.random.default_rng(5)

    def mat(*shape):
        a = rng.standard_normal(shape, dtype=np.float32)
        a *= 0.02
        return a.astype(np.float16).astype(np.float32)

    t0 = time.time()
    embed, gf = mat(V, D), np.ones(D, np.float32)
    layers = [[mat(D, D), mat(D, D), mat(D, D), mat(D, D), mat(D, F), mat(D, F), mat(D, F),
               np.ones(D, np.float32), np.ones(D, np.float32)] for _ in range(L)]
    ow = orc.Weights(embed, gf, layers)
    tok, tgt = tokens_uniform(72, V, 1, cfg.seq)
    print(f"7B width, {L} layers, seq {cfg.seq}: weights in {time.time() - t0:.0f} s", flush=True)

    def run(bits):
        oc = orc.make_config(D, F, cfg.heads, L, V, head_dim=cfg.hd, fp16_operands=bits)
        lg, _, _ = orc.forward(oc, ow, tok, tgt)
        return lg

    lg32 = run(0)

    def dev(bits):
        d = (run(bits) - lg32).astype(np.float64)
        return float(np.sqrt(np.mean(d * d))), float(np.abs(d).max())

    r, m = dev(orc.F16_ALL)
    print(f"{'all points':>14s}: rms {r:.3e} max {m:.3e}", flush=True)
    for name, bit in orc.F16_POINTS.items():
        r1, m1 = dev(bit)
        r2, m2 = dev(orc.F16_ALL & ~bit)
        print(f"{name:>14s}: alone rms {r1:.3e} max {m1:.3e}; all but it rms {r2:.3e} max {m2:.3e}", flush=True)


if __name__ == "__main__":
    main()
