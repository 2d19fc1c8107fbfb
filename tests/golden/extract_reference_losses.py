"""Writes reference_losses.json: the forward losses the reference publishes.

The reference's own init makes every layer an identity map (Wo = W2 = 0,
crates/engine/src/layer.rs:1516,1519), so with tokens (i*31+7) % 8192 these
losses depend only on the embedding LCG, the final RMSNorm, the tied logits
and the mean cross-entropy.  They are the only numeric golden values for the
path that the reference holds.  Sources (read as data, nothing executed):

  results/forward_utilization/scale_ladder.json   "loss" per probe (6 d.p.)
                                                  and "params_b" (model.rs:109-114 count)
  results/2026-03-18_1830_param-sweep.md          loss0 column (3 d.p.)
  README.md:58                                    600m-A "loss=9.0108"

Run in a checkout that has the reference at /root/reference; the fixture is
committed so the tests never read the reference.
"""
import json
import os
import re

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    out = []
    p = "results/forward_utilization/scale_ladder.json"
    lines = open(os.path.join(REF, p)).read().splitlines()
    for e in json.load(open(os.path.join(REF, p))):
        ln = next(i + 1 for i, l in enumerate(lines) if f'"loss": {e["loss"]}' in l
                  and any(f'"name": "{e["name"]}"' in x for x in lines[max(0, i - 16):i]))
        out.append({"name": e["name"], "dim": e["dim"], "hidden": e["hidden"], "heads": e["heads"],
                    "nlayers": e["nlayers"], "seq": e["seq"], "vocab": 8192, "loss": e["loss"],
                    "decimals": 6, "params_b": e["params_b"], "source": f"{p}:{ln}"})
    p = "results/2026-03-18_1830_param-sweep.md"
    for i, l in enumerate(open(os.path.join(REF, p)).read().splitlines()):
        cells = [c.strip().strip("*") for c in l.split("|")]
        if len(cells) < 17 or not re.match(r"^\d", cells[3] or ""):
            continue
        name = cells[1].split(" ")[0]
        dim, hidden, heads, nl, seq = (int(cells[k]) for k in (3, 4, 5, 6, 7))
        out.append({"name": name, "dim": dim, "hidden": hidden, "heads": heads, "nlayers": nl,
                    "seq": seq, "vocab": 8192, "loss": float(cells[14]), "decimals": 3,
                    "source": f"{p}:{i + 1}"})
    out.append({"name": "600m-A (README)", "dim": 1536, "hidden": 4096, "heads": 12, "nlayers": 20,
                "seq": 512, "vocab": 8192, "loss": 9.0108, "decimals": 4, "source": "README.md:58"})
    with open(os.path.join(HERE, "reference_losses.json"), "w") as f:
        json.dump({"tokens": "(i*31+7) % vocab, targets shifted by one",
                   "init": "ModelWeights::random (LCG, Wo = W2 = 0, embed scale 0.005)",
                   "entries": out}, f, indent=1)
    print(f"wrote {len(out)} entries")


if __name__ == "__main__":
    main()
