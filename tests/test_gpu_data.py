"""GPU side of the on-disk formats: RSTK checkpoints in and out of a context
(bin/train.rs:238-345) and the validation loop (bin/train.rs:196-236) over a
memory-mapped token file, against the CPU oracle's forward and compute_bpb's
definition (data.rs:75-91)."""
import math

import numpy as np
import pytest

from rustane_amd import hip_bridge as hb
from rustane_amd.engine import ModelWeights

from helpers import LOSS_RTOL, oracle_cfg, oracle_weights, random_gammas, rstk_bytes, small_cfg

pytestmark = pytest.mark.gpu


def _cfg():
    return small_cfg(dim=256, hidden=512, heads=2, hd=128, nlayers=2, vocab=1024, seq=64)


def test_checkpoint_load_equals_weight_upload(tmp_path):
    cfg = _cfg()
    w = random_gammas(ModelWeights.normal(cfg, seed=81), seed=82)
    p = tmp_path / "ckpt_000007.bin"
    p.write_bytes(rstk_bytes(cfg, w, 7))
    tok = np.random.default_rng(83).integers(0, cfg.vocab, size=(1, cfg.seq + 1)).astype(np.uint32)
    print("[case] checkpoint load, dim 256, 2 layers", flush=True)
    with hb.Context(cfg.to_rh(), 0, 1, 0) as a, hb.Context(cfg.to_rh(), 0, 1, 0) as b:
        assert a.load_checkpoint(str(p)) == 7
        b.load_weights(w.embed, w.gamma_final, [lw.tensors() for lw in w.layers])
        oa = a.forward(tok[:, :-1], tok[:, 1:])
        ob = b.forward(tok[:, :-1], tok[:, 1:])
        np.testing.assert_array_equal(oa.logits, ob.logits)
        e, gf, layers = a.read_weights()
    np.testing.assert_array_equal(e, w.embed)
    np.testing.assert_array_equal(gf, w.gamma_final)
    for lw, got in zip(w.layers, layers):
        for x, y in zip(lw.tensors(), got):
            np.testing.assert_array_equal(x, y)


def test_checkpoint_save_is_byte_exact(tmp_path):
    """Weights already fp16-representable survive the device round trip, so
    the saved file equals the format definition's bytes."""
    cfg = _cfg()
    w = random_gammas(ModelWeights.normal(cfg, seed=84), seed=85)
    p = tmp_path / "out.bin"
    with hb.Context(cfg.to_rh(), 0, 1, 0) as c:
        c.load_weights(w.embed, w.gamma_final, [lw.tensors() for lw in w.layers])
        c.save_checkpoint(str(p), 1234)
    assert p.read_bytes() == rstk_bytes(cfg, w, 1234)
    info = hb.checkpoint_info(str(p))
    assert (info.step, info.dim, info.nlayers, info.vocab, info.seq) == (1234, 256, 2, 1024, 64)


def test_checkpoint_rejects_other_shapes(tmp_path):
    cfg = _cfg()
    w = ModelWeights.normal(cfg, seed=86)
    good = rstk_bytes(cfg, w, 0)
    other = small_cfg(dim=256, hidden=512, heads=2, hd=128, nlayers=3, vocab=1024, seq=64)
    p = tmp_path / "c.bin"
    with hb.Context(other.to_rh(), 0, 1, 0) as c:  # 3 layers vs the file's 2
        p.write_bytes(good)
        with pytest.raises(hb.HipBridgeError) as e:
            c.load_checkpoint(str(p))
        assert e.value.code == hb.RH_EINVAL
    wide = small_cfg(dim=256, hidden=640, heads=2, hd=128, nlayers=2, vocab=1024, seq=64)
    with hb.Context(wide.to_rh(), 0, 1, 0) as c:  # hidden is not in the header: size mismatch
        with pytest.raises(hb.HipBridgeError) as e:
            c.load_checkpoint(str(p))
        assert e.value.code == hb.RH_EIO
    with hb.Context(cfg.to_rh(), 0, 1, 0) as c:
        p.write_bytes(good[:-4])  # truncated
        with pytest.raises(hb.HipBridgeError) as e:
            c.load_checkpoint(str(p))
        assert e.value.code == hb.RH_EIO
        p.write_bytes(good)
        c.load_checkpoint(str(p))  # still usable


@pytest.mark.parametrize("max_batch", [1, 2])
def test_validate_matches_oracle(orc, tmp_path, max_batch):
    """5 windows (batches of max_batch) of a 1000-token file; the loss average
    and val_bpb follow train.rs's window positions and f32 sums."""
    cfg = _cfg()
    w = ModelWeights.normal(cfg, seed=87, std=0.05)
    rng = np.random.default_rng(88)
    ids = rng.integers(0, cfg.vocab, size=1000).astype("<u2")
    p = tmp_path / "val.bin"
    p.write_bytes(ids.tobytes())
    tb = hb.TokenBytes(values=np.where(rng.random(cfg.vocab) < 0.05, 0, rng.integers(1, 7, cfg.vocab)))
    steps, S = 5, cfg.seq
    print(f"[case] validate max_batch={max_batch}", flush=True)
    with hb.Context(cfg.to_rh(), 0, max_batch, 0) as c:
        c.load_weights(w.embed, w.gamma_final, [lw.tensors() for lw in w.layers])
        val = hb.TokenData(str(p))
        loss, bpb = c.validate(val, tb, steps)
        loss_nb, bpb_nb = c.validate(val, None, steps)
    # oracle: the same windows, one forward each, then compute_bpb's definition
    max_pos = len(ids) - S - 1
    ocfg, ow = oracle_cfg(orc, cfg), oracle_weights(orc, w)
    all_l, all_t = [], []
    for s in range(steps):
        pos = (s * S) % max_pos
        inp = ids[pos:pos + S].astype(np.uint32)[None]
        tgt = ids[pos + 1:pos + 1 + S].astype(np.uint32)[None]
        _, tl, _ = orc.forward(ocfg, ow, inp, tgt)
        all_l.append(tl[0])
        all_t.append(tgt[0])
    L, T = np.concatenate(all_l).astype(np.float64), np.concatenate(all_t)
    keep = tb.bytes[T] > 0
    ref_bpb = L[keep].sum() / (math.log(2) * tb.bytes[T][keep].sum())
    print(f"[result] validate loss gpu={loss} cpu={L.mean()} bpb gpu={bpb} cpu={ref_bpb}", flush=True)
    assert loss == pytest.approx(L.mean(), rel=LOSS_RTOL)
    assert bpb == pytest.approx(ref_bpb, rel=LOSS_RTOL)
    assert loss_nb == loss and bpb_nb == 0.0
