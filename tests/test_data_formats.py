"""On-disk formats either side of the forward, host side (no GPU): token
files (data.rs:11-44), the RSTK checkpoint header (bin/train.rs:238-262,
296-300) and compute_bpb (data.rs:75-91), through the C-ABI.

The reference holds no sample files for these formats, so the checks are
byte-level constructions from the format definitions plus hand-computed
known answers."""
import math
import struct

import numpy as np
import pytest

from rustane_amd import hip_bridge as hb


def test_tokens_roundtrip_and_bounds(tmp_path):
    rng = np.random.default_rng(3)
    ids = rng.integers(0, 65536, size=1001, dtype=np.int64).astype("<u2")
    p = tmp_path / "tok.bin"
    p.write_bytes(ids.tobytes() + b"\x07")  # trailing odd byte is ignored
    t = hb.TokenData(str(p))
    assert len(t) == 1001
    np.testing.assert_array_equal(t.tokens(0, 1001), ids.astype(np.uint32))
    np.testing.assert_array_equal(t.tokens(500, 7), ids[500:507].astype(np.uint32))
    assert t.tokens(1001, 0).size == 0
    with pytest.raises(hb.HipBridgeError) as e:
        t.tokens(995, 7)
    assert e.value.code == hb.RH_ERANGE
    t.close()


def test_tokens_little_endian_and_empty(tmp_path):
    p = tmp_path / "le.bin"
    p.write_bytes(bytes([0x34, 0x12, 0xFF, 0xFF, 0x00, 0x01]))
    t = hb.TokenData(str(p))
    np.testing.assert_array_equal(t.tokens(0, 3), [0x1234, 0xFFFF, 0x0100])
    e = tmp_path / "empty.bin"
    e.write_bytes(b"")
    assert len(hb.TokenData(str(e))) == 0
    with pytest.raises(hb.HipBridgeError) as err:
        hb.TokenData(str(tmp_path / "missing.bin"))
    assert err.value.code == hb.RH_EIO


def test_checkpoint_header_fields(tmp_path):
    p = tmp_path / "ckpt_000042.bin"
    p.write_bytes(struct.pack("<4s6I", b"RSTK", 1, 42, 768, 6, 8192, 512) + b"\0" * 12)
    info = hb.checkpoint_info(str(p))
    assert (info.version, info.step, info.dim, info.nlayers, info.vocab, info.seq) == (1, 42, 768, 6, 8192, 512)
    assert info.file_bytes == 40
    bad = tmp_path / "bad.bin"
    bad.write_bytes(struct.pack("<4s6I", b"RSTX", 1, 0, 1, 1, 1, 1))
    short = tmp_path / "short.bin"
    short.write_bytes(b"RSTK" + b"\0" * 10)
    for q in (bad, short):
        with pytest.raises(hb.HipBridgeError) as e:
            hb.checkpoint_info(str(q))
        assert e.value.code == hb.RH_EIO


def test_compute_bpb_known_answers():
    tb = hb.TokenBytes(values=[2, 0, 3, 1])
    # token 1 has no bytes (special token): its loss is left out
    bpb, nats, nb = hb.compute_bpb([1.0, 2.0, 3.0], [0, 1, 2], tb)
    assert (nats, nb) == (4.0, 5)
    assert bpb == pytest.approx(4.0 / (math.log(2) * 5), rel=1e-6)
    # all special -> 0 bytes -> bpb 0 (data.rs:85-89)
    assert hb.compute_bpb([5.0, 6.0], [1, 1], tb) == (0.0, 0.0, 0)
    assert hb.compute_bpb([], [], tb) == (0.0, 0.0, 0)
    # uniform loss ln 2 per byte-weighted token: 1 bit per byte
    bpb, _, _ = hb.compute_bpb([math.log(2) * 3], [2], tb)
    assert bpb == pytest.approx(1.0, rel=1e-6)
    with pytest.raises(hb.HipBridgeError) as e:
        hb.compute_bpb([1.0], [4], tb)
    assert e.value.code == hb.RH_ERANGE


def test_compute_bpb_random_vs_float64():
    rng = np.random.default_rng(9)
    V = 500
    tb = hb.TokenBytes(values=np.where(rng.random(V) < 0.1, 0, rng.integers(1, 9, V)))
    losses = rng.random(4096).astype(np.float32) * 8
    targets = rng.integers(0, V, 4096).astype(np.uint32)
    bpb, nats, nb = hb.compute_bpb(losses, targets, tb)
    keep = tb.bytes[targets] > 0
    n64, b64 = float(losses[keep].astype(np.float64).sum()), int(tb.bytes[targets][keep].sum())
    assert nb == b64
    assert nats == pytest.approx(n64, rel=1e-5)
    assert bpb == pytest.approx(n64 / (math.log(2) * b64), rel=1e-5)
