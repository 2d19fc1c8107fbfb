"""The C-ABI library on the host (no GPU needed).

librustane_hip.so must load, export every function include/rustane_hip.h
declares, and reject invalid arguments with the documented codes before any
device work: these are the host-side rules of the boundary that replaces the
reference's ane-bridge (crates/ane-bridge/src/lib.rs:1-9), whose compile step
returns a Result and whose callers never see a partial forward
(crates/engine/src/layer.rs:1678,4459).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np
import pytest

from rustane_amd import hip_bridge as hb


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(hb.LIB_PATH):
        from rustane_amd import build
        build.build()
    return hb.lib()


def _cfg(**kw):
    base = dict(dim=256, hidden=512, heads=4, kv_heads=4, head_dim=64, seq=64, nlayers=2,
                vocab=1024, rms_eps=1e-5, rope_base=1e4, softcap=0.0)
    base.update(kw)
    return hb.RhConfig(**base)


def test_header_declares_the_boundary():
    names = hb.header_symbols()
    for required in ("rh_create", "rh_destroy", "rh_last_error", "rh_load_weights_f32",
                     "rh_forward", "rh_prefill", "rh_decode_step"):
        assert required in names


def test_library_exports_every_header_symbol(lib):
    missing = [n for n in hb.header_symbols() if not hasattr(lib, n)]
    assert not missing, missing


def test_exports_are_unmangled_c_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", hb.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert set(hb.header_symbols()) <= exported


def test_library_has_gfx950_code_object():
    """The device code in the library is built for gfx950 only."""
    blob = open(hb.LIB_PATH, "rb").read()
    assert b"gfx950" in blob
    for other in (b"gfx942", b"gfx90a", b"gfx1100"):
        assert b"amdgcn-amd-amdhsa--" + other not in blob


@pytest.mark.parametrize("bad", [
    dict(dim=200),                  # dim % 128
    dict(hidden=300),               # hidden % 128
    dict(kv_heads=2),               # GQA is not part of the reference forward
    dict(head_dim=96),              # head_dim 64 or 128
    dict(heads=2),                  # heads * head_dim != dim
    dict(nlayers=0),
    dict(vocab=1023),               # vocab % 4
    dict(seq=0),
    dict(rms_eps=0.0),
    dict(rope_base=-1.0),
    dict(softcap=-1.0),
])
def test_create_rejects_invalid_config(lib, bad):
    out = ctypes.c_void_p(123)
    rc = lib.rh_create(ctypes.byref(_cfg(**bad)), 0, 1, 0, ctypes.byref(out))
    assert rc == hb.RH_EINVAL
    assert out.value is None


def test_create_rejects_bad_sizes_and_nulls(lib):
    out = ctypes.c_void_p()
    assert lib.rh_create(ctypes.byref(_cfg()), 0, 0, 0, ctypes.byref(out)) == hb.RH_EINVAL
    assert lib.rh_create(ctypes.byref(_cfg()), 0, 1, -1, ctypes.byref(out)) == hb.RH_EINVAL
    assert lib.rh_create(None, 0, 1, 0, ctypes.byref(out)) == hb.RH_EINVAL
    assert lib.rh_create(ctypes.byref(_cfg()), 0, 1, 0, None) == hb.RH_EINVAL


def test_create_on_missing_device_is_edevice(lib):
    out = ctypes.c_void_p()
    rc = lib.rh_create(ctypes.byref(_cfg()), 4096, 1, 0, ctypes.byref(out))
    assert rc == hb.RH_EDEVICE
    assert out.value is None


def test_null_context_is_rejected_everywhere(lib):
    tok = np.zeros(4, np.uint32)
    tp = tok.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))
    f = ctypes.c_float()
    pos = ctypes.c_int()
    assert lib.rh_forward(None, tp, tp, 1, 4, None, None, ctypes.byref(f)) == hb.RH_EINVAL
    assert lib.rh_forward_dev(None, None, None, 1, 4, None, None, None) == hb.RH_EINVAL
    assert lib.rh_prefill(None, tp, 1, 4, None, None) == hb.RH_EINVAL
    assert lib.rh_decode_step(None, 1, tp, tp, None) == hb.RH_EINVAL
    assert lib.rh_decode(None, 1, tp, 1, tp) == hb.RH_EINVAL
    assert lib.rh_decode_step_noalloc(None, 1, None, None, None) == hb.RH_EINVAL
    assert lib.rh_decode_pos(None, ctypes.byref(pos)) == hb.RH_EINVAL
    assert lib.rh_set_softcap(None, 1.0) == hb.RH_EINVAL
    assert lib.rh_sync(None) == hb.RH_EINVAL
    assert lib.rh_init_weights_normal(None, 0, 0.02) == hb.RH_EINVAL
    assert lib.rh_load_weights_f32(None, None, None, None) == hb.RH_EINVAL
    assert lib.rh_read_weights_f32(None, None, None, None) == hb.RH_EINVAL
    assert lib.rh_profile_enable(None, 0, 1) == hb.RH_EINVAL
    assert lib.rh_set_graphs(None, 1) == hb.RH_EINVAL
    assert lib.rh_stream(None) is None
    assert lib.rh_context_info(None, None, None, None) == hb.RH_EINVAL
    assert lib.rh_load_checkpoint(None, b"x", None) == hb.RH_EINVAL
    assert lib.rh_save_checkpoint(None, b"x", 0) == hb.RH_EINVAL
    assert lib.rh_validate(None, None, None, 1, None, None) == hb.RH_EINVAL
    lib.rh_destroy(None)  # a no-op
    lib.rh_tokens_close(None)  # a no-op
    assert lib.rh_tokens_len(None) == 0
    assert lib.rh_sched_create(None, None, None) == hb.RH_EINVAL
    assert lib.rh_sched_submit(None, None) == hb.RH_EINVAL
    assert lib.rh_sched_wait(None, None) == hb.RH_EINVAL
    assert lib.rh_sched_run_batch(None, None, 0, None) == hb.RH_EINVAL
    lib.rh_sched_destroy(None)  # a no-op
    assert lib.rh_forward_backward(None, tp, tp, 1, 4, 1.0, None) == hb.RH_EINVAL
    assert lib.rh_zero_grads(None) == hb.RH_EINVAL
    assert lib.rh_read_grads_f32(None, None, None, None) == hb.RH_EINVAL
    assert lib.rh_grad_norm(None, None) == hb.RH_EINVAL
    assert lib.rh_update_weights(None, 1, 0.1, None, 1.0) == hb.RH_EINVAL
    assert lib.rh_train_step(None, None, 0, None, None, None) == hb.RH_EINVAL


def test_train_config_defaults_and_schedule():
    """TrainConfig::default (full_model.rs:59-78) and learning_rate
    (full_model.rs:903-913) are host-only and run without a GPU."""
    tc = hb.train_config()
    assert (tc.max_lr, tc.warmup_steps, tc.total_steps, tc.accum_steps) == (pytest.approx(3e-4), 100, 10000, 10)
    assert (tc.beta1, tc.beta2, tc.weight_decay) == (pytest.approx(0.9), pytest.approx(0.95), pytest.approx(0.1))
    assert (tc.loss_scale, tc.grad_clip, tc.softcap) == (256.0, 1.0, 0.0)
    import oracle
    otc = oracle.TrainConfig()
    for step in (0, 1, 50, 99, 100, 101, 2500, 5050, 9999, 10000):
        assert hb.learning_rate(step, tc) == oracle.learning_rate(step, otc)


def test_context_free_errors_are_per_thread(lib):
    """rh_last_error(NULL) reports the calling thread's last context-free
    failure."""
    import threading
    assert lib.rh_tokens_open(b"/nonexistent/tokens.bin", ctypes.byref(ctypes.c_void_p())) == hb.RH_EIO
    assert b"/nonexistent/tokens.bin" in lib.rh_last_error(None)
    seen = []
    th = threading.Thread(target=lambda: seen.append(lib.rh_last_error(None)))
    th.start()
    th.join()
    assert seen == [b""]
