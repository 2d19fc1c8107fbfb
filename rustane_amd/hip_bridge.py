"""ctypes binding of librustane_hip.so (include/rustane_hip.h).

This is the Python face of the C-ABI that stands in for the reference's
`ane-bridge` crate (crates/ane-bridge/src/lib.rs:1-9).  It loads the in-tree
library and fails loudly when it is missing: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librustane_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(HERE), "include", "rustane_hip.h")

RH_OK, RH_EINVAL, RH_ERANGE, RH_ENOMEM, RH_EDEVICE, RH_ESTATE, RH_EIO = 0, -1, -2, -3, -4, -5, -6
ERR_NAMES = {RH_EINVAL: "RH_EINVAL", RH_ERANGE: "RH_ERANGE", RH_ENOMEM: "RH_ENOMEM",
             RH_EDEVICE: "RH_EDEVICE", RH_ESTATE: "RH_ESTATE", RH_EIO: "RH_EIO"}

K_GEMM_QKV, K_GEMM_WO, K_GEMM_W13, K_GEMM_W2, K_GEMM_LOGITS, K_ATTN = range(6)
K_GEMV_QKV, K_GEMV_WO, K_GEMV_W13, K_GEMV_W2, K_GEMV_LOGITS, K_DECODE_ATTN = range(6, 12)

_f32p = ctypes.POINTER(ctypes.c_float)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_vp = ctypes.c_void_p


class HipBridgeError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{ERR_NAMES.get(code, code)}: {msg}")
        self.code = code


class RhConfig(ctypes.Structure):
    _fields_ = [("dim", ctypes.c_int32), ("hidden", ctypes.c_int32), ("heads", ctypes.c_int32),
                ("kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("seq", ctypes.c_int32), ("nlayers", ctypes.c_int32), ("vocab", ctypes.c_int32),
                ("rms_eps", ctypes.c_float), ("rope_base", ctypes.c_float),
                ("softcap", ctypes.c_float)]


class RhCkptInfo(ctypes.Structure):
    _fields_ = [("version", ctypes.c_uint32), ("step", ctypes.c_uint32), ("dim", ctypes.c_uint32),
                ("nlayers", ctypes.c_uint32), ("vocab", ctypes.c_uint32), ("seq", ctypes.c_uint32),
                ("file_bytes", ctypes.c_uint64)]


class RhTrainConfig(ctypes.Structure):
    """TrainConfig (full_model.rs:42-78)."""
    _fields_ = [("max_lr", ctypes.c_float), ("min_lr_frac", ctypes.c_float), ("warmup_steps", ctypes.c_uint32),
                ("total_steps", ctypes.c_uint32), ("beta1", ctypes.c_float), ("beta2", ctypes.c_float),
                ("eps", ctypes.c_float), ("weight_decay", ctypes.c_float), ("matrix_lr_scale", ctypes.c_float),
                ("embed_lr_scale", ctypes.c_float), ("loss_scale", ctypes.c_float),
                ("accum_steps", ctypes.c_uint32), ("grad_clip", ctypes.c_float), ("softcap", ctypes.c_float)]


def train_config(**overrides) -> RhTrainConfig:
    """TrainConfig::default with fields overridden by keyword."""
    tc = RhTrainConfig()
    lib().rh_train_config_default(ctypes.byref(tc))
    for k, v in overrides.items():
        assert hasattr(tc, k), k
        setattr(tc, k, v)
    return tc


def learning_rate(step: int, tc: RhTrainConfig) -> float:
    return float(lib().rh_learning_rate(step, ctypes.byref(tc)))


class RhSchedConfig(ctypes.Structure):
    _fields_ = [("max_batch", ctypes.c_int), ("queue_capacity", ctypes.c_int), ("max_wait_us", ctypes.c_int)]


class RhSchedRequest(ctypes.Structure):
    _fields_ = [("request_id", ctypes.c_uint64), ("kind", ctypes.c_int), ("len", ctypes.c_int),
                ("nsteps", ctypes.c_int), ("tokens", ctypes.POINTER(ctypes.c_uint32)),
                ("targets", ctypes.POINTER(ctypes.c_uint32)), ("out_tokens", ctypes.POINTER(ctypes.c_uint32))]


class RhSchedResult(ctypes.Structure):
    _fields_ = [("request_id", ctypes.c_uint64), ("kind", ctypes.c_int), ("status", ctypes.c_int),
                ("loss", ctypes.c_float), ("batch", ctypes.c_int), ("queue_wait_ms", ctypes.c_float),
                ("service_ms", ctypes.c_float), ("total_ms", ctypes.c_float), ("message", ctypes.c_char * 128)]


JOB_FORWARD, JOB_GENERATE = 0, 1

_lib = None


def lib():
    """Loads librustane_hip.so; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m rustane_amd.build` "
                           "(there is no CPU fallback for the HIP path)")
    L = ctypes.CDLL(LIB_PATH)
    ctxp = ctypes.c_void_p
    L.rh_create.argtypes = [ctypes.POINTER(RhConfig), ctypes.c_int, ctypes.c_int, ctypes.c_int,
                            ctypes.POINTER(ctxp)]
    L.rh_destroy.argtypes = [ctxp]
    L.rh_destroy.restype = None
    L.rh_last_error.argtypes = [ctxp]
    L.rh_last_error.restype = ctypes.c_char_p
    L.rh_load_weights_f32.argtypes = [ctxp, _f32p, _f32p, ctypes.POINTER(_f32p)]
    L.rh_read_weights_f32.argtypes = [ctxp, _f32p, _f32p, ctypes.POINTER(_f32p)]
    L.rh_init_weights_normal.argtypes = [ctxp, ctypes.c_uint64, ctypes.c_float]
    L.rh_forward.argtypes = [ctxp, _u32p, _u32p, ctypes.c_int, ctypes.c_int, _f32p, _f32p, _f32p]
    L.rh_forward_backward.argtypes = [ctxp, _u32p, _u32p, ctypes.c_int, ctypes.c_int, ctypes.c_float, _f32p]
    L.rh_forward_train.argtypes = [ctxp, _u32p, _u32p, ctypes.c_int, ctypes.c_int, ctypes.c_float, _f32p,
                                   ctypes.POINTER(ctypes.c_void_p)]
    L.rh_backward.argtypes = [ctxp, ctypes.c_void_p, _u32p, ctypes.c_float, ctypes.c_float, _f32p]
    L.rh_forward_result_free.argtypes = [ctypes.c_void_p]
    L.rh_forward_result_free.restype = None
    L.rh_set_fp32_masters.argtypes = [ctxp, ctypes.c_int]
    L.rh_zero_grads.argtypes = [ctxp]
    L.rh_train_config_default.argtypes = [ctypes.POINTER(RhTrainConfig)]
    L.rh_train_config_default.restype = None
    L.rh_learning_rate.argtypes = [ctypes.c_uint32, ctypes.POINTER(RhTrainConfig)]
    L.rh_learning_rate.restype = ctypes.c_float
    L.rh_grad_norm.argtypes = [ctxp, _f32p]
    L.rh_update_weights.argtypes = [ctxp, ctypes.c_uint32, ctypes.c_float, ctypes.POINTER(RhTrainConfig),
                                    ctypes.c_float]
    L.rh_train_step.argtypes = [ctxp, ctypes.c_void_p, ctypes.c_uint32, ctypes.POINTER(RhTrainConfig), _f32p,
                                _f32p]
    L.rh_read_grads_f32.argtypes = [ctxp, _f32p, _f32p, ctypes.POINTER(_f32p)]
    L.rh_forward_dev.argtypes = [ctxp, _vp, _vp, ctypes.c_int, ctypes.c_int, _vp, _vp, _vp]
    L.rh_prefill.argtypes = [ctxp, _u32p, ctypes.c_int, ctypes.c_int, _u32p, _f32p]
    L.rh_decode_step.argtypes = [ctxp, ctypes.c_int, _u32p, _u32p, _f32p]
    L.rh_decode.argtypes = [ctxp, ctypes.c_int, _u32p, ctypes.c_int, _u32p]
    L.rh_decode_step_noalloc.argtypes = [ctxp, ctypes.c_int, _vp, _vp, _vp]
    L.rh_decode_pos.argtypes = [ctxp, ctypes.POINTER(ctypes.c_int)]
    L.rh_set_softcap.argtypes = [ctxp, ctypes.c_float]
    L.rh_sync.argtypes = [ctxp]
    L.rh_stream.argtypes = [ctxp]
    L.rh_stream.restype = ctypes.c_void_p
    L.rh_profile_enable.argtypes = [ctxp, ctypes.c_int, ctypes.c_int]
    L.rh_profile_read.argtypes = [ctxp, ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                                  ctypes.POINTER(ctypes.c_int64)]
    L.rh_set_graphs.argtypes = [ctxp, ctypes.c_int]
    L.rh_context_info.argtypes = [ctxp, ctypes.POINTER(RhConfig), ctypes.POINTER(ctypes.c_int),
                                  ctypes.POINTER(ctypes.c_int)]
    L.rh_checkpoint_info.argtypes = [ctypes.c_char_p, ctypes.POINTER(RhCkptInfo)]
    L.rh_load_checkpoint.argtypes = [ctxp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32)]
    L.rh_save_checkpoint.argtypes = [ctxp, ctypes.c_char_p, ctypes.c_uint32]
    L.rh_tokens_open.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)]
    L.rh_tokens_close.argtypes = [ctypes.c_void_p]
    L.rh_tokens_close.restype = None
    L.rh_tokens_len.argtypes = [ctypes.c_void_p]
    L.rh_tokens_len.restype = ctypes.c_int64
    L.rh_tokens_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, _u32p]
    L.rh_compute_bpb.argtypes = [_f32p, _u32p, ctypes.c_int64, ctypes.POINTER(ctypes.c_int32), ctypes.c_int,
                                 _f32p, _f32p, ctypes.POINTER(ctypes.c_int64)]
    L.rh_validate.argtypes = [ctxp, ctypes.c_void_p, ctypes.POINTER(ctypes.c_int32), ctypes.c_int, _f32p,
                              _f32p]
    L.rh_sched_create.argtypes = [ctxp, ctypes.POINTER(RhSchedConfig), ctypes.POINTER(ctypes.c_void_p)]
    L.rh_sched_destroy.argtypes = [ctypes.c_void_p]
    L.rh_sched_destroy.restype = None
    L.rh_sched_submit.argtypes = [ctypes.c_void_p, ctypes.POINTER(RhSchedRequest)]
    L.rh_sched_wait.argtypes = [ctypes.c_void_p, ctypes.POINTER(RhSchedResult)]
    L.rh_sched_run_batch.argtypes = [ctypes.c_void_p, ctypes.POINTER(RhSchedRequest), ctypes.c_int,
                                     ctypes.POINTER(RhSchedResult)]
    _lib = L
    return L


def header_symbols() -> list[str]:
    """Names of every function declared in include/rustane_hip.h."""
    import re
    text = open(HEADER_PATH).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rh_[a-z0-9_]+)\s*\(", text)))


def _f(a):
    return None if a is None else a.ctypes.data_as(_f32p)


def _u(a):
    return None if a is None else a.ctypes.data_as(_u32p)


@dataclass
class ForwardOut:
    logits: np.ndarray | None        # [B, S, V]
    token_losses: np.ndarray | None  # [B, S]
    mean_loss: np.ndarray | None     # [B]


class ForwardResult:
    """ForwardResult (full_model.rs:120-129): a handle to a training forward's
    caches, which stay on the device; rh_forward_result_free on release."""

    def __init__(self, h: ctypes.c_void_p, tokens: np.ndarray):
        self.h = h
        self.tokens = tokens

    def close(self):
        if getattr(self, "h", None):
            lib().rh_forward_result_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Context:
    """One rh_ctx: a device, a stream, fp16 weights, KV cache and workspaces."""

    def __init__(self, cfg: RhConfig, device: int = 0, max_batch: int = 1, max_ctx: int = 0):
        self.cfg = cfg
        self.max_batch, self.max_ctx = max_batch, max_ctx
        h = ctypes.c_void_p()
        rc = lib().rh_create(ctypes.byref(cfg), device, max_batch, max_ctx, ctypes.byref(h))
        if rc != RH_OK:
            raise HipBridgeError(rc, "rh_create failed")
        self.h = h

    # -- lifetime ---------------------------------------------------------
    def close(self):
        if getattr(self, "h", None):
            lib().rh_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _ck(self, rc: int, what: str):
        if rc != RH_OK:
            msg = lib().rh_last_error(self.h)
            raise HipBridgeError(rc, f"{what}: {msg.decode() if msg else ''}")

    # -- weights ----------------------------------------------------------
    def load_weights(self, embed, gamma_final, layers):
        """layers: nlayers lists of 9 fp32 arrays in RSTK order (reference orientation)."""
        keep = [np.ascontiguousarray(embed, np.float32), np.ascontiguousarray(gamma_final, np.float32)]
        flat = [np.ascontiguousarray(t, np.float32) for lw in layers for t in lw]
        ptrs = (_f32p * len(flat))(*[_f(t) for t in flat])
        self._ck(lib().rh_load_weights_f32(self.h, _f(keep[0]), _f(keep[1]), ptrs), "rh_load_weights_f32")

    def set_fp32_masters(self, keep: bool = True):
        """Keep (or drop) fp32 master weights on the device (rh_set_fp32_masters)."""
        self._ck(lib().rh_set_fp32_masters(self.h, int(keep)), "rh_set_fp32_masters")

    def read_weights(self):
        c = self.cfg
        D, F, V, L = c.dim, c.hidden, c.vocab, c.nlayers
        embed = np.empty((V, D), np.float32)
        gf = np.empty(D, np.float32)
        shapes = [(D, D)] * 4 + [(D, F)] * 3 + [(D,), (D,)]
        layers = [[np.empty(s, np.float32) for s in shapes] for _ in range(L)]
        flat = [t for lw in layers for t in lw]
        ptrs = (_f32p * len(flat))(*[_f(t) for t in flat])
        self._ck(lib().rh_read_weights_f32(self.h, _f(embed), _f(gf), ptrs), "rh_read_weights_f32")
        return embed, gf, layers

    # -- training pass ----------------------------------------------------
    def forward_backward(self, tokens, targets, loss_scale: float = 1.0):
        """Adds loss_scale x d(mean loss)/d(params) of every sequence to the
        context's gradients; returns the mean losses [B]."""
        tokens = np.ascontiguousarray(tokens, np.uint32)
        if tokens.ndim == 1:
            tokens = tokens[None]
        B, S = tokens.shape
        tg = np.ascontiguousarray(targets, np.uint32).reshape(B, S)
        ml = np.empty((B,), np.float32)
        self._ck(lib().rh_forward_backward(self.h, _u(tokens), _u(tg), B, S, float(loss_scale), _f(ml)),
                 "rh_forward_backward")
        return ml

    def forward_train(self, tokens, targets, softcap: float = 0.0):
        """full_model::forward -> ForwardResult: the training forward with its
        caches kept on the device; returns (ForwardResult, mean losses [B])."""
        tokens = np.ascontiguousarray(tokens, np.uint32)
        if tokens.ndim == 1:
            tokens = tokens[None]
        B, S = tokens.shape
        tg = np.ascontiguousarray(targets, np.uint32).reshape(B, S)
        ml = np.empty((B,), np.float32)
        h = ctypes.c_void_p()
        self._ck(lib().rh_forward_train(self.h, _u(tokens), _u(tg), B, S, float(softcap), _f(ml), ctypes.byref(h)),
                 "rh_forward_train")
        return ForwardResult(h, tokens), ml

    def backward(self, fwd: "ForwardResult", tokens=None, softcap: float = 0.0, loss_scale: float = 1.0,
                 want_norm: bool = True):
        """full_model::backward(&fwd, tokens, softcap, loss_scale, grads):
        accumulates the gradients; returns the accumulated gradients' L2 norm
        (None when want_norm is False)."""
        tok = fwd.tokens if tokens is None else np.ascontiguousarray(tokens, np.uint32)
        norm = ctypes.c_float()
        self._ck(lib().rh_backward(self.h, fwd.h, _u(tok), float(softcap), float(loss_scale),
                                   ctypes.byref(norm) if want_norm else None), "rh_backward")
        return norm.value if want_norm else None

    def zero_grads(self):
        self._ck(lib().rh_zero_grads(self.h), "rh_zero_grads")

    def read_grads(self):
        """(dembed [V, D], dgamma_final [D], [[9 per layer]]) in the weights'
        orientation and RSTK order."""
        c = self.cfg
        D, F, V, L = c.dim, c.hidden, c.vocab, c.nlayers
        embed = np.empty((V, D), np.float32)
        gf = np.empty(D, np.float32)
        shapes = [(D, D)] * 4 + [(D, F)] * 3 + [(D,), (D,)]
        layers = [[np.empty(s, np.float32) for s in shapes] for _ in range(L)]
        flat = [t for lw in layers for t in lw]
        ptrs = (_f32p * len(flat))(*[_f(t) for t in flat])
        self._ck(lib().rh_read_grads_f32(self.h, _f(embed), _f(gf), ptrs), "rh_read_grads_f32")
        return embed, gf, layers

    def grad_norm(self) -> float:
        out = ctypes.c_float()
        self._ck(lib().rh_grad_norm(self.h, ctypes.byref(out)), "rh_grad_norm")
        return out.value

    def update_weights(self, t: int, lr: float, tc: RhTrainConfig, grad_scale: float):
        self._ck(lib().rh_update_weights(self.h, t, lr, ctypes.byref(tc), grad_scale), "rh_update_weights")

    def train_step(self, data: "TokenData", step: int, tc: RhTrainConfig):
        """train_step (full_model.rs:1488-1600); returns (mean loss, clipped-norm input)."""
        loss, norm = ctypes.c_float(), ctypes.c_float()
        self._ck(lib().rh_train_step(self.h, data.h, step, ctypes.byref(tc), ctypes.byref(loss), ctypes.byref(norm)),
                 "rh_train_step")
        return loss.value, norm.value

    def init_normal(self, seed: int, std: float = 0.02):
        self._ck(lib().rh_init_weights_normal(self.h, seed, std), "rh_init_weights_normal")

    def set_softcap(self, c: float):
        self._ck(lib().rh_set_softcap(self.h, c), "rh_set_softcap")

    # -- forward ----------------------------------------------------------
    def forward(self, tokens, targets=None, want_logits=True, want_token_losses=True) -> ForwardOut:
        tokens = np.ascontiguousarray(tokens, np.uint32)
        if tokens.ndim == 1:
            tokens = tokens[None]
        B, S = tokens.shape
        tg = None if targets is None else np.ascontiguousarray(targets, np.uint32).reshape(B, S)
        logits = np.empty((B, S, self.cfg.vocab), np.float32) if want_logits else None
        tl = np.empty((B, S), np.float32) if (tg is not None and want_token_losses) else None
        ml = np.empty((B,), np.float32) if tg is not None else None
        self._ck(lib().rh_forward(self.h, _u(tokens), _u(tg), B, S, _f(logits), _f(tl), _f(ml)),
                 "rh_forward")
        return ForwardOut(logits, tl, ml)

    def forward_dev(self, tokens_ptr: int, targets_ptr: int | None, batch: int, seq: int,
                    logits_ptr=None, token_losses_ptr=None, mean_ptr=None):
        self._ck(lib().rh_forward_dev(self.h, tokens_ptr, targets_ptr, batch, seq, logits_ptr,
                                      token_losses_ptr, mean_ptr), "rh_forward_dev")

    # -- decode -----------------------------------------------------------
    def prefill(self, tokens, want_logits=False):
        tokens = np.ascontiguousarray(tokens, np.uint32)
        if tokens.ndim == 1:
            tokens = tokens[None]
        B, n = tokens.shape
        nxt = np.empty(B, np.uint32)
        lg = np.empty((B, self.cfg.vocab), np.float32) if want_logits else None
        self._ck(lib().rh_prefill(self.h, _u(tokens), B, n, _u(nxt), _f(lg)), "rh_prefill")
        return nxt, lg

    def decode_step(self, in_tok, want_logits=False):
        in_tok = np.ascontiguousarray(in_tok, np.uint32).reshape(-1)
        out = np.empty_like(in_tok)
        lg = np.empty((len(in_tok), self.cfg.vocab), np.float32) if want_logits else None
        self._ck(lib().rh_decode_step(self.h, len(in_tok), _u(in_tok), _u(out), _f(lg)), "rh_decode_step")
        return out, lg

    def decode_step_noalloc(self, batch: int, in_tok_ptr: int, out_tok_ptr: int, logits_ptr=None):
        """rh_decode_step_noalloc: device pointers, enqueued without a sync."""
        self._ck(lib().rh_decode_step_noalloc(self.h, batch, in_tok_ptr, out_tok_ptr, logits_ptr),
                 "rh_decode_step_noalloc")

    def decode(self, in_tok, nsteps: int):
        in_tok = np.ascontiguousarray(in_tok, np.uint32).reshape(-1)
        out = np.empty((nsteps, len(in_tok)), np.uint32)
        self._ck(lib().rh_decode(self.h, len(in_tok), _u(in_tok), nsteps, _u(out)), "rh_decode")
        return out

    @property
    def pos(self) -> int:
        p = ctypes.c_int()
        self._ck(lib().rh_decode_pos(self.h, ctypes.byref(p)), "rh_decode_pos")
        return p.value

    # -- misc -------------------------------------------------------------
    def sync(self):
        self._ck(lib().rh_sync(self.h), "rh_sync")

    @property
    def stream(self) -> int:
        return lib().rh_stream(self.h)

    def profile_enable(self, kclass: int, on: bool = True):
        self._ck(lib().rh_profile_enable(self.h, kclass, int(on)), "rh_profile_enable")

    def profile_read(self, kclass: int):
        ms = ctypes.c_double()
        n = ctypes.c_int64()
        self._ck(lib().rh_profile_read(self.h, kclass, ctypes.byref(ms), ctypes.byref(n)),
                 "rh_profile_read")
        return ms.value, n.value

    def set_graphs(self, on: bool):
        self._ck(lib().rh_set_graphs(self.h, int(on)), "rh_set_graphs")

    # -- on-disk formats ----------------------------------------------------
    def load_checkpoint(self, path: str) -> int:
        """load_checkpoint (bin/train.rs:296-345); returns the stored step."""
        step = ctypes.c_uint32()
        self._ck(lib().rh_load_checkpoint(self.h, os.fsencode(path), ctypes.byref(step)),
                 "rh_load_checkpoint")
        return step.value

    def save_checkpoint(self, path: str, step: int):
        """save_checkpoint (bin/train.rs:238-275) of the device weights."""
        self._ck(lib().rh_save_checkpoint(self.h, os.fsencode(path), step), "rh_save_checkpoint")

    def validate(self, val: "TokenData", token_bytes: "TokenBytes | None", steps: int):
        """validate (bin/train.rs:196-236) -> (avg_loss, bpb)."""
        loss, bpb = ctypes.c_float(), ctypes.c_float()
        tb = None if token_bytes is None else token_bytes.ptr()
        self._ck(lib().rh_validate(self.h, val.h, tb, steps, ctypes.byref(loss), ctypes.byref(bpb)),
                 "rh_validate")
        return loss.value, bpb.value


def _ck_free(rc: int, what: str):
    if rc != RH_OK:
        raise HipBridgeError(rc, f"{what}: {lib().rh_last_error(None).decode(errors='replace')}")


def checkpoint_info(path: str) -> RhCkptInfo:
    """RSTK header fields (bin/train.rs:249-256)."""
    info = RhCkptInfo()
    _ck_free(lib().rh_checkpoint_info(os.fsencode(path), ctypes.byref(info)), "rh_checkpoint_info")
    return info


class TokenData:
    """TokenData (data.rs:11-44): a memory-mapped uint16 token file."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        _ck_free(lib().rh_tokens_open(os.fsencode(path), ctypes.byref(h)), "rh_tokens_open")
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            lib().rh_tokens_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self) -> int:
        return int(lib().rh_tokens_len(self.h))

    def tokens(self, start: int, n: int) -> np.ndarray:
        out = np.empty(n, np.uint32)
        _ck_free(lib().rh_tokens_read(self.h, start, n, _u(out)), "rh_tokens_read")
        return out


class TokenBytes:
    """TokenBytes (data.rs:46-71): int32 byte length per token id."""

    def __init__(self, path: str | None = None, values=None):
        self.bytes = (np.fromfile(path, dtype="<i4") if path is not None
                      else np.ascontiguousarray(values, dtype=np.int32))

    def ptr(self):
        return self.bytes.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))


def compute_bpb(losses, targets, token_bytes: TokenBytes):
    """compute_bpb (data.rs:75-91) -> (bpb, total_nats, total_bytes)."""
    losses = np.ascontiguousarray(losses, np.float32).ravel()
    targets = np.ascontiguousarray(targets, np.uint32).ravel()
    if losses.size != targets.size:
        raise ValueError("losses and targets differ in length")
    bpb, nats, nb = ctypes.c_float(), ctypes.c_float(), ctypes.c_int64()
    _ck_free(lib().rh_compute_bpb(_f(losses), _u(targets), losses.size, token_bytes.ptr(),
                                  token_bytes.bytes.size, ctypes.byref(bpb), ctypes.byref(nats),
                                  ctypes.byref(nb)), "rh_compute_bpb")
    return bpb.value, nats.value, nb.value


@dataclass
class SchedResult:
    request_id: int
    kind: int
    status: int
    loss: float
    batch: int
    queue_wait_ms: float
    service_ms: float
    total_ms: float
    message: str
    tokens: np.ndarray | None = None  # generate requests


class Scheduler:
    """rh_sched over one Context (multistream::ForwardScheduler,
    multistream.rs:54-161): forward requests (tokens, targets) -> loss and
    generation requests (prompt, nsteps) -> greedy tokens, served in batches by
    one worker thread.  While it exists only the worker uses the context."""

    def __init__(self, ctx: Context, max_batch: int, queue_capacity: int | None = None,
                 max_wait_us: int = 0):
        cfg = RhSchedConfig(max_batch, queue_capacity or 2 * max_batch, max_wait_us)
        h = ctypes.c_void_p()
        ctx._ck(lib().rh_sched_create(ctx.h, ctypes.byref(cfg), ctypes.byref(h)), "rh_sched_create")
        self.h, self.ctx = h, ctx

    def close(self):
        if getattr(self, "h", None):
            lib().rh_sched_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @staticmethod
    def _request(rid, kind, tokens, targets=None, nsteps=0):
        tok = np.ascontiguousarray(tokens, np.uint32).ravel()
        tgt = None if targets is None else np.ascontiguousarray(targets, np.uint32).ravel()
        out = np.zeros(nsteps, np.uint32) if kind == JOB_GENERATE else None
        rq = RhSchedRequest(rid, kind, tok.size, nsteps, _u(tok), _u(tgt), _u(out))
        return rq, (tok, tgt, out)

    def run_batch(self, requests):
        """ForwardScheduler::run_batch.  requests: (id, tokens, targets) for a
        forward or (id, prompt, None, nsteps) for a generation; results sorted
        by id."""
        built = [self._request(r[0], JOB_GENERATE if len(r) > 3 else JOB_FORWARD, r[1], r[2],
                               r[3] if len(r) > 3 else 0) for r in requests]
        arr = (RhSchedRequest * len(built))(*[b[0] for b in built])
        res = (RhSchedResult * len(built))()
        rc = lib().rh_sched_run_batch(self.h, arr, len(built), res)
        if rc != RH_OK:
            raise HipBridgeError(rc, "rh_sched_run_batch")
        outs = {r[0]: keep[2] for r, (_, keep) in zip(requests, built)}
        return [SchedResult(x.request_id, x.kind, x.status, x.loss, x.batch, x.queue_wait_ms, x.service_ms,
                            x.total_ms, x.message.decode(errors="replace"), outs.get(x.request_id))
                for x in res]
