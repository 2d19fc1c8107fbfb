"""ctypes binding of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY.  This is the parity checker for the HIP path and
the timed CPU baseline; only tests/, the smoke check and the benchmark's
CPU-baseline leg import it.  The product package (rustane_amd) never does.

The C restatement lives in oracle.cpp; each function there cites the
reference file:line it follows.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_u32p = ctypes.POINTER(ctypes.c_uint32)


class OrcConfig(ctypes.Structure):
    _fields_ = [
        ("dim", ctypes.c_int32), ("hidden", ctypes.c_int32), ("heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("nlayers", ctypes.c_int32), ("vocab", ctypes.c_int32),
        ("rms_eps", ctypes.c_float), ("rope_base", ctypes.c_float), ("softcap", ctypes.c_float),
        ("fp16_operands", ctypes.c_int32),
    ]


class OrcWeights(ctypes.Structure):
    _fields_ = [("embed", _f32p), ("gamma_final", _f32p), ("layers", ctypes.POINTER(_f32p))]


class OrcGrads(ctypes.Structure):
    _fields_ = [("dembed", _f32p), ("dgamma_final", _f32p), ("layers", ctypes.POINTER(_f32p))]


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE] + (["-B"] if force else []),
                       check=True, stdout=subprocess.DEVNULL)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        sz = ctypes.c_size_t
        L.orc_vsma.argtypes = [_f32p, ctypes.c_float, _f32p, _f32p, sz]
        L.orc_vsub.argtypes = [_f32p, _f32p, _f32p, sz]
        L.orc_mtrans.argtypes = [_f32p, sz, _f32p, sz, sz, sz]
        L.orc_sgemm_at.argtypes = [_f32p, sz, sz, _f32p, sz, _f32p]
        L.orc_random_vec.argtypes = [_f32p, sz, ctypes.c_float]
        L.orc_embedding_forward.argtypes = [_f32p, sz, _u32p, sz, _f32p]
        L.orc_rmsnorm_forward.argtypes = [_f32p, _f32p, _f32p, sz, ctypes.c_float]
        L.orc_rmsnorm_forward.restype = ctypes.c_float
        L.orc_rmsnorm_forward_channel_first.argtypes = [_f32p, _f32p, _f32p, _f32p, sz, sz,
                                                        ctypes.c_float]
        L.orc_silu_gate.argtypes = [_f32p, _f32p, _f32p, sz]
        L.orc_cross_entropy_forward.argtypes = [_f32p, sz, ctypes.c_uint32, _f32p]
        L.orc_cross_entropy_forward.restype = ctypes.c_float
        L.orc_cross_entropy_forward_backward_batch.argtypes = [_f32p, _u32p, sz, sz, _f32p,
                                                               ctypes.c_float]
        L.orc_cross_entropy_forward_backward_batch.restype = ctypes.c_float
        L.orc_rope_table.argtypes = [sz, sz, ctypes.c_float, _f32p, _f32p]
        L.orc_sdpa_fwd.argtypes = [ctypes.POINTER(OrcConfig), sz, _f32p, _f32p, _f32p, _f32p,
                                   _f32p, _f32p, _f32p, _f32p]
        L.orc_layer_forward.argtypes = [ctypes.POINTER(OrcConfig), sz, ctypes.POINTER(_f32p),
                                        _f32p, _f32p]
        L.orc_forward.argtypes = [ctypes.POINTER(OrcConfig), ctypes.POINTER(OrcWeights), _u32p,
                                  _u32p, ctypes.c_int, ctypes.c_int, _f32p, _f32p, _f32p]
        L.orc_forward.restype = ctypes.c_int
        L.orc_kv_create.argtypes = [ctypes.POINTER(OrcConfig), ctypes.c_int]
        L.orc_kv_create.restype = ctypes.c_void_p
        L.orc_kv_destroy.argtypes = [ctypes.c_void_p]
        L.orc_kv_pos.argtypes = [ctypes.c_void_p]
        L.orc_prefill.argtypes = [ctypes.POINTER(OrcConfig), ctypes.POINTER(OrcWeights),
                                  ctypes.c_void_p, _u32p, ctypes.c_int, _f32p]
        L.orc_decode_step.argtypes = [ctypes.POINTER(OrcConfig), ctypes.POINTER(OrcWeights),
                                      ctypes.c_void_p, ctypes.c_uint32, _f32p]
        L.orc_prefill_batch.argtypes = [ctypes.POINTER(OrcConfig), ctypes.POINTER(OrcWeights),
                                        ctypes.POINTER(ctypes.c_void_p), ctypes.c_int, _u32p, ctypes.c_int, _f32p]
        L.orc_decode_step_batch.argtypes = [ctypes.POINTER(OrcConfig), ctypes.POINTER(OrcWeights),
                                            ctypes.POINTER(ctypes.c_void_p), ctypes.c_int, _u32p, _f32p,
                                            ctypes.POINTER(ctypes.c_int32)]
        L.orc_num_threads.restype = ctypes.c_int
        L.orc_forward_backward.argtypes = [ctypes.POINTER(OrcConfig), ctypes.POINTER(OrcWeights),
                                           _u32p, _u32p, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                           ctypes.POINTER(OrcGrads), _f32p]
        L.orc_forward_backward.restype = ctypes.c_int
        L.orc_rmsnorm_backward_channel_first.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
                                                         sz, sz]
        L.orc_silu_gate_backward.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, sz]
        L.orc_sdpa_backward.argtypes = [ctypes.POINTER(OrcConfig), sz, _f32p, _f32p, _f32p, _f32p,
                                        _f32p, _f32p, _f32p]
        L.orc_rope_backward.argtypes = [ctypes.POINTER(OrcConfig), _f32p, sz]
        L.orc_adam_step_fused.argtypes = [_f32p, _f32p, _f32p, _f32p, sz, ctypes.c_uint32, ctypes.c_float,
                                          ctypes.c_float, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                                          ctypes.c_float]
        L.orc_powi.argtypes = [ctypes.c_float, ctypes.c_uint32]
        L.orc_powi.restype = ctypes.c_float
        L.orc_svesq.argtypes = [_f32p, sz]
        L.orc_svesq.restype = ctypes.c_float
        L.orc_learning_rate.argtypes = [ctypes.c_uint32, ctypes.c_float, ctypes.c_float, ctypes.c_uint32,
                                        ctypes.c_uint32]
        L.orc_learning_rate.restype = ctypes.c_float
        _lib = L
    return _lib


def fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_f32p)


def up(a: np.ndarray):
    assert a.dtype == np.uint32 and a.flags.c_contiguous
    return a.ctypes.data_as(_u32p)


# fp16 rounding points of the oracle's fp16-operand mode (oracle.h ORC_F16_*)
F16_POINTS = {"xn": 1, "q": 2, "k": 4, "v": 8, "p": 16, "attn": 32, "xn2": 64, "gate": 128, "xf": 256}
F16_ALL = 511


def make_config(dim, hidden, heads, nlayers, vocab, head_dim=None, rms_eps=1e-5,
                rope_base=1e4, softcap=0.0, fp16_operands=0) -> OrcConfig:
    """fp16_operands: True (every point) or a set of F16_POINTS bits at which
    the forward and decode round to fp16, where an fp16-operand device path
    does; 0 = the reference's fp32 arithmetic."""
    hd = head_dim if head_dim is not None else dim // heads
    bits = F16_ALL if fp16_operands is True else int(fp16_operands)
    return OrcConfig(dim, hidden, heads, hd, nlayers, vocab, rms_eps, rope_base, softcap, bits)


class Weights:
    """Holds numpy fp32 arrays (reference orientation) and the ctypes view."""

    def __init__(self, embed, gamma_final, layers):
        self.embed = np.ascontiguousarray(embed, dtype=np.float32)
        self.gamma_final = np.ascontiguousarray(gamma_final, dtype=np.float32)
        self.layers = [[np.ascontiguousarray(t, dtype=np.float32) for t in lw] for lw in layers]
        flat = [t for lw in self.layers for t in lw]
        self._ptrs = (_f32p * len(flat))(*[fp(t) for t in flat])
        self.c = OrcWeights(fp(self.embed), fp(self.gamma_final), self._ptrs)


def forward(cfg: OrcConfig, w: Weights, tokens: np.ndarray, targets: np.ndarray | None,
            want_logits: bool = True):
    """Returns (logits [B,S,V] | None, token_losses [B,S] | None, mean_loss [B] | None)."""
    tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
    if tokens.ndim == 1:
        tokens = tokens[None, :]
    B, S = tokens.shape
    logits = np.zeros((B, S, cfg.vocab), np.float32) if want_logits else None
    tl = ml = None
    tg = None
    if targets is not None:
        tg = np.ascontiguousarray(targets, dtype=np.uint32).reshape(B, S)
        tl = np.zeros((B, S), np.float32)
        ml = np.zeros((B,), np.float32)
    rc = lib().orc_forward(ctypes.byref(cfg), ctypes.byref(w.c), up(tokens),
                           up(tg) if tg is not None else None, B, S,
                           fp(logits) if logits is not None else None,
                           fp(tl) if tl is not None else None, fp(ml) if ml is not None else None)
    if rc != 0:
        raise ValueError(f"orc_forward failed: {rc}")
    return logits, tl, ml


class KV:
    def __init__(self, cfg: OrcConfig, max_ctx: int):
        self.cfg = cfg
        self.h = lib().orc_kv_create(ctypes.byref(cfg), max_ctx)

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_kv_destroy(self.h)
            self.h = None

    @property
    def pos(self):
        return lib().orc_kv_pos(self.h)

    def prefill(self, w: Weights, tokens: np.ndarray) -> np.ndarray:
        tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.zeros(self.cfg.vocab, np.float32)
        rc = lib().orc_prefill(ctypes.byref(self.cfg), ctypes.byref(w.c), self.h, up(tokens),
                               len(tokens), fp(out))
        if rc != 0:
            raise ValueError(f"orc_prefill failed: {rc}")
        return out

    def step(self, w: Weights, token: int):
        out = np.zeros(self.cfg.vocab, np.float32)
        best = lib().orc_decode_step(ctypes.byref(self.cfg), ctypes.byref(w.c), self.h,
                                     int(token), fp(out))
        if best < 0:
            raise ValueError(f"orc_decode_step failed: {best}")
        return best, out


class KVBatch:
    """B sequences with their own caches, stepped together
    (orc_prefill_batch / orc_decode_step_batch)."""

    def __init__(self, cfg: OrcConfig, batch: int, max_ctx: int):
        self.cfg = cfg
        self.kvs = [KV(cfg, max_ctx) for _ in range(batch)]
        self._h = (ctypes.c_void_p * batch)(*[kv.h for kv in self.kvs])

    @property
    def pos(self):
        return [kv.pos for kv in self.kvs]

    def prefill(self, w: Weights, tokens: np.ndarray) -> np.ndarray:
        """tokens [B, len] -> last-position logits [B, V]."""
        tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
        B, n = tokens.shape
        assert B == len(self.kvs)
        out = np.zeros((B, self.cfg.vocab), np.float32)
        rc = lib().orc_prefill_batch(ctypes.byref(self.cfg), ctypes.byref(w.c), self._h, B, up(tokens), n,
                                     fp(out))
        if rc != 0:
            raise ValueError(f"orc_prefill_batch failed: {rc}")
        return out

    def step(self, w: Weights, tokens) -> tuple[np.ndarray, np.ndarray]:
        """tokens [B] -> (argmax [B], logits [B, V])."""
        tokens = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
        B = tokens.size
        assert B == len(self.kvs)
        out = np.zeros((B, self.cfg.vocab), np.float32)
        best = np.zeros(B, np.int32)
        rc = lib().orc_decode_step_batch(ctypes.byref(self.cfg), ctypes.byref(w.c), self._h, B, up(tokens),
                                         fp(out), best.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)))
        if rc != 0:
            raise ValueError(f"orc_decode_step_batch failed: {rc}")
        return best, out


class Grads:
    """Zero-initialised fp32 gradient arrays shaped like Weights (reference
    orientation, RSTK order); the oracle accumulates into them."""

    def __init__(self, w: Weights):
        self.embed = np.zeros_like(w.embed)
        self.gamma_final = np.zeros_like(w.gamma_final)
        self.layers = [[np.zeros_like(t) for t in lw] for lw in w.layers]
        flat = [t for lw in self.layers for t in lw]
        self._ptrs = (_f32p * len(flat))(*[fp(t) for t in flat])
        self.c = OrcGrads(fp(self.embed), fp(self.gamma_final), self._ptrs)


def forward_backward(cfg: OrcConfig, w: Weights, tokens: np.ndarray, targets: np.ndarray,
                     grads: Grads | None = None, loss_scale: float = 1.0):
    """Adds loss_scale x the gradient of each sequence's mean loss into grads
    (new zero grads when None).  Returns (grads, mean_loss [B])."""
    tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
    if tokens.ndim == 1:
        tokens = tokens[None, :]
    B, S = tokens.shape
    tg = np.ascontiguousarray(targets, dtype=np.uint32).reshape(B, S)
    g = grads if grads is not None else Grads(w)
    ml = np.zeros((B,), np.float32)
    rc = lib().orc_forward_backward(ctypes.byref(cfg), ctypes.byref(w.c), up(tokens), up(tg), B, S,
                                    float(loss_scale), ctypes.byref(g.c), fp(ml))
    if rc != 0:
        raise ValueError(f"orc_forward_backward failed: {rc}")
    return g, ml


# ---------------------------------------------------------------- optimizer
class TrainConfig:
    """TrainConfig and its defaults (full_model.rs:42-78)."""

    def __init__(self, **kw):
        self.max_lr, self.min_lr_frac, self.warmup_steps, self.total_steps = 3e-4, 0.1, 100, 10000
        self.beta1, self.beta2, self.eps, self.weight_decay = 0.9, 0.95, 1e-8, 0.1
        self.matrix_lr_scale, self.embed_lr_scale, self.loss_scale = 0.05, 5.0, 256.0
        self.accum_steps, self.grad_clip, self.softcap = 10, 1.0, 0.0
        for k, v in kw.items():
            assert hasattr(self, k), k
            setattr(self, k, v)


def adam_step_fused(param, grad, m, v, t, lr, beta1, beta2, eps, wd, grad_scale):
    """step_fused (cpu/adam.rs:95-132) in place on fp32 numpy arrays."""
    lib().orc_adam_step_fused(fp(param), fp(grad) if grad is not None else None, fp(m), fp(v), param.size,
                              int(t), lr, beta1, beta2, eps, wd, grad_scale)


def learning_rate(step, tc: TrainConfig) -> float:
    return float(lib().orc_learning_rate(int(step), tc.max_lr, tc.min_lr_frac, int(tc.warmup_steps),
                                         int(tc.total_steps)))


def grad_norm(g: Grads) -> float:
    """grad_norm (full_model.rs:1403-1450): per-tensor vDSP_svesq, summed as
    (embed + gamma_final + first half of the layers) + (second half), sqrt."""
    sq = lambda a: float(lib().orc_svesq(fp(a), a.size))
    mid = len(g.layers) // 2
    s1 = np.float32(sq(g.embed))
    s1 = np.float32(s1 + np.float32(sq(g.gamma_final)))
    for lw in g.layers[:mid]:
        for t in lw:
            s1 = np.float32(s1 + np.float32(sq(t)))
    s2 = np.float32(0.0)
    for lw in g.layers[mid:]:
        for t in lw:
            s2 = np.float32(s2 + np.float32(sq(t)))
    return float(np.sqrt(np.float32(s1 + s2)))


class OptState:
    """ModelOptState: zero first and second moments shaped like the weights."""

    def __init__(self, w: Weights):
        self.embed_m, self.embed_v = np.zeros_like(w.embed), np.zeros_like(w.embed)
        self.gf_m, self.gf_v = np.zeros_like(w.gamma_final), np.zeros_like(w.gamma_final)
        self.m = [[np.zeros_like(t) for t in lw] for lw in w.layers]
        self.v = [[np.zeros_like(t) for t in lw] for lw in w.layers]


def update_weights(w: Weights, g: Grads, o: OptState, t: int, lr: float, tc: TrainConfig, grad_scale: float):
    """update_weights (full_model.rs:1123-1241) + update_layer (:1243-1400):
    embed at lr * embed_lr_scale and gamma_final at lr, both without weight
    decay; per layer the seven matrices at lr * matrix_lr_scale with
    weight_decay, the two gammas at lr without."""
    b1, b2, eps = tc.beta1, tc.beta2, tc.eps
    f32 = np.float32
    embed_lr = float(f32(lr) * f32(tc.embed_lr_scale))   # fp32 products, as in the reference
    matrix_lr = float(f32(lr) * f32(tc.matrix_lr_scale))
    adam_step_fused(w.embed, g.embed, o.embed_m, o.embed_v, t, embed_lr, b1, b2, eps, 0.0, grad_scale)
    adam_step_fused(w.gamma_final, g.gamma_final, o.gf_m, o.gf_v, t, lr, b1, b2, eps, 0.0, grad_scale)
    for lw, lg, lm, lv in zip(w.layers, g.layers, o.m, o.v):
        for j in range(9):
            mat = j < 7
            adam_step_fused(lw[j], lg[j], lm[j], lv[j], t, matrix_lr if mat else lr, b1, b2, eps,
                            tc.weight_decay if mat else 0.0, grad_scale)


def train_update(w: Weights, g: Grads, o: OptState, step: int, tc: TrainConfig):
    """The update half of train_step_with_options (full_model.rs:1573-1600):
    gsc = 1/(accum_steps*loss_scale); clip by the global norm; update_weights
    at t = step + 1.  Returns (scaled_norm, combined_scale, lr)."""
    gsc = np.float32(1.0) / (np.float32(tc.accum_steps) * np.float32(tc.loss_scale))
    raw = np.float32(grad_norm(g))
    scaled = np.float32(raw * gsc)
    combined = np.float32(tc.grad_clip) / raw if scaled > np.float32(tc.grad_clip) else gsc
    lr = learning_rate(step, tc)
    update_weights(w, g, o, step + 1, lr, tc, float(combined))
    return float(scaled), float(combined), lr
