"""Host-side mirror of rustane's engine forward/loss API over the HIP path.

Names, argument meaning and error behaviour follow the reference crate
`engine` (crates/engine/src/):

  ModelConfig, presets, param_count      model.rs:5-151
  LayerWeights / ModelWeights + random   layer.rs:52-63,1509-1567; full_model.rs:19-23,132-141
  CompiledKernels.compile                layer.rs:843-969 (here: creates the GPU context)
  ModelForwardWorkspace.new / new_lean   full_model.rs:206-264
  forward -> ForwardResult               full_model.rs:915-991
  forward_ws / forward_only_ws -> loss   full_model.rs:378-472, 494-588
  forward_losses -> per-token losses     full_model.rs:1603-1660

Every call runs on the GPU through librustane_hip.so; weights are uploaded
once per ModelWeights generation (the reference re-stages them into ANE
IOSurfaces on every layer call, layer.rs:4670-4705).  Like the reference,
shape mismatches raise (Rust `assert!` panics -> AssertionError here).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import hip_bridge as hb


# --------------------------------------------------------------------------- config
@dataclass
class ModelConfig:
    dim: int
    hidden: int
    heads: int
    kv_heads: int
    hd: int
    seq: int
    nlayers: int
    vocab: int
    q_dim: int = 0
    kv_dim: int = 0
    gqa_ratio: int = 1

    def __post_init__(self):
        if not self.q_dim:
            self.q_dim = self.heads * self.hd
        if not self.kv_dim:
            self.kv_dim = self.kv_heads * self.hd
        self.gqa_ratio = self.heads // self.kv_heads

    @staticmethod
    def custom(dim, hidden, heads, nlayers, seq, vocab=8192, hd=128) -> "ModelConfig":
        """custom_config of the probes (tests/bench_fwd_only_scale.rs:24-44)."""
        return ModelConfig(dim, hidden, heads, heads, hd, seq, nlayers, vocab)

    # presets (model.rs:21-151)
    @staticmethod
    def gpt_karpathy():
        return ModelConfig(768, 2048, 6, 6, 128, 512, 6, 8192)

    @staticmethod
    def gpt_1024():
        return ModelConfig(1024, 2816, 8, 8, 128, 512, 8, 8192)

    @staticmethod
    def target_600m():
        return ModelConfig(1536, 4096, 12, 12, 128, 512, 20, 8192)

    @staticmethod
    def target_800m():
        return ModelConfig(1792, 4864, 14, 14, 128, 512, 24, 8192)

    @staticmethod
    def target_1b():
        return ModelConfig(2048, 5632, 16, 16, 128, 512, 28, 8192)

    @staticmethod
    def target_1_5b():
        return ModelConfig(2304, 6144, 18, 18, 128, 512, 32, 8192)

    @staticmethod
    def mha_28l():
        return ModelConfig(1024, 3072, 8, 8, 128, 256, 28, 8192)

    def param_count(self) -> int:
        """model.rs:109-114."""
        per_layer = 4 * self.dim * self.dim + 3 * self.dim * self.hidden
        return self.nlayers * per_layer + self.vocab * self.dim + self.dim * (2 * self.nlayers + 1)

    def to_rh(self, softcap: float = 0.0) -> hb.RhConfig:
        assert self.kv_heads == self.heads, "MHA only (sdpa_fwd.rs reshapes K/V with `heads`)"
        return hb.RhConfig(self.dim, self.hidden, self.heads, self.kv_heads, self.hd, self.seq,
                           self.nlayers, self.vocab, 1e-5, 1e4, softcap)


# Workloads of the measured configurations (weights N(0, 0.02), uniform tokens).
def tiny_config():
    return ModelConfig(512, 1408, 8, 8, 64, 256, 8, 8192)


def cfg_600m():
    return ModelConfig(1536, 4096, 12, 12, 128, 512, 20, 32000)


def cfg_5b_deep():
    return ModelConfig(2560, 6912, 20, 20, 128, 512, 60, 32000)


def cfg_7b():
    return ModelConfig(4096, 11008, 32, 32, 128, 512, 32, 32000)


# --------------------------------------------------------------------------- weights
_LCG_A = np.uint64(6364136223846793005)
_LCG_C = np.uint64(1442695040888963407)


def random_vec(n: int, scale: float) -> np.ndarray:
    """random_vec (layer.rs:1556-1567): wrapping-u64 LCG seeded with 42 + n,
    r = ((s >> 32) as f32 / u32::MAX as f32) * 2 - 1, x = r * scale.
    Vectorised with LCG jump-ahead: s_{j*B+k} = A_k * s_{j*B} + C_k."""
    B = 4096
    Ak = np.empty(B, np.uint64)
    Ck = np.empty(B, np.uint64)
    a, c = np.uint64(1), np.uint64(0)
    with np.errstate(over="ignore"):
        for k in range(B):  # (A_k, C_k) for k+1 steps
            a = a * _LCG_A
            c = c * _LCG_A + _LCG_C
            Ak[k], Ck[k] = a, c
        out = np.empty(n, np.float32)
        s = np.uint64(42 + n)
        umax = np.float32(4294967295.0)
        sc = np.float32(scale)
        for j in range(0, n, B):
            m = min(B, n - j)
            st = Ak[:m] * s + Ck[:m]
            r = ((st >> np.uint64(32)).astype(np.float32) / umax) * np.float32(2.0) - np.float32(1.0)
            out[j:j + m] = r * sc
            s = st[m - 1]
    return out


@dataclass
class LayerWeights:
    wq: np.ndarray      # [DIM, Q_DIM]  (in x out)
    wk: np.ndarray      # [DIM, KV_DIM]
    wv: np.ndarray      # [DIM, KV_DIM]
    wo: np.ndarray      # [Q_DIM, DIM]
    w1: np.ndarray      # [DIM, HIDDEN]
    w3: np.ndarray      # [DIM, HIDDEN]
    w2: np.ndarray      # [DIM, HIDDEN] (used transposed)
    gamma1: np.ndarray  # [DIM]
    gamma2: np.ndarray  # [DIM]

    @staticmethod
    def random(cfg: ModelConfig) -> "LayerWeights":
        """layer.rs:1509-1524: Wq/Wk/Wv 1/sqrt(D), W1/W3 1/sqrt(F), Wo = W2 = 0 (DeepNet)."""
        sq = np.float32(1.0) / np.sqrt(np.float32(cfg.dim))
        sf = np.float32(1.0) / np.sqrt(np.float32(cfg.hidden))
        D, F = cfg.dim, cfg.hidden
        return LayerWeights(
            random_vec(D * cfg.q_dim, sq).reshape(D, cfg.q_dim),
            random_vec(D * cfg.kv_dim, sq).reshape(D, cfg.kv_dim),
            random_vec(D * cfg.kv_dim, sq).reshape(D, cfg.kv_dim),
            np.zeros((cfg.q_dim, D), np.float32),
            random_vec(D * F, sf).reshape(D, F),
            random_vec(D * F, sf).reshape(D, F),
            np.zeros((D, F), np.float32),
            np.ones(D, np.float32), np.ones(D, np.float32))

    def tensors(self):
        """RSTK order (bin/train.rs:238-345)."""
        return [self.wq, self.wk, self.wv, self.wo, self.w1, self.w3, self.w2, self.gamma1,
                self.gamma2]


@dataclass
class ModelWeights:
    embed: np.ndarray        # [VOCAB, DIM]
    layers: list             # [LayerWeights]
    gamma_final: np.ndarray  # [DIM]
    # Upload-cache key.  None (the default): a forward uploads the weights on
    # every call, as the reference re-stages them on every call
    # (layer.rs:4670-4705), so in-place changes are always seen.  An int:
    # the context keeps the upload while (object, version) is unchanged, and
    # every in-place write must be followed by bump().
    version: int | None = field(default=None)

    @staticmethod
    def random(cfg: ModelConfig) -> "ModelWeights":
        """full_model.rs:132-141 (embed scale 0.005, gammas 1).  Same-size
        tensors are identical in the reference (seed = 42 + n), so layers share
        arrays here too."""
        lw = LayerWeights.random(cfg)
        return ModelWeights(random_vec(cfg.vocab * cfg.dim, 0.005).reshape(cfg.vocab, cfg.dim),
                            [lw] * cfg.nlayers, np.ones(cfg.dim, np.float32))

    @staticmethod
    def normal(cfg: ModelConfig, seed: int, std: float = 0.02, fp16_round: bool = True):
        """Every matrix N(0, std^2) from numpy's PCG64(seed), gammas 1; rounded
        through fp16 so the device copy and a CPU check see identical values."""
        rng = np.random.default_rng(seed)

        def mat(*shape):
            a = rng.standard_normal(shape, dtype=np.float32) * np.float32(std)
            return a.astype(np.float16).astype(np.float32) if fp16_round else a

        D, F = cfg.dim, cfg.hidden
        layers = [LayerWeights(mat(D, cfg.q_dim), mat(D, cfg.kv_dim), mat(D, cfg.kv_dim),
                               mat(cfg.q_dim, D), mat(D, F), mat(D, F), mat(D, F),
                               np.ones(D, np.float32), np.ones(D, np.float32))
                  for _ in range(cfg.nlayers)]
        return ModelWeights(mat(cfg.vocab, D), layers, np.ones(D, np.float32))

    def bump(self):
        """Marks the weights as changed and opts into upload caching (the
        reference's w2_generation idea, training.rs:121)."""
        self.version = 1 if self.version is None else self.version + 1


# --------------------------------------------------------------------------- kernels
class CompiledKernels:
    """CompiledKernels::compile (layer.rs:843-969) -> a GPU context.  Holds the
    device-resident fp16 copy of the last ModelWeights passed to a forward."""

    def __init__(self, cfg: ModelConfig, device: int = 0, max_batch: int = 1, max_ctx: int = 0,
                 softcap: float = 0.0):
        self.cfg = cfg
        self.ctx = hb.Context(cfg.to_rh(softcap), device, max_batch, max_ctx)
        self._softcap = softcap
        self._loaded = None

    @staticmethod
    def compile(cfg: ModelConfig, **kw) -> "CompiledKernels":
        return CompiledKernels(cfg, **kw)

    compile_forward_only = compile
    try_compile = compile

    def ensure_weights(self, weights: ModelWeights):
        """Uploads the weights unless they carry a version and that
        (object, version) is the one uploaded last."""
        key = None if weights.version is None else (id(weights), weights.version)
        if key is None or self._loaded != key:
            self.ctx.load_weights(weights.embed, weights.gamma_final,
                                  [lw.tensors() for lw in weights.layers])
            self._loaded = key

    def ensure_softcap(self, softcap: float):
        if softcap != self._softcap:
            self.ctx.set_softcap(softcap)
            self._softcap = softcap

    def close(self):
        self.ctx.close()


@dataclass
class ForwardResult:
    """full_model.rs:121-129 (the backward-only fields are not produced)."""
    loss: float
    logits: np.ndarray  # [SEQ, VOCAB] (post-softcap)


class ModelForwardWorkspace:
    """full_model.rs:206-264.  Device workspaces live in the context; this
    keeps the host-side outputs of the last call."""

    def __init__(self, cfg: ModelConfig):
        self.cfg = cfg
        self.logits = None

    @staticmethod
    def new(cfg):
        return ModelForwardWorkspace(cfg)

    new_lean = new


def _check(cfg: ModelConfig, tokens, targets):
    tokens = np.asarray(tokens, np.uint32)
    if tokens.shape != (cfg.seq,):
        raise ValueError(f"tokens must be [{cfg.seq}], got {tokens.shape}")
    if targets is not None:
        targets = np.asarray(targets, np.uint32)
        if targets.shape != (cfg.seq,):
            raise ValueError(f"targets must be [{cfg.seq}], got {targets.shape}")
    return tokens, targets


def forward(cfg, kernels: CompiledKernels, weights: ModelWeights, tokens, targets,
            softcap: float = 0.0) -> ForwardResult:
    tokens, targets = _check(cfg, tokens, targets)
    kernels.ensure_weights(weights)
    kernels.ensure_softcap(softcap)
    out = kernels.ctx.forward(tokens, targets, want_logits=True, want_token_losses=False)
    return ForwardResult(float(out.mean_loss[0]), out.logits[0])


def forward_ws(cfg, kernels: CompiledKernels, weights: ModelWeights, tokens, targets,
               softcap: float, ws: ModelForwardWorkspace) -> float:
    tokens, targets = _check(cfg, tokens, targets)
    kernels.ensure_weights(weights)
    kernels.ensure_softcap(softcap)
    out = kernels.ctx.forward(tokens, targets, want_logits=True, want_token_losses=False)
    ws.logits = out.logits[0]
    return float(out.mean_loss[0])


def forward_only_ws(cfg, kernels: CompiledKernels, weights: ModelWeights, tokens, targets,
                    softcap: float, ws: ModelForwardWorkspace) -> float:
    tokens, targets = _check(cfg, tokens, targets)
    kernels.ensure_weights(weights)
    kernels.ensure_softcap(softcap)
    out = kernels.ctx.forward(tokens, targets, want_logits=False, want_token_losses=False)
    return float(out.mean_loss[0])


def forward_losses(cfg, kernels: CompiledKernels, weights: ModelWeights, tokens, targets,
                   softcap: float = 0.0) -> np.ndarray:
    tokens, targets = _check(cfg, tokens, targets)
    kernels.ensure_weights(weights)
    kernels.ensure_softcap(softcap)
    out = kernels.ctx.forward(tokens, targets, want_logits=False, want_token_losses=True)
    return out.token_losses[0]


# --------------------------------------------------------------------------- work model
def prefill_flops(cfg: ModelConfig, seq: int | None = None, batch: int = 1) -> dict:
    """Algorithmic FLOPs per forward: GEMM 2*S*L*(4D^2 + 3DF), causal attention
    2*D*S*(S+1)*L, logits 2*S*D*V (elementwise work excluded)."""
    S = seq or cfg.seq
    D, F, L, V = cfg.dim, cfg.hidden, cfg.nlayers, cfg.vocab
    gemm = 2 * S * L * (4 * D * D + 3 * D * F)
    attn = 2 * D * S * (S + 1) * L
    logits = 2 * S * D * V
    per = {"gemm": gemm, "attn": attn, "logits": logits, "total": gemm + attn + logits,
           "w13": 2 * S * L * 2 * D * F, "w13_per_launch": 2 * S * 2 * D * F}
    return {k: v * batch for k, v in per.items()}


def train_step_flops(cfg: ModelConfig, seq: int | None = None, batch: int = 1) -> int:
    """Algorithmic FLOPs of one forward + backward: every forward product is
    matched by a data-gradient and a weight-gradient product of the same size
    (GEMMs and the tied logits), and attention's backward is dQ, dK, dV, dP
    (twice the forward's QK^T and PV), so 3x the forward's count."""
    return 3 * prefill_flops(cfg, seq, batch)["total"]


def decode_bytes(cfg: ModelConfig, ctx_len: float, batch: int = 1) -> dict:
    """Compulsory HBM bytes of one decode step: fp16 weights (layers + tied
    vocab projection) + per sequence K/V read at ctx_len and the K/V append."""
    D, F, L, V = cfg.dim, cfg.hidden, cfg.nlayers, cfg.vocab
    weights = 2 * (L * (4 * D * D + 3 * D * F) + V * D)
    kv = batch * (2 * L * ctx_len * D * 2 + 2 * L * D * 2)
    return {"weights": weights, "kv": kv, "total": weights + kv}
