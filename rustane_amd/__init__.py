"""rustane_amd -- MI355X (gfx950) forward token loop and greedy decode for
rustane's engine: hand-written HIP kernels behind a C-ABI
(include/rustane_hip.h, librustane_hip.so) and a Python mirror of the
reference engine API (rustane_amd.engine)."""
from . import hip_bridge  # noqa: F401
from .engine import (  # noqa: F401
    CompiledKernels, ForwardResult, LayerWeights, ModelConfig, ModelForwardWorkspace,
    ModelWeights, forward, forward_losses, forward_only_ws, forward_ws, random_vec)
