"""PyTorch-ROCm layers whose spline part runs on the HIP kernels."""

from .layers import GRKAN, KAN, KANLinear, from_mlp, layer_inputs, rebuild_kan
from .science import derivative, gradient, laplacian
from .transformer import KANFFN, KATBlock, kanify

__all__ = [
    "GRKAN",
    "KAN",
    "KANFFN",
    "KANLinear",
    "KATBlock",
    "derivative",
    "from_mlp",
    "gradient",
    "kanify",
    "laplacian",
    "layer_inputs",
    "rebuild_kan",
]
