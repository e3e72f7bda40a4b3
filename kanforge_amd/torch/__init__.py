"""PyTorch-ROCm layers whose spline part runs on the HIP kernels."""

from .layers import GRKAN, KAN, KANLinear, layer_inputs, rebuild_kan
from .science import derivative, gradient, laplacian

__all__ = ["GRKAN", "KAN", "KANLinear", "derivative", "gradient", "laplacian", "layer_inputs", "rebuild_kan"]
