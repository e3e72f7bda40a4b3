"""Deployable forms of KAN models (kanforge/export/__init__.py): lookup tables evaluated by the
HIP gather + lerp kernel."""

from .lut import ActivationLayer, DenseLayer, LUTLayer, LUTModel, end_slopes, input_ranges, quantize, to_lut

__all__ = ["ActivationLayer", "DenseLayer", "LUTLayer", "LUTModel", "end_slopes", "input_ranges", "quantize", "to_lut"]
