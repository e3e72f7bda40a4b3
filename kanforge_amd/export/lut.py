"""Lookup-table form of KAN models, evaluated on the GPU (kanforge/export/lut.py).

Every edge phi_oi of a layer is tabulated at ``size`` uniform points over its input's range
[lo_i, hi_i]; a layer then computes, per row,

    t = (x_i - lo_i) / step_i,  j = clip(floor(t), 0, size - 2),  f = clip(t, 0, size - 1) - j
    y_o = b_o + sum_i T[i, j, o] + f (T[i, j+1, o] - T[i, j, o])

plus, with ``extrapolate="linear"``, each edge's end slope times how far t leaves [0, size - 1]
(``"clamp"`` holds the end values). ``quantize`` stores the tables as int8/int16 with one scale per
output and the per-edge centre folded into the bias. The tables are built with the layer's own
``edge_derivative(x, 0)`` (HIP kernels) and every layer is evaluated by ``kf_lut_forward``: one
lane per (row, output), gathers contiguous over outputs. Host arrays are NumPy, as in the
reference; device copies are made on first use and reused while the arrays are the same objects.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np
import torch
from torch import nn

from ..convert import activation_name, make_activation
from ..torch import _lib
from ..torch.layers import KANLinear


def end_slopes(tables: np.ndarray):
    """(slope_lo, slope_hi), each (in, out), per index step: the mean slope over the last 1/32 of
    each end of the float tables (kanforge/export/lut.py:131-135)."""
    size = tables.shape[1]
    k = max(1, (size - 1) // 32)
    t = np.asarray(tables, dtype=np.float64)
    return (t[:, k] - t[:, 0]) / k, (t[:, -1] - t[:, -1 - k]) / k


def input_ranges(layer: KANLinear, x=None, margin: float = 0.0) -> np.ndarray:
    """(in, 2) ranges: of the samples ``x`` when given, else the B-spline grid's ends, else
    [-1, 1]; widened by ``margin`` times the width (kanforge/interpret/analysis.py:24-35)."""
    if x is not None:
        xs = torch.as_tensor(x).detach().reshape(-1, layer.in_features).double()
        r = torch.stack([xs.min(0).values, xs.max(0).values], -1).cpu().numpy()
    elif getattr(layer, "basis_grid", None) is not None:
        g = layer.basis_grid.detach().double().cpu().numpy()
        r = np.stack([g[..., 0], g[..., -1]], -1).reshape(layer.in_features, 2)
    else:
        r = np.tile([-1.0, 1.0], (layer.in_features, 1))
    pad = margin * (r[:, 1] - r[:, 0])
    return np.stack([r[:, 0] - pad, r[:, 1] + pad], -1)


def _device_of(x, default="cuda"):
    return x.device if isinstance(x, torch.Tensor) else torch.device(default)


@dataclass
class LUTLayer:
    """Tables ``(in, size, out)`` over per-input ranges [lo, hi] (kanforge/export/lut.py:45-89)."""

    tables: np.ndarray
    lo: np.ndarray
    hi: np.ndarray
    bias: np.ndarray
    n_sum: int | None = None
    n_mult: int = 0
    arity: int = 2
    scale: np.ndarray | None = None
    bits: int | None = None
    slope_lo: np.ndarray | None = None
    slope_hi: np.ndarray | None = None
    _dev: tuple | None = field(default=None, repr=False, compare=False)

    kind = "kan"

    @property
    def size(self) -> int:
        return self.tables.shape[1]

    @property
    def step(self) -> np.ndarray:
        return (self.hi - self.lo) / (self.size - 1)

    def _device_arrays(self, device):
        key = (str(device), id(self.tables), id(self.lo), id(self.hi), id(self.bias), id(self.scale), id(self.slope_lo), id(self.slope_hi))
        if self._dev is None or self._dev[0] != key:
            def f32(a):
                return None if a is None else torch.as_tensor(np.ascontiguousarray(a, dtype=np.float32), device=device)

            tab = np.ascontiguousarray(self.tables)
            if tab.dtype not in (np.int8, np.int16):
                tab = tab.astype(np.float32)
            inv = (self.size - 1) / (np.asarray(self.hi, np.float64) - np.asarray(self.lo, np.float64))
            arrays = {
                "tables": torch.as_tensor(tab, device=device),
                "lo": f32(self.lo),
                "inv_step": f32(inv),
                "bias": f32(self.bias),
                "scale": f32(self.scale),
                "slope_lo": f32(self.slope_lo),
                "slope_hi": f32(self.slope_hi),
            }
            self._dev = (key, arrays)
        return self._dev[1]

    def __call__(self, x: torch.Tensor, extrapolate: str = "linear") -> torch.Tensor:
        """(B, out) float32 on x's device for x (B, in)."""
        if extrapolate not in ("linear", "clamp"):
            raise ValueError("extrapolate must be 'linear' or 'clamp'")
        n_in, size, n_out = self.tables.shape
        x2 = x.reshape(-1, n_in).to(torch.float32).contiguous()
        a = self._device_arrays(x2.device)
        codes = {torch.float32: _lib.KF_F32, torch.int8: _lib.KF_I8, torch.int16: _lib.KF_I16}
        if a["tables"].dtype not in codes:
            raise TypeError(f"tables must be float, int8 or int16, not {a['tables'].dtype}")
        linear = extrapolate == "linear" and a["slope_lo"] is not None
        y = torch.empty(x2.shape[0], n_out, dtype=torch.float32, device=x2.device)

        def ptr(t):
            return None if t is None else ctypes.c_void_p(t.data_ptr())

        with torch.cuda.device(x2.device):
            rc = _lib.load().kf_lut_forward(
                codes[a["tables"].dtype], x2.shape[0], n_in, size, n_out, ptr(x2), ptr(a["tables"]), ptr(a["lo"]),
                ptr(a["inv_step"]), ptr(a["bias"]), ptr(a["scale"]), ptr(a["slope_lo"] if linear else None),
                ptr(a["slope_hi"] if linear else None), ptr(y), ctypes.c_void_p(torch.cuda.current_stream(x2.device).cuda_stream),
            )
        _lib.check(rc, "kf_lut_forward")
        if self.n_mult:
            tail = y[:, self.n_sum :].reshape(-1, self.n_mult, self.arity).prod(-1)
            y = torch.cat([y[:, : self.n_sum], tail], -1)
        return y.reshape(*x.shape[:-1], y.shape[-1])


@dataclass
class DenseLayer:
    """A kept ``Linear``: weight (out, in), bias (out) or None."""

    weight: np.ndarray
    bias: np.ndarray | None
    kind = "linear"

    def __call__(self, x: torch.Tensor, extrapolate: str = "linear") -> torch.Tensor:
        w = torch.as_tensor(self.weight, dtype=torch.float32, device=x.device)
        b = None if self.bias is None else torch.as_tensor(self.bias, dtype=torch.float32, device=x.device)
        return torch.nn.functional.linear(x.to(torch.float32), w, b)


@dataclass
class ActivationLayer:
    """A kept activation, by portable name."""

    name: str
    kind = "activation"

    def __call__(self, x: torch.Tensor, extrapolate: str = "linear") -> torch.Tensor:
        return make_activation(self.name)(x.to(torch.float32))


@dataclass
class LUTModel:
    """The layers in order; called on a NumPy array it returns NumPy (float64), on a tensor a
    float32 tensor on that tensor's device."""

    layers: list = field(default_factory=list)
    extrapolate: str = "linear"

    def __call__(self, x):
        numpy_in = not isinstance(x, torch.Tensor)
        h = torch.as_tensor(np.asarray(x, dtype=np.float32), device=_device_of(x)) if numpy_in else x
        for layer in self.layers:
            h = layer(h, self.extrapolate)
        return h.double().cpu().numpy() if numpy_in else h

    @property
    def n_inputs(self) -> int:
        first = self.layers[0]
        return first.tables.shape[0] if first.kind == "kan" else first.weight.shape[1]

    def nbytes(self) -> int:
        return int(sum(layer.tables.nbytes for layer in self.layers if layer.kind == "kan"))


def _tables(layer: KANLinear, lo: np.ndarray, hi: np.ndarray, size: int) -> np.ndarray:
    """(in, size, out) float32 values of every edge at ``size`` uniform points of each range."""
    pts = lo + (hi - lo) * np.linspace(0.0, 1.0, size)[:, None]
    like = layer.coef
    with torch.no_grad():
        edges = layer.edge_derivative(torch.as_tensor(pts, dtype=like.dtype, device=like.device), 0)
    return np.ascontiguousarray(edges.float().cpu().numpy().transpose(2, 0, 1))


def to_lut(model, x=None, size: int = 256, margin: float = 0.05, extrapolate: str = "linear") -> LUTModel:
    """Tabulate a ``KANLinear`` or a sequence of layers (``KAN``, ``nn.Sequential``): ranges from
    the activations each KAN layer receives for the samples ``x`` (widened by ``margin``), else
    from the grids (kanforge/export/lut.py:144-172). ``Linear`` layers and activations are kept."""
    if size < 2:
        raise ValueError("size must be >= 2")
    children = [model] if isinstance(model, KANLinear) else list(model)
    out = LUTModel(extrapolate=extrapolate)
    h = x
    for m in children:
        if isinstance(m, KANLinear):
            if h is not None:
                h = torch.as_tensor(h).to(m.coef.device, m.coef.dtype)
            r = input_ranges(m, h, margin)
            bias = np.zeros(m.out_features) if m.bias is None else m.bias.detach().double().cpu().numpy()
            tables = _tables(m, r[:, 0], r[:, 1], size)
            s_lo, s_hi = end_slopes(tables)
            out.layers.append(LUTLayer(tables, r[:, 0], r[:, 1], bias, slope_lo=s_lo, slope_hi=s_hi))
        elif isinstance(m, nn.Linear):
            b = None if m.bias is None else m.bias.detach().double().cpu().numpy()
            out.layers.append(DenseLayer(m.weight.detach().double().cpu().numpy(), b))
        else:
            out.layers.append(ActivationLayer(activation_name(m)))
        if h is not None:
            with torch.no_grad():
                h = m(h)
    return out


def quantize(lut: LUTModel, bits: int = 8) -> LUTModel:
    """Integer tables: T[i, :, o] = centre[i, o] + scale[o] q[i, :, o] with |q| <= 2^(bits-1) - 1,
    the centres summed into the bias (kanforge/export/lut.py:175-197)."""
    if not 2 <= bits <= 16:
        raise ValueError("bits must be in [2, 16]")
    qmax = 2 ** (bits - 1) - 1
    layers = []
    for layer in lut.layers:
        if layer.kind != "kan":
            layers.append(layer)
            continue
        t = np.asarray(layer.tables, dtype=np.float64)
        centre = 0.5 * (t.max(1) + t.min(1))
        spread = np.abs(t - centre[:, None, :]).max((0, 1))
        scale = np.where(spread > 0, spread / qmax, 1.0)
        q = np.round((t - centre[:, None, :]) / scale).astype(np.int8 if bits <= 8 else np.int16)
        layers.append(
            LUTLayer(q, layer.lo, layer.hi, layer.bias + centre.sum(0), layer.n_sum, layer.n_mult, layer.arity,
                     scale=scale, bits=bits, slope_lo=layer.slope_lo, slope_hi=layer.slope_hi)
        )
    return LUTModel(layers, lut.extrapolate)
