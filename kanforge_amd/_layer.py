"""Parameter layout and initialisation shared by the layers
(kanforge/_layer.py:18-83): groups, per-input buffers, init std schemes."""

from __future__ import annotations

import math

import numpy as np

COEF_INITS = ("normal", "zero", "variance", "lecun", "glorot")


def resolve_groups(in_features: int, groups: int | None) -> int:
    """Number of parameter groups: ``None`` means one group per input."""
    if groups is None:
        return in_features
    if groups < 1 or in_features % groups:
        raise ValueError(f"groups={groups} must divide in_features={in_features}")
    return groups


def basis_param_values(basis, groups: int, in_features: int, grid_ranges=None):
    """Initial basis state: trainable ``(groups, *shape)`` and buffers ``(in, *shape)``."""
    trainable, buffers = {}, {}
    for name, spec in basis.param_specs().items():
        if spec.trainable:
            trainable[name] = np.broadcast_to(spec.value, (groups, *spec.shape)).copy()
            continue
        value = np.broadcast_to(spec.value, (in_features, *spec.shape)).astype(np.float64)
        if grid_ranges is not None and name in basis.grid_names():
            r = np.broadcast_to(np.asarray(grid_ranges, dtype=np.float64), (in_features, 2))
            value = r[:, :1] + (r[:, 1:] - r[:, :1]) * np.linspace(0, 1, spec.shape[-1])
        buffers[name] = value.copy()
    return trainable, buffers


def _gauss_hermite(points: int = 96):
    x, w = np.polynomial.hermite_e.hermegauss(points)
    return x, w / math.sqrt(2 * math.pi)


def basis_second_moment(basis) -> float:
    """E[sum_k B_k(x)^2] for x ~ N(0, 1) with default parameters."""
    x, w = _gauss_hermite()
    return float(w @ (basis.host_values(x) ** 2).sum(-1))


def _silu(x):
    return x / (1.0 + np.exp(-x))


SILU_SECOND_MOMENT = float(_gauss_hermite()[1] @ _silu(_gauss_hermite()[0]) ** 2)


def init_stds(basis, in_features, out_features, coef_init, coef_init_std, has_base):
    """(coef std, base weight std or None for torch's kaiming-uniform default)."""
    if coef_init not in COEF_INITS:
        raise ValueError(f"coef_init must be one of {COEF_INITS}")
    if coef_init == "normal":
        return coef_init_std / math.sqrt(in_features), None
    if coef_init == "zero":
        return 0.0, None
    m2 = max(basis_second_moment(basis), 1e-12)
    if coef_init == "variance":
        return 1.0 / math.sqrt(in_features * m2), None
    fan = in_features if coef_init == "lecun" else (in_features + out_features) / 2
    share = 0.5 if has_base else 1.0
    return math.sqrt(share / (fan * m2)), math.sqrt(share / (fan * SILU_SECOND_MOMENT)) if has_base else None
