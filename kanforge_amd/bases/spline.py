"""B-spline basis on a per-input grid (kanforge/bases/spline.py:22-92 semantics).

The grid buffer ``(in, G+1)`` is extended by ``order`` knots on each side with
the mean grid step (pykan). The HIP kernels read two float32 knot tables
built here in float64:

* comparison table: every knot rounded toward +inf, so that for a float32
  x, ``x >= t`` in float64 holds exactly when ``x >= ceil32(t)``; the
  half-open interval search ``t_j <= x < t_{j+1}`` of the reference
  (spline.py:80) is therefore reproduced bit for bit;
* arithmetic table: knots rounded to nearest, padded with ``order`` extra
  strictly increasing knots per side so the local de Boor recurrence never
  leaves the table.
"""

from __future__ import annotations

from typing import Any

import numpy as np

from .base import Basis, ParamSpec, _check_range


def extend_grid(grid, k: int):
    """Add ``k`` points on each side of ``grid`` (``(..., G+1)``) with the mean step."""
    grid = np.asarray(grid, dtype=np.float64)
    if k == 0:
        return grid.copy()
    h = (grid[..., -1:] - grid[..., :1]) / (grid.shape[-1] - 1)
    i = np.arange(k, dtype=np.float64)
    left = grid[..., :1] - h * (k - i)
    right = grid[..., -1:] + h * (i + 1)
    return np.concatenate([left, grid, right], -1)


def ceil_f32(t: np.ndarray) -> np.ndarray:
    """Smallest float32 >= t (elementwise, t float64)."""
    t = np.asarray(t, dtype=np.float64)
    f = t.astype(np.float32)
    low = f.astype(np.float64) < t
    f[low] = np.nextafter(f[low], np.float32(np.inf))
    return f


def uniform_table(grid, k: int, rtol: float = 1e-7) -> np.ndarray | None:
    """``(in, 2)`` float32 ``(t_0, 1/h)`` of the extended knots when every input's knots are evenly
    spaced by its own h (relative tolerance ``rtol``), else None. The kernels use it to locate a
    point's interval in constant time; the interval itself is still decided by the comparison
    table, and the values by the knots being even."""
    t = extend_grid(np.atleast_2d(np.asarray(grid, dtype=np.float64)), k)
    if t.shape[1] < 2:
        return None
    d = np.diff(t, axis=1)
    h = (t[:, -1] - t[:, 0]) / (t.shape[1] - 1)
    if not (h > 0).all() or not (np.abs(d - h[:, None]) <= rtol * h[:, None]).all():
        return None
    return np.ascontiguousarray(np.stack([t[:, 0], 1.0 / h], 1).astype(np.float32))


def knot_tables(grid, k: int) -> tuple[np.ndarray, np.ndarray]:
    """(arithmetic table (in, nk + 2k), comparison table (in, nk)), float32."""
    t = extend_grid(np.atleast_2d(np.asarray(grid, dtype=np.float64)), k)
    cmp_ = ceil_f32(t)
    if k:
        hl = t[:, 1:2] - t[:, :1]
        hr = t[:, -1:] - t[:, -2:-1]
        r = np.arange(1, k + 1, dtype=np.float64)
        left = t[:, :1] - hl * r[::-1]
        right = t[:, -1:] + hr * r
        pad = np.concatenate([left, t, right], 1)
    else:
        pad = t
    return np.ascontiguousarray(pad.astype(np.float32)), np.ascontiguousarray(cmp_)


class _Gridded(Basis):
    def __init__(self, grid_size: int = 5, order: int = 3, grid_range: tuple[float, float] = (-1.0, 1.0)):
        if grid_size < 1 or order < 0:
            raise ValueError("grid_size must be >= 1 and order >= 0")
        self.grid_size = int(grid_size)
        self.order = int(order)
        self.grid_range = _check_range(grid_range)

    @property
    def size(self) -> int:
        return self.grid_size + self.order

    @property
    def support(self) -> int:
        return self.order + 1

    def param_specs(self):
        return {"grid": ParamSpec(np.linspace(*self.grid_range, self.grid_size + 1), trainable=False)}

    def knots(self, p=None):
        grid = np.linspace(*self.grid_range, self.grid_size + 1) if p is None else np.asarray(p["grid"], np.float64)
        return extend_grid(grid, self.order)

    def config(self) -> dict[str, Any]:
        return {"name": self.name, "grid_size": self.grid_size, "order": self.order, "grid_range": self.grid_range}


class BSpline(_Gridded):
    """B-splines of ``order`` on ``grid_size`` intervals: ``grid_size + order``
    functions, zero outside the extended grid (kanforge/bases/spline.py:95-128)."""

    name = "bspline"
    local = True

    def host_values(self, x, params=None):
        x = np.asarray(x, dtype=np.float64)[..., None]
        t = self.knots(params)
        k = self.order
        b = ((x >= t[..., :-1]) & (x < t[..., 1:])).astype(np.float64)
        for q in range(1, k + 1):
            left = (x - t[..., : -(q + 1)]) / (t[..., q:-1] - t[..., : -(q + 1)])
            right = (t[..., q + 1 :] - x) / (t[..., q + 1 :] - t[..., 1:-q])
            b = left * b[..., :-1] + right * b[..., 1:]
        return b
