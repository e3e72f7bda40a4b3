"""Grid tools of the KAN layers, host-side NumPy float64 (kanforge/grid.py:1-84).

* ``adaptive_grid``: per-input grids from samples, quantiles blended with a
  uniform grid over the samples' range (weight ``grid_eps`` on the uniform
  part, which keeps every grid strictly increasing).
* ``refit``: coefficients of a new basis (or grid) that reproduce the old
  edge functions at sample points, by least squares per input. Grid update,
  grid refinement and conversion between bases are all this one operation.

They run off the hot path (once per grid change); the layers' device tables
(B-spline knots) are rebuilt on the next call because they are keyed on the
grid tensor's version.
"""

from __future__ import annotations

import numpy as np


def adaptive_grid(x: np.ndarray, n_points: int, margin: float = 0.0, grid_eps: float = 0.02) -> np.ndarray:
    """Grids ``(in, n_points)`` from samples ``x`` ``(N, in)`` (kanforge/grid.py:19-32).

    Point j of input i is ``grid_eps * u_j + (1 - grid_eps) * q_j``: ``u`` uniform over
    ``[min - margin, max + margin]``, ``q`` the sample of rank ``round(j (N - 1) / (n - 1))``.
    An input whose samples span less than 1e-8 gets the uniform grid over +-0.5 around them.
    """
    if not 0 < grid_eps <= 1:
        raise ValueError("grid_eps must be in (0, 1]: the uniform part keeps the grid increasing")
    xs = np.sort(np.asarray(x, dtype=np.float64), axis=0)
    ranks = np.rint(np.linspace(0, len(xs) - 1, n_points)).astype(int)
    quant = xs[ranks].T  # (in, n)
    lo, hi = xs[0] - margin, xs[-1] + margin
    flat = hi - lo < 1e-8
    lo = np.where(flat, lo - 0.5, lo)
    hi = np.where(flat, hi + 0.5, hi)
    uniform = lo[:, None] + (hi - lo)[:, None] * np.linspace(0.0, 1.0, n_points)
    quant = np.where(flat[:, None], uniform, quant)
    return grid_eps * uniform + (1.0 - grid_eps) * quant


def resample_grid(grid: np.ndarray, n_points: int) -> np.ndarray:
    """Grids ``(in, n)`` linearly interpolated to ``n_points`` points (kanforge/grid.py:35-39)."""
    grid = np.asarray(grid, dtype=np.float64)
    src = np.linspace(0.0, 1.0, grid.shape[-1])
    dst = np.linspace(0.0, 1.0, n_points)
    return np.stack([np.interp(dst, src, row) for row in grid])


def grid_ranges(basis, params: dict) -> np.ndarray | None:
    """``(in, 2)`` first and last point of the basis grid, or None for grid-free bases."""
    names = basis.grid_names()
    if not names:
        return None
    g = np.asarray(params[names[0]], dtype=np.float64)
    return np.stack([g[..., 0], g[..., -1]], axis=-1)


def sample_inputs(ranges: np.ndarray, n: int) -> np.ndarray:
    """``(n, in)`` evenly spaced points spanning each input's range."""
    t = np.linspace(0.0, 1.0, n)[:, None]
    return ranges[:, 0] + t * (ranges[:, 1] - ranges[:, 0])


def refit(old_basis, old_params: dict, old_coef: np.ndarray, new_basis, new_params: dict, x: np.ndarray,
          ridge: float = 0.0) -> np.ndarray:
    """Coefficients ``(out, in, new_basis.size)`` whose edge functions match the old ones at
    ``x`` ``(N, in)`` in the least-squares sense, input by input (kanforge/grid.py:56-84).

    Params are per input (trainable group parameters already repeated). Minimum-norm
    solutions (``lstsq``) where a new basis function has no samples; ``ridge`` > 0 adds
    Tikhonov damping scaled by the mean squared basis value. A new basis that spans the old
    edge functions reproduces them to rounding error.
    """
    x = np.asarray(x, dtype=np.float64)
    phi_old = old_basis.host_values(x, old_params)        # (N, in, n)
    target = np.einsum("Nin,oin->iNo", phi_old, np.asarray(old_coef, dtype=np.float64))
    phi_new = np.moveaxis(new_basis.host_values(x, new_params), 1, 0)  # (in, N, n')
    out = []
    for a, y in zip(phi_new, target):
        if ridge:
            lam = np.sqrt(ridge * np.mean(a * a) * len(a))
            a = np.concatenate([a, lam * np.eye(a.shape[1])])
            y = np.concatenate([y, np.zeros((a.shape[1], y.shape[1]))])
        out.append(np.linalg.lstsq(a, y, rcond=None)[0])  # (n', out)
    return np.moveaxis(np.stack(out), 2, 0)  # (out, in, n')
