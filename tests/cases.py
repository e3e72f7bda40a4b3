"""Shared test cases: the same seeded inputs for the HIP path and the oracle."""

from __future__ import annotations

import numpy as np
import torch

import kanforge_amd as kf
from kanforge_amd.bases.spline import extend_grid as host_extend_grid
from kanforge_amd.kernels import plan_for
from oracle import kan64 as o

BASES = {
    "chebyshev8": kf.Chebyshev(8),
    "chebyshev5": kf.Chebyshev(5),
    "legendre_identity": kf.Legendre(4, input_map="identity"),
    "jacobi6": kf.Jacobi(6, 0.5, 0.5),
    "jacobi_ab": kf.Jacobi(4, 0.5, 1.5),
    "gram": kf.Gram(4),
    "taylor": kf.Taylor(3),
    "bspline53": kf.BSpline(5, 3),
    "bspline83": kf.BSpline(8, 3),
    "bspline41": kf.BSpline(4, 1),
    "bspline20": kf.BSpline(2, 0),
    "rational": kf.Rational(5, 4, "gelu"),
}

FAMILY_KW = {
    "chebyshev": ("chebyshev", {}),
    "legendre": ("legendre", {}),
    "jacobi": ("jacobi", None),
    "gram": None,
    "taylor": ("taylor", {}),
}


def random_grid(n_in, n_points, rng, lo=-1.0, hi=1.0):
    """Strictly increasing non-uniform grids (n_in, n_points)."""
    inc = rng.uniform(0.5, 1.5, size=(n_in, n_points - 1))
    g = np.concatenate([np.zeros((n_in, 1)), np.cumsum(inc, 1)], 1)
    return lo + (hi - lo) * g / g[:, -1:]


def oracle_basis(basis, n_in, params=None):
    """The oracle's view (Basis64) of a host basis with per-input params."""
    plan = plan_for(basis)
    if plan.kind == "cheb":
        return o.Basis64("poly", A=np.asarray(basis._cheb, np.float64), input_map=basis.input_map)
    if plan.kind == "bspline":
        grid = np.broadcast_to(np.linspace(*basis.grid_range, basis.grid_size + 1), (n_in, basis.grid_size + 1))
        if params is not None and "grid" in params:
            grid = np.asarray(params["grid"], np.float64)
        return o.Basis64("bspline", grid=grid, k=basis.order)
    num = np.asarray(params["num"], np.float64)
    den = np.asarray(params["den"], np.float64)
    rep = n_in // num.shape[0]  # groups of inputs share one parameter row
    return o.Basis64("rational", num=np.repeat(num, rep, 0), den=np.repeat(den, rep, 0))


def to_dev(a, dtype, device="cuda"):
    return torch.as_tensor(np.asarray(a, dtype=np.float32)).to(device=device, dtype=dtype)


def rounded(a, dtype):
    """float64 copy of what the device sees after casting to dtype."""
    a = np.asarray(a, dtype=np.float64)
    if dtype == torch.bfloat16:
        return o.round_bf16(a)
    return a.astype(np.float32).astype(np.float64)
