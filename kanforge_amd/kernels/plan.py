"""What the HIP kernels compute for a basis (kanforge/kernels/plan.py:39-121).

A ``KernelPlan`` names the per-input *kernel features* the device evaluates
and how derivatives are obtained:

* ``cheb``: features T_j(z), z = tanh(x) or x. The m-th x-derivative of every
  basis function is a fixed combination of them,
  phi_k^(m) = sum_j R_m[k, j] T_j(z) (``fold``), applied to the coefficients
  (and to coefficient gradients), so the kernels never differentiate.
  Every polynomial family with a tanh or identity map reduces to this.
* ``bspline``: features are the B-splines themselves; the derivative order
  is native to the kernel (Cox-de Boor to degree k - m, then m derivative
  steps).
* ``rational``: P/(1+|Q|) with trainable P, Q shared by groups of inputs;
  native derivative order (quotient rule). The reference sends this basis to
  plain ops only (plan.py:107-108); here it has a plan.
"""

from __future__ import annotations

from dataclasses import dataclass
from functools import lru_cache

import numpy as np
from numpy.polynomial import chebyshev as C

from ..bases import BSpline, PolynomialBasis, Rational

ONE_MINUS_Z2 = np.array([0.5, 0.0, -0.5])  # 1 - z^2 in the Chebyshev basis

# Plan kinds that backend="auto" sends to the HIP kernels, per torch device
# type. On ROCm torch reports "cuda"; every plan kind has a kernel.
AUTO_KINDS = {"cuda": ("cheb", "bspline", "rational")}

MAX_ORDER = 8  # largest derivative order of the kernel features
MAX_BASIS = 16  # basis functions per edge the kernels hold (KF_MAX_K)


@dataclass(frozen=True)
class KernelPlan:
    kind: str  # "cheb" | "bspline" | "rational"
    consts: tuple  # cheb: (degree, input_map); bspline: (grid_size, order); rational: (num_degree, den_degree)
    size: int
    fold_key: tuple = ()  # cheb: flattened Chebyshev coefficient matrix A
    grid: bool = False  # reads the per-input grid buffer

    @property
    def folded(self) -> bool:
        return self.kind == "cheb"

    def n_features(self, m: int) -> int:
        """Kernel features evaluated for derivative order m."""
        if self.kind == "cheb":
            d, input_map = self.consts
            return d + 1 + m if input_map == "tanh" else d + 1
        return self.size

    def native_order(self, m: int) -> int:
        return 0 if self.folded else m

    def fold(self, m: int) -> np.ndarray | None:
        """R_m ``(size, n_features(m))`` for folded plans, None otherwise."""
        if not self.folded:
            return None
        return _fold(self.consts, self.fold_key, m)

    def device_fold(self, m: int) -> tuple[np.ndarray, bool]:
        """The fold the HIP kernels evaluate for order m, and whether their features carry the
        factor (1 - z^2).

        For a tanh map and m >= 1 every row of R_m is (1 - z^2) times a polynomial of degree
        deg + m - 2 (d/dx = (1 - z^2) d/dz), so the kernels use R_m with that factor divided out
        and weight each element's features by (1 - z^2): two Chebyshev features fewer per edge,
        the same values."""
        d, input_map = self.consts
        if input_map != "tanh" or m == 0:
            return self.fold(m), False
        return _reduced_fold(self.consts, self.fold_key, m), True


@lru_cache(maxsize=None)
def _fold(consts, fold_key, m):
    d, input_map = consts
    a = np.asarray(fold_key, dtype=np.float64).reshape(d + 1, -1)
    n_t = d + 1 + m if input_map == "tanh" else d + 1
    cols = []
    for k in range(a.shape[1]):
        col = a[:, k]
        for _ in range(m):
            col = C.chebder(col) if len(col) > 1 else np.zeros(1)
            if input_map == "tanh":
                col = C.chebmul(col, ONE_MINUS_Z2)  # d/dx f(tanh x) = f'(z) (1 - z^2)
        out = np.zeros(n_t)
        out[: min(len(col), n_t)] = col[:n_t]
        cols.append(out)
    r = np.stack(cols)
    r.setflags(write=False)
    return r


@lru_cache(maxsize=None)
def _reduced_fold(consts, fold_key, m):
    d, _ = consts
    r = _fold(consts, fold_key, m)
    n_t = max(1, d + m - 1)
    rows = []
    for row in r:
        q, rem = C.chebdiv(row, ONE_MINUS_Z2)
        scale = max(1.0, float(np.abs(row).max()))
        if np.abs(rem).max() > 1e-9 * scale:  # exact division for tanh maps and m >= 1
            raise AssertionError("fold row is not divisible by (1 - z^2)")
        out = np.zeros(n_t)
        out[: min(len(q), n_t)] = q[:n_t]
        rows.append(out)
    out = np.stack(rows)
    out.setflags(write=False)
    return out


def plan_for(basis) -> KernelPlan | None:
    """The kernel plan of ``basis``, or None when the HIP path has no kernel for it."""
    if isinstance(basis, PolynomialBasis) and basis.input_map in ("tanh", "identity"):
        a = basis._cheb
        return KernelPlan("cheb", (basis.degree, basis.input_map), basis.size, tuple(a.ravel().tolist()))
    if type(basis) is BSpline:
        return KernelPlan("bspline", (basis.grid_size, basis.order), basis.size, grid=True)
    if type(basis) is Rational:
        return KernelPlan("rational", (basis.num_degree, basis.den_degree), 1)
    return None
