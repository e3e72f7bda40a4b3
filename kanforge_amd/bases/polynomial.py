"""Polynomial bases evaluated through Chebyshev features.

Every family is a matrix A of Chebyshev coefficients (family(z) =
[T_0(z)..T_D(z)] @ A, interpolated at Chebyshev nodes as in
kanforge/bases/polynomial.py:51-56) of z = tanh(x) or z = x. The kernels only
ever evaluate T_j(z); A and the derivative chain rule are folded into the
coefficients (kanforge/kernels/plan.py:88-101).
"""

from __future__ import annotations

import math
from functools import cached_property
from typing import Any

import numpy as np
from numpy.polynomial import chebyshev as C
from numpy.polynomial import hermite as H
from numpy.polynomial import laguerre as La
from numpy.polynomial import legendre as Le

from .base import Basis

INPUT_MAPS = ("tanh", "identity")


class PolynomialBasis(Basis):
    default_input_map = "tanh"

    def __init__(self, degree: int = 5, input_map: str | None = None):
        if degree < 0:
            raise ValueError("degree must be >= 0")
        input_map = input_map or self.default_input_map
        if input_map not in INPUT_MAPS:
            raise ValueError(f"input_map must be one of {INPUT_MAPS} on the HIP path")
        self.degree = int(degree)
        self.input_map = input_map

    @property
    def size(self) -> int:
        return self.degree + 1

    def _family(self, z: np.ndarray) -> np.ndarray:
        raise NotImplementedError

    @cached_property
    def _cheb(self) -> np.ndarray:
        """Chebyshev coefficients of every basis polynomial, ``(D+1, size)``."""
        d = self.degree
        nodes = np.cos(np.pi * (np.arange(d + 1) + 0.5) / (d + 1))
        return np.linalg.solve(C.chebvander(nodes, d), self._family(nodes))

    def host_values(self, x, params=None):
        x = np.asarray(x, dtype=np.float64)
        z = np.tanh(x) if self.input_map == "tanh" else x
        return C.chebvander(z, self.degree) @ self._cheb

    def config(self) -> dict[str, Any]:
        return {"name": self.name, "degree": self.degree, "input_map": self.input_map}


class Chebyshev(PolynomialBasis):
    """T_n(tanh x), as in ChebyKAN."""

    name = "chebyshev"

    def _family(self, z):
        return C.chebvander(z, self.degree)

    @cached_property
    def _cheb(self) -> np.ndarray:
        return np.eye(self.degree + 1)


class Chebyshev2(PolynomialBasis):
    name = "chebyshev2"

    def _family(self, z):
        u = [np.ones_like(z), 2 * z]
        for _ in range(2, self.degree + 1):
            u.append(2 * z * u[-1] - u[-2])
        return np.stack(u[: self.degree + 1], -1)


class Legendre(PolynomialBasis):
    name = "legendre"

    def _family(self, z):
        return Le.legvander(z, self.degree)


class Jacobi(PolynomialBasis):
    """P_n^(alpha, beta), as in JacobiKAN."""

    name = "jacobi"

    def __init__(self, degree: int = 5, alpha: float = 1.0, beta: float = 1.0, input_map: str | None = None):
        if alpha <= -1 or beta <= -1:
            raise ValueError("alpha and beta must be > -1")
        super().__init__(degree, input_map)
        self.alpha, self.beta = float(alpha), float(beta)

    def _family(self, z):
        a, b = self.alpha, self.beta
        out = [np.ones_like(z), (a + 1) + (a + b + 2) * (z - 1) / 2]
        for n in range(2, self.degree + 1):
            c = 2 * n + a + b
            num = (c - 1) * (c * (c - 2) * z + a * a - b * b) * out[-1] - 2 * (n + a - 1) * (n + b - 1) * c * out[-2]
            out.append(num / (2 * n * (n + a + b) * (c - 2)))
        return np.stack(out[: self.degree + 1], -1)

    def config(self):
        return {**super().config(), "alpha": self.alpha, "beta": self.beta}


class Gegenbauer(PolynomialBasis):
    name = "gegenbauer"

    def __init__(self, degree: int = 5, lam: float = 1.0, input_map: str | None = None):
        if lam <= -0.5 or lam == 0:
            raise ValueError("lam must be > -1/2 and non-zero")
        super().__init__(degree, input_map)
        self.lam = float(lam)

    def _family(self, z):
        lam = self.lam
        out = [np.ones_like(z), 2 * lam * z]
        for n in range(2, self.degree + 1):
            out.append((2 * z * (n + lam - 1) * out[-1] - (n + 2 * lam - 2) * out[-2]) / n)
        return np.stack(out[: self.degree + 1], -1)

    def config(self):
        return {**super().config(), "lam": self.lam}


class Hermite(PolynomialBasis):
    name = "hermite"

    def _family(self, z):
        return H.hermvander(z, self.degree)


class Laguerre(PolynomialBasis):
    name = "laguerre"

    def _family(self, z):
        return La.lagvander(z, self.degree)


class Bernstein(PolynomialBasis):
    name = "bernstein"

    def _family(self, z):
        t, n = (z + 1) / 2, self.degree
        return np.stack([math.comb(n, j) * t**j * (1 - t) ** (n - j) for j in range(n + 1)], -1)


class Gram(PolynomialBasis):
    """Orthonormal on ``points`` equally spaced points of [-1, 1]."""

    name = "gram"

    def __init__(self, degree: int = 5, points: int | None = None, input_map: str | None = None):
        super().__init__(degree, input_map)
        self.points = int(points) if points is not None else 2 * (self.degree + 1)
        if self.points <= self.degree:
            raise ValueError("points must be > degree")

    @cached_property
    def _cheb(self):
        grid = np.linspace(-1, 1, self.points)
        _, r = np.linalg.qr(C.chebvander(grid, self.degree))
        sign = np.sign(np.diag(r))
        return np.linalg.inv(r) * sign * math.sqrt(self.points)

    def config(self):
        return {**super().config(), "points": self.points}


class Taylor(PolynomialBasis):
    """Monomials 1, x, ..., x^degree; identity input map by default."""

    name = "taylor"
    default_input_map = "identity"

    def _family(self, z):
        return np.stack([z**j for j in range(self.degree + 1)], -1)
