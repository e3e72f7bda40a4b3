"""Bases on the HIP path: B-splines, the Chebyshev-reducible polynomial
families (tanh or identity input map) and the group rational of GR-KAN."""

from .base import BASES, Basis, ParamSpec, make_basis
from .polynomial import (
    Bernstein,
    Chebyshev,
    Chebyshev2,
    Gegenbauer,
    Gram,
    Hermite,
    Jacobi,
    Laguerre,
    Legendre,
    PolynomialBasis,
    Taylor,
)
from .rational import Rational, fit_rational
from .spline import BSpline, extend_grid

__all__ = [
    "BASES",
    "BSpline",
    "Basis",
    "Bernstein",
    "Chebyshev",
    "Chebyshev2",
    "Gegenbauer",
    "Gram",
    "Hermite",
    "Jacobi",
    "Laguerre",
    "Legendre",
    "ParamSpec",
    "PolynomialBasis",
    "Rational",
    "Taylor",
    "extend_grid",
    "fit_rational",
    "make_basis",
]
