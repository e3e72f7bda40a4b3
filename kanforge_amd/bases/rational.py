"""Rational activation P(x) / (1 + |Q(x)|): the GR-KAN basis of KAT.

One trainable function per input (``size == 1``): numerator coefficients
a_0..a_p and denominator b_1..b_q (kanforge/bases/rational.py:64-104). Layers
share them within groups of inputs; the layer coefficients act as KAT's
linear weight.
"""

from __future__ import annotations

import math
from functools import lru_cache

import numpy as np

from .base import Basis, ParamSpec

TARGETS = {
    "identity": lambda x: x,
    "silu": lambda x: x / (1 + np.exp(-x)),
    "gelu": lambda x: 0.5 * x * (1 + np.vectorize(math.erf)(x / math.sqrt(2))),
    "tanh": np.tanh,
}


def _design(x, num_degree, den_degree):
    """Monomial columns of P (x^0..x^p) and of Q (x^1..x^q)."""
    return x[:, None] ** np.arange(num_degree + 1), x[:, None] ** np.arange(1, den_degree + 1)


def _sk_start(vp, vq, y, sweeps=25):
    """Sanathanan-Koerner iteration for P/(1+|Q|) ~ y.

    With the sign pattern s = sign(Q) and the denominator D = 1 + |Q| of the previous sweep held
    fixed, (P - y (1 + s Q)) / D is linear in the coefficients: each sweep is one weighted linear
    least-squares solve, and its solution gives the next s and D."""
    n_p = vp.shape[1]
    s = np.ones_like(y)
    d = np.ones_like(y)
    theta = np.zeros(n_p + vq.shape[1])
    for _ in range(sweeps):
        rows = np.hstack([vp, -(y * s)[:, None] * vq]) / d[:, None]
        theta = np.linalg.lstsq(rows, y / d, rcond=None)[0]
        q = vq @ theta[n_p:]
        s = np.where(q < 0, -1.0, 1.0)
        d = 1.0 + np.abs(q)
    return theta


def _gauss_newton(vp, vq, y, theta, iters=60):
    """Gauss-Newton on the true residual P/(1+|Q|) - y, each step shortened by halving until the
    sum of squares decreases (stops when no shortened step does)."""
    n_p = vp.shape[1]

    def residual(th):
        q = vq @ th[n_p:]
        return (vp @ th[:n_p]) / (1.0 + np.abs(q)) - y, q

    r, q = residual(theta)
    for _ in range(iters):
        d = 1.0 + np.abs(q)
        p = vp @ theta[:n_p]
        jac = np.hstack([vp / d[:, None], (-p * np.sign(q) / d**2)[:, None] * vq])
        step = np.linalg.lstsq(jac, -r, rcond=None)[0]
        t = 1.0
        while t > 1e-6:
            r_new, q_new = residual(theta + t * step)
            if r_new @ r_new < r @ r:
                theta, r, q = theta + t * step, r_new, q_new
                break
            t *= 0.5
        else:
            break
    return theta


@lru_cache(maxsize=None)
def fit_rational(target: str, num_degree: int, den_degree: int, lim: float = 3.0):
    """(a, b) of P/(1+|Q|) fitted to ``target`` on [-lim, lim] in the least-squares sense:
    a Sanathanan-Koerner start (reweighted linear solves) polished by Gauss-Newton."""
    x = np.linspace(-lim, lim, 2001)
    y = TARGETS[target](x)
    vp, vq = _design(x, num_degree, den_degree)
    theta = _gauss_newton(vp, vq, y, _sk_start(vp, vq, y))
    n_p = num_degree + 1
    return theta[:n_p].copy(), theta[n_p:].copy()


class Rational(Basis):
    name = "rational"

    def __init__(self, num_degree: int = 5, den_degree: int = 4, init: str = "silu"):
        if num_degree < 0 or den_degree < 1:
            raise ValueError("num_degree must be >= 0 and den_degree >= 1")
        if init not in TARGETS:
            raise ValueError(f"init must be one of {sorted(TARGETS)}")
        self.num_degree = int(num_degree)
        self.den_degree = int(den_degree)
        self.init = init

    @property
    def size(self) -> int:
        return 1

    def param_specs(self):
        a, b = fit_rational(self.init, self.num_degree, self.den_degree)
        return {"numerator": ParamSpec(a), "denominator": ParamSpec(b)}

    def host_values(self, x, params=None):
        x = np.asarray(x, dtype=np.float64)
        if params is None:
            a, b = fit_rational(self.init, self.num_degree, self.den_degree)
        else:
            a, b = np.asarray(params["numerator"], np.float64), np.asarray(params["denominator"], np.float64)
        P = sum(a[..., j] * x**j for j in range(self.num_degree + 1))
        Q = sum(b[..., j] * x ** (j + 1) for j in range(self.den_degree))
        return (P / (1 + np.abs(Q)))[..., None]

    def config(self):
        return {"name": self.name, "num_degree": self.num_degree, "den_degree": self.den_degree, "init": self.init}
