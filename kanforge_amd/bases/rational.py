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


@lru_cache(maxsize=None)
def fit_rational(target: str, num_degree: int, den_degree: int, lim: float = 3.0):
    """(a, b) of P/(1+|Q|) fitted to ``target`` on [-lim, lim].

    Start: the linear least-squares solution of P - f Q = f. Then damped
    Gauss-Newton (Levenberg-Marquardt) on the true residual P/(1+|Q|) - f.
    """
    f = TARGETS[target]
    x = np.linspace(-lim, lim, 2001)
    y = f(x)
    vp = x[:, None] ** np.arange(num_degree + 1)
    vq = x[:, None] ** np.arange(1, den_degree + 1)
    theta = np.linalg.lstsq(np.hstack([vp, -y[:, None] * vq]), y, rcond=None)[0]
    npar = num_degree + 1

    def resid(th):
        q = vq @ th[npar:]
        return (vp @ th[:npar]) / (1 + np.abs(q)) - y, q

    r, q = resid(theta)
    damping = 1e-3
    for _ in range(300):
        d = 1 + np.abs(q)
        jac = np.hstack([vp / d[:, None], (-(vp @ theta[:npar]) * np.sign(q) / d**2)[:, None] * vq])
        jtj = jac.T @ jac
        step = np.linalg.solve(jtj + damping * (np.diag(np.diag(jtj)) + 1e-12 * np.eye(len(theta))), -jac.T @ r)
        r2, q2 = resid(theta + step)
        if r2 @ r2 < r @ r:
            theta, r, q = theta + step, r2, q2
            damping = max(damping / 3, 1e-12)
        else:
            damping *= 4
            if damping > 1e8:
                break
    return theta[:npar].copy(), theta[npar:].copy()


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
