"""Writes the golden vectors of tests/golden/*.npz from independent library
routines (scipy.interpolate, scipy.special, numpy.polynomial), NOT from the
oracle, so that tests/test_oracle.py can pin the oracle against them.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import os

import numpy as np
from numpy.polynomial import chebyshev as C
from scipy import special
from scipy.interpolate import BSpline

HERE = os.path.dirname(os.path.abspath(__file__))


def knots(grid, k):
    """Extended knot vector (mean step extension), written out independently."""
    g = np.asarray(grid, np.float64)
    h = (g[-1] - g[0]) / (len(g) - 1)
    return np.concatenate([g[0] - h * np.arange(k, 0, -1), g, g[-1] + h * np.arange(1, k + 1)])


def bspline_cases():
    rng = np.random.default_rng(10)
    out = {}
    for name, grid, k in [
        ("u5k3", np.linspace(-1, 1, 6), 3),
        ("u8k3", np.linspace(-1, 1, 9), 3),
        ("u4k1", np.linspace(-1, 1, 5), 1),
        ("nu6k2", np.sort(np.concatenate([[-1.0, 1.0], rng.uniform(-0.9, 0.9, 5)])), 2),
        ("u3k5", np.linspace(-1.5, 2.0, 4), 5),
    ]:
        t = knots(grid, k)
        x = np.concatenate([rng.uniform(grid[0], grid[-1], 64), grid[:-1]])
        size = len(t) - 1 - k
        vals = [BSpline.design_matrix(x, t, k).toarray()]
        for m in range(1, k + 2):
            if m > k:
                vals.append(np.zeros((len(x), size)))
            else:
                vals.append(np.stack([BSpline(t, np.eye(size)[j], k)(x, nu=m) for j in range(size)], -1))
        out[name] = dict(grid=grid, k=np.array(k), x=x, values=np.stack(vals))
    return out


def family_cases():
    z = np.linspace(-0.95, 0.95, 41)
    out = {
        "chebyshev": np.stack([special.eval_chebyt(n, z) for n in range(9)], -1),
        "chebyshev2": np.stack([special.eval_chebyu(n, z) for n in range(6)], -1),
        "legendre": np.stack([special.eval_legendre(n, z) for n in range(6)], -1),
        "jacobi_0.5_0.5": np.stack([special.eval_jacobi(n, 0.5, 0.5, z) for n in range(7)], -1),
        "jacobi_0.5_1.5": np.stack([special.eval_jacobi(n, 0.5, 1.5, z) for n in range(5)], -1),
        "gegenbauer_0.75": np.stack([special.eval_gegenbauer(n, 0.75, z) for n in range(6)], -1),
    }
    # d/dz P_n^(a,b) = (n+a+b+1)/2 P_{n-1}^(a+1,b+1): first derivative of Jacobi(6, .5, .5)
    a = b = 0.5
    dj = [np.zeros_like(z)] + [0.5 * (n + a + b + 1) * special.eval_jacobi(n - 1, a + 1, b + 1, z) for n in range(1, 7)]
    out["jacobi_0.5_0.5_dz"] = np.stack(dj, -1)
    # T_n' = n U_{n-1}
    out["chebyshev_dz"] = np.stack([np.zeros_like(z)] + [n * special.eval_chebyu(n - 1, z) for n in range(1, 9)], -1)
    return z, out


def main():
    b = bspline_cases()
    np.savez(os.path.join(HERE, "bspline_scipy.npz"), **{f"{n}__{k}": v for n, d in b.items() for k, v in d.items()})
    z, f = family_cases()
    np.savez(os.path.join(HERE, "families_scipy.npz"), z=z, **f)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
