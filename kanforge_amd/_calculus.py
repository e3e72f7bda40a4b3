"""Host-side polynomial helpers (float64 NumPy) used to prepare kernel constants.

Same definitions as kanforge/_calculus.py:18-44 (Horner evaluation and the
chain polynomials of the tanh/sigmoid maps).
"""

from __future__ import annotations

import math

import numpy as np
from numpy.polynomial import polynomial as P

TANH_FACTOR = np.array([1.0, 0.0, -1.0])  # d/du tanh = 1 - tanh^2
SIGMOID_FACTOR = np.array([0.0, 1.0, -1.0])  # d/du sigmoid = s - s^2


def horner(coefs, x):
    """sum_j coefs[j] * x**j for NumPy arrays."""
    y = np.zeros_like(np.asarray(x, dtype=np.float64)) + (coefs[-1] if len(coefs) else 0.0)
    for c in reversed(list(coefs)[:-1]):
        y = y * x + c
    return y


def falling(n: int, k: int) -> int:
    """n (n-1) ... (n-k+1); 0 when k > n."""
    return math.perm(n, k) if 0 <= k <= n else 0


def chain_polys(start, factor, m: int) -> list[np.ndarray]:
    """[p_0 .. p_m], p_0 = start, p_{j+1} = p_j' * factor (power basis)."""
    out = [np.asarray(start, dtype=np.float64)]
    for _ in range(m):
        out.append(P.polymul(P.polyder(out[-1]), factor))
    return out
