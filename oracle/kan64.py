"""Float64 NumPy oracle for the fused KAN basis hot path.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or the timed CPU baseline). The product path never calls it.

Every function restates, from the mathematics, what the reference computes in
float64; the reference file:line it follows is named in each docstring
(paths relative to the kanforge repository). How each function is pinned
(independently of this file's own formulas) is listed in ``PINNING`` at the
bottom and exercised by ``tests/test_oracle.py``.

Notation: a layer has ``n_in`` inputs, ``n_out`` outputs and ``K`` basis
functions per edge; ``x`` is ``(B, n_in)``, ``coef`` is ``(n_out, n_in, K)``.
"""

from __future__ import annotations

import math

import numpy as np
from numpy.polynomial import chebyshev as npcheb
from numpy.polynomial import polynomial as nppoly

# --------------------------------------------------------------------------
# scalar calculus helpers


def chain_polys(start, factor, m):
    """[p_0..p_m], p_{j+1} = p_j' * factor (power-basis coefficients).

    Follows ``kanforge/_calculus.py:35-44``. With factor 1 - t^2, p_j(tanh u)
    is the j-th u-derivative of p_0(tanh u); with s - s^2 likewise for sigmoid.
    """
    out = [np.asarray(start, dtype=np.float64)]
    for _ in range(m):
        out.append(nppoly.polymul(nppoly.polyder(out[-1]), factor))
    return out


TANH_FACTOR = np.array([1.0, 0.0, -1.0])
SIGMOID_FACTOR = np.array([0.0, 1.0, -1.0])


def sigmoid(x):
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * (1.0 + np.tanh(0.5 * x))


def silu_derivative(x, m):
    """d^m/dx^m of x*sigmoid(x) = x p_m(s) + m p_{m-1}(s), s = sigmoid(x).

    Follows ``kanforge/_calculus.py:90-96``.
    """
    x = np.asarray(x, dtype=np.float64)
    s = sigmoid(x)
    if m == 0:
        return x * s
    p = chain_polys([0.0, 1.0], SIGMOID_FACTOR, m)
    return x * nppoly.polyval(s, p[m]) + m * nppoly.polyval(s, p[m - 1])


def tanh_map(x, m):
    """[g, g', ..., g^(m)] for g = tanh (``kanforge/bases/polynomial.py:71-73``)."""
    z = np.tanh(np.asarray(x, dtype=np.float64))
    p = chain_polys([0.0, 1.0], TANH_FACTOR, m)
    return [z] + [nppoly.polyval(z, p[j]) for j in range(1, m + 1)]


def _bell_partial(inner, m):
    """Partial Bell polynomials B_{m,k}(g', g'', ...) for k=1..m (dict k -> array)."""
    bell = {(0, 0): 1.0}
    for n in range(1, m + 1):
        for k in range(1, n + 1):
            acc = 0.0
            for i in range(1, n - k + 2):
                prev = bell.get((n - i, k - 1))
                if prev is None:
                    continue
                acc = acc + math.comb(n - 1, i - 1) * inner[i] * prev
            bell[(n, k)] = acc
    return {k: bell[(m, k)] for k in range(1, m + 1)}


def faa_di_bruno(outer, inner, m):
    """m-th derivative of f(g(x)) from f^(k)(g) and g^(k) (``kanforge/_calculus.py:51-76``)."""
    if m == 0:
        return outer[0]
    b = _bell_partial(inner, m)
    out = 0.0
    for k in range(1, m + 1):
        out = out + outer[k] * b[k]
    return out


def quotient(num, den, m):
    """m-th derivative of N/D from N^(0..m), D^(0..m) (``kanforge/_calculus.py:79-87``)."""
    out = [num[0] / den[0]]
    for n in range(1, m + 1):
        acc = num[n]
        for k in range(1, n + 1):
            acc = acc - math.comb(n, k) * den[k] * out[n - k]
        out.append(acc / den[0])
    return out[m]


# --------------------------------------------------------------------------
# B-splines


def extend_grid(grid, k):
    """Knots: k points added each side with the mean grid step.

    Follows ``kanforge/bases/spline.py:22-30``: h = (g_G - g_0)/G,
    left r = g_0 - h (k - r), right r = g_G + h (r + 1).
    """
    grid = np.asarray(grid, dtype=np.float64)
    if k == 0:
        return grid.copy()
    h = (grid[..., -1:] - grid[..., :1]) / (grid.shape[-1] - 1)
    i = np.arange(k, dtype=np.float64)
    left = grid[..., :1] - h * (k - i)
    right = grid[..., -1:] + h * (i + 1)
    return np.concatenate([left, grid, right], -1)


def bspline_interval(x, knots):
    """Index j with knots[j] <= x < knots[j+1], or -1 when there is none.

    The level-0 indicator of ``kanforge/bases/spline.py:80`` is the half-open
    test above; at most one j satisfies it. ``x`` (..., n_in), ``knots``
    (n_in, n_knots) or (n_knots,). Brute force over all knots in float64.
    """
    x = np.asarray(x, dtype=np.float64)
    t = np.asarray(knots, dtype=np.float64)
    ge = x[..., None] >= t[..., :-1]
    lt = x[..., None] < t[..., 1:]
    hit = ge & lt
    idx = np.where(hit.any(-1), hit.argmax(-1), -1)
    return idx.astype(np.int64)


def bspline_basis(x, knots, k, m=0):
    """d^m/dx^m of the B-splines of degree k on ``knots``: (..., n_in, n_knots-1-k).

    Dense Cox-de Boor from the half-open indicators, then m derivative steps,
    as in ``kanforge/bases/spline.py:74-92``; m > k gives zeros.
    """
    x = np.asarray(x, dtype=np.float64)[..., None]
    t = np.asarray(knots, dtype=np.float64)
    size = t.shape[-1] - 1 - k
    if m > k:
        return np.zeros(x.shape[:-1] + (size,))
    b = ((x >= t[..., :-1]) & (x < t[..., 1:])).astype(np.float64)
    for q in range(1, k - m + 1):
        left = (x - t[..., : -(q + 1)]) / (t[..., q:-1] - t[..., : -(q + 1)])
        right = (t[..., q + 1 :] - x) / (t[..., q + 1 :] - t[..., 1:-q])
        b = left * b[..., :-1] + right * b[..., 1:]
    for q in range(k - m + 1, k + 1):
        n = b.shape[-1] - 1
        b = q * (b[..., :-1] / (t[..., q : q + n] - t[..., :n]) - b[..., 1:] / (t[..., q + 1 : q + 1 + n] - t[..., 1 : 1 + n]))
    return b


# --------------------------------------------------------------------------
# polynomial families (all evaluated through Chebyshev coefficients)


def family_values(name, z, degree, **kw):
    """Values of the polynomial family at float64 points z: (len(z), degree+1).

    The three-term recurrences of ``kanforge/bases/polynomial.py:114-262``.
    """
    z = np.asarray(z, dtype=np.float64)
    d = degree
    if name == "chebyshev":
        return npcheb.chebvander(z, d)
    if name == "chebyshev2":
        u = [np.ones_like(z), 2 * z]
        for _ in range(2, d + 1):
            u.append(2 * z * u[-1] - u[-2])
        return np.stack(u[: d + 1], -1)
    if name == "legendre":
        p = [np.ones_like(z), z]
        for n in range(2, d + 1):
            p.append(((2 * n - 1) * z * p[-1] - (n - 1) * p[-2]) / n)
        return np.stack(p[: d + 1], -1)
    if name == "jacobi":
        a, b = kw.get("alpha", 1.0), kw.get("beta", 1.0)
        out = [np.ones_like(z), (a + 1) + (a + b + 2) * (z - 1) / 2]
        for n in range(2, d + 1):
            c = 2 * n + a + b
            num = (c - 1) * (c * (c - 2) * z + a * a - b * b) * out[-1] - 2 * (n + a - 1) * (n + b - 1) * c * out[-2]
            out.append(num / (2 * n * (n + a + b) * (c - 2)))
        return np.stack(out[: d + 1], -1)
    if name == "gegenbauer":
        lam = kw.get("lam", 1.0)
        out = [np.ones_like(z), 2 * lam * z]
        for n in range(2, d + 1):
            out.append((2 * z * (n + lam - 1) * out[-1] - (n + 2 * lam - 2) * out[-2]) / n)
        return np.stack(out[: d + 1], -1)
    if name == "taylor":
        return np.stack([z**j for j in range(d + 1)], -1)
    raise ValueError(name)


def cheb_coefficients(name, degree, **kw):
    """A (degree+1, degree+1): family(z) = chebvander(z) @ A.

    Interpolation at Chebyshev nodes, ``kanforge/bases/polynomial.py:51-56``.
    """
    nodes = np.cos(np.pi * (np.arange(degree + 1) + 0.5) / (degree + 1))
    return np.linalg.solve(npcheb.chebvander(nodes, degree), family_values(name, nodes, degree, **kw))


def polynomial_basis(x, A, input_map="tanh", m=0):
    """d^m/dx^m of [T_0(z)..T_D(z)] @ A with z = tanh(x) or z = x: (..., n_in, size).

    Follows ``kanforge/bases/polynomial.py:66-106`` (Faa di Bruno over the
    input map, derivatives of the family in z by chebder).
    """
    x = np.asarray(x, dtype=np.float64)
    A = np.asarray(A, dtype=np.float64)
    d = A.shape[0] - 1
    if input_map == "tanh":
        g = tanh_map(x, m)
    elif input_map == "identity":
        g = [x] + ([np.ones_like(x)] + [np.zeros_like(x)] * (m - 1) if m else [])
    else:
        raise ValueError(input_map)
    z = g[0]
    T = npcheb.chebvander(z, d)
    outer = []
    for k in range(m + 1):
        a = npcheb.chebder(A, k, axis=0) if k else A
        outer.append(T[..., : a.shape[0]] @ a if a.shape[0] else np.zeros(z.shape + (A.shape[1],)))
    return faa_di_bruno(outer, [gi[..., None] if np.ndim(gi) else gi for gi in g], m) if m else outer[0]


ONE_MINUS_Z2 = np.array([0.5, 0.0, -0.5])  # 1 - z^2 in the Chebyshev basis


def fold_matrix(A, input_map, m):
    """R_m (size, n_t): d^m/dx^m family_k(g(x)) = sum_j R_m[k, j] T_j(g(x)).

    Follows ``kanforge/kernels/plan.py:88-101``: chebder, then for the tanh
    map multiplication by 1 - z^2 in the Chebyshev basis, m times.
    n_t = D + 1 + m for tanh, D + 1 for identity.
    """
    A = np.asarray(A, dtype=np.float64)
    d = A.shape[0] - 1
    n_t = d + 1 + m if input_map == "tanh" else d + 1
    cols = []
    for k in range(A.shape[1]):
        col = A[:, k]
        for _ in range(m):
            col = npcheb.chebder(col) if len(col) > 1 else np.zeros(1)
            if input_map == "tanh":
                col = npcheb.chebmul(col, ONE_MINUS_Z2)
        out = np.zeros(n_t)
        out[: min(len(col), n_t)] = col[:n_t]
        cols.append(out)
    return np.stack(cols)


# --------------------------------------------------------------------------
# rational P / (1 + |Q|)


def _poly_derivative(coef, first, k, x):
    """k-th derivative of sum_j coef[..., j] x^(j+first) at x (coef per input)."""
    coef = np.asarray(coef, dtype=np.float64)
    n = coef.shape[-1]
    out = np.zeros(np.broadcast_shapes(np.shape(x), coef.shape[:-1]))
    for j in range(n):
        p = j + first
        if p < k:
            continue
        out = out + coef[..., j] * math.perm(p, k) * np.asarray(x, dtype=np.float64) ** (p - k)
    return out


def rational_basis(x, num, den, m=0):
    """d^m/dx^m of P(x)/(1+|Q(x)|): (..., n_in, 1).

    P = sum_{j=0..} num[j] x^j, Q = sum_{j=1..} den[j-1] x^j, |Q|' = sign(Q) Q'
    (``kanforge/bases/rational.py:84-101``); num (n_in, nP), den (n_in, nQ).
    """
    x = np.asarray(x, dtype=np.float64)
    P = [_poly_derivative(num, 0, k, x) for k in range(m + 1)]
    Q = [_poly_derivative(den, 1, k, x) for k in range(m + 1)]
    s = np.sign(Q[0])
    D = [1.0 + np.abs(Q[0])] + [s * q for q in Q[1:]]
    return quotient(P, D, m)[..., None]


def rational_param_grads(x, num, den):
    """(dphi/dnum (..., n_in, nP), dphi/dden (..., n_in, nQ)) of phi = P/(1+|Q|)."""
    x = np.asarray(x, dtype=np.float64)
    num = np.asarray(num, dtype=np.float64)
    den = np.asarray(den, dtype=np.float64)
    P = _poly_derivative(num, 0, 0, x)
    Q = _poly_derivative(den, 1, 0, x)
    D = 1.0 + np.abs(Q)
    dnum = np.stack([x**j / D for j in range(num.shape[-1])], -1)
    dden = np.stack([-P * np.sign(Q) * x ** (j + 1) / D**2 for j in range(den.shape[-1])], -1)
    return dnum, dden


# --------------------------------------------------------------------------
# basis descriptions used by the layer-level functions below


class Basis64:
    """A basis as the oracle sees it: kind plus per-input parameters.

    kind "poly": A (D+1, size) Chebyshev coefficients, input_map;
    kind "bspline": per-input grid (n_in, G+1), order k;
    kind "rational": per-input num (n_in, nP), den (n_in, nQ).
    """

    def __init__(self, kind, **kw):
        self.kind = kind
        self.kw = kw

    @property
    def size(self):
        if self.kind == "poly":
            return self.kw["A"].shape[1]
        if self.kind == "bspline":
            g = np.asarray(self.kw["grid"])
            return g.shape[-1] - 1 + self.kw["k"]
        return 1

    def __call__(self, x, m=0):
        """d^m/dx^m of every basis function: (..., n_in, size)."""
        if self.kind == "poly":
            return polynomial_basis(x, self.kw["A"], self.kw.get("input_map", "tanh"), m)
        if self.kind == "bspline":
            k = self.kw["k"]
            t = extend_grid(self.kw["grid"], k)
            return bspline_basis(x, t, k, m)
        return rational_basis(x, self.kw["num"], self.kw["den"], m)


def kan_linear(x, coef, basis, base_weight=None, bias=None, edge_scale=None):
    """y = sum_{i,k} s_oi c[o,i,k] phi_k(x_i) + sum_i w_oi silu(x_i) + b_o.

    Follows ``kanforge/reference.py:18-44``.
    """
    x = np.asarray(x, dtype=np.float64)
    coef = np.asarray(coef, dtype=np.float64)
    if edge_scale is not None:
        coef = coef * np.asarray(edge_scale, dtype=np.float64)[..., None]
    y = np.einsum("...ik,oik->...o", basis(x), coef, optimize=True)
    if base_weight is not None:
        y = y + silu_derivative(x, 0) @ np.asarray(base_weight, dtype=np.float64).T
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64)
    return y


# --------------------------------------------------------------------------
# the three primitives and edge_derivative (``kanforge/kernels/__init__.py:1-13``)


def prim_F(x, c, w, basis, m=0):
    """F_m[b,o] = sum_{i,k} w[b,i] c[o,i,k] phi_k^(m)(x[b,i]); w None means ones."""
    phi = basis(x, m)
    if w is not None:
        phi = phi * np.asarray(w, dtype=np.float64)[..., None]
    return np.einsum("bik,oik->bo", phi, np.asarray(c, dtype=np.float64), optimize=True)


def prim_G(x, g, w, basis, m=0):
    """G_m[o,i,k] = sum_b w[b,i] g[b,o] phi_k^(m)(x[b,i])."""
    phi = basis(x, m)
    if w is not None:
        phi = phi * np.asarray(w, dtype=np.float64)[..., None]
    return np.einsum("bik,bo->oik", phi, np.asarray(g, dtype=np.float64), optimize=True)


def prim_P(x, g, c, basis, m=0):
    """P_m[b,i] = sum_{o,k} g[b,o] c[o,i,k] phi_k^(m)(x[b,i])."""
    phi = basis(x, m)
    h = np.einsum("bo,oik->bik", np.asarray(g, dtype=np.float64), np.asarray(c, dtype=np.float64), optimize=True)
    return (h * phi).sum(-1)


def edge_derivative(x, coef_eff, basis, m=0, base_weight_eff=None):
    """d[b,o,i] = sum_k c[o,i,k] phi_k^(m)(x[b,i]) + W[o,i] silu^(m)(x[b,i]).

    Follows ``kanforge/torch/layers.py:206-226`` (SiLU base only).
    """
    d = np.einsum("bik,oik->boi", basis(x, m), np.asarray(coef_eff, dtype=np.float64), optimize=True)
    if base_weight_eff is not None:
        d = d + silu_derivative(x, m)[:, None, :] * np.asarray(base_weight_eff, dtype=np.float64)[None]
    return d


# --------------------------------------------------------------------------
# symbolic edges (``kanforge/_layer.py:256-272``, ``kanforge/interpret/library.py:34-55``)

SYMBOLIC = (
    ("0", lambda u: 0 * u), ("x", lambda u: u), ("x^2", lambda u: u * u), ("x^3", lambda u: u * u * u),
    ("x^4", lambda u: (u * u) * (u * u)), ("1/x", lambda u: 1 / u), ("1/x^2", lambda u: 1 / (u * u)),
    ("sqrt", np.sqrt), ("1/sqrt", lambda u: 1 / np.sqrt(u)), ("exp", np.exp), ("log", np.log), ("sin", np.sin),
    ("cos", np.cos), ("tanh", np.tanh), ("sigmoid", lambda u: 1 / (1 + np.exp(-u))), ("gaussian", lambda u: np.exp(-u * u)),
    ("abs", np.abs), ("arctan", np.arctan),
)


def symbolic_edges(x, code, params):
    """(..., out, in): c f_code(a x_i + b) + d on edges with code >= 0, zero elsewhere.

    ``code`` (out, in) indexes ``SYMBOLIC`` (the reference's function order); ``params`` (out, in, 4).
    """
    x = np.asarray(x, dtype=np.float64)
    code = np.asarray(code)
    p = np.asarray(params, dtype=np.float64)
    u = p[..., 0] * x[..., None, :] + p[..., 1]
    out = np.zeros(u.shape)
    for k in np.unique(code[code >= 0]):
        sel = code == k
        with np.errstate(all="ignore"):
            v = p[..., 2] * SYMBOLIC[k][1](np.where(sel, u, 1.0)) + p[..., 3]
        out = np.where(sel, v, out)
    return out


# --------------------------------------------------------------------------
# rounding helpers: the oracle always sees the dtype-rounded inputs


def round_bf16(a):
    """Round-to-nearest-even float64 -> bfloat16 -> float64 (via float32)."""
    f = np.asarray(a, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    out = u.astype(np.uint32).view(np.float32).astype(np.float64)
    return np.where(nan, np.nan, out)


def normwise_err(got, want):
    """max|got - want| / max|want| (0 when both vanish)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    scale = np.abs(want).max() if want.size else 0.0
    diff = np.abs(got - want).max() if want.size else 0.0
    return diff / scale if scale > 0 else diff


def ref_metric(got, want):
    """The reference's own closeness measure: max|d| / max(1, max|want|) (``tests/test_kernels.py:96-99``)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return np.abs(got - want).max() / max(1.0, np.abs(want).max())


PINNING = {
    "extend_grid": "knot vectors fed to scipy.interpolate.BSpline.design_matrix (tests/test_oracle.py)",
    "bspline_interval": "brute force over knots in float64 at, next to and between every knot; scipy design_matrix support",
    "bspline_basis": "scipy.interpolate.BSpline.design_matrix and BSpline(t, e_j, k)(x, nu=m); partition of unity",
    "family_values": "scipy.special eval_chebyt/eval_chebyu/eval_legendre/eval_jacobi/eval_gegenbauer",
    "polynomial_basis": "chebvander(tanh x) (m=0); central finite differences of order m in float64",
    "fold_matrix": "T(z) @ R_m.T == polynomial_basis(x, m) (tests/test_kernels.py:31-44 invariant)",
    "rational_basis": "direct polynomial evaluation for m=0; finite differences for m>0",
    "rational_param_grads": "finite differences in the parameters",
    "silu_derivative": "finite differences; closed form sigma(x)(1+x(1-sigma(x))) for m=1",
    "prim_F/prim_G/prim_P": "brute-force Python loops on tiny shapes; y = F_0(x,c,1) equals kan_linear",
    "edge_derivative": "sum over i of order-0 edges plus bias equals kan_linear (tests/test_layers.py:62-63)",
    "kan_linear": "per-edge manual sum (tests/test_bases.py:64-74)",
    "symbolic_edges": "defining values of every library function (x^2(3) = 9, sin(pi/2) = 1, ...); affine map inside and out",
}


# --------------------------------------------------------------------------
# lookup tables (kanforge/export/lut.py)


def lut_layer(x, tables, lo, hi, bias, scale=None, slope_lo=None, slope_hi=None, extrapolate="linear"):
    """LUTLayer.__call__ (kanforge/export/lut.py:70-89) in float64: x (B, in), tables
    (in, size, out); y (B, out) = bias + [scale *] sum_i lerp of T[i, j], T[i, j+1] at
    t = (x - lo) / step (step = (hi - lo) / (size - 1)), plus the end slopes times how far t
    leaves [0, size - 1] when extrapolating linearly."""
    x = np.asarray(x, dtype=np.float64)
    T = np.asarray(tables, dtype=np.float64)
    size = T.shape[1]
    step = (np.asarray(hi, np.float64) - np.asarray(lo, np.float64)) / (size - 1)
    t_raw = (x - lo) / step
    t = np.clip(t_raw, 0, size - 1)
    j = np.clip(np.floor(t), 0, size - 2).astype(np.int64)
    f = t - j
    i = np.arange(x.shape[-1])
    t0, t1 = T[i, j], T[i, j + 1]
    acc = (t0 + f[..., None] * (t1 - t0)).sum(-2)
    y = acc * scale + bias if scale is not None else acc + bias
    if extrapolate == "linear" and slope_lo is not None:
        below = np.minimum(t_raw, 0.0)[..., None]
        above = np.maximum(t_raw - (size - 1), 0.0)[..., None]
        y = y + (below * slope_lo + above * slope_hi).sum(-2)
    return y


def lut_end_slopes(tables):
    """Per index step, over the first and last max(1, (size-1) // 32) steps
    (kanforge/export/lut.py:131-135): (slope_lo, slope_hi), each (in, out)."""
    T = np.asarray(tables, dtype=np.float64)
    k = max(1, (T.shape[1] - 1) // 32)
    return (T[:, k] - T[:, 0]) / k, (T[:, -1] - T[:, -1 - k]) / k


def lut_quantize(tables, bias, bits=8):
    """(q, scale, bias') with T ~ centre + scale q (kanforge/export/lut.py:175-197): centre the
    (max + min) / 2 of each edge, scale per output the largest deviation over qmax."""
    T = np.asarray(tables, dtype=np.float64)
    qmax = 2 ** (bits - 1) - 1
    centre = 0.5 * (T.max(1) + T.min(1))
    dev = np.abs(T - centre[:, None, :]).max((0, 1))
    scale = np.where(dev > 0, dev / qmax, 1.0)
    q = np.round((T - centre[:, None, :]) / scale).astype(np.int8 if bits <= 8 else np.int16)
    return q, scale, np.asarray(bias, np.float64) + centre.sum(0)
