"""Pins the float64 oracle (oracle/kan64.py) against independent references:
scipy/numpy library routines, the committed golden vectors written from them
(tests/golden/make_golden.py), closed forms, finite differences and brute
force. Each oracle function is checked by something other than its own
formula; a planted mistake must fail here (see test_planted_mistakes_fail)."""

import math
import os

import numpy as np
import pytest
from numpy.polynomial import chebyshev as C
from scipy import special
from scipy.interpolate import BSpline

from oracle import kan64 as o

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
rng = np.random.default_rng(0)


def fd(f, x, m, h=None):
    """m-th central finite difference of f at x (float64)."""
    h = h or {1: 1e-5, 2: 1e-4, 3: 2e-3}[m]
    coeffs = {1: [(-0.5, -1), (0.5, 1)], 2: [(1, -1), (-2, 0), (1, 1)], 3: [(-0.5, -2), (1, -1), (-1, 1), (0.5, 2)]}[m]
    return sum(c * f(x + s * h) for c, s in coeffs) / h**m


# --- B-splines ------------------------------------------------------------------


def test_bspline_matches_scipy_golden():
    data = np.load(os.path.join(GOLDEN, "bspline_scipy.npz"))
    names = sorted({k.split("__")[0] for k in data.files})
    assert names
    for n in names:
        grid, k, x, vals = (data[f"{n}__{f}"] for f in ("grid", "k", "x", "values"))
        k = int(k)
        t = o.extend_grid(grid, k)
        for m in range(vals.shape[0]):
            got = o.bspline_basis(x, t, k, m)
            np.testing.assert_allclose(got, vals[m], atol=1e-9 * max(1.0, np.abs(vals[m]).max()), err_msg=f"{n} m={m}")


@pytest.mark.parametrize("k", [0, 1, 2, 3, 5])
@pytest.mark.parametrize("grid_size", [1, 4, 9])
def test_bspline_matches_scipy_live(k, grid_size):
    grid = np.linspace(-1.5, 2.0, grid_size + 1)
    t = o.extend_grid(grid, k)
    x = rng.uniform(-1.5, 2.0, 200)
    np.testing.assert_allclose(o.bspline_basis(x, t, k), BSpline.design_matrix(x, t, k).toarray(), atol=1e-12)


def test_bspline_invariants():
    t = o.extend_grid(np.linspace(-2, 3, 8), 3)
    x = np.linspace(-2, 3, 1001)[:-1]
    b = o.bspline_basis(x, t, 3)
    np.testing.assert_allclose(b.sum(-1), 1.0, atol=1e-12)  # partition of unity inside the grid
    assert ((np.abs(b) > 1e-14).sum(-1) <= 4).all()  # support k + 1
    far = np.array([-10.0, t[0] - 1e-9, t[-1], 10.0])
    assert np.all(o.bspline_basis(far, t, 3) == 0)  # zero outside [t_0, t_last)
    # non-finite inputs propagate NaN through the recurrence (as the reference's arithmetic does)
    assert np.isnan(o.bspline_basis(np.array([np.nan, np.inf]), t, 3)).all()


def test_extend_grid_by_hand():
    np.testing.assert_allclose(o.extend_grid([0.0, 1.0, 2.0], 2), [-2.0, -1.0, 0.0, 1.0, 2.0, 3.0, 4.0])
    g = np.array([[0.0, 0.5, 2.0]])  # non-uniform: mean step (2 - 0) / 2 = 1
    np.testing.assert_allclose(o.extend_grid(g, 1), [[-1.0, 0.0, 0.5, 2.0, 3.0]])


def test_bspline_interval_brute_force():
    t = o.extend_grid(np.sort(rng.uniform(-1, 1, 7)), 3)
    t32 = t.astype(np.float32).astype(np.float64)
    x = np.concatenate([t, t32, np.nextafter(t, -np.inf), np.nextafter(t, np.inf), rng.uniform(-3, 3, 300), [np.nan]])
    idx = o.bspline_interval(x, t)
    # independent formula: last knot <= x, half-open, -1 outside [t0, t_last)
    ref = np.searchsorted(t, x, side="right") - 1
    ref = np.where((x >= t[0]) & (x < t[-1]), ref, -1)
    np.testing.assert_array_equal(idx, ref)
    # agrees with the support scipy reports for the degree-0 design matrix
    inside = (x >= t[0]) & (x < t[-1])
    d0 = BSpline.design_matrix(x[inside], t, 0).toarray()
    np.testing.assert_array_equal(d0.argmax(-1), idx[inside])


# --- polynomial families -----------------------------------------------------------


def test_families_match_scipy_golden():
    data = np.load(os.path.join(GOLDEN, "families_scipy.npz"))
    z = data["z"]
    np.testing.assert_allclose(o.family_values("chebyshev", z, 8), data["chebyshev"], atol=1e-12)
    np.testing.assert_allclose(o.family_values("chebyshev2", z, 5), data["chebyshev2"], atol=1e-12)
    np.testing.assert_allclose(o.family_values("legendre", z, 5), data["legendre"], atol=1e-12)
    np.testing.assert_allclose(o.family_values("jacobi", z, 6, alpha=0.5, beta=0.5), data["jacobi_0.5_0.5"], atol=1e-11)
    np.testing.assert_allclose(o.family_values("jacobi", z, 4, alpha=0.5, beta=1.5), data["jacobi_0.5_1.5"], atol=1e-11)
    np.testing.assert_allclose(o.family_values("gegenbauer", z, 5, lam=0.75), data["gegenbauer_0.75"], atol=1e-11)


@pytest.mark.parametrize("name,kw,deg", [("jacobi", {"alpha": 0.5, "beta": 0.5}, 6), ("legendre", {}, 5), ("gegenbauer", {"lam": 0.75}, 4)])
def test_cheb_coefficients_reproduce_family(name, kw, deg):
    A = o.cheb_coefficients(name, deg, **kw)
    z = rng.uniform(-1, 1, 50)
    np.testing.assert_allclose(C.chebvander(z, deg) @ A, o.family_values(name, z, deg, **kw), atol=1e-11)


def test_polynomial_basis_values_and_closed_form_derivative():
    data = np.load(os.path.join(GOLDEN, "families_scipy.npz"))
    z = data["z"]
    x = np.arctanh(z)
    A = o.cheb_coefficients("jacobi", 6, alpha=0.5, beta=0.5)
    np.testing.assert_allclose(o.polynomial_basis(x, A, "tanh", 0), data["jacobi_0.5_0.5"], atol=1e-11)
    # d/dx P(tanh x) = P'(z) (1 - z^2), P' from the scipy closed form
    want = data["jacobi_0.5_0.5_dz"] * (1 - z**2)[:, None]
    np.testing.assert_allclose(o.polynomial_basis(x, A, "tanh", 1), want, atol=1e-10)
    want_cheb = data["chebyshev_dz"] * (1 - z**2)[:, None]
    np.testing.assert_allclose(o.polynomial_basis(x, np.eye(9), "tanh", 1), want_cheb, atol=1e-10)


@pytest.mark.parametrize("m", [1, 2, 3])
@pytest.mark.parametrize("input_map", ["tanh", "identity"])
def test_polynomial_basis_derivatives_match_finite_differences(m, input_map):
    A = o.cheb_coefficients("jacobi", 5, alpha=0.5, beta=1.5)
    x = rng.uniform(-0.8, 0.8, 25)
    got = o.polynomial_basis(x, A, input_map, m)
    want = fd(lambda v: o.polynomial_basis(v, A, input_map, 0), x, m)
    tol = 2e-4 if m == 3 else 2e-5  # O(h^2) truncation of the third difference
    np.testing.assert_allclose(got, want, atol=tol * max(1, np.abs(want).max()))


@pytest.mark.parametrize("m", [0, 1, 2, 3])
@pytest.mark.parametrize("name", ["chebyshev", "jacobi"])
def test_fold_matrix_reproduces_derivatives(m, name):
    # the invariant of tests/test_kernels.py:31-44 on the independently pinned polynomial_basis
    kw = {"alpha": 0.5, "beta": 0.5} if name == "jacobi" else {}
    A = o.cheb_coefficients(name, 6, **kw)
    x = np.linspace(-1.2, 1.2, 41)
    for input_map in ("tanh", "identity"):
        r = o.fold_matrix(A, input_map, m)
        z = np.tanh(x) if input_map == "tanh" else x
        feats = C.chebvander(z, r.shape[1] - 1)
        want = o.polynomial_basis(x, A, input_map, m)
        np.testing.assert_allclose(feats @ r.T, want, atol=1e-9 * max(1, np.abs(want).max()))


# --- rational and SiLU --------------------------------------------------------------


def test_rational_values_and_derivatives():
    num = rng.normal(0, 0.3, (3, 6))
    den = rng.normal(0, 0.3, (3, 4))
    x = rng.normal(0, 1, (11, 3))
    direct = np.stack(
        [sum(num[i, j] * x[:, i] ** j for j in range(6)) / (1 + np.abs(sum(den[i, j] * x[:, i] ** (j + 1) for j in range(4)))) for i in range(3)],
        -1,
    )
    np.testing.assert_allclose(o.rational_basis(x, num, den, 0)[..., 0], direct, atol=1e-13)
    for m in (1, 2):
        got = o.rational_basis(x, num, den, m)[..., 0]
        want = fd(lambda v: o.rational_basis(v, num, den, 0)[..., 0], x, m)
        np.testing.assert_allclose(got, want, atol=1e-5 * max(1, np.abs(want).max()))


def test_rational_param_grads_match_finite_differences():
    num = rng.normal(0, 0.3, (1, 6))
    den = rng.normal(0, 0.3, (1, 4))
    x = rng.normal(0, 1, (20, 1))
    dn, dd = o.rational_param_grads(x, num, den)
    h = 1e-6
    for j in range(6):
        e = np.zeros_like(num)
        e[0, j] = h
        want = (o.rational_basis(x, num + e, den)[..., 0] - o.rational_basis(x, num - e, den)[..., 0]) / (2 * h)
        np.testing.assert_allclose(dn[..., j], want, atol=1e-7)
    for j in range(4):
        e = np.zeros_like(den)
        e[0, j] = h
        want = (o.rational_basis(x, num, den + e)[..., 0] - o.rational_basis(x, num, den - e)[..., 0]) / (2 * h)
        np.testing.assert_allclose(dd[..., j], want, atol=1e-6)


def test_silu_derivatives():
    x = np.linspace(-4, 4, 33)
    s = 1 / (1 + np.exp(-x))
    np.testing.assert_allclose(o.silu_derivative(x, 0), x * s, atol=1e-14)
    np.testing.assert_allclose(o.silu_derivative(x, 1), s * (1 + x * (1 - s)), atol=1e-13)
    for m in (2, 3):
        want = fd(lambda v: o.silu_derivative(v, 0), x, m)
        np.testing.assert_allclose(o.silu_derivative(x, m), want, atol=1e-5)


# --- primitives and the layer ------------------------------------------------------


def tiny():
    B, IN, OUT = 3, 2, 2
    basis = o.Basis64("poly", A=o.cheb_coefficients("jacobi", 2, alpha=0.5, beta=0.5), input_map="tanh")
    x = rng.uniform(-0.9, 0.9, (B, IN))
    c = rng.normal(size=(OUT, IN, 3))
    g = rng.normal(size=(B, OUT))
    w = rng.uniform(0.5, 1.5, (B, IN))
    return basis, x, c, g, w


@pytest.mark.parametrize("m", [0, 1, 2])
def test_primitives_match_brute_force_loops(m):
    basis, x, c, g, w = tiny()
    B, IN = x.shape
    OUT, _, K = c.shape
    phi = basis(x, m)
    F = np.zeros((B, OUT))
    G = np.zeros((OUT, IN, K))
    P = np.zeros((B, IN))
    for b in range(B):
        for i in range(IN):
            for k in range(K):
                for oo in range(OUT):
                    F[b, oo] += w[b, i] * c[oo, i, k] * phi[b, i, k]
                    G[oo, i, k] += w[b, i] * g[b, oo] * phi[b, i, k]
                    P[b, i] += g[b, oo] * c[oo, i, k] * phi[b, i, k]
    np.testing.assert_allclose(o.prim_F(x, c, w, basis, m), F, atol=1e-12)
    np.testing.assert_allclose(o.prim_G(x, g, w, basis, m), G, atol=1e-12)
    np.testing.assert_allclose(o.prim_P(x, g, c, basis, m), P, atol=1e-12)


def test_closure_identities():
    # dF/dx = w * P_{m+1}: finite differences of F_0 along x[b, i]
    basis, x, c, g, w = tiny()
    loss = lambda xx: (o.prim_F(xx, c, None, basis, 0) * g).sum()  # noqa: E731
    h = 1e-6
    got = o.prim_P(x, g, c, basis, 1)
    for b in range(x.shape[0]):
        for i in range(x.shape[1]):
            e = np.zeros_like(x)
            e[b, i] = h
            assert abs((loss(x + e) - loss(x - e)) / (2 * h) - got[b, i]) < 1e-6


def test_kan_linear_is_sum_over_edges_and_edge_derivative():
    t_grid = np.linspace(-1, 1, 6)
    basis = o.Basis64("bspline", grid=np.broadcast_to(t_grid, (3, 6)), k=3)
    x = rng.uniform(-1, 1, (8, 3))
    coef = rng.normal(size=(2, 3, 8))
    W = rng.normal(size=(2, 3))
    b = rng.normal(size=2)
    y = o.kan_linear(x, coef, basis, W, b)
    t = o.extend_grid(t_grid, 3)
    silu = x / (1 + np.exp(-x))
    for oo in range(2):
        manual = b[oo] + sum(BSpline.design_matrix(x[:, i], t, 3).toarray() @ coef[oo, i] + W[oo, i] * silu[:, i] for i in range(3))
        np.testing.assert_allclose(y[:, oo], manual, atol=1e-12)
    d = o.edge_derivative(x, coef, basis, 0, W)
    np.testing.assert_allclose(d.sum(-1) + b, y, atol=1e-12)


def test_bf16_rounding_matches_torch():
    torch = pytest.importorskip("torch")
    v = rng.normal(0, 3, 1000)
    want = torch.tensor(v, dtype=torch.float32).to(torch.bfloat16).double().numpy()
    np.testing.assert_array_equal(o.round_bf16(v), want)


def test_planted_mistakes_fail():
    """Plausible mistakes in the oracle's formulas are caught by the pins above."""
    data = np.load(os.path.join(GOLDEN, "bspline_scipy.npz"))
    grid, k, x, vals = (data[f"u5k3__{f}"] for f in ("grid", "k", "x", "values"))
    t = o.extend_grid(grid, int(k))
    # closed interval instead of half-open changes values at the knots
    closed = ((x[:, None] >= t[:-1]) & (x[:, None] <= t[1:])).astype(float)
    assert not np.allclose(closed, BSpline.design_matrix(x, t, 0).toarray())
    # a dropped tanh chain factor fails the closed-form derivative
    fam = np.load(os.path.join(GOLDEN, "families_scipy.npz"))
    z = fam["z"]
    wrong = fam["chebyshev_dz"]  # without (1 - z^2)
    assert not np.allclose(o.polynomial_basis(np.arctanh(z), np.eye(9), "tanh", 1), wrong, atol=1e-6)
    # a transposed coefficient operand fails the brute-force loop check
    basis, xx, c, g, w = tiny()
    assert not np.allclose(o.prim_F(xx, c[::-1], w, basis, 0), o.prim_F(xx, c, w, basis, 0))


def test_symbolic_edges_follow_the_function_table():
    """Each code's function at a defining point, the affine maps inside and outside, zeros on the
    other edges, and the table order of the reference's library (codes are stored in models)."""
    names = [n for n, _ in o.SYMBOLIC]
    assert names[:5] == ["0", "x", "x^2", "x^3", "x^4"] and names[11] == "sin" and names[-1] == "arctan"
    at = {"0": (2.0, 0.0), "x": (2.0, 2.0), "x^2": (3.0, 9.0), "x^3": (2.0, 8.0), "x^4": (2.0, 16.0), "1/x": (4.0, 0.25),
          "1/x^2": (2.0, 0.25), "sqrt": (4.0, 2.0), "1/sqrt": (4.0, 0.5), "exp": (0.0, 1.0), "log": (np.e, 1.0),
          "sin": (np.pi / 2, 1.0), "cos": (0.0, 1.0), "tanh": (0.0, 0.0), "sigmoid": (0.0, 0.5), "gaussian": (0.0, 1.0),
          "abs": (-3.0, 3.0), "arctan": (1.0, np.pi / 4)}
    for k, name in enumerate(names):
        u, want = at[name]
        code = np.array([[k, -1]])
        params = np.array([[[2.0, u - 2.0 * 0.5, 3.0, -1.0], [1, 0, 1, 0]]])  # a x + b = u at x = 0.5
        d = o.symbolic_edges(np.array([[0.5, 0.7]]), code, params)
        assert np.isclose(d[0, 0, 0], 3.0 * want - 1.0), name
        assert d[0, 0, 1] == 0.0


# --- lookup tables (kanforge/export/lut.py) ---------------------------------------------------


def _linear_tables(rng, n_in=3, size=17, n_out=4):
    lo = rng.uniform(-2, -0.5, n_in)
    hi = rng.uniform(0.5, 2, n_in)
    a, b = rng.normal(size=(n_in, n_out)), rng.normal(size=(n_in, n_out))
    pts = lo[:, None] + (hi - lo)[:, None] * np.linspace(0, 1, size)[None, :]  # (in, size)
    return lo, hi, a, b, a[:, None, :] + b[:, None, :] * pts[..., None]


def test_lut_reproduces_linear_edges_inside_and_outside():
    """A table of linear edges a + b x is reproduced exactly by the lerp inside the range and,
    with its own end slopes (b times the step, per index step), by linear extrapolation outside."""
    rng = np.random.default_rng(0)
    lo, hi, a, b, T = _linear_tables(rng)
    bias = rng.normal(size=4)
    x = rng.uniform(-4, 4, (200, 3))
    s_lo, s_hi = o.lut_end_slopes(T)
    step = (hi - lo) / (T.shape[1] - 1)
    np.testing.assert_allclose(s_lo, b * step[:, None], rtol=1e-12)
    got = o.lut_layer(x, T, lo, hi, bias, slope_lo=s_lo, slope_hi=s_hi)
    want = (a[None] + b[None] * x[..., None]).sum(1) + bias
    np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-10)


def test_lut_hits_table_values_and_clamps():
    rng = np.random.default_rng(1)
    n_in, size, n_out = 2, 9, 3
    T = rng.normal(size=(n_in, size, n_out))
    lo, hi = np.array([-1.0, 0.5]), np.array([1.0, 2.5])
    s = np.array([[0, 8], [3, 5], [8, 0]])  # table indices per row and input
    x = lo + s * (hi - lo) / (size - 1)
    got = o.lut_layer(x, T, lo, hi, np.zeros(n_out), extrapolate="clamp")
    want = np.stack([T[0, s[r, 0]] + T[1, s[r, 1]] for r in range(3)])
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    far = o.lut_layer(np.array([[50.0, -50.0]]), T, lo, hi, np.zeros(n_out), extrapolate="clamp")
    np.testing.assert_allclose(far[0], T[0, -1] + T[1, 0], rtol=1e-12)


def test_lut_quantize_error_bound():
    """Dequantised entries are within half a step of the float tables, so a row's sum over n_in
    inputs is within n_in scale / 2 per output."""
    rng = np.random.default_rng(2)
    T = rng.normal(size=(5, 33, 4)) * np.array([1.0, 0.1, 3.0, 0.0])
    bias = rng.normal(size=4)
    for bits in (8, 12):
        q, scale, bias_q = o.lut_quantize(T, bias, bits)
        assert q.dtype == (np.int8 if bits <= 8 else np.int16)
        assert np.abs(q).max() <= 2 ** (bits - 1) - 1
        centre = 0.5 * (T.max(1) + T.min(1))
        deq = centre[:, None, :] + scale * q
        assert np.all(np.abs(deq - T) <= scale / 2 + 1e-12)
        np.testing.assert_allclose(bias_q, bias + centre.sum(0))
        x = rng.uniform(-1, 1, (50, 5))
        lo, hi = -np.ones(5), np.ones(5)
        yq = o.lut_layer(x, q, lo, hi, bias_q, scale=scale, extrapolate="clamp")
        yf = o.lut_layer(x, T, lo, hi, bias, extrapolate="clamp")
        assert np.all(np.abs(yq - yf) <= 5 * scale / 2 + 1e-9)
