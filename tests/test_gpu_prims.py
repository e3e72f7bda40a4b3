"""Parity of the HIP primitives (through the C ABI) with the float64 oracle.

Every case feeds the device and the oracle the same seeded, dtype-rounded
inputs. Tolerances (normwise max|d|/max|ref|): float32 1e-5, bfloat16 2e-2;
B-spline interval indices bit-exact.
"""

import math

import numpy as np
import pytest
import torch

import kanforge_amd as kf
from cases import BASES, oracle_basis, random_grid, rounded, to_dev
from kanforge_amd.kernels import plan_for
from kanforge_amd.torch import kernels as K
from oracle import kan64 as o

pytestmark = pytest.mark.gpu
DEV = "cuda"

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}
DTYPES = [torch.float32, torch.bfloat16]
SHAPES = [(150, 45, 70), (256, 64, 128), (300, 265, 40)]  # ragged, aligned, several input tiles


def setup(name, B, IN, seed=0):
    rng = np.random.default_rng(seed)
    basis = BASES[name]
    plan = plan_for(basis)
    params, st = None, None
    if plan.kind == "bspline":
        grid = random_grid(IN, basis.grid_size + 1, rng)
        params = {"grid": grid}
        st = K.bspline_state(torch.as_tensor(grid, device="cuda"), basis.order)
        x = rng.uniform(-1.15, 1.15, (B, IN))
    elif plan.kind == "rational":
        groups = math.gcd(IN, 5) if IN % 5 == 0 else 1
        num = rounded(rng.normal(0, math.sqrt(0.1), (groups, 6)), torch.float32)
        den = rounded(rng.normal(0, math.sqrt(0.1), (groups, 4)), torch.float32)
        params = {"num": num, "den": den}
        st = K.rational_state(torch.as_tensor(num, device="cuda"), torch.as_tensor(den, device="cuda"), IN // groups)
        x = rng.normal(0, 1, (B, IN))
    else:
        x = rng.normal(0, 1, (B, IN)) * (0.6 if basis.input_map == "identity" else 1.0)
    return basis, plan, st, oracle_basis(basis, IN, params), x, rng


def err(got, want):
    return o.normwise_err(got.detach().float().cpu().double().numpy(), want)


PRIM_CASES = [
    ("chebyshev8", 0), ("chebyshev8", 1), ("chebyshev8", 2),
    ("legendre_identity", 0), ("legendre_identity", 1),
    ("jacobi6", 0), ("jacobi6", 2),
    ("gram", 1),
    ("bspline53", 0), ("bspline53", 1), ("bspline53", 3), ("bspline53", 4),
    ("bspline41", 0), ("bspline20", 0),
    ("rational", 0), ("rational", 1), ("rational", 2),
]  # fmt: skip


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16"])
@pytest.mark.parametrize("shape", SHAPES, ids=["ragged", "aligned", "wide"])
@pytest.mark.parametrize("name,m", PRIM_CASES)
def test_F_matches_oracle(name, m, shape, dtype):
    B, IN, OUT = shape
    basis, plan, st, ob, x, rng = setup(name, B, IN)
    Kb = basis.size
    c = rng.normal(0, 1 / math.sqrt(IN * Kb), (OUT, IN, Kb))
    for weighted in (False, True):
        w = rng.uniform(0.5, 1.5, (B, IN)) if weighted else None
        y = K._raw("F", plan, m, to_dev(x, dtype), None if w is None else to_dev(w, dtype), to_dev(c, dtype), st, OUT)
        want = o.prim_F(rounded(x, dtype), rounded(c, dtype), None if w is None else rounded(w, dtype), ob, m)
        e = err(y, want)
        assert e <= TOL[dtype], (name, m, weighted, e)


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16"])
@pytest.mark.parametrize("shape", SHAPES, ids=["ragged", "aligned", "wide"])
@pytest.mark.parametrize("name,m", PRIM_CASES)
def test_G_matches_oracle(name, m, shape, dtype):
    B, IN, OUT = shape
    basis, plan, st, ob, x, rng = setup(name, B, IN, seed=1)
    g = rng.normal(0, 1, (B, OUT))
    for weighted in (False, True):
        w = rng.uniform(0.5, 1.5, (B, IN)) if weighted else None
        dc = K._raw("G", plan, m, to_dev(x, dtype), None if w is None else to_dev(w, dtype), to_dev(g, dtype), st, OUT)
        want = o.prim_G(rounded(x, dtype), rounded(g, dtype), None if w is None else rounded(w, dtype), ob, m)
        assert dc.shape == want.shape
        e = err(dc, want)
        assert e <= TOL[dtype], (name, m, weighted, e)


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16"])
@pytest.mark.parametrize("shape", SHAPES, ids=["ragged", "aligned", "wide"])
@pytest.mark.parametrize("name,m", PRIM_CASES)
def test_P_matches_oracle(name, m, shape, dtype):
    B, IN, OUT = shape
    basis, plan, st, ob, x, rng = setup(name, B, IN, seed=2)
    Kb = basis.size
    c = rng.normal(0, 1 / math.sqrt(IN * Kb), (OUT, IN, Kb))
    g = rng.normal(0, 1, (B, OUT))
    p = K._raw("P", plan, m, to_dev(x, dtype), to_dev(g, dtype), to_dev(c, dtype), st, OUT)
    want = o.prim_P(rounded(x, dtype), rounded(g, dtype), rounded(c, dtype), ob, m)
    e = err(p, want)
    assert e <= TOL[dtype], (name, m, e)


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16"])
@pytest.mark.parametrize("name,m", PRIM_CASES + [("chebyshev8", 5), ("bspline83", 2)])
def test_features_match_oracle(name, m, dtype):
    basis, plan, st, ob, x, rng = setup(name, 97, 13, seed=3)
    phi = K._features_raw(plan, m, st, to_dev(x, dtype))
    want = ob(rounded(x, dtype), m)
    assert phi.shape == want.shape
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert err(phi, want) <= tol


@pytest.mark.parametrize("name", ["bspline53", "bspline83", "bspline41", "bspline20"])
def test_bspline_interval_bit_exact(name):
    rng = np.random.default_rng(4)
    basis = BASES[name]
    IN = 7
    grid = random_grid(IN, basis.grid_size + 1, rng, -0.8, 1.3)
    t = o.extend_grid(grid, basis.order)  # float64 knots (IN, nk)
    # points on, one float32 ulp around, and between every knot, plus far outside and NaN
    t32 = t.astype(np.float32)
    cols = [t32, np.nextafter(t32, np.float32(-np.inf)), np.nextafter(t32, np.float32(np.inf))]
    mids = ((t[:, 1:] + t[:, :-1]) / 2).astype(np.float32)
    far = np.tile(np.array([-1e6, 1e6, np.nan], np.float32), (IN, 1))
    xt = np.concatenate(cols + [mids, far], 1)  # (IN, n)
    x = np.ascontiguousarray(xt.T)  # (n, IN)
    st = K.bspline_state(torch.as_tensor(grid, device="cuda"), basis.order)
    got = K.bspline_interval(torch.as_tensor(x, device="cuda"), st.knots_cmp).cpu().numpy()
    want = np.stack([o.bspline_interval(x[:, i].astype(np.float64), t[i]) for i in range(IN)], 1)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16"])
@pytest.mark.parametrize("name,m", [("chebyshev8", 0), ("chebyshev8", 2), ("jacobi6", 2), ("bspline53", 1), ("rational", 1), ("legendre_identity", 2)])
@pytest.mark.parametrize("base", [False, True])
def test_edge_derivative_matches_oracle(name, m, base, dtype):
    B, IN, OUT = 83, 70, 9
    basis, plan, st, ob, x, rng = setup(name, B, IN, seed=5)
    c = rng.normal(0, 0.5, (OUT, IN, basis.size))
    bw = rng.normal(0, 0.5, (OUT, IN)) if base else None
    d = K._edge_raw(plan, m, st, to_dev(x, dtype), to_dev(c, dtype), None if bw is None else to_dev(bw, dtype))
    want = o.edge_derivative(rounded(x, dtype), rounded(c, dtype), ob, m, None if bw is None else rounded(bw, dtype))
    assert d.shape == want.shape
    assert err(d, want) <= TOL[dtype]


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16"])
@pytest.mark.parametrize("name,m", [("bspline53", 0), ("bspline83", 1), ("bspline41", 0), ("rational", 0), ("rational", 1)])
def test_F_many_tiles(name, m, dtype):
    """Unweighted B-spline and rational F over at least half a round of 256 x 256 tiles take
    the flat GEMM route (features in (B, in K) layout times coef^T); ragged batch and outputs."""
    B, IN, OUT = 4000, 64, 2100
    basis, plan, st, ob, x, rng = setup(name, B, IN, seed=12)
    c = rng.normal(0, 1 / math.sqrt(IN * basis.size), (OUT, IN, basis.size))
    y = K._raw("F", plan, m, to_dev(x, dtype), None, to_dev(c, dtype), st, OUT)
    want = o.prim_F(rounded(x, dtype), rounded(c, dtype), None, ob, m)
    assert y.shape == want.shape
    assert err(y, want) <= TOL[dtype]


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16"])
@pytest.mark.parametrize("name,m", [("bspline53", 0), ("bspline83", 1)])
def test_G_many_output_tiles(name, m, dtype):
    """Grids of at least two rounds of tiles take G's unsplit B-spline route (a flat GEMM
    over the precomputed features); the small shapes above take the batch-split route."""
    B, IN, OUT = 80, 2050, 1030
    basis, plan, st, ob, x, rng = setup(name, B, IN, seed=11)
    g = rng.normal(0, 1, (B, OUT))
    w = rng.uniform(0.5, 1.5, (B, IN))
    for wt in (None, w):
        dc = K._raw("G", plan, m, to_dev(x, dtype), None if wt is None else to_dev(wt, dtype), to_dev(g, dtype), st, OUT)
        want = o.prim_G(rounded(x, dtype), rounded(g, dtype), None if wt is None else rounded(wt, dtype), ob, m)
        assert dc.shape == want.shape
        assert err(dc, want) <= TOL[dtype], (name, m, wt is None)


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16"])
@pytest.mark.parametrize("name,m", [("jacobi6", 2), ("bspline53", 1), ("rational", 1)])
@pytest.mark.parametrize("shape", [(70, 2, 64), (70, 64, 1), (33, 3, 5), (40, 1, 1)], ids=["2to64", "64to1", "3to5", "1to1"])
def test_edge_derivative_narrow_layers(shape, name, m, dtype):
    """Layers narrower than a half-wave in inputs or outputs (the PINN's first and last layers)."""
    B, IN, OUT = shape
    basis, plan, st, ob, x, rng = setup(name, B, IN, seed=7)
    c = rng.normal(0, 0.5, (OUT, IN, basis.size))
    bw = rng.normal(0, 0.5, (OUT, IN))
    d = K._edge_raw(plan, m, st, to_dev(x, dtype), to_dev(c, dtype), to_dev(bw, dtype))
    want = o.edge_derivative(rounded(x, dtype), rounded(c, dtype), ob, m, rounded(bw, dtype))
    assert d.shape == want.shape
    assert err(d, want) <= TOL[dtype]


def test_rational_param_grad_matches_oracle():
    B, IN, OUT = 300, 40, 24
    basis, plan, st, ob, x, rng = setup("rational", B, IN, seed=6)
    c = rng.normal(0, 0.3, (OUT, IN, 1))
    g = rng.normal(0, 1, (B, OUT))
    w = rng.uniform(0.5, 1.5, (B, IN))
    xd = to_dev(x, torch.float32)
    h = torch.empty(B, IN, dtype=torch.float32, device="cuda")
    K._raw("P", plan, 1, xd, to_dev(g, torch.float32), to_dev(c, torch.float32), st, OUT, h=h)
    hw = np.einsum("bo,oi->bi", rounded(g, torch.float32), rounded(c, torch.float32)[..., 0])
    assert o.normwise_err(h.cpu().double().numpy(), hw) <= 1e-5
    dnum, dden = K._rational_param_grad(plan, st, xd, h, to_dev(w, torch.float32))
    xr = rounded(x, torch.float32)
    gn, gd = o.rational_param_grads(xr, ob.kw["num"], ob.kw["den"])
    wr = rounded(w, torch.float32)
    groups = st.num.shape[0]
    want_n = np.einsum("bi,bij->ij", hw * wr, gn).reshape(groups, -1, gn.shape[-1]).sum(1)
    want_d = np.einsum("bi,bij->ij", hw * wr, gd).reshape(groups, -1, gd.shape[-1]).sum(1)
    assert o.normwise_err(dnum.cpu().double().numpy(), want_n) <= 1e-5
    assert o.normwise_err(dden.cpu().double().numpy(), want_d) <= 1e-5


@pytest.mark.parametrize("m", [1, 2, 3])
def test_rational_param_grad_of_derivative_features_matches_finite_differences(m):
    """d/dtheta of sum_{b,i} h w phi^(m)(x) (the parameter gradients a gradient penalty needs)
    against central differences of the oracle's float64 phi^(m) in each of the group's ten
    parameters."""
    B, IN = 200, 40
    basis, plan, st, ob, x, rng = setup("rational", B, IN, seed=7 + m)
    h = rng.normal(0, 1, (B, IN))
    w = rng.uniform(0.5, 1.5, (B, IN))
    xd = to_dev(x, torch.float32)
    dnum, dden = K._rational_param_grad(plan, st, xd, to_dev(h, torch.float32), to_dev(w, torch.float32), m)
    xr, hr, wr = rounded(x, torch.float32), rounded(h, torch.float32), rounded(w, torch.float32)
    num, den = st.num.double().cpu().numpy(), st.den.double().cpu().numpy()
    groups, gs = num.shape[0], IN // num.shape[0]

    def total(nm, dn):
        phi = o.rational_basis(xr, np.repeat(nm, gs, 0), np.repeat(dn, gs, 0), m)[..., 0]
        return (hr * wr * phi).reshape(B, groups, gs).sum((0, 2))  # per group

    want_n, want_d = np.zeros_like(num), np.zeros_like(den)
    for arr, want in ((num, want_n), (den, want_d)):
        for j in range(arr.shape[1]):
            eps = 1e-6
            up, dn_ = arr.copy(), arr.copy()
            up[:, j] += eps
            dn_[:, j] -= eps
            args_up = (up, den) if arr is num else (num, up)
            args_dn = (dn_, den) if arr is num else (num, dn_)
            want[:, j] = (total(*args_up) - total(*args_dn)) / (2 * eps)
    assert o.normwise_err(dnum.cpu().double().numpy(), want_n) <= 1e-4
    assert o.normwise_err(dden.cpu().double().numpy(), want_d) <= 1e-4


def test_zero_batch_and_errors():
    basis, plan, st, ob, x, rng = setup("chebyshev8", 4, 8)
    xd = torch.zeros(0, 8, device="cuda")
    c = torch.randn(5, 8, 9, device="cuda")
    y = K._raw("F", plan, 0, xd, None, c, st, 5)
    assert y.shape == (0, 5)
    dc = K._raw("G", plan, 0, xd, None, torch.zeros(0, 5, device="cuda"), st, 5)
    assert dc.shape == (5, 8, 9) and float(dc.abs().max()) == 0.0
    with pytest.raises(TypeError):
        K._raw("F", plan, 0, torch.zeros(3, 8, device="cuda", dtype=torch.float16), None, c.half(), st, 5)
    with pytest.raises(NotImplementedError):
        K._raw("F", plan, 9, torch.zeros(3, 8, device="cuda"), None, c, st, 5)


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16"])
def test_bspline_nonfinite_and_outside_inputs(dtype):
    # NaN / inf propagate NaN through the recurrence; finite points outside the
    # extended grid give zeros (kanforge/bases/spline.py:74-92 arithmetic)
    basis, plan, st, ob, x, rng = setup("bspline53", 4, 3, seed=7)
    xs = np.array([[np.nan, np.inf, -np.inf], [-50.0, 50.0, 0.1], [0.2, np.nan, 0.3], [0.0, 0.0, 0.0]])
    phi = K._features_raw(plan, 0, st, torch.as_tensor(xs, dtype=torch.float32).to("cuda", dtype)).float().cpu().numpy()
    want = ob(rounded(xs, dtype), 0)
    np.testing.assert_array_equal(np.isnan(phi), np.isnan(want))
    finite = ~np.isnan(want)
    np.testing.assert_allclose(phi[finite], want[finite], atol=2e-2 if dtype == torch.bfloat16 else 1e-6)


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16"])
def test_bspline_nonfinite_and_outside_inputs_through_F_P_G(dtype):
    """Rows with a NaN or infinite input give NaN wherever the dense float64 contraction does (F:
    the row's outputs; P: that input; G: every feature of that input), points outside the grid
    contribute nothing; the rest matches the oracle (float32 layers run the sparse k + 1 route)."""
    B, IN, OUT = 70, 5, 9
    basis, plan, st, ob, x, rng = setup("bspline53", B, IN, seed=11)
    x[3, 1], x[10, 4], x[20, 0], x[21, 2], x[30, 3] = np.nan, np.inf, -np.inf, -50.0, 50.0
    c = rng.normal(0, 0.3, (OUT, IN, basis.size))
    g = rng.normal(0, 1, (B, OUT))
    w = rng.uniform(0.5, 1.5, (B, IN))
    xd, cd, gd, wd = (to_dev(a, dtype) for a in (x, c, g, w))
    xr, cr, gr, wr = (rounded(a, dtype) for a in (x, c, g, w))
    atol = 2e-2 if dtype == torch.bfloat16 else 1e-5
    for got, want in (
        (K._raw("F", plan, 0, xd, wd, cd, st, OUT), o.prim_F(xr, cr, wr, ob, 0)),
        (K._raw("P", plan, 1, xd, gd, cd, st, OUT), o.prim_P(xr, gr, cr, ob, 1)),
        (K._raw("G", plan, 0, xd, wd, gd, st, OUT), o.prim_G(xr, gr, wr, ob, 0)),
    ):
        got = got.float().cpu().double().numpy()
        np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
        fin = ~np.isnan(want)
        scale = max(1.0, np.abs(want[fin]).max())
        np.testing.assert_allclose(got[fin], want[fin], rtol=0, atol=atol * scale)


@pytest.mark.parametrize("k,m", [(3, 0), (3, 1), (3, 2), (2, 0), (1, 1), (0, 0)])
def test_uniform_grid_features_equal_the_general_path(k, m):
    """The even-knot fast path (constant-time interval estimate checked against the ceil32 table,
    de Boor in the normalised coordinate) gives the general path's features at, one ulp around and
    between every knot, and outside the extended grid."""
    G, IN = 8, 3
    grid = np.stack([np.linspace(-1, 1, G + 1), np.linspace(-0.3, 2.1, G + 1), np.linspace(-5, -2, G + 1)])
    basis = kf.BSpline(G, k)
    plan = plan_for(basis)
    st = K.bspline_state(torch.as_tensor(grid, device=DEV), k)
    assert st.knots_u is not None
    general = K.BasisState(knots=st.knots, knots_cmp=st.knots_cmp)
    t = o.extend_grid(grid, k).astype(np.float32)  # (IN, nk)
    pts = []
    for row in t.T:
        for v in row:
            pts += [np.nextafter(v, np.float32(-np.inf)), v, np.nextafter(v, np.float32(np.inf))]
    mids = (t[:, 1:] + t[:, :-1]) / 2
    cols = np.array(pts, dtype=np.float32).reshape(-1, IN)
    x = np.concatenate([cols, mids.T, t[:, :1].T - 1.0, t[:, -1:].T + 1.0]).astype(np.float32)
    xd = torch.as_tensor(x, device=DEV)
    fast = K._features_raw(plan, m, st, xd).cpu().double().numpy()
    slow = K._features_raw(plan, m, general, xd).cpu().double().numpy()
    scale = max(1.0, np.abs(slow).max())
    np.testing.assert_allclose(fast, slow, rtol=0, atol=2e-6 * scale)
    want = o.Basis64("bspline", grid=grid, k=k)(x.astype(np.float64), m)
    np.testing.assert_allclose(fast, want, rtol=0, atol=1e-5 * max(1.0, np.abs(want).max()))


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16"])
@pytest.mark.parametrize("shape", [(2048, 2, 64), (1500, 64, 1), (1300, 3, 40), (1100, 17, 5), (1024, 4, 70),
                                   (1200, 8, 3), (1100, 100, 1), (1030, 96, 8), (1024, 200, 2)],
                         ids=["2to64", "64to1", "3to40", "17to5", "4to70", "8to3", "100to1", "96to8", "200to2"])
@pytest.mark.parametrize("name,m", [("jacobi6", 0), ("jacobi6", 1), ("jacobi6", 2), ("chebyshev5", 1), ("bspline53", 0), ("bspline53", 2)])
def test_F_narrow_layers_stream_and_match_oracle(name, m, shape, dtype):
    """Layers with at most 8 outputs or at most 4 inputs stream rows: Chebyshev-family layers with
    at most 8 outputs and 128 inputs one lane per (row, input) with 16 or 64 lanes per row and one
    or two inputs per lane, the rest one thread per row with the fold in registers; weighted and
    unweighted, against the oracle."""
    B, IN, OUT = shape
    basis, plan, st, ob, x, rng = setup(name, B, IN)
    Kb = basis.size
    c = rng.normal(0, 1 / math.sqrt(IN * Kb), (OUT, IN, Kb))
    for weighted in (False, True):
        w = rng.uniform(0.5, 1.5, (B, IN)) if weighted else None
        y = K._raw("F", plan, m, to_dev(x, dtype), None if w is None else to_dev(w, dtype), to_dev(c, dtype), st, OUT)
        want = o.prim_F(rounded(x, dtype), rounded(c, dtype), None if w is None else rounded(w, dtype), ob, m)
        e = err(y, want)
        assert e <= TOL[dtype], (name, m, weighted, e)
