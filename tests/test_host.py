"""Host-side logic without a GPU: plans and fold matrices, knot tables,
parameter layout and state_dict names, error behaviour, the C ABI library
(loads, exports every declared symbol, validates arguments before any
launch), and the CPU baseline route."""

import ctypes
import math
import os
import re

import numpy as np
import pytest
import torch

import kanforge_amd as kf
from kanforge_amd.bases.spline import ceil_f32, knot_tables
from kanforge_amd.kernels import plan_for
from kanforge_amd.torch import GRKAN, KAN, KANLinear
from kanforge_amd.torch import _lib
from oracle import kan64 as o

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
rng = np.random.default_rng(0)


# --- plans and fold matrices ------------------------------------------------------


@pytest.mark.parametrize(
    "basis,name,kw",
    [
        (kf.Chebyshev(8), "chebyshev", {}),
        (kf.Jacobi(6, 0.5, 0.5), "jacobi", {"alpha": 0.5, "beta": 0.5}),
        (kf.Legendre(4, input_map="identity"), "legendre", {}),
        (kf.Gegenbauer(5, 0.75), "gegenbauer", {"lam": 0.75}),
        (kf.Taylor(3), "taylor", {}),
    ],
)
@pytest.mark.parametrize("m", [0, 1, 2, 3])
def test_plan_fold_matches_oracle(basis, name, kw, m):
    plan = plan_for(basis)
    assert plan.kind == "cheb" and plan.size == basis.size
    A = o.cheb_coefficients(name, basis.degree, **kw)
    np.testing.assert_allclose(basis._cheb, A, atol=1e-12)
    np.testing.assert_allclose(plan.fold(m), o.fold_matrix(A, basis.input_map, m), atol=1e-12)
    assert plan.n_features(m) == plan.fold(m).shape[1]


@pytest.mark.parametrize("basis", [kf.Chebyshev(8), kf.Jacobi(6, 0.5, 0.5), kf.Chebyshev(0), kf.Gegenbauer(5, 0.75)])
@pytest.mark.parametrize("m", [0, 1, 2, 3, 5])
def test_device_fold_equals_reference_fold(basis, m):
    """What the kernels evaluate: for tanh maps and m >= 1, R_m with (1 - z^2) divided out and the
    features weighted by (1 - z^2) (two features fewer); it must reproduce R_m's polynomials."""
    plan = plan_for(basis)
    r, (rd, factored) = plan.fold(m), plan.device_fold(m)
    assert factored == (m >= 1)
    if factored:
        assert rd.shape == (basis.size, max(1, basis.degree + m - 1))
    z = np.linspace(-0.999, 0.999, 41)
    want = np.polynomial.chebyshev.chebval(z, r.T)
    got = np.polynomial.chebyshev.chebval(z, rd.T) * ((1 - z * z) if factored else 1.0)
    np.testing.assert_allclose(got, want, atol=1e-9 * max(1.0, np.abs(want).max()))


def test_plans_for_every_kind():
    assert plan_for(kf.BSpline(8, 3)).kind == "bspline" and plan_for(kf.BSpline(8, 3)).size == 11
    assert plan_for(kf.Rational(5, 4)).kind == "rational"
    assert plan_for(kf.Gram(4)).kind == "cheb"
    with pytest.raises(ValueError):
        kf.Chebyshev(4, input_map="fractional")


def test_gram_coefficients_orthonormal():
    b = kf.Gram(4)
    grid = np.linspace(-1, 1, b.points)
    v = b.host_values(np.arctanh(np.clip(grid, -0.999999, 0.999999)))  # tanh map undone
    gram = v.T @ v / b.points
    np.testing.assert_allclose(gram, np.eye(5), atol=1e-4)


# --- knot tables --------------------------------------------------------------------


def test_ceil32_comparisons_are_exact():
    t = np.sort(rng.uniform(-2, 2, 50)) + rng.uniform(-1e-9, 1e-9, 50)
    c = ceil_f32(t)
    assert (c.astype(np.float64) >= t).all()
    assert (np.nextafter(c, np.float32(-np.inf)).astype(np.float64) < t).all()  # smallest such float32
    x = np.concatenate([t.astype(np.float32), np.nextafter(t.astype(np.float32), np.float32(np.inf)), rng.uniform(-2, 2, 500).astype(np.float32)])
    for tk, ck in zip(t, c):
        np.testing.assert_array_equal(x.astype(np.float64) >= tk, x >= ck)


def test_knot_tables_layout():
    grid = np.stack([np.linspace(-1, 1, 9), np.linspace(-0.5, 2, 9)])
    pad, cmp_ = knot_tables(grid, 3)
    t = o.extend_grid(grid, 3)
    assert cmp_.shape == (2, 15) and pad.shape == (2, 21)
    np.testing.assert_allclose(pad[:, 3:-3], t.astype(np.float32))
    assert (np.diff(pad, axis=1) > 0).all()  # padding knots keep the table strictly increasing


# --- layer layout and errors -----------------------------------------------------------


def test_kanlinear_parameter_layout_matches_reference():
    layer = KANLinear(5, 3, kf.BSpline(5, 3), edge_scale=True)
    names = dict(layer.named_parameters())
    assert set(names) == {"coef", "base_weight", "bias", "edge_scale"}
    assert layer.coef.shape == (3, 5, 8) and layer.base_weight.shape == (3, 5) and layer.bias.shape == (3,)
    sd = layer.state_dict()
    assert set(sd) == {"coef", "base_weight", "bias", "edge_scale", "edge_mask", "sym_code", "sym_params", "basis_grid"}
    assert sd["basis_grid"].shape == (5, 6) and sd["sym_code"].dtype == torch.int32
    cheb = KANLinear(3, 2, "chebyshev", base_activation=None, bias=False)
    assert set(dict(cheb.named_parameters())) == {"coef"}


def test_grkan_layout_and_init():
    torch.manual_seed(0)
    layer = GRKAN(64, 64, groups=8)
    assert layer.base_weight is None
    assert layer.basis_numerator.shape == (8, 6) and layer.basis_denominator.shape == (8, 4)
    # coef_init "variance": std = 1 / sqrt(in * E[phi^2]) for x ~ N(0, 1)
    x, w = np.polynomial.hermite_e.hermegauss(96)
    m2 = float((w / math.sqrt(2 * math.pi)) @ layer.basis.host_values(x)[:, 0] ** 2)
    assert abs(layer.coef.std().item() - 1 / math.sqrt(64 * m2)) < 0.01
    z = np.linspace(-3, 3, 301)
    gelu = 0.5 * z * (1 + np.vectorize(math.erf)(z / math.sqrt(2)))
    assert np.abs(layer.basis.host_values(z)[:, 0] - gelu).max() < 2e-2  # rationals start as GELU


def test_errors_and_backend_selection():
    with pytest.raises(ValueError):
        KANLinear(3, 2, backend="fast")
    with pytest.raises(ValueError, match="must divide"):
        KANLinear(5, 2, "rational", groups=2)
    with pytest.raises(ValueError):
        KANLinear(3, 2, edge_dropout=1.0)
    with pytest.raises(RuntimeError, match="ROCm|device"):
        KANLinear(3, 2, "chebyshev")(torch.zeros(1, 3))  # CPU tensors: no silent fallback
    with pytest.raises(RuntimeError, match="ops"):
        KANLinear(3, 2, "chebyshev", backend="ops")(torch.zeros(1, 3))
    with pytest.raises(ValueError):
        KAN([3])
    with pytest.raises(ValueError, match="unknown basis"):
        kf.make_basis("nope")
    assert kf.make_basis(kf.Chebyshev(4).config()) == kf.Chebyshev(4)


# --- the C ABI ------------------------------------------------------------------------


def declared_symbols():
    header = open(os.path.join(ROOT, "include", "kfhip.h")).read()
    header = re.sub(r"/\*.*?\*/", "", header, flags=re.S)
    return sorted(set(re.findall(r"\b(kf_[A-Za-z_0-9]+)\s*\(", header)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    syms = declared_symbols()
    assert "kf_F" in syms and "kf_G" in syms and "kf_P" in syms
    for name in syms:
        assert hasattr(lib, name), name
    assert set(syms) == set(_lib.EXPORTS)
    assert _lib.load().kf_version().decode().startswith("kfhip")


def test_abi_struct_matches_header():
    header = open(os.path.join(ROOT, "include", "kfhip.h")).read()
    body = header[header.index("typedef struct kf_basis") : header.index("} kf_basis;")]
    fields = re.findall(r"\b(?:int32_t|const float \*)\s*([a-z_]+);", body)
    assert fields == [f for f, _ in _lib.KfBasis._fields_]
    for name in ("KF_F32", "KF_BF16", "KF_KIND_CHEB", "KF_KIND_BSPLINE", "KF_KIND_RATIONAL", "KF_MAX_K", "KF_MAX_NT"):
        value = int(re.search(rf"#define {name} (-?\d+)", header).group(1))
        assert getattr(_lib, name) == value, name


def test_abi_rejects_bad_arguments_without_launching():
    lib = _lib.load()
    b = _lib.KfBasis()
    rc = lib.kf_F(None, 0, 4, 4, 4, None, None, None, None, None, 0, None)
    assert rc == -1 and b"NULL" in lib.kf_last_error()
    b.kind, b.size, b.order, b.n_t = _lib.KF_KIND_CHEB, 9, 0, 9
    rc = lib.kf_F(ctypes.byref(b), 0, 4, 4, 4, None, None, None, None, None, 0, None)
    assert rc == -1 and b"fold" in lib.kf_last_error()
    fold = np.eye(9, dtype=np.float32)
    b.fold = fold.ctypes.data_as(ctypes.c_void_p)
    rc = lib.kf_F(ctypes.byref(b), 7, 4, 4, 4, None, None, None, None, None, 0, None)
    assert rc == -1 and b"dtype" in lib.kf_last_error()
    rc = lib.kf_F(ctypes.byref(b), 1, 4, 4, 4, None, None, None, None, None, 0, None)
    assert rc == -1 and b"NULL" in lib.kf_last_error()
    b.order = 12
    assert lib.kf_G(ctypes.byref(b), 1, 4, 4, 4, None, None, None, None, None, 0, None) == -4
    b.order = 0
    assert lib.kf_workspace_bytes(0, ctypes.byref(b), 1, 8192, 768, 3072) > 0
    # a workspace that is too small is rejected before any launch
    rc = lib.kf_F(ctypes.byref(b), 1, 4, 4, 4, ctypes.c_void_p(256), None, ctypes.c_void_p(256), ctypes.c_void_p(256), ctypes.c_void_p(256), 1, None)
    assert rc == -2 and b"workspace" in lib.kf_last_error()
    b.kind, b.size, b.n_t, b.spline_k, b.n_knots = _lib.KF_KIND_BSPLINE, 8, 8, 3, 99
    rc = lib.kf_features(ctypes.byref(b), 0, 4, 4, None, None, None)
    assert rc == -1 and b"n_knots" in lib.kf_last_error()


def _needed_bytes(lib, fn, b, w):
    """The workspace size an entry point asks for, read from its error text (1-byte workspace)."""
    p = ctypes.c_void_p(256)
    if fn is lib.kf_F:  # (x, w, c, y)
        rc = fn(ctypes.byref(b), _lib.KF_BF16, 8192, 768, 3072, p, w, p, p, p, 1, None)
    else:  # kf_G: (x, g, w, dc)
        rc = fn(ctypes.byref(b), _lib.KF_BF16, 8192, 768, 3072, p, p, w, p, p, 1, None)
    assert rc == -2
    return int(re.search(rb"workspace of (\d+) bytes needed", lib.kf_last_error()).group(1))


@pytest.mark.parametrize("op", ["kf_F", "kf_G"])
def test_workspace_check_uses_the_layout_of_reduced_tanh_folds(op):
    """A reduced tanh fold (input map TANH_SQ) carries the (1 - z^2) weight even when w is NULL:
    the size check must ask for the weighted layout the kernels then carve."""
    lib = _lib.load()
    fn = getattr(lib, op)
    b = _lib.KfBasis()
    fold = np.ones((9, 8), dtype=np.float32)
    b.kind, b.size, b.order, b.n_t = _lib.KF_KIND_CHEB, 9, 1, 8
    b.fold = fold.ctypes.data_as(ctypes.c_void_p)
    b.input_map = _lib.KF_MAP_TANH_SQ
    unweighted_call = _needed_bytes(lib, fn, b, None)
    weighted_call = _needed_bytes(lib, fn, b, ctypes.c_void_p(256))
    assert unweighted_call == weighted_call
    assert unweighted_call <= lib.kf_workspace_bytes(_lib.KF_OP_F if op == "kf_F" else _lib.KF_OP_G, ctypes.byref(b), 1, 8192, 768, 3072)
    b.input_map = _lib.KF_MAP_TANH  # a plain tanh map without w has the smaller unweighted layout
    assert _needed_bytes(lib, fn, b, None) < weighted_call


# --- CPU baseline route ------------------------------------------------------------


def test_cpu_baseline_route_matches_oracle():
    from oracle.torch_cpu import kan_step

    g = torch.Generator().manual_seed(0)
    x = torch.randn(16, 12, generator=g, dtype=torch.float64)
    coef = torch.randn(7, 12, 9, generator=g, dtype=torch.float64) * 0.1
    gy = torch.randn(16, 7, generator=g, dtype=torch.float64)
    y, gx, gc = kan_step(x, coef, gy, 8)
    ob = o.Basis64("poly", A=np.eye(9), input_map="tanh")
    xn, cn, gn = x.numpy(), coef.numpy(), gy.numpy()
    np.testing.assert_allclose(y.detach().numpy(), o.prim_F(xn, cn, None, ob, 0), atol=1e-12)
    np.testing.assert_allclose(gx.numpy(), o.prim_P(xn, gn, cn, ob, 1), atol=1e-12)
    np.testing.assert_allclose(gc.numpy(), o.prim_G(xn, gn, None, ob, 0), atol=1e-12)


def test_noalloc_F_rejects_shapes_beyond_its_static_scratch_before_any_launch():
    lib = _lib.load()
    b = _lib.KfBasis()
    fold = np.eye(9, dtype=np.float32)
    b.kind, b.size, b.order, b.n_t, b.input_map = _lib.KF_KIND_CHEB, 9, 0, 9, _lib.KF_MAP_TANH
    b.fold = fold.ctypes.data_as(ctypes.c_void_p)
    p = ctypes.c_void_p(256)
    rc = lib.kf_F_noalloc(ctypes.byref(b), _lib.KF_BF16, 8192, 768, 4096, p, p, p, p, None)
    assert rc == _lib.KF_EWORKSPACE and b"static scratch" in lib.kf_last_error()
    need = lib.kf_workspace_bytes(_lib.KF_OP_F, ctypes.byref(b), _lib.KF_BF16, 8192, 768, 4096)
    assert need > _lib.KF_NOALLOC_SCRATCH_BYTES


# --- the custom-op boundary (no GPU: plan keys and fake kernels) ---------------------------


@pytest.mark.parametrize("basis", [kf.Chebyshev(8), kf.Jacobi(6, 0.5, 0.5), kf.Legendre(4, input_map="identity"), kf.BSpline(8, 3), kf.Rational(5, 4)])
def test_plan_key_round_trip_is_exact(basis):
    from kanforge_amd.torch import kernels as K

    plan = plan_for(basis)
    key = K.plan_key(plan)
    assert K.plan_of(key) == plan and K.plan_key(key) is key


def test_custom_op_fake_kernels_give_shapes_on_meta_tensors():
    from kanforge_amd.torch import kernels as K

    key = K.plan_key(plan_for(kf.BSpline(8, 3)))
    x = torch.empty(33, 7, device="meta")
    c = torch.empty(5, 7, 11, device="meta")
    g = torch.empty(33, 5, device="meta")
    kn, kc, ku = torch.empty(7, 21, device="meta"), torch.empty(7, 15, device="meta"), torch.empty(7, 2, device="meta")
    assert torch.ops.kf.F(x, None, c, kn, kc, ku, None, None, key, 0).shape == (33, 5)
    assert torch.ops.kf.G(x, g, None, kn, kc, ku, None, None, key, 0).shape == (5, 7, 11)
    assert torch.ops.kf.P(x, g, c, kn, kc, None, None, None, key, 1).shape == (33, 7)
    assert torch.ops.kf.features(x, kn, kc, ku, None, None, key, 2).shape == (33, 7, 11)
    assert torch.ops.kf.edge_derivative(x, c, None, kn, kc, ku, None, None, key, 1).shape == (33, 5, 7)
    rkey = K.plan_key(plan_for(kf.Rational(5, 4)))
    num, den = torch.empty(7, 6, device="meta"), torch.empty(7, 4, device="meta")
    p, dn, dd = torch.ops.kf.rational_bwd(x, g, torch.empty(5, 7, 1, device="meta"), None, num, den, rkey, 0)
    assert p.shape == (33, 7) and dn.shape == (7, 6) and dd.shape == (7, 4)


def test_symbolic_table_and_functions_match_the_oracle():
    from kanforge_amd import symbolic as sym

    assert list(sym.NAMES) == [n for n, _ in o.SYMBOLIC]
    x = np.linspace(0.3, 2.5, 23)
    for k, (name, fn) in enumerate(o.SYMBOLIC):
        got = sym.function(k)(torch.as_tensor(x)).numpy()
        np.testing.assert_allclose(got, fn(x), rtol=1e-12, atol=1e-14, err_msg=name)
    layer = KANLinear(3, 2, kf.Chebyshev(3))
    layer.fix_symbolic(1, 0, "x^2", (1.0, 0.5, 2.0, 0.25))
    layer.fix_symbolic(0, 2, "sin", (2.0, 0.0, 1.0, 0.0))
    assert layer.symbolic_edges() == {(0, 2): ("sin", (2.0, 0.0, 1.0, 0.0)), (1, 0): ("x^2", (1.0, 0.5, 2.0, 0.25))}
    assert layer.edge_mask[1, 0] == 0 and layer.active_edges().all()
    layer.unfix_symbolic(1, 0)
    assert layer.symbolic_edges().keys() == {(0, 2)} and layer.edge_mask[1, 0] == 1
    with pytest.raises(ValueError, match="unknown symbolic"):
        layer.fix_symbolic(0, 0, "sinc")


def test_bases_beyond_the_kernel_limit_are_rejected_up_front():
    from kanforge_amd.kernels.plan import MAX_BASIS

    assert MAX_BASIS == _lib.KF_MAX_K
    with pytest.raises(ValueError, match="at most 16"):
        KANLinear(3, 2, kf.BSpline(20, 3))
    layer = KANLinear(3, 2, kf.BSpline(5, 3))
    before = layer.coef.detach().clone()
    with pytest.raises(ValueError, match="at most 16"):
        layer.refine_grid(20)
    assert torch.equal(layer.coef, before) and layer.basis.grid_size == 5  # untouched
    layer.refine_grid(13)  # 16 basis functions: the largest supported
    assert layer.coef.shape == (2, 3, 16)


def test_uniform_knot_table():
    from kanforge_amd.bases.spline import uniform_table

    grid = np.stack([np.linspace(-1, 1, 9), np.linspace(-0.5, 2, 9)])
    tab = uniform_table(grid, 3)
    t = o.extend_grid(grid, 3)
    np.testing.assert_allclose(tab[:, 0], t[:, 0].astype(np.float32))
    np.testing.assert_allclose(tab[:, 1], (1 / (t[:, 1] - t[:, 0])).astype(np.float32), rtol=1e-6)
    bent = grid.copy()
    bent[1, 4] += 1e-3  # one uneven input: the whole layer takes the general path
    assert uniform_table(bent, 3) is None
