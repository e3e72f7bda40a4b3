"""KANLinear with its SiLU base branch and bias fused into the HIP contractions (kf_F_base,
kf_P_base, kf_G_base), and F and G with the bias alone (kf_F_bias, kf_G_bias), against the float64
oracle: y and every first-order gradient on layers
whose three entries all fuse (Chebyshev degrees 8, 7 and 5: chunks of 9 features, and even counts
on the runtime-count F kernel) and on cubic B-spline layers, ragged shapes (inputs not a multiple of 16, outputs not of 8,
batch not of 64), the headline shape 768 -> 3072 at batch 8192 against a plain PyTorch float32
reference, double backward through the fused layer (its backward composes differentiable ops
there) against the unfused layer, the routes the library reports, and bitwise determinism.
Tolerance: bfloat16 normwise 2e-2.
"""

import math

import numpy as np
import pytest
import torch

import kanforge_amd as kf
from cases import oracle_basis, rounded
from kanforge_amd.torch import KANLinear
from kanforge_amd.torch import kernels as K
from oracle import kan64 as o

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16
TOL = 2e-2


def np64(t):
    return t.detach().float().cpu().double().numpy()


def make_layer(deg, IN, OUT, seed=0, edge_scale=False, bias=True):
    torch.manual_seed(seed)
    layer = KANLinear(IN, OUT, kf.Chebyshev(deg), edge_scale=edge_scale, bias=bias)
    with torch.no_grad():
        layer.coef.normal_(0, 0.5 / math.sqrt(IN))
        layer.base_weight.normal_(0, 1 / math.sqrt(IN))
        if edge_scale:
            layer.edge_scale.uniform_(0.5, 1.5)
        if bias:
            layer.bias.normal_()
    return layer.to(device=DEV, dtype=BF)


def make_spline_layer(IN, OUT, grid=8, seed=0, grid_range=(-3.0, 3.0)):
    torch.manual_seed(seed)
    layer = KANLinear(IN, OUT, kf.BSpline(grid, 3, grid_range=grid_range))
    with torch.no_grad():
        layer.coef.normal_(0, 0.5 / math.sqrt(IN))
        layer.base_weight.normal_(0, 1 / math.sqrt(IN))
        layer.bias.normal_()
    return layer.to(device=DEV, dtype=BF)


def unfused(layer):
    """The same layer on the unfused route (F, P, G plus torch base-branch ops)."""
    layer._base_fused = lambda x: False
    return layer


def test_routes_reported_by_the_library():
    plan = make_layer(8, 48, 8)._plan_key
    assert K.base_fused(plan, None, BF, 8192, 768, 3072) == (True, True, True)
    assert K.base_fused(plan, None, torch.float32, 8192, 768, 3072) == (False, False, False)
    assert not K.base_fused(plan, None, BF, 4096, 64, 4)[0]  # narrow: F's streaming route
    plan6 = make_layer(6, 48, 8)._plan_key  # 7 features a chunk: not fused
    assert not K.base_fused(plan6, None, BF, 8192, 768, 3072)[0]
    sp = make_spline_layer(768, 3072)  # cubic B-splines on 8 intervals: all three
    assert K.base_fused(sp._plan_key, sp._basis_state(), BF, 16384, 768, 3072) == (True, True, True)
    sp5 = make_spline_layer(768, 3072, grid=5)  # 8 basis functions: no spare slot in P's tile
    assert K.base_fused(sp5._plan_key, sp5._basis_state(), BF, 16384, 768, 3072) == (True, False, True)


# (batch, in, out, degree): every case has >= 128 G tiles of 192 x 48 (g96_kernel)
CASES = [
    (256, 3072, 384, 8),
    (333, 3000, 400, 8),  # ragged: in % 16, out % 8, batch % 64
    (200, 3072, 384, 7),  # 8 features a chunk (runtime count)
    (130, 3072, 384, 5),  # 6 features a chunk; P of order 1 not on p8 (composed)
]


@pytest.mark.parametrize("B,IN,OUT,deg", CASES)
def test_fused_layer_against_oracle(B, IN, OUT, deg):
    layer = make_layer(deg, IN, OUT, edge_scale=True)
    fused = K.base_fused(layer._plan_key, None, BF, B, IN, OUT)
    print(f"case B={B} in={IN} out={OUT} deg={deg} fused={fused}", flush=True)
    assert fused[0] and fused[2]
    assert fused[1] == (deg != 5)
    ob = oracle_basis(layer.basis, IN, None)
    rng = np.random.default_rng(B)
    x0 = rng.normal(0, 1, (B, IN))
    gy0 = rng.normal(0, 1, (B, OUT))
    x = torch.as_tensor(x0, dtype=torch.float32).to(DEV, BF).requires_grad_()
    gy = torch.as_tensor(gy0, dtype=torch.float32).to(DEV, BF)
    y = layer(x)
    y.backward(gy)
    torch.cuda.synchronize()
    xr, gyr = rounded(x0, BF), rounded(gy0, BF)
    c, s, W, b = np64(layer.coef), np64(layer.edge_scale), np64(layer.base_weight), np64(layer.bias)
    assert o.normwise_err(np64(y), o.kan_linear(xr, c, ob, W, b, s)) <= TOL
    ceff = c * s[..., None]
    G0 = o.prim_G(xr, gyr, None, ob, 0)
    checks = {
        "x": (x.grad, o.prim_P(xr, gyr, ceff, ob, 1) + (gyr @ W) * o.silu_derivative(xr, 1)),
        "coef": (layer.coef.grad, G0 * s[..., None]),
        "edge_scale": (layer.edge_scale.grad, (G0 * c).sum(-1)),
        "base_weight": (layer.base_weight.grad, gyr.T @ o.silu_derivative(xr, 0)),
        "bias": (layer.bias.grad, gyr.sum(0)),
    }
    for key, (got, want) in checks.items():
        err = o.normwise_err(np64(got), want)
        print(f"  {key}: {err:.3e}", flush=True)
        assert err <= TOL, (key, err)


@pytest.mark.parametrize("B,IN,OUT,grid", [(300, 768, 200, 8), (257, 136, 300, 8), (200, 96, 130, 5)])
def test_fused_bspline_layer_against_oracle(B, IN, OUT, grid):
    """Cubic B-splines: F with silu(x) and a ones column after each row's features, G with dW on
    the GEMM core, and on 8 intervals (11 basis functions, P's 12-slot tiles) P with W^T in the
    spare feature slot; the second shape is ragged, the third has 8 basis functions (P composed)."""
    layer = make_spline_layer(IN, OUT, grid)
    fused = K.base_fused(layer._plan_key, layer._basis_state(), BF, B, IN, OUT)
    print(f"B-spline case B={B} in={IN} out={OUT} grid={grid} fused={fused}", flush=True)
    assert fused == (True, grid == 8, True)
    ob = oracle_basis(layer.basis, IN, {"grid": np64(layer.basis_grid)})
    rng = np.random.default_rng(B)
    x0 = rng.normal(0, 1.2, (B, IN))
    gy0 = rng.normal(0, 1, (B, OUT))
    x = torch.as_tensor(x0, dtype=torch.float32).to(DEV, BF).requires_grad_()
    gy = torch.as_tensor(gy0, dtype=torch.float32).to(DEV, BF)
    y = layer(x)
    y.backward(gy)
    torch.cuda.synchronize()
    xr, gyr = rounded(x0, BF), rounded(gy0, BF)
    c, W, b = np64(layer.coef), np64(layer.base_weight), np64(layer.bias)
    checks = {
        "y": (y, o.kan_linear(xr, c, ob, W, b)),
        "x": (x.grad, o.prim_P(xr, gyr, c, ob, 1) + (gyr @ W) * o.silu_derivative(xr, 1)),
        "coef": (layer.coef.grad, o.prim_G(xr, gyr, None, ob, 0)),
        "base_weight": (layer.base_weight.grad, gyr.T @ o.silu_derivative(xr, 0)),
        "bias": (layer.bias.grad, gyr.sum(0)),
    }
    for key, (got, want) in checks.items():
        err = o.normwise_err(np64(got), want)
        print(f"  {key}: {err:.3e}", flush=True)
        assert err <= TOL, (key, err)


def test_headline_shape_with_base_and_bias():
    """768 -> 3072 Chebyshev(8), batch 8192: y, dX, dCoef, dW, db against float32 torch."""
    B, IN, OUT, KB = 8192, 768, 3072, 9
    torch.manual_seed(0)
    layer = KANLinear(IN, OUT, kf.Chebyshev(8), device=DEV, dtype=BF)
    with torch.no_grad():
        layer.coef.copy_(torch.randn(OUT, IN, KB, device=DEV) / math.sqrt(IN * KB))
        layer.bias.normal_()
    assert K.base_fused(layer._plan_key, None, BF, B, IN, OUT) == (True, True, True)
    x = torch.randn(B, IN, device=DEV).to(BF).requires_grad_()
    gy = torch.randn(B, OUT, device=DEV).to(BF)
    y = layer(x)
    dx, dc, dw, db = torch.autograd.grad(y, [x, layer.coef, layer.base_weight, layer.bias], gy)
    torch.cuda.synchronize()
    a = torch.as_tensor(np.asarray(layer.basis._cheb), dtype=torch.float32, device=DEV)
    xf, g32 = x.detach().float(), gy.float()
    z = torch.tanh(xf)
    t, dt = [torch.ones_like(z), z], [torch.zeros_like(z), torch.ones_like(z)]
    for j in range(2, KB):
        t.append(2 * z * t[j - 1] - t[j - 2])
        dt.append(2 * t[j - 1] + 2 * z * dt[j - 1] - dt[j - 2])
    phi = (torch.stack(t, -1) @ a).reshape(B, IN * KB)
    dphi = torch.stack(dt, -1) * (1 - z * z).unsqueeze(-1) @ a
    c2 = layer.coef.detach().float().reshape(OUT, IN * KB)
    W = layer.base_weight.detach().float()
    sx = torch.nn.functional.silu(xf)
    sig = torch.sigmoid(xf)
    dsx = sig * (1 + xf * (1 - sig))
    refs = {
        "y": (y, phi @ c2.t().contiguous() + sx @ W.t().contiguous() + layer.bias.detach().float()),
        "dx": (dx, (g32 @ c2).reshape(B, IN, KB).mul_(dphi).sum(-1) + (g32 @ W) * dsx),
        "dcoef": (dc, (g32.t().contiguous() @ phi).reshape(OUT, IN, KB)),
        "dbase_w": (dw, g32.t().contiguous() @ sx),
        "dbias": (db, g32.sum(0)),
    }
    for key, (got, want) in refs.items():
        err = ((got.float() - want).abs().max() / want.abs().max()).item()
        print(f"headline {key}: {err:.3e}", flush=True)
        assert torch.isfinite(got).all() and err < TOL, (key, err)


def test_double_backward_through_the_fused_layer():
    """Gradient penalty d/dtheta sum (dy/dx)^2: the fused layer's backward composes kf::P and
    torch ops under create_graph; the unfused layer gives the same values."""
    B, IN, OUT = 256, 3072, 384
    rng = np.random.default_rng(5)
    x0 = torch.as_tensor(rng.normal(0, 1, (B, IN)), dtype=torch.float32).to(DEV, BF)
    grads = []
    for fuse in (True, False):
        layer = make_layer(8, IN, OUT, seed=3)
        if not fuse:
            unfused(layer)
        x = x0.clone().requires_grad_()
        y = layer(x)
        (gx,) = torch.autograd.grad(y.float().sum(), x, create_graph=True)
        (gx.float() ** 2).sum().backward()
        grads.append([p.grad.detach().float().clone() for p in (layer.coef, layer.base_weight)] + [gx.detach().float()])
    torch.cuda.synchronize()
    for got, want in zip(*grads):
        err = ((got - want).abs().max() / want.abs().max()).item()
        assert err < TOL, err


def test_fused_calls_are_deterministic():
    B, IN, OUT = 1024, 768, 3072
    layer = make_layer(8, IN, OUT, seed=7)
    x = torch.randn(B, IN, device=DEV).to(BF).requires_grad_()
    gy = torch.randn(B, OUT, device=DEV).to(BF)
    outs = []
    for _ in range(2):
        y = layer(x)
        outs.append([y.detach()] + list(torch.autograd.grad(y, [x, layer.coef, layer.base_weight, layer.bias], gy)))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)


BIAS_CASES = [
    ("cheb8", kf.Chebyshev(8), torch.bfloat16, 300, 96, 200),  # register-A kernel: per-output constant
    ("bspline83", kf.BSpline(8, 3), torch.bfloat16, 257, 64, 130),  # GEMM core epilogue
    ("rational", kf.Rational(5, 4), torch.bfloat16, 300, 128, 96),  # GEMM core epilogue
    ("cheb8_f32", kf.Chebyshev(8), torch.float32, 77, 24, 19),  # one more pass
    ("bspline53_f32", kf.BSpline(5, 3), torch.float32, 4096, 64, 64),  # sparse route, one more pass
]


@pytest.mark.parametrize("name,basis,dtype,B,IN,OUT", BIAS_CASES, ids=[c[0] for c in BIAS_CASES])
def test_F_bias_is_F_plus_bias(name, basis, dtype, B, IN, OUT):
    """kf_F_bias against kf_F plus the bias in float32 (bf16: the fused routes add the bias before
    the one rounding, so within two bf16 roundings of it; float32 routes add it exactly)."""
    torch.manual_seed(1)
    layer = KANLinear(IN, OUT, basis, base_activation=None, groups=8 if name == "rational" else None).to(DEV, dtype)
    with torch.no_grad():
        layer.bias.normal_()
    x = torch.randn(B, IN, device=DEV).to(dtype) * 0.8
    st = layer._basis_state()
    num = den = None
    if layer._plan.kind == "rational":
        num, den = layer.basis_numerator, layer.basis_denominator
    with torch.no_grad():
        fused = K.spline_forward(x, layer.coef, st, layer._plan_key, num, den, bias=layer.bias)
        plain = K.spline_forward(x, layer.coef, st, layer._plan_key, num, den)
    torch.cuda.synchronize()
    want = plain.float() + layer.bias.float()
    if dtype == torch.float32:
        torch.testing.assert_close(fused, want, rtol=1e-6, atol=1e-6)
    else:
        err = ((fused.float() - want).abs().max() / want.abs().max()).item()
        assert err <= 1e-2, err


G_BIAS_CASES = [
    ("cheb8_g96", kf.Chebyshev(8), torch.bfloat16, 200, 3072, 384),  # column sums of the T_0 term
    ("cheb8_small", kf.Chebyshev(8), torch.bfloat16, 77, 24, 19),  # precomputed features, own sums
    ("bspline83", kf.BSpline(8, 3), torch.bfloat16, 257, 64, 130),  # GEMM core route
    ("rational", kf.Rational(5, 4), torch.bfloat16, 300, 128, 96),  # GEMM core route
    ("cheb8_f32", kf.Chebyshev(8), torch.float32, 333, 96, 200),
    ("bspline53_f32", kf.BSpline(5, 3), torch.float32, 4096, 64, 64),  # sparse route: G's slice sums of g
]


@pytest.mark.parametrize("name,basis,dtype,B,IN,OUT", G_BIAS_CASES, ids=[c[0] for c in G_BIAS_CASES])
def test_G_bias_is_G_plus_column_sums(name, basis, dtype, B, IN, OUT):
    """kf_G_bias: dc bitwise equal to kf_G's (the same kernels), dbias against float64 column sums
    of g at the dtype's tolerance."""
    torch.manual_seed(2)
    layer = KANLinear(IN, OUT, basis, base_activation=None, groups=8 if name == "rational" else None).to(DEV, dtype)
    x = (torch.randn(B, IN, device=DEV) * 0.8).to(dtype)
    g = torch.randn(B, OUT, device=DEV).to(dtype)
    st = layer._basis_state()
    num = den = None
    if layer._plan.kind == "rational":
        num, den = K._rat(st, layer.basis_numerator, layer.basis_denominator)
    key = layer._plan_key
    with torch.no_grad():
        dc, db = K._G_BIAS(x, g, None, *K._tables(st), num, den, key, 0)
        dc0 = K._G(x, g, None, *K._tables(st), num, den, key, 0)
    torch.cuda.synchronize()
    assert torch.equal(dc, dc0)
    want = g.double().sum(0)
    err = ((db.double() - want).abs().max() / want.abs().max()).item()
    assert err <= (1e-5 if dtype == torch.float32 else 1e-2), err


@pytest.mark.parametrize("B,IN,OUT,grid,k", [(4096, 64, 64, 5, 3), (333, 70, 45, 8, 3), (200, 40, 33, 5, 1), (300, 200, 150, 5, 3)])
def test_fused_sparse_float32_layer_against_oracle(B, IN, OUT, grid, k):
    """float32 B-splines on the sparse route: W as basis function K (feature silu(x)) in F, P and
    G, the bias in F's stores; the first shape is the 64 -> 64 benchmark layer (the small-layer
    kernels, like the next two: ragged, degree 1), the last runs the staged kernels (sides above 128). Tolerance: float32 normwise 1e-5."""
    torch.manual_seed(4)
    layer = KANLinear(IN, OUT, kf.BSpline(grid, k, grid_range=(-2.0, 2.0)))
    with torch.no_grad():
        layer.coef.normal_(0, 0.5 / math.sqrt(IN))
        layer.bias.normal_()
    layer = layer.to(DEV)
    fused = K.base_fused(layer._plan_key, layer._basis_state(), torch.float32, B, IN, OUT)
    print(f"sparse case B={B} in={IN} out={OUT} grid={grid} k={k} fused={fused}", flush=True)
    assert fused == (True, True, True)
    ob = oracle_basis(layer.basis, IN, {"grid": np64(layer.basis_grid)})
    rng = np.random.default_rng(B)
    x0 = rng.uniform(-2.2, 2.2, (B, IN))
    gy0 = rng.normal(0, 1, (B, OUT))
    x = torch.as_tensor(x0, dtype=torch.float32, device=DEV).requires_grad_()
    gy = torch.as_tensor(gy0, dtype=torch.float32, device=DEV)
    y = layer(x)
    y.backward(gy)
    torch.cuda.synchronize()
    c, W, b = np64(layer.coef), np64(layer.base_weight), np64(layer.bias)
    checks = {
        "y": (y, o.kan_linear(x0, c, ob, W, b)),
        "x": (x.grad, o.prim_P(x0, gy0, c, ob, 1) + (gy0 @ W) * o.silu_derivative(x0, 1)),
        "coef": (layer.coef.grad, o.prim_G(x0, gy0, None, ob, 0)),
        "base_weight": (layer.base_weight.grad, gy0.T @ o.silu_derivative(x0, 0)),
        "bias": (layer.bias.grad, gy0.sum(0)),
    }
    for key, (got, want) in checks.items():
        err = o.normwise_err(np64(got), want)
        print(f"  {key}: {err:.3e}", flush=True)
        assert err <= 1e-5, (key, err)



def test_sparse_base_entries_take_a_null_workspace():
    """On the float32 sparse route kf_F_base and kf_P_base need no workspace
    (kf_workspace_bytes is 0): called through the C ABI with NULL they give the same bits as with
    one (the same kernels)."""
    import ctypes

    from kanforge_amd.torch import _lib

    torch.manual_seed(5)
    B, IN, OUT = 333, 64, 48
    layer = KANLinear(IN, OUT, kf.BSpline(5, 3)).to(DEV)
    pl, st = layer._plan, layer._basis_state()
    x = (torch.rand(B, IN, device=DEV) * 2 - 1).contiguous()
    g = torch.randn(B, OUT, device=DEV).contiguous()
    c, bw, bias = (t.detach().contiguous() for t in (layer.coef, layer.base_weight, layer.bias))
    lib = _lib.load()
    d0, _k0 = K._desc(pl, 0, st)
    d1, _k1 = K._desc(pl, 1, st)
    for op, d in ((_lib.KF_OP_F_BASE, d0), (_lib.KF_OP_P_BASE, d1)):
        assert lib.kf_workspace_bytes(op, ctypes.byref(d), _lib.KF_F32, B, IN, OUT) == 0
    stream = torch.cuda.current_stream().cuda_stream
    y = torch.empty(B, OUT, device=DEV)
    p = torch.empty(B, IN, device=DEV)
    print(f"null workspace case B={B} in={IN} out={OUT}", flush=True)
    rc = lib.kf_F_base(ctypes.byref(d0), _lib.KF_F32, B, IN, OUT, x.data_ptr(), c.data_ptr(), bw.data_ptr(),
                       bias.data_ptr(), y.data_ptr(), None, 0, stream)
    assert rc == 0, lib.kf_last_error()
    rc = lib.kf_P_base(ctypes.byref(d1), _lib.KF_F32, B, IN, OUT, x.data_ptr(), g.data_ptr(), c.data_ptr(),
                       bw.data_ptr(), p.data_ptr(), None, 0, stream)
    assert rc == 0, lib.kf_last_error()
    torch.cuda.synchronize()
    assert torch.equal(y, K._f_base_raw(pl, st, x, c, bw, bias))
    assert torch.equal(p, K._p_base_raw(pl, st, x, g, c, bw))
