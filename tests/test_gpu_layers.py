"""KANLinear / GRKAN / KAN on the HIP path against the float64 oracle:
values, every first-order gradient, higher input derivatives through the
F/G/P closure, the gradient penalty (double backward into coef), and the
chained PINN Laplacian."""

import math

import numpy as np
import pytest
import torch

import kanforge_amd as kf
from cases import BASES, oracle_basis, rounded
from kanforge_amd.torch import GRKAN, KAN, KANLinear, laplacian
from oracle import kan64 as o

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}


def np64(t):
    return t.detach().float().cpu().double().numpy()


def make_layer(name, IN, OUT, dtype, seed=0, edge_scale=True, base=True):
    torch.manual_seed(seed)
    layer = KANLinear(IN, OUT, BASES[name], edge_scale=edge_scale, base_activation=torch.nn.functional.silu if base else None)
    with torch.no_grad():
        layer.coef.normal_(0, 0.5 / math.sqrt(IN))
        if edge_scale:
            layer.edge_scale.uniform_(0.5, 1.5)
        if layer.bias is not None:
            layer.bias.normal_()
        if name.startswith("bspline"):
            rng = np.random.default_rng(seed)
            from cases import random_grid

            layer.basis_grid.copy_(torch.as_tensor(random_grid(IN, BASES[name].grid_size + 1, rng)))
    return layer.to(device=DEV, dtype=dtype)


def oracle_of(layer):
    params = None
    if layer._plan.kind == "bspline":
        params = {"grid": np64(layer.basis_grid)}
    elif layer._plan.kind == "rational":
        params = {"num": np64(layer.basis_numerator), "den": np64(layer.basis_denominator)}
    return oracle_basis(layer.basis, layer.in_features, params)


LAYER_CASES = ["chebyshev8", "jacobi6", "legendre_identity", "bspline53", "bspline41"]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("name", LAYER_CASES)
def test_layer_forward_and_gradients(name, dtype):
    B, IN, OUT = 77, 24, 19
    layer = make_layer(name, IN, OUT, dtype)
    ob = oracle_of(layer)
    rng = np.random.default_rng(1)
    x0 = rng.uniform(-0.95, 0.95, (B, IN))
    gy0 = rng.normal(0, 1, (B, OUT))
    x = torch.as_tensor(x0, dtype=torch.float32).to(DEV, dtype).requires_grad_()
    gy = torch.as_tensor(gy0, dtype=torch.float32).to(DEV, dtype)
    y = layer(x)
    assert y.dtype == dtype and y.shape == (B, OUT)
    y.backward(gy)

    xr, gyr = rounded(x0, dtype), rounded(gy0, dtype)
    c, s, W, b = np64(layer.coef), np64(layer.edge_scale), np64(layer.base_weight), np64(layer.bias)
    want_y = o.kan_linear(xr, c, ob, W, b, s)
    assert o.normwise_err(np64(y), want_y) <= TOL[dtype]
    ceff = c * s[..., None]
    want_gx = o.prim_P(xr, gyr, ceff, ob, 1) + (gyr @ W) * o.silu_derivative(xr, 1)
    G0 = o.prim_G(xr, gyr, None, ob, 0)
    checks = {
        "x": (x.grad, want_gx),
        "coef": (layer.coef.grad, G0 * s[..., None]),
        "edge_scale": (layer.edge_scale.grad, (G0 * c).sum(-1)),
        "base_weight": (layer.base_weight.grad, gyr.T @ o.silu_derivative(xr, 0)),
        "bias": (layer.bias.grad, gyr.sum(0)),
    }
    for key, (got, want) in checks.items():
        err = o.normwise_err(np64(got), want)
        print(f"{name} {dtype} {key}: {err:.3e}", flush=True)
        assert err <= TOL[dtype], (key, err)


@pytest.mark.parametrize("name", ["chebyshev5", "jacobi_ab", "bspline53", "taylor"])
def test_higher_input_derivatives_and_gradient_penalty(name):
    # what tests/test_kernels.py:102-121 checks, here against float64
    B, IN, OUT = 37, 4, 5
    layer = make_layer(name, IN, OUT, torch.float32, edge_scale=False)
    ob = oracle_of(layer)
    rng = np.random.default_rng(2)
    x0 = rng.uniform(-0.9, 0.9, (B, IN))
    x = torch.as_tensor(x0, dtype=torch.float32, device=DEV).requires_grad_()
    wts = torch.linspace(-1, 1, OUT, device=DEV)
    loss = (layer(x) * wts).sum()
    (gx,) = torch.autograd.grad(loss, x, create_graph=True)
    (gxx,) = torch.autograd.grad(gx.sum(), x, create_graph=True)
    (gxxx,) = torch.autograd.grad(gxx.sum(), x, create_graph=True)
    (gc,) = torch.autograd.grad((gx**2).sum(), layer.coef)
    xr = rounded(x0, torch.float32)
    gyr = np.broadcast_to(np64(wts), (B, OUT))
    c, W = np64(layer.coef), np64(layer.base_weight)
    for m, got in ((1, gx), (2, gxx), (3, gxxx)):
        want = o.prim_P(xr, gyr, c, ob, m) + (gyr @ W) * o.silu_derivative(xr, m)
        err = o.normwise_err(np64(got), want)
        print(f"{name} d{m}x: {err:.3e}", flush=True)
        assert err <= 1e-5, (m, err)
    gx64 = o.prim_P(xr, gyr, c, ob, 1) + (gyr @ W) * o.silu_derivative(xr, 1)
    want_gc = 2 * o.prim_G(xr, gyr, gx64, ob, 1)
    err = o.normwise_err(np64(gc), want_gc)
    print(f"{name} gradient penalty: {err:.3e}", flush=True)
    assert err <= 1e-5, err


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("name,order", [("chebyshev8", 0), ("chebyshev8", 2), ("bspline53", 1), ("jacobi6", 2)])
def test_layer_edge_derivative(name, order, dtype):
    B, IN, OUT = 50, 12, 7
    layer = make_layer(name, IN, OUT, dtype)
    ob = oracle_of(layer)
    x0 = np.random.default_rng(3).uniform(-0.9, 0.9, (B, IN))
    x = torch.as_tensor(x0, dtype=torch.float32).to(DEV, dtype)
    d = layer.edge_derivative(x, order)
    assert d.shape == (B, OUT, IN)
    ceff = np64(layer.coef) * np64(layer.edge_scale)[..., None]
    want = o.edge_derivative(rounded(x0, dtype), ceff, ob, order, np64(layer.base_weight))
    assert o.normwise_err(np64(d), want) <= TOL[dtype]
    if order == 0 and dtype == torch.float32:
        # sum over inputs plus bias is the layer output (tests/test_layers.py:62-63)
        np.testing.assert_allclose(np64(d.sum(-1) + layer.bias), np64(layer(x)), atol=2e-5)


@pytest.mark.parametrize("name,order", [("chebyshev8", 0), ("chebyshev8", 2), ("bspline53", 1), ("jacobi6", 2)])
def test_edge_derivative_gradients(name, order):
    """Backward of edge_derivative: x through the order+1 edges, coef through the features,
    base_weight through silu^(order), against the float64 oracle."""
    B, IN, OUT = 45, 10, 6
    layer = make_layer(name, IN, OUT, torch.float32)
    ob = oracle_of(layer)
    rng = np.random.default_rng(8)
    x0 = rng.uniform(-0.9, 0.9, (B, IN))
    r0 = rng.normal(0, 1, (B, OUT, IN))
    x = torch.as_tensor(x0, dtype=torch.float32, device=DEV).requires_grad_()
    d = layer.edge_derivative(x, order)
    gx, gc, gs, gw = torch.autograd.grad(d, [x, layer.coef, layer.edge_scale, layer.base_weight], torch.as_tensor(r0, dtype=torch.float32, device=DEV))
    xr = rounded(x0, torch.float32)
    c, s, W = np64(layer.coef), np64(layer.edge_scale), np64(layer.base_weight)
    e1 = o.edge_derivative(xr, c * s[..., None], ob, order + 1, W)
    phi = ob(xr, order)
    gce = np.einsum("boi,bik->oik", r0, phi)
    checks = {
        "x": (gx, (r0 * e1).sum(1)),
        "coef": (gc, gce * s[..., None]),
        "edge_scale": (gs, (gce * c).sum(-1)),
        "base_weight": (gw, np.einsum("boi,bi->oi", r0, o.silu_derivative(xr, order))),
    }
    for key, (got, want) in checks.items():
        err = o.normwise_err(np64(got), want)
        print(f"edge {name} order {order} d{key}: {err:.3e}", flush=True)
        assert err <= 1e-5, (key, err)


@pytest.mark.parametrize("name", ["bspline53", "chebyshev8", "rational"])
def test_edge_dropout_training_step_matches_oracle(name):
    """KANLinear's edge_dropout training forward (kanforge/torch/layers.py:171-176) and its backward,
    with the dropout mask regenerated from the same torch seed: every parameter gradient, the
    rational numerator/denominator included."""
    B, IN, OUT, p = 40, 16, 12, 0.3
    if name == "rational":
        torch.manual_seed(0)
        layer = KANLinear(IN, OUT, kf.Rational(5, 4, "gelu"), groups=4, base_activation=None, edge_dropout=p)
        with torch.no_grad():
            layer.basis_numerator.add_(0.05 * torch.randn_like(layer.basis_numerator))
            layer.basis_denominator.add_(0.05 * torch.randn_like(layer.basis_denominator))
            layer.bias.normal_()
        layer = layer.to(DEV)
    else:
        layer = make_layer(name, IN, OUT, torch.float32)
        layer.edge_dropout = p
    layer.train()
    ob = oracle_of(layer)
    rng = np.random.default_rng(9)
    x0, gy0 = rng.uniform(-0.9, 0.9, (B, IN)), rng.normal(0, 1, (B, OUT))
    x = torch.as_tensor(x0, dtype=torch.float32, device=DEV).requires_grad_()
    torch.manual_seed(123)
    y = layer(x)
    torch.manual_seed(123)
    keep = (torch.rand(B, OUT, IN, device=DEV) >= p).double().cpu().numpy()
    params = [x] + [t for t in (layer.coef, layer.edge_scale, layer.base_weight, layer.bias) if t is not None]
    if name == "rational":
        params += [layer.basis_numerator, layer.basis_denominator]
    grads = dict(zip(range(len(params)), torch.autograd.grad(y, params, torch.as_tensor(gy0, dtype=torch.float32, device=DEV))))
    xr = rounded(x0, torch.float32)
    c = np64(layer.coef)
    s = np64(layer.edge_scale) if layer.edge_scale is not None else np.ones(c.shape[:2])
    W = np64(layer.base_weight) if layer.base_weight is not None else None
    ceff = c * s[..., None]
    e0 = o.edge_derivative(xr, ceff, ob, 0, W)
    e1 = o.edge_derivative(xr, ceff, ob, 1, W)
    M = gy0[:, :, None] * keep / (1 - p)  # d loss / d edge
    want = {"y": (keep * e0).sum(-1) / (1 - p) + np64(layer.bias), "x": (M * e1).sum(1)}
    gce = np.einsum("boi,bik->oik", M, ob(xr, 0))
    want["coef"] = gce * s[..., None]
    got = {"y": y, "x": grads[0], "coef": grads[1]}
    k = 2
    if layer.edge_scale is not None:
        want["edge_scale"], got["edge_scale"] = (gce * c).sum(-1), grads[k]
        k += 1
    if W is not None:
        want["base_weight"], got["base_weight"] = np.einsum("boi,bi->oi", M, o.silu_derivative(xr, 0)), grads[k]
        k += 1
    want["bias"], got["bias"] = gy0.sum(0), grads[k]
    if name == "rational":
        h = np.einsum("boi,oi->bi", M, ceff[..., 0])
        dn, dd = o.rational_param_grads(xr, ob.kw["num"], ob.kw["den"])
        g = layer.basis_numerator.shape[0]
        want["numerator"] = np.einsum("bi,bij->ij", h, dn).reshape(g, -1, 6).sum(1)
        want["denominator"] = np.einsum("bi,bij->ij", h, dd).reshape(g, -1, 4).sum(1)
        got["numerator"], got["denominator"] = grads[k + 1], grads[k + 2]
    for key in want:
        err = o.normwise_err(np64(got[key]), want[key])
        print(f"edge_dropout {name} {key}: {err:.3e}", flush=True)
        assert err <= 1e-5, (key, err)


@pytest.mark.parametrize("name", ["bspline53", "chebyshev8"])
def test_masked_and_symbolic_layer_matches_oracle(name):
    """Pruned and symbolic edges on the kernel path (kanforge tests/test_interpret.py:116-133):
    forward, x/coef/base_weight gradients and the order-0 edge derivative against the oracle."""
    B, IN, OUT = 41, 5, 4
    layer = make_layer(name, IN, OUT, torch.float32, edge_scale=False)
    mask = np.ones((OUT, IN))
    mask[0, 1] = mask[2, 3] = mask[3, 0] = 0
    layer.set_edge_mask(mask)
    layer.fix_symbolic(1, 0, "x^2", (1.0, 0.5, 2.0, 0.25))
    layer.fix_symbolic(3, 4, "sin", (2.0, 0.1, 1.5, -0.2))
    layer.fix_symbolic(0, 2, "gaussian", (1.5, 0.0, 0.7, 0.0))
    ob = oracle_of(layer)
    rng = np.random.default_rng(10)
    x0, gy0 = rng.uniform(-0.9, 0.9, (B, IN)), rng.normal(0, 1, (B, OUT))
    x = torch.as_tensor(x0, dtype=torch.float32, device=DEV).requires_grad_()
    y = layer(x)
    gx, gc, gw = torch.autograd.grad(y, [x, layer.coef, layer.base_weight], torch.as_tensor(gy0, dtype=torch.float32, device=DEV))
    xr = rounded(x0, torch.float32)
    m = np64(layer.edge_mask)
    code, sp = layer.sym_code.cpu().numpy(), np64(layer.sym_params)
    c, W = np64(layer.coef) * m[..., None], np64(layer.base_weight) * m
    e0 = o.edge_derivative(xr, c, ob, 0, W) + o.symbolic_edges(xr, code, sp)
    # d/dx of a symbolic edge c f(a x + b) + d by central differences of the oracle (float64)
    h = 1e-6
    dsym = (o.symbolic_edges(xr + h, code, sp) - o.symbolic_edges(xr - h, code, sp)) / (2 * h)
    checks = {
        "y": (y, e0.sum(-1) + np64(layer.bias)),
        "edges": (layer.edge_derivative(x, 0), e0),
        "x": (gx, o.prim_P(xr, gy0, c, ob, 1) + (gy0 @ W) * o.silu_derivative(xr, 1) + np.einsum("bo,boi->bi", gy0, dsym)),
        "coef": (gc, o.prim_G(xr, gy0, None, ob, 0) * m[..., None]),
        "base_weight": (gw, (gy0.T @ o.silu_derivative(xr, 0)) * m),
    }
    for key, (got, want) in checks.items():
        err = o.normwise_err(np64(got), want)
        print(f"masked/symbolic {name} {key}: {err:.3e}", flush=True)
        assert err <= 1e-5, (key, err)


def test_edge_derivative_order0_with_another_base_activation():
    """Order-0 edges of a layer whose base activation is not SiLU (kanforge/torch/layers.py:213-216)."""
    torch.manual_seed(0)
    layer = KANLinear(6, 5, kf.BSpline(5, 3), base_activation=torch.nn.functional.gelu).to(DEV)
    x0 = np.random.default_rng(11).uniform(-0.9, 0.9, (30, 6))
    x = torch.as_tensor(x0, dtype=torch.float32, device=DEV)
    d = layer.edge_derivative(x, 0)
    xr = rounded(x0, torch.float32)
    from scipy.special import erf

    gelu = 0.5 * xr * (1 + erf(xr / np.sqrt(2)))
    want = o.edge_derivative(xr, np64(layer.coef), oracle_of(layer), 0) + gelu[:, None, :] * np64(layer.base_weight)
    assert o.normwise_err(np64(d), want) <= 1e-5
    np.testing.assert_allclose(np64(d.sum(-1) + layer.bias), np64(layer(x)), atol=2e-6)
    with pytest.raises(NotImplementedError):
        layer.edge_derivative(x, 1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_grkan_forward_and_all_gradients(dtype):
    B, IN, OUT = 96, 32, 40
    torch.manual_seed(0)
    layer = GRKAN(IN, OUT, groups=8)
    with torch.no_grad():
        layer.basis_numerator.add_(0.05 * torch.randn_like(layer.basis_numerator))
        layer.basis_denominator.add_(0.05 * torch.randn_like(layer.basis_denominator))
        layer.bias.normal_()
    layer = layer.to(DEV, dtype)
    rng = np.random.default_rng(4)
    x0, gy0 = rng.normal(0, 1, (B, IN)), rng.normal(0, 1, (B, OUT))
    x = torch.as_tensor(x0, dtype=torch.float32).to(DEV, dtype).requires_grad_()
    y = layer(x)
    y.backward(torch.as_tensor(gy0, dtype=torch.float32).to(DEV, dtype))
    num, den = np64(layer.basis_numerator), np64(layer.basis_denominator)
    ob = o.Basis64("rational", num=np.repeat(num, IN // 8, 0), den=np.repeat(den, IN // 8, 0))
    xr, gyr = rounded(x0, dtype), rounded(gy0, dtype)
    c = np64(layer.coef)
    h = gyr @ c[..., 0]  # (B, IN)
    dn, dd = o.rational_param_grads(xr, ob.kw["num"], ob.kw["den"])
    checks = {
        "y": (y, o.kan_linear(xr, c, ob, None, np64(layer.bias))),
        "x": (x.grad, o.prim_P(xr, gyr, c, ob, 1)),
        "coef": (layer.coef.grad, o.prim_G(xr, gyr, None, ob, 0)),
        "numerator": (layer.basis_numerator.grad, np.einsum("bi,bij->ij", h, dn).reshape(8, -1, 6).sum(1)),
        "denominator": (layer.basis_denominator.grad, np.einsum("bi,bij->ij", h, dd).reshape(8, -1, 4).sum(1)),
    }
    for key, (got, want) in checks.items():
        err = o.normwise_err(np64(got), want)
        print(f"grkan {dtype} {key}: {err:.3e}", flush=True)
        assert err <= TOL[dtype], (key, err)


def test_grkan_gradient_penalty_reaches_the_rational_parameters():
    """Double backward through a GR-KAN layer with trainable P/Q: the gradient of the penalty
    sum (dL/dx)^2, L = <y, gy>, with respect to numerator and denominator, against central
    differences of the oracle's float64 penalty."""
    B, IN, OUT = 40, 16, 8
    torch.manual_seed(3)
    layer = GRKAN(IN, OUT, groups=4)
    with torch.no_grad():
        layer.basis_numerator.add_(0.1 * torch.randn_like(layer.basis_numerator))
        layer.basis_denominator.add_(0.1 * torch.randn_like(layer.basis_denominator))
    layer = layer.to(DEV)
    rng = np.random.default_rng(5)
    x0, gy0 = rng.normal(0, 1, (B, IN)), rng.normal(0, 1, (B, OUT))
    x = torch.as_tensor(x0, dtype=torch.float32, device=DEV).requires_grad_()
    gy = torch.as_tensor(gy0, dtype=torch.float32, device=DEV)
    (gx,) = torch.autograd.grad((layer(x) * gy).sum(), x, create_graph=True)
    (gx * gx).sum().backward()
    xr, gyr = rounded(x0, torch.float32), rounded(gy0, torch.float32)
    c = np64(layer.coef)
    num, den = np64(layer.basis_numerator), np64(layer.basis_denominator)

    def penalty(nm, dn):
        ob = o.Basis64("rational", num=np.repeat(nm, IN // 4, 0), den=np.repeat(dn, IN // 4, 0))
        return (o.prim_P(xr, gyr, c, ob, 1) ** 2).sum()

    for name, arr, got in (("numerator", num, layer.basis_numerator.grad), ("denominator", den, layer.basis_denominator.grad)):
        want = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            eps = 1e-6
            up, dn = arr.copy(), arr.copy()
            up[idx] += eps
            dn[idx] -= eps
            hi = penalty(up, den) if arr is num else penalty(num, up)
            lo = penalty(dn, den) if arr is num else penalty(num, dn)
            want[idx] = (hi - lo) / (2 * eps)
        err = o.normwise_err(np64(got), want)
        print(f"grkan penalty d{name}: {err:.3e}", flush=True)
        assert err <= 1e-4, (name, err)


def _chained_second_derivative(layers, x, dim):
    """Forward-mode (h, h', h'') through KAN layers in float64."""
    h = x
    hp = np.zeros_like(x)
    hp[:, dim] = 1.0
    hpp = np.zeros_like(x)
    for lay in layers:
        ob, ceff, W, b = lay
        e0 = o.edge_derivative(h, ceff, ob, 0, W)
        e1 = o.edge_derivative(h, ceff, ob, 1, W)
        e2 = o.edge_derivative(h, ceff, ob, 2, W)
        h_new = e0.sum(-1) + b
        hp_new = np.einsum("boi,bi->bo", e1, hp)
        hpp_new = np.einsum("boi,bi->bo", e2, hp**2) + np.einsum("boi,bi->bo", e1, hpp)
        h, hp, hpp = h_new, hp_new, hpp_new
    return hpp[:, 0]


def test_pinn_laplacian_matches_forward_mode_oracle():
    torch.manual_seed(0)
    model = KAN([2, 16, 16, 1], kf.Jacobi(6, 0.5, 0.5)).to(DEV)
    rng = np.random.default_rng(5)
    x0 = rng.uniform(-1, 1, (300, 2))
    x = torch.as_tensor(x0, dtype=torch.float32, device=DEV)
    lap = laplacian(model, x)
    layers = []
    for lay in model:
        layers.append((oracle_of(lay), np64(lay.coef), np64(lay.base_weight), np64(lay.bias)))
    xr = rounded(x0, torch.float32)
    want = sum(_chained_second_derivative(layers, xr, d) for d in range(2))
    err = o.normwise_err(np64(lap), want)
    print(f"laplacian: {err:.3e}", flush=True)
    assert err <= 1e-5, err


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_saved_model_reloads_with_identical_outputs(tmp_path, dtype):
    """kanforge.save/load round trip (kanforge tests/test_export.py:67-77): the reloaded model
    gives bit-identical outputs on the HIP path."""
    from kanforge_amd import convert as cv

    torch.manual_seed(0)
    model = torch.nn.Sequential(KAN([4, 16, 8], kf.BSpline(5, 3)), GRKAN(8, 8, groups=4)).to(device=DEV, dtype=dtype)
    path = tmp_path / "m.npz"
    cv.save(model, path)
    back = cv.load(path, device=DEV)
    x = (torch.rand(33, 4, device=DEV) * 2 - 1).to(dtype)
    with torch.no_grad():
        torch.testing.assert_close(back(x), model(x), rtol=0, atol=0)


def test_forward_after_grid_update_uses_the_new_grid():
    """After update_grid / refine_grid the kernel route sees the new grid and coefficients
    (kanforge tests/test_kernels.py:136-143): the device knot tables are rebuilt."""
    torch.manual_seed(0)
    model = KAN([3, 5, 2], kf.BSpline(5, 3)).to(DEV)
    x = torch.randn(64, 3, device=DEV) * 0.4
    model(x)  # device tables of the initial grids
    model.update_grid(x)
    model[0].refine_grid(8)
    for layer, h in [(model[0], x), (model[1], model[0](x).detach())]:
        ob = oracle_of(layer)
        want = o.kan_linear(np64(h), np64(layer.coef), ob, np64(layer.base_weight), np64(layer.bias))
        assert o.normwise_err(np64(layer(h)), want) <= TOL[torch.float32]
    assert model[0].basis.grid_size == 8 and model[0].basis_grid.shape == (3, 9)


@pytest.mark.parametrize("kind", ["kan", "grkan"])
def test_kanffn_forward_matches_oracle(kind):
    """KANFFN (kanforge/torch/transformer.py:25-52): two KAN layers back to back."""
    from kanforge_amd.torch import KANFFN

    torch.manual_seed(0)
    ffn = KANFFN(16, 48, kind=kind, basis=kf.Chebyshev(6), groups=4).to(DEV)
    x = torch.randn(40, 16, device=DEV) * 0.7
    with torch.no_grad():
        y = ffn(x)
    def arr(t):
        return None if t is None else np64(t)

    h = o.kan_linear(np64(x), np64(ffn.fc1.coef), oracle_of(ffn.fc1), arr(ffn.fc1.base_weight), arr(ffn.fc1.bias))
    want = o.kan_linear(h, np64(ffn.fc2.coef), oracle_of(ffn.fc2), arr(ffn.fc2.base_weight), arr(ffn.fc2.bias))
    err = o.normwise_err(np64(y), want)
    print(f"kanffn {kind}: {err:.3e}", flush=True)
    assert err <= 1e-5, err


def test_kanify_exact_keeps_outputs_and_katblock_runs():
    """kanify(mode="exact") (kanforge/torch/transformer.py:127-167) keeps the model's function:
    the spline parts start at zero."""
    from kanforge_amd.torch import KATBlock, kanify

    torch.manual_seed(1)

    class Mlp(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.fc1, self.act, self.fc2 = torch.nn.Linear(12, 32), torch.nn.GELU(), torch.nn.Linear(32, 12)

        def forward(self, x):
            return self.fc2(self.act(self.fc1(x)))

    model = torch.nn.Sequential(Mlp(), torch.nn.LayerNorm(12), Mlp()).to(DEV)
    x = torch.randn(2, 9, 12, device=DEV)
    with torch.no_grad():
        before = model(x)
        assert kanify(model, "exact", basis=kf.BSpline(5, 3)) == ["0", "2"]
        after = model(x)
    torch.testing.assert_close(after, before, rtol=1e-5, atol=1e-6)

    blk = KATBlock(16, 4, mlp_ratio=2.0, groups=4).to(DEV).eval()
    z = torch.randn(3, 7, 16, device=DEV)
    with torch.no_grad():
        out = blk(z)
        h = blk.norm1(z)
        ref = z + blk.attn(h, h, h, need_weights=False)[0]
        ref = ref + blk.ffn(blk.norm2(ref))
    assert out.shape == z.shape
    torch.testing.assert_close(out, ref, rtol=0, atol=0)


@pytest.mark.parametrize("basis", [kf.Jacobi(6, 0.5, 0.5), kf.BSpline(5, 3)], ids=["jacobi6", "bspline53"])
def test_forward_mode_laplacian_equals_reverse_mode_and_trains(basis):
    """laplacian() on a KAN chain propagates Taylor coefficients forward (F with w); on any other
    callable it differentiates twice with autograd (kanforge/torch/science.py:25-46). Both give
    the same field and the same gradients of a PINN loss with respect to every parameter."""
    torch.manual_seed(0)
    model = KAN([2, 16, 16, 1], basis).to(DEV)
    with torch.no_grad():
        for layer in model:
            layer.bias.normal_(0, 0.1)
    x = torch.rand(500, 2, device=DEV) * 1.8 - 0.9
    lap_f = laplacian(model, x)
    lap_r = laplacian(lambda z: model(z), x)
    err = o.normwise_err(np64(lap_f), np64(lap_r))
    print(f"forward vs reverse laplacian {basis!r}: {err:.3e}", flush=True)
    assert err <= 1e-5
    params = [p for p in model.parameters()]
    # (the last layer's bias does not enter second derivatives: no gradient in either mode)
    g_f = torch.autograd.grad((lap_f**2).mean(), params, allow_unused=True)
    g_r = torch.autograd.grad((laplacian(lambda z: model(z), x) ** 2).mean(), params, allow_unused=True)
    for p, a, b in zip(params, g_f, g_r):
        assert (a is None) == (b is None)
        if a is not None:
            e = o.normwise_err(np64(a), np64(b))
            assert e <= 1e-5, (p.shape, e)
    assert g_f[-1] is None  # model[-1].bias
