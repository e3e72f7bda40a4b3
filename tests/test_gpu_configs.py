"""Every benchmark configuration at its own workload on the HIP path, against the float64 oracle.

The workloads are the ones bench.py times (same shapes, dtypes, seeds and layer defaults):
  * KANLinear 64 -> 64 B-spline(5, 3), float32, batch 4096, SiLU base: every output and
    gradient of the whole step against the oracle;
  * KANLinear 768 -> 3072 Chebyshev(8), bfloat16, batch 8192: rows of y and dX, and blocks of
    dCoef over the whole batch (tests/test_gpu_headline.py holds the float32-reference and
    identity checks of the same step);
  * GR-KAN FFN 768 -> 3072 -> 768 (8 groups, P 5 / Q 4) and the B-spline(8, 3) FFN
    768 -> 3072 -> 768, bfloat16, 16384 tokens, forward + backward at full size: rows of the
    output and of dX through the two layers, blocks of every coefficient gradient over all
    16384 tokens, the rational parameter gradients, and the adjoint identity of each layer;
  * the PINN KAN [2, 64, 64, 1] Jacobi(6, 1/2, 1/2), float32, 65536 points: edge_derivative
    of order 2 of every layer and the chained Laplacian, checked on row subsets.

Rows of a layer are independent, so a row subset of a full-size run is checked exactly; sums
over the batch (coefficient gradients) are checked on blocks of (output, input) edges with the
whole batch. Primitive-level checks feed the oracle the inputs each layer actually received on
the device; chain-level checks run the oracle through the whole network from the inputs.
Tolerances: normwise (max|d| / max|ref|) 1e-5 for float32 and 2e-2 for bfloat16.
"""

import math

import numpy as np
import pytest
import torch

import kanforge_amd as kf
from cases import rounded
from kanforge_amd.torch import KAN, KANLinear, laplacian
from kanforge_amd.torch import kernels as K
from kanforge_amd.torch.layers import layer_inputs
from oracle import kan64 as o

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}


def np64(t):
    return t.detach().float().cpu().double().numpy()


def randn(shape, seed, scale=1.0):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)) * scale


def check(what, got, want, tol):
    err = o.normwise_err(got, want)
    print(f"{what}: normwise error {err:.3e} (tol {tol:.0e})", flush=True)
    assert err <= tol, f"{what}: {err:.3e} > {tol:.0e}"


def oracle_of(layer):
    """The oracle's view of a layer's basis with its per-input parameters (float64)."""
    plan = layer._plan
    n_in = layer.in_features
    if plan.kind == "cheb":
        return o.Basis64("poly", A=np.asarray(layer.basis._cheb, np.float64), input_map=layer.basis.input_map)
    if plan.kind == "bspline":
        return o.Basis64("bspline", grid=np64(layer.basis_grid), k=layer.basis.order)
    rep = n_in // layer.basis_numerator.shape[0]
    return o.Basis64(
        "rational", num=np.repeat(np64(layer.basis_numerator), rep, 0), den=np.repeat(np64(layer.basis_denominator), rep, 0)
    )


def restrict(ob, idx):
    """The oracle basis of the inputs ``idx`` only."""
    if ob.kind == "poly":
        return ob
    if ob.kind == "bspline":
        return o.Basis64("bspline", grid=ob.kw["grid"][idx], k=ob.kw["k"])
    return o.Basis64("rational", num=ob.kw["num"][idx], den=ob.kw["den"][idx])


def layer_np(layer):
    arr = lambda t: None if t is None else np64(t)  # noqa: E731
    return oracle_of(layer), np64(layer.effective_coef()), arr(layer.effective_base_weight()), arr(layer.bias)


def oracle_layer(x, lay):
    ob, c, W, b = lay
    return o.kan_linear(x, c, ob, W, b)


def oracle_layer_dx(x, g, lay):
    """d(sum g * layer(x))/dx, float64."""
    ob, c, W, b = lay
    gx = o.prim_P(x, g, c, ob, 1)
    if W is not None:
        gx = gx + (g @ W) * o.silu_derivative(x, 1)
    return gx


def check_coef_grad_block(what, layer, x_in, g_out, got, tol, rng, n_o=48, n_i=48):
    """dCoef[o, i, :] = sum_b g[b, o] phi(x[b, i]) over the whole batch for a block of edges."""
    ob = oracle_of(layer)
    o_idx = np.sort(rng.choice(layer.out_features, n_o, replace=False))
    i_idx = np.sort(rng.choice(layer.in_features, n_i, replace=False))
    want = o.prim_G(x_in[:, i_idx], g_out[:, o_idx], None, restrict(ob, i_idx), 0)
    if layer.edge_scale is not None:
        want = want * np64(layer.edge_scale)[np.ix_(o_idx, i_idx)][..., None]
    check(what, np64(got)[np.ix_(o_idx, i_idx)], want, tol)


# --- KANLinear 64 -> 64 B-spline(5, 3), float32, batch 4096 ----------------------------------


def test_kan64_bspline_fp32_step_matches_oracle():
    torch.manual_seed(0)
    layer = KANLinear(64, 64, kf.BSpline(5, 3)).to(DEV)
    with torch.no_grad():
        layer.coef.copy_(randn(layer.coef.shape, 1, 1 / math.sqrt(64 * 8)))
        layer.bias.copy_(randn((64,), 4, 0.1))
    x0 = torch.rand(4096, 64, generator=torch.Generator().manual_seed(0)) * 2 - 1
    gy0 = randn((4096, 64), 3)
    x = x0.to(DEV).requires_grad_()
    gy = gy0.to(DEV)
    y = layer(x)
    gx, gc, gw, gb = torch.autograd.grad(y, [x, layer.coef, layer.base_weight, layer.bias], gy)
    ob, c, W, b = lay = layer_np(layer)
    xr, g = x0.double().numpy(), gy0.double().numpy()
    check("kan64 y", np64(y), oracle_layer(xr, lay), 1e-5)
    check("kan64 dx", np64(gx), oracle_layer_dx(xr, g, lay), 1e-5)
    check("kan64 dcoef", np64(gc), o.prim_G(xr, g, None, ob, 0), 1e-5)
    check("kan64 dbase_weight", np64(gw), g.T @ o.silu_derivative(xr, 0), 1e-5)
    check("kan64 dbias", np64(gb), g.sum(0), 1e-5)


# --- KANLinear 768 -> 3072 Chebyshev(8), bfloat16, batch 8192 ---------------------------------


def test_cheb768_step_rows_and_dcoef_blocks_match_oracle():
    B, IN, OUT, KB = 8192, 768, 3072, 9
    layer = KANLinear(IN, OUT, kf.Chebyshev(8), base_activation=None, bias=False, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        layer.coef.copy_(randn((OUT, IN, KB), 1, 1 / math.sqrt(IN * KB)).to(torch.bfloat16))
    x = randn((B, IN), 0).to(DEV, torch.bfloat16).requires_grad_()
    gy = randn((B, OUT), 3).to(DEV, torch.bfloat16)
    y = layer(x)
    dx, dc = torch.autograd.grad(y, [x, layer.coef], gy)
    rng = np.random.default_rng(7)
    rows = np.sort(rng.choice(B, 384, replace=False))
    xr, g = np64(x), np64(gy)
    lay = layer_np(layer)
    check("cheb768 y rows", np64(y)[rows], oracle_layer(xr[rows], lay), 2e-2)
    check("cheb768 dx rows", np64(dx)[rows], oracle_layer_dx(xr[rows], g[rows], lay), 2e-2)
    check_coef_grad_block("cheb768 dcoef block", layer, xr, g, dc, 2e-2, rng)


# --- the two-layer FFNs, bfloat16, 16384 tokens ---------------------------------------------


def _ffn_step(ffn, x0, gy0):
    """Full-size forward + backward; returns the layer inputs and upstream gradients it saw."""
    x = x0.to(DEV, torch.bfloat16).requires_grad_()
    gy = gy0.to(DEV, torch.bfloat16)
    h = ffn.fc1(x)
    h.retain_grad()
    y = ffn.fc2(h)
    params = list(ffn.parameters())
    y.backward(gy)
    torch.cuda.synchronize()
    return {"x": x, "h": h, "y": y, "gy": gy, "gh": h.grad, "params": params}


def _check_ffn(name, ffn, run, rng):
    x, h, y = np64(run["x"]), np64(run["h"]), np64(run["y"])
    gy, gh = np64(run["gy"]), np64(run["gh"])
    l1, l2 = layer_np(ffn.fc1), layer_np(ffn.fc2)
    rows = np.sort(rng.choice(x.shape[0], 256, replace=False))
    # primitive level: each layer against the oracle on the inputs it received
    check(f"{name} fc1 y rows", h[rows], oracle_layer(x[rows], l1), 2e-2)
    check(f"{name} fc2 y rows", y[rows], oracle_layer(h[rows], l2), 2e-2)
    check(f"{name} fc2 dx rows", gh[rows], oracle_layer_dx(h[rows], gy[rows], l2), 2e-2)
    check(f"{name} fc1 dx rows", np64(run["x"].grad)[rows], oracle_layer_dx(x[rows], gh[rows], l1), 2e-2)
    # chain level: the oracle through both layers from x (the hidden state and its gradient are
    # bfloat16 tensors between the layers, so the oracle rounds them there too)
    h64 = o.round_bf16(oracle_layer(x[rows], l1))
    check(f"{name} chain y rows", y[rows], oracle_layer(h64, l2), 2e-2)
    if ffn.fc2._plan.kind != "rational":
        # A rational basis' derivative jumps where Q changes sign (d|Q| = sign(Q) dQ): where the
        # device's h and the oracle's h are neighbouring bfloat16 values across such a root,
        # phi'(h) differs by O(1), so dX through the chain is ill-posed at bfloat16. The
        # per-layer dX checks above (on the hidden state the device computed) cover it.
        gh64 = o.round_bf16(oracle_layer_dx(h64, gy[rows], l2))
        check(f"{name} chain dx rows", np64(run["x"].grad)[rows], oracle_layer_dx(x[rows], gh64, l1), 2e-2)
    # sums over all tokens
    check_coef_grad_block(f"{name} fc2 dcoef block", ffn.fc2, h, gy, ffn.fc2.coef.grad, 2e-2, rng)
    check_coef_grad_block(f"{name} fc1 dcoef block", ffn.fc1, x, gh, ffn.fc1.coef.grad, 2e-2, rng)
    for lay, xin, g in ((ffn.fc1, x, gh), (ffn.fc2, h, gy)):
        tag = f"{name} {'fc1' if lay is ffn.fc1 else 'fc2'}"
        if lay.base_weight is not None:
            o_idx = np.sort(rng.choice(lay.out_features, 64, replace=False))
            want = g[:, o_idx].T @ o.silu_derivative(xin, 0)
            check(f"{tag} dbase_weight rows", np64(lay.base_weight.grad)[o_idx], want, 2e-2)
        if lay.bias is not None:
            check(f"{tag} dbias", np64(lay.bias.grad), g.sum(0), 2e-2)
        # adjoint identity over the whole layer: <F_0(x, c), g> = <c, G_0(x, g)>
        st = lay._basis_state()
        xs = run["x"].detach() if lay is ffn.fc1 else run["h"].detach()
        gs = run["gh"] if lay is ffn.fc1 else run["gy"]
        c = lay.coef.detach()
        f0 = K.prim_F(xs, c, None, st, lay._plan, 0)
        g0 = K.prim_G(xs, gs, None, st, lay._plan, 0)
        lhs = (f0.double() * gs.double()).sum().item()
        rhs = (c.double() * g0.double()).sum().item()
        scale = (f0.double() * gs.double()).abs().sum().item()
        print(f"{tag} adjoint: {abs(lhs - rhs) / scale:.3e}", flush=True)
        assert abs(lhs - rhs) <= 2e-3 * scale


def test_grkan_ffn_full_size_matches_oracle():
    from kanforge_amd.torch import KANFFN

    ffn = KANFFN(768, 3072, kind="grkan", groups=8).to(DEV, torch.bfloat16)
    with torch.no_grad():
        for i, layer in enumerate((ffn.fc1, ffn.fc2)):
            layer.basis_numerator.copy_(randn(layer.basis_numerator.shape, 2 + 2 * i, math.sqrt(0.1)))
            layer.basis_denominator.copy_(randn(layer.basis_denominator.shape, 3 + 2 * i, math.sqrt(0.1)))
    x0, gy0 = randn((16384, 768), 0), randn((16384, 768), 3)
    run = _ffn_step(ffn, x0, gy0)
    rng = np.random.default_rng(11)
    _check_ffn("grkan", ffn, run, rng)
    # rational parameter gradients: sums over every token and every input of a group
    for lay, xin, g in ((ffn.fc1, np64(run["x"]), np64(run["gh"])), (ffn.fc2, np64(run["h"]), np64(run["gy"]))):
        ob = oracle_of(lay)
        hsum = g @ np64(lay.coef)[..., 0]  # (B, in): sum_o g[b, o] c[o, i]
        dn, dd = o.rational_param_grads(xin, ob.kw["num"], ob.kw["den"])
        groups = lay.basis_numerator.shape[0]
        want_n = np.einsum("bi,bij->ij", hsum, dn, optimize=True).reshape(groups, -1, dn.shape[-1]).sum(1)
        want_d = np.einsum("bi,bij->ij", hsum, dd, optimize=True).reshape(groups, -1, dd.shape[-1]).sum(1)
        tag = "fc1" if lay is ffn.fc1 else "fc2"
        check(f"grkan {tag} dnum", np64(lay.basis_numerator.grad), want_n, 2e-2)
        check(f"grkan {tag} dden", np64(lay.basis_denominator.grad), want_d, 2e-2)


def test_bspline_ffn_full_size_matches_oracle():
    from kanforge_amd.torch import KANFFN

    dim, hid, k = 768, 3072, 11
    ffn = KANFFN(dim, hid, kind="kan", basis=kf.BSpline(8, 3)).to(DEV, torch.bfloat16)
    with torch.no_grad():
        ffn.fc1.coef.copy_(randn(ffn.fc1.coef.shape, 1, 1 / math.sqrt(dim * k)))
        ffn.fc2.coef.copy_(randn(ffn.fc2.coef.shape, 1, 1 / math.sqrt(hid * k)))
        ffn.fc1.bias.copy_(randn((hid,), 5, 0.1))
        ffn.fc2.bias.copy_(randn((dim,), 6, 0.1))
    x0, gy0 = randn((16384, dim), 0), randn((16384, dim), 3)
    run = _ffn_step(ffn, x0, gy0)
    _check_ffn("bspline", ffn, run, np.random.default_rng(12))


# --- PINN KAN [2, 64, 64, 1] Jacobi(6, 1/2, 1/2), float32, 65536 points ---------------------


def _pinn():
    model = KAN([2, 64, 64, 1], kf.Jacobi(6, 0.5, 0.5)).to(DEV)
    with torch.no_grad():
        for i, layer in enumerate(model):
            layer.coef.copy_(randn(layer.coef.shape, 1 + i, 1 / math.sqrt(layer.in_features * 7)))
    x = (torch.rand(65536, 2, generator=torch.Generator().manual_seed(0)) * 2 - 1).to(DEV)
    return model, x


def test_pinn_edge_derivative_order2_full_size_matches_oracle():
    model, x = _pinn()
    with torch.no_grad():
        edges = model.edge_derivative(x, 2)
        inputs = [h for _, h in layer_inputs(model, x)]
    rows = np.sort(np.random.default_rng(13).choice(x.shape[0], 2048, replace=False))
    h64 = np64(x)[rows]
    for li, (layer, d, hin) in enumerate(zip(model, edges, inputs)):
        lay = layer_np(layer)
        ob, c, W, b = lay
        assert d.shape == (65536, layer.out_features, layer.in_features)
        # on the inputs the layer received on the device, and through the oracle chain
        check(f"pinn layer {li} edge order 2", np64(d[rows]), o.edge_derivative(np64(hin)[rows], c, ob, 2, W), 1e-5)
        check(f"pinn layer {li} edge order 2 (chain)", np64(d[rows]), o.edge_derivative(h64, c, ob, 2, W), 1e-5)
        h64 = oracle_layer(h64, lay)


def _chained_second_derivative(layers, x, dim):
    """Forward-mode (h, h', h'') through KAN layers in float64."""
    h = x
    hp = np.zeros_like(x)
    hp[:, dim] = 1.0
    hpp = np.zeros_like(x)
    for ob, ceff, W, b in layers:
        e1 = o.edge_derivative(h, ceff, ob, 1, W)
        e2 = o.edge_derivative(h, ceff, ob, 2, W)
        h, hp, hpp = (
            o.kan_linear(h, ceff, ob, W, b),
            np.einsum("boi,bi->bo", e1, hp),
            np.einsum("boi,bi->bo", e2, hp**2) + np.einsum("boi,bi->bo", e1, hpp),
        )
    return hpp[:, 0]


def test_pinn_laplacian_full_size_matches_forward_mode_oracle():
    model, x = _pinn()
    lap = laplacian(model, x)
    assert lap.shape == (65536,)
    rows = np.sort(np.random.default_rng(14).choice(x.shape[0], 4096, replace=False))
    layers = [layer_np(layer) for layer in model]
    xr = np64(x)[rows]
    want = sum(_chained_second_derivative(layers, xr, d) for d in range(2))
    check("pinn laplacian rows", np64(lap)[rows], want, 1e-5)
