"""The torch-CPU plain routes the benchmark times as its CPU baseline agree with the oracle
(B-spline and GR-KAN layers, edge second derivatives) and with finite differences (Laplacian)."""

import numpy as np
import pytest
import torch

import kanforge_amd as kf
from kanforge_amd.torch import GRKAN, KAN, KANLinear
from oracle import kan64 as o
from oracle import torch_cpu as tc


def test_bspline_layer_matches_oracle():
    torch.manual_seed(0)
    layer = KANLinear(8, 5, kf.BSpline(5, 3))
    x = torch.rand(50, 8, dtype=torch.float64) * 2.2 - 1.1
    got = tc.CpuLayer(layer, torch.float64)(x).detach().numpy()
    basis = o.Basis64("bspline", grid=layer.basis_grid.double().numpy(), k=3)
    want = o.kan_linear(x.numpy(), layer.coef.double().detach().numpy(), basis,
                        layer.base_weight.double().detach().numpy(), layer.bias.double().detach().numpy())
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-12)


def test_grkan_layer_matches_oracle():
    torch.manual_seed(1)
    layer = GRKAN(16, 8, groups=4)
    with torch.no_grad():
        layer.basis_numerator.normal_(0, 0.3)
        layer.basis_denominator.normal_(0, 0.3)
    x = torch.randn(30, 16, dtype=torch.float64)
    got = tc.CpuLayer(layer, torch.float64)(x).detach().numpy()
    rep = lambda t: np.repeat(t.double().detach().numpy(), 4, 0)
    basis = o.Basis64("rational", num=rep(layer.basis_numerator), den=rep(layer.basis_denominator))
    want = o.kan_linear(x.numpy(), layer.coef.double().detach().numpy(), basis, None, layer.bias.double().detach().numpy())
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-12)


def test_edge_second_derivative_matches_oracle():
    torch.manual_seed(2)
    net = KAN([2, 6, 1], kf.Jacobi(6, 0.5, 0.5, input_map="tanh"))
    x = torch.rand(20, 2, dtype=torch.float64) * 2 - 1
    got = tc.CpuLayer(net[0], torch.float64).edge_second(x).numpy()
    basis = o.Basis64("poly", A=net[0].basis._cheb, input_map="tanh")
    want = o.edge_derivative(x.numpy(), net[0].coef.double().detach().numpy(), basis, 2,
                             net[0].base_weight.double().detach().numpy())
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-12 * np.abs(want).max())


def test_laplacian_matches_finite_differences():
    torch.manual_seed(3)
    net = KAN([2, 6, 1], kf.Jacobi(6, 0.5, 0.5, input_map="tanh"))
    layers = [tc.CpuLayer(m, torch.float64) for m in net]
    x = torch.rand(5, 2, dtype=torch.float64)
    xr = x.clone().requires_grad_()
    u = xr
    for layer in layers:
        u = layer(u)
    (g,) = torch.autograd.grad(u.sum(), xr, create_graph=True)
    lap = sum(torch.autograd.grad(g[:, d].sum(), xr, retain_graph=True)[0][:, d] for d in range(2))

    def f(p):
        h = p
        for layer in layers:
            h = layer(h)
        return h[:, 0].detach()

    eps, eye = 1e-4, torch.eye(2, dtype=x.dtype)
    fd = sum((f(x + eps * eye[d]) - 2 * f(x) + f(x - eps * eye[d])) / eps**2 for d in range(2))
    assert (lap - fd).abs().max().item() < 1e-5
    assert tc.time_laplacian_step(layers, x, reps=1)[0] > 0
