"""Grid tools (kanforge/grid.py:1-84, kanforge/_layer.py:99-191), host side: adaptive grids
against their definition and edge cases, and the refit pinned by what the mathematics fixes:
when the new basis spans the old edge functions (a Chebyshev degree raised, a uniform
B-spline grid refined by an integer factor, whose knots nest) the refit reproduces them to
rounding error at fresh points; edge scales are kept."""

import numpy as np
import pytest
import torch

import kanforge_amd as kf
from kanforge_amd import grid as gt
from kanforge_amd.torch import GRKAN, KANLinear

rng = np.random.default_rng(0)


def edge_functions(layer, x):
    """(N, out, in) edge function values of a layer at host points x (N, in), float64."""
    snap = layer._snapshot()
    phi = layer.basis.host_values(x, snap.per_input())
    return np.einsum("nik,oik->noi", phi, snap.effective_coef())


def test_adaptive_grid_definition():
    x = rng.normal(0, 1, (500, 3))
    g = gt.adaptive_grid(x, 9, margin=0.1, grid_eps=0.02)
    xs = np.sort(x, axis=0)
    ranks = np.rint(np.linspace(0, 499, 9)).astype(int)
    lo, hi = xs[0] - 0.1, xs[-1] + 0.1
    uni = lo[:, None] + (hi - lo)[:, None] * np.linspace(0, 1, 9)
    np.testing.assert_allclose(g, 0.02 * uni + 0.98 * xs[ranks].T, rtol=0, atol=1e-14)
    np.testing.assert_allclose(gt.adaptive_grid(x, 9, 0.1, 1.0), uni, atol=1e-14)  # all uniform
    assert (np.diff(g, axis=1) > 0).all()


def test_adaptive_grid_edge_cases():
    x = np.concatenate([np.zeros((50, 1)), np.full((50, 1), 2.0)], axis=0)  # repeated values
    assert (np.diff(gt.adaptive_grid(x, 6), axis=1) > 0).all()  # the uniform part keeps it increasing
    flat = gt.adaptive_grid(np.full((10, 2), 0.3), 5)
    np.testing.assert_allclose(flat, np.tile(np.linspace(-0.2, 0.8, 5), (2, 1)), atol=1e-14)
    with pytest.raises(ValueError):
        gt.adaptive_grid(x, 6, grid_eps=0.0)


def test_resample_grid_keeps_ends_and_shape():
    g = np.stack([np.linspace(-1, 1, 5), np.array([-2.0, -1.0, 0.0, 2.0, 3.0])])
    r = gt.resample_grid(g, 9)
    np.testing.assert_allclose(r[:, [0, -1]], g[:, [0, -1]])
    np.testing.assert_allclose(r[0], np.linspace(-1, 1, 9), atol=1e-15)
    np.testing.assert_allclose(r[1, ::2], g[1], atol=1e-15)  # old points kept


def test_change_basis_to_a_larger_polynomial_space_is_exact():
    torch.manual_seed(0)
    layer = KANLinear(3, 4, kf.Chebyshev(4), dtype=torch.float64, edge_scale=True)
    with torch.no_grad():
        layer.edge_scale.uniform_(0.5, 1.5)
    x_fit = rng.uniform(-2, 2, (400, 3))
    x_new = rng.uniform(-2, 2, (50, 3))
    before = edge_functions(layer, x_new)
    scale = layer.edge_scale.detach().clone()
    layer.change_basis(kf.Chebyshev(8), x_fit)
    assert layer.basis == kf.Chebyshev(8) and layer.coef.shape == (4, 3, 9)
    torch.testing.assert_close(layer.edge_scale.detach(), scale, rtol=0, atol=0)
    np.testing.assert_allclose(edge_functions(layer, x_new), before, atol=1e-10)


def test_refine_uniform_bspline_grid_is_exact():
    torch.manual_seed(1)
    layer = KANLinear(2, 3, kf.BSpline(4, 3), dtype=torch.float64)
    x_new = rng.uniform(-0.99, 0.99, (60, 2))
    before = edge_functions(layer, x_new)
    layer.refine_grid(8)
    assert layer.basis.grid_size == 8 and layer.coef.shape == (3, 2, 11) and layer.basis_grid.shape == (2, 9)
    np.testing.assert_allclose(edge_functions(layer, x_new), before, atol=1e-10)


def test_update_grid_moves_the_grid_to_the_data():
    torch.manual_seed(2)
    layer = KANLinear(2, 3, kf.BSpline(5, 3), dtype=torch.float64)
    x = rng.normal(0, 0.3, (300, 2))
    layer.update_grid(torch.as_tensor(x))
    np.testing.assert_allclose(layer.basis_grid.numpy(), gt.adaptive_grid(x, 6), atol=1e-14)
    assert layer.coef.shape == (3, 2, 8)


def test_change_basis_without_samples_uses_the_grid_range():
    torch.manual_seed(3)
    layer = KANLinear(2, 2, kf.BSpline(6, 3), dtype=torch.float64)
    layer.change_basis(kf.Chebyshev(6, input_map="identity"))
    assert layer.coef.shape == (2, 2, 7) and layer._plan.kind == "cheb"


def test_grid_free_bases_refuse_grid_updates():
    layer = GRKAN(8, 4, groups=4, dtype=torch.float64)
    with pytest.raises(TypeError):
        layer.update_grid(torch.zeros(10, 8))
    with pytest.raises(TypeError):
        layer.refine_grid(8)
    with pytest.raises(ValueError):
        KANLinear(2, 2, kf.Chebyshev(3)).change_basis(kf.Chebyshev(5))  # no grid and no samples
