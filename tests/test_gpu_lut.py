"""Lookup-table inference (kanforge/export/lut.py) on the HIP gather + lerp kernel, against the
float64 oracle: float32, int8 and int16 tables, ragged shapes, both extrapolation modes; and the
tabulation of real models (kanforge tests/test_export.py:95-120)."""

import numpy as np
import pytest
import torch

import kanforge_amd as kf
from kanforge_amd.export import LUTLayer, LUTModel, quantize, to_lut
from kanforge_amd.torch import KAN
from oracle import kan64 as o

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("shape", [(300, 7, 1), (257, 3, 5), (130, 64, 64), (100, 16, 100), (70, 1, 33)],
                         ids=["7to1", "3to5", "64to64", "16to100", "1to33"])
@pytest.mark.parametrize("kind", ["f32", "int8", "int16"])
@pytest.mark.parametrize("extrapolate", ["linear", "clamp"])
def test_lut_kernel_matches_oracle(shape, kind, extrapolate):
    B, n_in, n_out = shape
    rng = np.random.default_rng(B + n_in)
    size = 37
    T = rng.normal(size=(n_in, size, n_out))
    lo = rng.uniform(-2, -0.5, n_in)
    hi = rng.uniform(0.5, 2, n_in)
    bias = rng.normal(size=n_out)
    s_lo, s_hi = o.lut_end_slopes(T)
    x = rng.uniform(-3, 3, (B, n_in)).astype(np.float32)
    x[: min(B, 5)] = lo + (hi - lo) * rng.integers(0, size, (min(B, 5), n_in)) / (size - 1)  # on table points
    if kind == "f32":
        tables, scale, b = T.astype(np.float32), None, bias
    else:
        tables, scale, b = o.lut_quantize(T, bias, 8 if kind == "int8" else 16)
    layer = LUTLayer(tables, lo, hi, b, scale=scale, slope_lo=s_lo, slope_hi=s_hi)
    got = layer(torch.as_tensor(x, device=DEV), extrapolate).double().cpu().numpy()
    want = o.lut_layer(x, tables, lo, hi, b, scale, s_lo, s_hi, extrapolate)
    assert o.normwise_err(got, want) <= 1e-5


def test_lut_of_a_kan_converges_and_quantizes():
    """Tables of 64, 256, 1024 points approach the model (the largest within 1e-4 of its scale);
    int8 tables stay within 3e-2 and take less than a third of the bytes."""
    torch.manual_seed(0)
    model = KAN([3, 5, 2], kf.BSpline(5, 3)).to(DEV)
    x = torch.rand(3000, 3, device=DEV) * 2 - 1
    xin = torch.rand(500, 3, device=DEV) * 1.8 - 0.9
    with torch.no_grad():
        ref = model(xin).double().cpu().numpy()
    scale = np.abs(ref).max()
    errs = [np.abs(to_lut(model, x, size)(xin).double().cpu().numpy() - ref).max() / scale for size in (64, 256, 1024)]
    assert errs[2] < 1e-4 and errs[2] < errs[0], errs
    lut = to_lut(model, x, 256)
    q = quantize(lut)
    assert np.abs(q(xin).double().cpu().numpy() - ref).max() / scale < 3e-2
    assert q.nbytes() < lut.nbytes() / 3
    # NumPy in, NumPy out
    got = lut(xin.cpu().numpy())
    assert isinstance(got, np.ndarray) and got.shape == (500, 2)


def test_lut_extrapolation_modes():
    """Beyond the range, linear extrapolation adds the end slope per unit of x; clamp holds the
    end value (kanforge tests/test_export.py:110-120)."""
    torch.manual_seed(1)
    model = KAN([1, 1], kf.BSpline(5, 3)).to(DEV)
    lut = to_lut(model, torch.rand(500, 1, device=DEV) * 2 - 1, 256, margin=0.0)
    layer = lut.layers[0]
    slope = layer.slope_hi[0, 0] / layer.step[0]
    far = np.array([[3.0]])
    lin = lut(far)
    lut.extrapolate = "clamp"
    clamp = lut(far)
    np.testing.assert_allclose(clamp, lut(np.array([[layer.hi[0]]])), rtol=1e-6)
    np.testing.assert_allclose(lin - clamp, slope * (3.0 - layer.hi[0]), rtol=1e-5)


def test_lut_tables_match_the_oracle_edges():
    """The tables are the model's edges at uniform points: each column equals the oracle's
    edge_derivative(x, 0) at those points (B-spline + SiLU base)."""
    torch.manual_seed(2)
    model = KAN([2, 3], kf.BSpline(4, 3)).to(DEV)
    lut = to_lut(model, None, 33, margin=0.0)
    layer, kan = lut.layers[0], model[0]
    pts = layer.lo + (layer.hi - layer.lo) * np.linspace(0, 1, 33)[:, None]
    ob = o.Basis64("bspline", grid=kan.basis_grid.double().cpu().numpy(), k=3)
    want = o.edge_derivative(pts, kan.effective_coef().double().detach().cpu().numpy(), ob, 0,
                             kan.effective_base_weight().double().detach().cpu().numpy())  # (size, out, in)
    np.testing.assert_allclose(layer.tables, want.transpose(2, 0, 1), rtol=0, atol=1e-5 * np.abs(want).max())


def test_lut_rejects_bad_arguments():
    layer = LUTLayer(np.zeros((2, 4, 3), np.float32), np.zeros(2), np.ones(2), np.zeros(3))
    with pytest.raises(ValueError):
        layer(torch.zeros(5, 2, device=DEV), "cubic")
    bad = LUTLayer(np.zeros((2, 4, 3), np.int8), np.zeros(2), np.ones(2), np.zeros(3))  # int tables, no scale
    with pytest.raises(RuntimeError):
        bad(torch.zeros(5, 2, device=DEV))
    assert LUTModel([layer])(np.zeros((0, 2))).shape == (0, 3)
