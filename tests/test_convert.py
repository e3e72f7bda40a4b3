"""kanforge's model file format (kanforge/convert.py:110-172, 313-324): save -> load
round trips are exact for every array and dtype, the file holds the spec and the arrays
under the names kanforge uses, and activations map to the same portable names
(kanforge tests/test_export.py:67-84). Host only: no kernel runs here."""

import functools
import json

import numpy as np
import pytest
import torch

import kanforge_amd as kf
from kanforge_amd import convert as cv
from kanforge_amd.torch import GRKAN, KAN, KANLinear


def arrays_equal(a, b):
    sa, sb = a.state_dict(), b.state_dict()
    assert sa.keys() == sb.keys()
    for k in sa:
        assert sa[k].dtype == sb[k].dtype, k
        assert torch.equal(sa[k], sb[k]), k


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16])
def test_kan_round_trip_is_exact(tmp_path, dtype):
    torch.manual_seed(0)
    model = KAN([2, 3, 1], kf.BSpline(4, 3), dtype=dtype)
    model[0].update_grid(torch.randn(100, 2, dtype=torch.float64) * 0.4)  # as kanforge's test does
    with torch.no_grad():
        model[1].edge_mask[0, 1] = 0
    path = tmp_path / "m.npz"
    cv.save(model, path)
    back = cv.load(path)
    assert isinstance(back, KAN) and back.widths == [2, 3, 1]
    assert back[0].coef.dtype == dtype
    arrays_equal(model, back)


def test_file_layout_matches_kanforge(tmp_path):
    model = KAN([2, 3, 1], kf.Chebyshev(8), bias=False)
    path = tmp_path / "m.npz"
    cv.save(model, path)
    with np.load(path, allow_pickle=False) as data:
        meta = json.loads(str(data["__spec__"]))
        keys = set(data.files)
        assert data["0.coef"].dtype == np.float64 and data["0.coef"].shape == (3, 2, 9)
    assert meta["format"] == 1 and meta["source"] == "torch"
    spec = meta["model"]
    assert spec["type"] == "KAN" and spec["widths"] == [2, 3, 1] and len(spec["layers"]) == 2
    layer = spec["layers"][0]
    assert layer["type"] == "KANLinear" and (layer["in"], layer["out"]) == (2, 3)
    assert layer["basis"] == kf.Chebyshev(8).config() and layer["base_activation"] == "silu"
    assert layer["bias"] is False and layer["dtype"] == "float32"
    assert {"0.coef", "0.base_weight", "0.edge_mask", "0.sym_code", "0.sym_params", "1.coef"} <= keys
    assert "0.bias" not in keys and "0.edge_scale" not in keys


def test_grkan_and_sequential_round_trip(tmp_path):
    torch.manual_seed(1)
    model = torch.nn.Sequential(
        torch.nn.Linear(8, 16),
        torch.nn.GELU(approximate="tanh"),
        GRKAN(16, 8, groups=4),
        KANLinear(8, 4, kf.Jacobi(6, 0.5, 0.5), edge_scale=True, base_activation=torch.nn.functional.gelu),
    )
    path = tmp_path / "m.npz"
    cv.save(model, path)
    back = cv.load(path)
    assert isinstance(back[0], torch.nn.Linear) and isinstance(back[2], KANLinear) and isinstance(back[3], KANLinear)
    assert back[2].basis == model[2].basis and back[3].basis == model[3].basis
    assert cv.activation_name(back[1]) == "gelu_tanh"
    arrays_equal(model, back)


def test_activation_names():
    assert cv.activation_name(torch.nn.functional.silu) == "silu"
    assert cv.activation_name(torch.nn.GELU()) == "gelu"
    assert cv.activation_name(torch.nn.GELU(approximate="tanh")) == "gelu_tanh"
    assert cv.activation_name(functools.partial(torch.nn.functional.gelu, approximate="tanh")) == "gelu_tanh"
    assert cv.activation_name(torch.nn.Identity()) == "identity"
    assert cv.activation_name(None) is None
    for name in ("silu", "gelu", "gelu_tanh", "tanh", "relu", "sigmoid", "identity"):
        assert cv.activation_name(cv.make_activation(name)) == name
    with pytest.raises(ValueError):
        cv.make_activation("swishy")


def test_unknown_format_raises(tmp_path):
    path = tmp_path / "m.npz"
    np.savez(path, __spec__=np.array(json.dumps({"format": 99, "source": "torch", "model": {}})))
    with pytest.raises(ValueError, match="format"):
        cv.load(path)
