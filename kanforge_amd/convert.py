"""Model files in kanforge's backend-independent format.

``save(model, path)`` writes one ``.npz``: every array of the model under its
dotted name (``"0.coef"``, ``"1.basis_grid"``, ...) plus ``__spec__``, a JSON
string ``{"format": 1, "source": "torch", "model": spec}`` describing the
architecture; ``load(path)`` rebuilds the model from it. The format is the one
of kanforge/convert.py:110-172 (spec and arrays) and :313-324 (save/load), so a
file moves between kanforge and this package unchanged; arrays are stored as
float64 like kanforge's ``_to_numpy`` (kanforge/torch/layers.py:231-232) and
cast back to the layer's dtype on load, which is exact for float32, bfloat16
and float64 layers. Only the torch backend exists here.
"""

from __future__ import annotations

import functools
import json

import numpy as np
import torch
import torch.nn.functional as F
from torch import nn

from .torch.layers import GRKAN, KAN, KANLinear, rebuild_kan

FORMAT = 1


# --- activations by portable name (kanforge/convert.py:28-105) ----------------------------


def activation_name(act) -> str | None:
    """Portable name of a base activation or activation layer (None = absent)."""
    if act is None:
        return None
    if isinstance(act, _Lambda):
        act = act.fn
    if isinstance(act, functools.partial) and getattr(act.func, "__name__", "") == "gelu":
        return "gelu_tanh" if act.keywords.get("approximate") in (True, "tanh") else "gelu"
    if isinstance(act, nn.GELU):
        return "gelu_tanh" if act.approximate == "tanh" else "gelu"
    names = (type(act).__name__.lower(), getattr(act, "__name__", "").lower())
    for name in names:
        if name in ("identity", "_identity"):
            return "identity"
        if name in ("silu", "swish"):
            return "silu"
        if name in ("tanh", "relu", "sigmoid", "gelu"):
            return name
    raise ValueError(f"no portable name for activation {act!r}")


def make_activation(name: str | None):
    """The torch callable for a portable activation name."""
    if name is None:
        return None
    table = {
        "identity": nn.Identity(),
        "silu": F.silu,
        "gelu": F.gelu,
        "gelu_tanh": functools.partial(F.gelu, approximate="tanh"),
        "tanh": nn.Tanh(),
        "relu": nn.ReLU(),
        "sigmoid": nn.Sigmoid(),
    }
    if name not in table:
        raise ValueError(f"unknown activation {name!r}")
    return table[name]


class _Lambda(nn.Module):
    """A plain activation function as a module (for ``Sequential`` models)."""

    def __init__(self, fn):
        super().__init__()
        self.fn = fn

    def forward(self, x):
        return self.fn(x)


def _dtype_name(t: torch.Tensor) -> str:
    return str(t.dtype).replace("torch.", "")


def _np(t: torch.Tensor) -> np.ndarray:
    """NumPy copy; dtypes NumPy lacks (bfloat16, float16) as float64 (exact)."""
    t = t.detach().cpu()
    return t.numpy() if t.dtype in (torch.float32, torch.float64) else t.double().numpy()


# --- model -> (spec, arrays) ------------------------------------------------------------------


def _layer_spec(layer: KANLinear) -> tuple[dict, dict]:
    kw = layer._init_kwargs
    spec = {
        "type": "GRKAN" if isinstance(layer, GRKAN) else "KANLinear",
        "in": layer.in_features,
        "out": layer.out_features,
        "basis": layer.basis.config(),
        "bias": bool(kw["bias"]),
        "base_activation": activation_name(kw["base_activation"]),
        "groups": kw["groups"],
        "edge_scale": bool(kw["edge_scale"]),
        "edge_dropout": float(kw["edge_dropout"]),
        "backend": kw["backend"],
        "dtype": _dtype_name(layer.coef),
    }
    return spec, {k: v for k, v in layer._export_full().items() if v is not None}


def to_spec(model: nn.Module) -> tuple[dict, dict[str, np.ndarray]]:
    """(spec, arrays) of a model made of ``KANLinear``/``GRKAN`` layers, ``KAN`` stacks,
    ``nn.Sequential``, ``nn.Linear`` and activation modules."""
    arrays: dict[str, np.ndarray] = {}

    def walk(m, prefix):
        if isinstance(m, KANLinear):
            spec, arr = _layer_spec(m)
            arrays.update({prefix + k: v for k, v in arr.items()})
            return spec
        if isinstance(m, KAN):
            return {"type": "KAN", "widths": [int(w) for w in m.widths], "layers": [walk(c, f"{prefix}{k}.") for k, c in enumerate(m)]}
        if isinstance(m, nn.Sequential):
            return {"type": "Sequential", "layers": [walk(c, f"{prefix}{k}.") for k, c in enumerate(m)]}
        if isinstance(m, nn.Linear):
            arrays[prefix + "weight"] = _np(m.weight)
            if m.bias is not None:
                arrays[prefix + "bias"] = _np(m.bias)
            return {"type": "Linear", "in": m.in_features, "out": m.out_features, "bias": m.bias is not None, "dtype": _dtype_name(m.weight)}
        return {"type": "Activation", "name": activation_name(m)}

    return walk(model, ""), arrays


# --- (spec, arrays) -> model ------------------------------------------------------------------


def _build(spec: dict, arrays: dict, prefix: str, device) -> nn.Module:
    t = spec["type"]
    if t in ("KANLinear", "GRKAN"):
        layer = KANLinear(
            spec["in"],
            spec["out"],
            spec["basis"],
            bias=spec["bias"],
            base_activation=make_activation(spec["base_activation"]),
            groups=spec["groups"],
            edge_scale=spec["edge_scale"],
            edge_dropout=spec["edge_dropout"],
            backend=spec["backend"],
            dtype=getattr(torch, spec.get("dtype", "float32")),
            device=device,
        )
        state = {k[len(prefix) :]: v for k, v in arrays.items() if k.startswith(prefix) and "." not in k[len(prefix) :]}
        layer._import_full(state)
        return layer
    if t in ("KAN", "Sequential"):
        children = [_build(c, arrays, f"{prefix}{k}.", device) for k, c in enumerate(spec["layers"])]
        return rebuild_kan(children) if t == "KAN" else nn.Sequential(*children)
    if t == "Linear":
        lin = nn.Linear(spec["in"], spec["out"], bias=spec["bias"], dtype=getattr(torch, spec.get("dtype", "float32")), device=device)
        with torch.no_grad():
            lin.weight.copy_(torch.as_tensor(arrays[prefix + "weight"]))
            if spec["bias"]:
                lin.bias.copy_(torch.as_tensor(arrays[prefix + "bias"]))
        return lin
    if t == "Activation":
        act = make_activation(spec["name"])
        return act if isinstance(act, nn.Module) else _Lambda(act)
    raise ValueError(f"layer type {t!r} is not part of this build")


def from_spec(spec: dict, arrays: dict, device=None) -> nn.Module:
    """Build the model described by ``spec`` and load ``arrays`` into it."""
    return _build(spec, arrays, "", device)


def save(model: nn.Module, path) -> None:
    """Write ``model`` to ``path`` (``.npz``) in kanforge's file format."""
    spec, arrays = to_spec(model)
    np.savez(path, __spec__=np.array(json.dumps({"format": FORMAT, "source": "torch", "model": spec})), **arrays)


def load(path, device=None) -> nn.Module:
    """Load a file written by ``save`` here or by kanforge (any of its backends)."""
    with np.load(path, allow_pickle=False) as data:
        meta = json.loads(str(data["__spec__"]))
        arrays = {k: data[k] for k in data.files if k != "__spec__"}
    if meta.get("format") != FORMAT:
        raise ValueError(f"unsupported file format {meta.get('format')!r}")
    return from_spec(meta["model"], arrays, device)
