"""Transformer feed-forward blocks built from KAN layers, and FFN replacement in existing models.

API of kanforge/torch/transformer.py:1-167 (``KANFFN``, ``KATBlock``, ``kanify``); the module
layout (``fc1``/``fc2`` inside ``KANFFN``) is kept so state_dicts and kanforge.save files match.

The model surgery is table-driven: ``FFN_PATTERNS`` lists the feed-forward layouts of the common
transformer families as dotted attribute paths (projection in, activation, projection out), and
``find_ffns`` resolves every pattern against every submodule into ``FFNSite`` records whose slots
can be read and replaced. Gated FFNs (``down(act(gate(x)) * up(x))``) have a pattern of their own.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from .layers import GRKAN, KANLinear

__all__ = ["KANFFN", "KATBlock", "kanify", "find_ffns", "FFN_PATTERNS", "GATED_PATTERN"]


class KANFFN(nn.Module):
    """``dim -> hidden -> dim`` with two KAN layers.

    ``kind="grkan"``: KAT's two group-rational layers, the first rational starting as the
    identity and the second as ``activation``; ``kind="kan"``: two ``KANLinear`` of ``basis``
    with ``kan_kwargs``. Dropout (``dropout``) follows each layer.
    """

    def __init__(self, dim: int, hidden: int | None = None, kind: str = "grkan", basis="bspline", groups: int = 8,
                 activation: str = "gelu", dropout: float = 0.0, **kan_kwargs):
        super().__init__()
        width = 4 * dim if hidden is None else hidden
        builders = {
            "grkan": lambda i, o, init: GRKAN(i, o, groups=groups, init=init),
            "kan": lambda i, o, init: KANLinear(i, o, basis, **kan_kwargs),
        }
        if kind not in builders:
            raise ValueError("kind must be 'grkan' or 'kan'")
        make = builders[kind]
        self.fc1 = make(dim, width, "identity")
        self.fc2 = make(width, dim, activation)
        self.drop = nn.Dropout(dropout)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        h = self.drop(self.fc1(x))
        return self.drop(self.fc2(h))


class KATBlock(nn.Module):
    """Pre-norm Kolmogorov-Arnold Transformer block: self-attention, then ``KANFFN``, each on the
    layer-normalised stream and added back to it."""

    def __init__(self, dim: int, heads: int, mlp_ratio: float = 4.0, kind: str = "grkan", dropout: float = 0.0,
                 **ffn_kwargs):
        super().__init__()
        self.norm1 = nn.LayerNorm(dim)
        self.attn = nn.MultiheadAttention(dim, heads, dropout=dropout, batch_first=True)
        self.norm2 = nn.LayerNorm(dim)
        self.ffn = KANFFN(dim, int(dim * mlp_ratio), kind, dropout=dropout, **ffn_kwargs)

    def forward(self, x: torch.Tensor, attn_mask=None, key_padding_mask=None) -> torch.Tensor:
        q = self.norm1(x)
        attended, _ = self.attn(q, q, q, attn_mask=attn_mask, key_padding_mask=key_padding_mask, need_weights=False)
        x = x + attended
        return x + self.ffn(self.norm2(x))


# --- model surgery ---------------------------------------------------------------------------


@dataclass(frozen=True)
class FFNPattern:
    """A feed-forward layout as dotted paths relative to the block that owns it. ``act`` lists
    candidate paths of the activation (the first one present is used)."""

    family: str
    proj_in: str
    act: tuple[str, ...]
    proj_out: str


FFN_PATTERNS = (
    FFNPattern("vit/clip/encoder", "fc1", ("activation_fn", "act", "act_fn", "activation"), "fc2"),
    FFNPattern("gpt2", "c_fc", ("act",), "c_proj"),
    FFNPattern("bert", "intermediate.dense", ("intermediate.intermediate_act_fn",), "output.dense"),
)
GATED_PATTERN = ("gate_proj", "up_proj", "down_proj")  # LLaMA, Mistral, Qwen, Gemma

# activation class-name fragments (or functions) -> rational initialisation target
_RATIONAL_TARGETS = (("gelu", "gelu"), ("silu", "silu"), ("swish", "silu"), ("tanh", "tanh"))
_FUNCTION_TARGETS = {F.gelu: "gelu", F.silu: "silu", torch.tanh: "tanh"}


@dataclass
class _Slot:
    """An attribute of a module, addressed by a dotted path from a root module."""

    owner: nn.Module
    attr: str

    @classmethod
    def resolve(cls, root: nn.Module, path: str) -> "_Slot | None":
        *parents, attr = path.split(".")
        owner = root
        for part in parents:
            owner = getattr(owner, part, None)
            if owner is None:
                return None
        return cls(owner, attr) if hasattr(owner, attr) else None

    def get(self):
        return getattr(self.owner, self.attr)

    def set(self, value) -> None:
        setattr(self.owner, self.attr, value)


@dataclass
class FFNSite:
    name: str
    pattern: FFNPattern
    proj_in: _Slot
    act: _Slot
    proj_out: _Slot


def find_ffns(model: nn.Module) -> list[FFNSite]:
    """Every submodule of ``model`` that matches one of ``FFN_PATTERNS`` (the first pattern that
    matches a module wins), in ``named_modules`` order."""
    sites = []
    for name, module in model.named_modules():
        for pattern in FFN_PATTERNS:
            pin, pout = _Slot.resolve(module, pattern.proj_in), _Slot.resolve(module, pattern.proj_out)
            act = next((s for s in (_Slot.resolve(module, p) for p in pattern.act) if s is not None), None)
            if pin is not None and pout is not None and act is not None:
                sites.append(FFNSite(name, pattern, pin, act, pout))
                break
    return sites


def _to_linear(module: nn.Module) -> nn.Linear:
    """``module`` as an ``nn.Linear``: itself, or the transpose of a GPT-2 ``Conv1D``
    (weight ``(in, out)``, ``y = x W + b``)."""
    if isinstance(module, nn.Linear):
        return module
    if type(module).__name__ != "Conv1D":
        raise TypeError(f"not a linear layer: {type(module).__name__}")
    weight = module.weight
    linear = nn.Linear(weight.shape[0], weight.shape[1], device=weight.device, dtype=weight.dtype)
    with torch.no_grad():
        linear.weight.copy_(weight.t())
        linear.bias.copy_(module.bias)
    return linear


def rational_target(act) -> str:
    """The rational initialisation that approximates an activation module or function."""
    if act in _FUNCTION_TARGETS:
        return _FUNCTION_TARGETS[act]
    cls = type(act).__name__.lower()
    for fragment, target in _RATIONAL_TARGETS:
        if fragment in cls:
            return target
    raise ValueError(f"no rational initialisation for activation {type(act).__name__}")


def _grkan_from(linear: nn.Linear, groups: int, init: str) -> GRKAN:
    """A GR-KAN layer carrying ``linear``'s weight as its coefficients and its bias."""
    layer = GRKAN(linear.in_features, linear.out_features, groups=groups, init=init, bias=linear.bias is not None)
    layer = layer.to(device=linear.weight.device, dtype=linear.weight.dtype)
    with torch.no_grad():
        layer.coef.copy_(linear.weight.unsqueeze(-1))
        if linear.bias is not None:
            layer.bias.copy_(linear.bias)
    return layer


def kanify(model: nn.Module, mode: str = "exact", basis="bspline", groups: int = 8, **kan_kwargs) -> list[str]:
    """Replace the feed-forward blocks of ``model`` in place and return the names of the blocks
    replaced.

    ``mode="exact"`` keeps the model's function: the output projection becomes a ``KANLinear``
    whose base branch is the activation with the projection's weights and whose splines start at
    zero, and the activation slot becomes an identity. A gated FFN's down projection becomes a
    ``KANLinear`` with an identity base branch.
    ``mode="grkan"`` moves the weights into GR-KAN layers as KAT does: the input projection's
    rationals start as the identity, the output projection's as the activation (approximately,
    to ~1e-2); gated FFNs are left as they are.
    """
    if mode not in ("exact", "grkan"):
        raise ValueError("mode must be 'exact' or 'grkan'")
    replaced = []
    for site in find_ffns(model):
        act = site.act.get()
        lin_in, lin_out = _to_linear(site.proj_in.get()), _to_linear(site.proj_out.get())
        if mode == "exact":
            site.proj_in.set(lin_in)
            site.proj_out.set(KANLinear.from_linear(lin_out, act, basis, **kan_kwargs))
        else:
            site.proj_in.set(_grkan_from(lin_in, groups, "identity"))
            site.proj_out.set(_grkan_from(lin_out, groups, rational_target(act)))
        site.act.set(nn.Identity())
        replaced.append(site.name)
    if mode == "exact":
        for name, module in model.named_modules():
            if not all(hasattr(module, a) for a in GATED_PATTERN) or isinstance(module.down_proj, KANLinear):
                continue
            module.down_proj = KANLinear.from_linear(module.down_proj, nn.Identity(), basis, **kan_kwargs)
            replaced.append(name)
    return replaced
