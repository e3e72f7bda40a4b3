"""KAN feed-forward blocks for transformers, and FFN replacement in existing models
(kanforge/torch/transformer.py:1-167).

* ``KANFFN``: dim -> hidden -> dim with two ``KANLinear`` (``kind="kan"``, any basis) or
  two group-rational layers (``kind="grkan"``, KAT: the first rational starts as the
  identity, the second as the activation).
* ``KATBlock``: pre-norm block, ``x + attn(norm(x))`` then ``x + KANFFN(norm(x))``.
* ``kanify(model)``: replace the FFNs of a model in place. ``mode="exact"`` keeps the
  outputs (the activation becomes the base branch of a ``KANLinear`` whose splines start at
  zero); ``mode="grkan"`` moves the weights into GR-KAN layers as KAT does from ViT (the
  rationals approximate the activation to about 1e-2).

Every KAN layer here runs the HIP kernels; nothing else in these modules is on that path.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from .layers import GRKAN, KANLinear

# activation (class or function name fragment) -> rational initialisation target
ACT_TARGETS = {"gelu": "gelu", "silu": "silu", "swish": "silu", "tanh": "tanh"}


class KANFFN(nn.Module):
    """dim -> hidden -> dim with KAN layers (``kind="kan"``) or GR-KAN (``kind="grkan"``)."""

    def __init__(
        self,
        dim: int,
        hidden: int | None = None,
        kind: str = "grkan",
        basis="bspline",
        groups: int = 8,
        activation: str = "gelu",
        dropout: float = 0.0,
        **kan_kwargs,
    ):
        super().__init__()
        hidden = hidden or 4 * dim
        if kind == "grkan":
            self.fc1 = GRKAN(dim, hidden, groups=groups, init="identity")
            self.fc2 = GRKAN(hidden, dim, groups=groups, init=activation)
        elif kind == "kan":
            self.fc1 = KANLinear(dim, hidden, basis, **kan_kwargs)
            self.fc2 = KANLinear(hidden, dim, basis, **kan_kwargs)
        else:
            raise ValueError("kind must be 'grkan' or 'kan'")
        self.drop = nn.Dropout(dropout)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.drop(self.fc2(self.drop(self.fc1(x))))


class KATBlock(nn.Module):
    """``x + attn(norm(x))``; ``x + KANFFN(norm(x))`` (the Kolmogorov-Arnold Transformer block)."""

    def __init__(self, dim: int, heads: int, mlp_ratio: float = 4.0, kind: str = "grkan", dropout: float = 0.0, **ffn_kwargs):
        super().__init__()
        self.norm1 = nn.LayerNorm(dim)
        self.attn = nn.MultiheadAttention(dim, heads, dropout=dropout, batch_first=True)
        self.norm2 = nn.LayerNorm(dim)
        self.ffn = KANFFN(dim, int(dim * mlp_ratio), kind, dropout=dropout, **ffn_kwargs)

    def forward(self, x: torch.Tensor, attn_mask=None, key_padding_mask=None) -> torch.Tensor:
        h = self.norm1(x)
        x = x + self.attn(h, h, h, attn_mask=attn_mask, key_padding_mask=key_padding_mask, need_weights=False)[0]
        return x + self.ffn(self.norm2(x))


# --- FFN replacement in existing models -------------------------------------------------------


def _as_linear(module) -> nn.Linear:
    """An ``nn.Linear`` computing the same map as ``module`` (``nn.Linear``, or a ``Conv1D``
    with weight ``(in, out)`` as in GPT-2: ``y = x W + b``)."""
    if isinstance(module, nn.Linear):
        return module
    if type(module).__name__ == "Conv1D":
        w = module.weight
        lin = nn.Linear(w.shape[0], w.shape[1], device=w.device, dtype=w.dtype)
        with torch.no_grad():
            lin.weight.copy_(w.T)
            lin.bias.copy_(module.bias)
        return lin
    raise TypeError(f"not a linear layer: {type(module).__name__}")


def _rational_target(act) -> str:
    name = type(act).__name__.lower()
    for key, target in ACT_TARGETS.items():
        if key in name:
            return target
    if act is F.gelu:
        return "gelu"
    if act is F.silu:
        return "silu"
    raise ValueError(f"no rational initialisation for activation {type(act).__name__}")


def _ffn_sites(model: nn.Module) -> list[tuple]:
    """(name, owner and attribute of the first projection, of the activation, of the second
    projection) for every feed-forward block found: ``fc1, act, fc2`` (ViT, CLIP and most
    encoders), ``c_fc, act, c_proj`` (GPT-2), ``intermediate.dense,
    intermediate.intermediate_act_fn, output.dense`` (BERT-like)."""
    sites = []
    for name, m in model.named_modules():
        act_attr = next((a for a in ("activation_fn", "act", "act_fn", "activation") if hasattr(m, a)), None)
        if hasattr(m, "fc1") and hasattr(m, "fc2") and act_attr is not None:
            sites.append((name, m, "fc1", m, act_attr, m, "fc2"))
        elif hasattr(m, "c_fc") and hasattr(m, "c_proj") and hasattr(m, "act"):
            sites.append((name, m, "c_fc", m, "act", m, "c_proj"))
        elif hasattr(m, "intermediate") and hasattr(m, "output") and hasattr(m.intermediate, "intermediate_act_fn"):
            sites.append((name, m.intermediate, "dense", m.intermediate, "intermediate_act_fn", m.output, "dense"))
    return sites


def _gated_sites(model: nn.Module) -> list[tuple[str, nn.Module]]:
    """Gated FFNs ``down_proj(act(gate_proj(x)) * up_proj(x))`` (LLaMA, Mistral, Qwen, Gemma)."""
    return [(name, m) for name, m in model.named_modules() if all(hasattr(m, a) for a in ("gate_proj", "up_proj", "down_proj"))]


def kanify(model: nn.Module, mode: str = "exact", basis="bspline", groups: int = 8, **kan_kwargs) -> list[str]:
    """Replace the feed-forward blocks of ``model`` in place; returns their module names.

    ``mode="exact"``: the second projection becomes ``KANLinear.from_linear`` with the
    activation as its base branch and the activation slot an identity; a gated FFN's down
    projection becomes a ``KANLinear`` with an identity base. The model computes the same
    function until the splines are trained.
    ``mode="grkan"``: first projection -> GR-KAN with identity rationals, second -> GR-KAN
    with rationals fitted to the activation, weights copied (approximate). Gated FFNs are left
    alone in this mode.
    """
    if mode not in ("exact", "grkan"):
        raise ValueError("mode must be 'exact' or 'grkan'")
    done = []
    for name, own_in, a_in, own_act, a_act, own_out, a_out in _ffn_sites(model):
        act = getattr(own_act, a_act)
        lin_in, lin_out = _as_linear(getattr(own_in, a_in)), _as_linear(getattr(own_out, a_out))
        if mode == "exact":
            setattr(own_in, a_in, lin_in)
            setattr(own_out, a_out, KANLinear.from_linear(lin_out, act, basis, **kan_kwargs))
        else:
            target = _rational_target(act)
            fc1 = GRKAN(lin_in.in_features, lin_in.out_features, groups=groups, init="identity", bias=lin_in.bias is not None)
            fc2 = GRKAN(lin_out.in_features, lin_out.out_features, groups=groups, init=target, bias=lin_out.bias is not None)
            for layer, lin in ((fc1, lin_in), (fc2, lin_out)):
                layer.to(lin.weight.device, lin.weight.dtype)
                with torch.no_grad():
                    layer.coef.copy_(lin.weight[..., None])
                    if lin.bias is not None:
                        layer.bias.copy_(lin.bias)
            setattr(own_in, a_in, fc1)
            setattr(own_out, a_out, fc2)
        setattr(own_act, a_act, nn.Identity())
        done.append(name)
    if mode == "exact":
        for name, m in _gated_sites(model):
            if not isinstance(m.down_proj, KANLinear):
                m.down_proj = KANLinear.from_linear(m.down_proj, nn.Identity(), basis, **kan_kwargs)
                done.append(name)
    return done
