"""PINN derivatives of a field u(x) kept in the autograd graph (kanforge/torch/science.py:25-46).

``derivative``, ``gradient`` and ``laplacian`` accept any callable, as in the reference, and
differentiate it with autograd (through KAN layers every node is an F, G or P launch of the HIP
kernels). For a chain of KAN layers (``KAN``, or an ``nn.Sequential`` of ``KANLinear`` with SiLU or
no base branch) ``laplacian`` instead propagates second-order Taylor coefficients forward. Per
layer, with h'_d = dh/dx_d for every input dimension d and S = sum_d d2h/dx_d2:
    h_out    = F_0(h, c) + W silu(h) + b
    h'_out,d = F_1(h, c, w=h'_d)                          + W (silu'(h) h'_d)
    S_out    = F_2(h, c, w=sum_d h'_d^2) + F_1(h, c, w=S) + W (silu''(h) sum_d h'_d^2 + silu'(h) S)
F is linear in its weight w, so the second-order terms of all dimensions collapse into one F_2
and one F_1 row block: each layer runs F on (D + 3) rows per point (the first layer D + 2), the
rows of the first-order launches stacked into one call. The result is the same function of x
and of the parameters, and stays differentiable (F's own autograd).
"""

from __future__ import annotations

from collections.abc import Callable

import torch
import torch.nn.functional as F
from torch import nn


def derivative(fn: Callable, x: torch.Tensor, order: int = 1, dim: int = 0) -> torch.Tensor:
    """d^order u / dx_dim^order for u = fn(x), x ``(N, d)``, u ``(N,)`` or ``(N, 1)``."""
    x = x if x.requires_grad else x.detach().requires_grad_()
    u = fn(x).reshape(x.shape[0])
    for _ in range(order):
        (g,) = torch.autograd.grad(u.sum(), x, create_graph=True)
        u = g[:, dim]
    return u


def gradient(fn: Callable, x: torch.Tensor) -> torch.Tensor:
    """(N, d) gradient of u = fn(x)."""
    x = x if x.requires_grad else x.detach().requires_grad_()
    (g,) = torch.autograd.grad(fn(x).reshape(x.shape[0]).sum(), x, create_graph=True)
    return g


def laplacian(fn: Callable, x: torch.Tensor) -> torch.Tensor:
    """(N,) sum of second derivatives of u = fn(x); forward-mode for chains of KAN layers."""
    layers = kan_chain(fn)
    if layers is not None and x.dim() == 2:
        return _laplacian_forward(layers, x)
    x = x if x.requires_grad else x.detach().requires_grad_()
    g = gradient(fn, x)
    return sum(torch.autograd.grad(g[:, k].sum(), x, create_graph=True)[0][:, k] for k in range(x.shape[1]))


def kan_chain(fn) -> list | None:
    """The KANLinear layers of ``fn`` when it is exactly a chain of them whose edges the Taylor
    pass covers (SiLU or no base branch, no symbolic edges, no edge dropout in training), else
    None."""
    from .layers import KANLinear

    if isinstance(fn, KANLinear):
        mods = [fn]
    elif isinstance(fn, nn.Sequential):
        mods = list(fn)
    else:
        return None
    for m in mods:
        if not isinstance(m, KANLinear):
            return None
        if m.base_weight is not None and m.base_activation is not F.silu:
            return None
        if m._sym_codes or (m.training and m.edge_dropout > 0):
            return None
    return mods


def _taylor_layer(layer, h: torch.Tensor, hps: torch.Tensor, has_S: bool):
    """A layer's (h, h', S) from its input's: h (B, in) and hps (n1, B, in), the first derivatives
    along every input dimension followed, when has_S, by the sum of the second derivatives S
    (absent: zero). Returns h_out and the same stack (D + 1, B, out) for the next layer: the
    layer's outputs are computed as one row stack [h; h'_1 .. h'_D; S], whose lower rows are that
    stack already (no copy)."""
    from . import kernels as K

    n1, B, n_in = hps.shape
    D = n1 - 1 if has_S else n1
    hp, S = hps[:D], (hps[D] if has_S else None)
    st = layer._basis_state()
    key = layer._plan_key
    c = layer.effective_coef()
    dt = c.dtype
    hk = h.to(dt)
    num = den = None
    if layer._plan.kind == "rational":
        num, den = layer.basis_numerator, layer.basis_denominator
    W = layer.effective_base_weight()
    if W is not None:
        # the base branch's operands of all three orders in one pass, and sum_d h'_d^2
        A, sq = K.silu_taylor(h, hp, S)
    else:
        sq = (hp * hp).sum(0)
    # value, first order (the D directions and S stacked into one launch), second order
    y = K.prim_F(hk, c, None, st, key, 0, num, den)
    f1 = K.prim_F(hk.repeat(n1, 1), c, hps.reshape(n1 * B, n_in).to(dt), st, key, 1, num, den).reshape(n1, B, -1)
    f2 = K.prim_F(hk, c, sq.to(dt), st, key, 2, num, den)
    S_spline = f2 if S is None else f2 + f1[D]
    n_out = y.shape[-1]
    Z = torch.cat([y, f1[:D].reshape(D * B, n_out), S_spline], 0)
    if W is not None:
        Z = torch.addmm(Z, A.to(dt), W.t())  # the base branch of y, every h'_d and S: one GEMM
    y, hps_out = Z[:B], Z[B:].reshape(D + 1, B, n_out)
    if layer.bias is not None:
        y = y + layer.bias
    return y.to(h.dtype), hps_out.to(h.dtype)


def _laplacian_forward(layers, x: torch.Tensor) -> torch.Tensor:
    B, D = x.shape
    h = x
    hps = torch.eye(D, dtype=x.dtype, device=x.device)[:, None, :].expand(D, B, D)  # dx/dx_d
    has_S = False
    for layer in layers:
        h, hps = _taylor_layer(layer, h, hps, has_S)
        has_S = True
    if h.shape[-1] != 1:
        raise ValueError(f"laplacian needs a scalar field, the network has {h.shape[-1]} outputs")
    return hps[-1][:, 0]
