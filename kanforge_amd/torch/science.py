"""PINN derivatives of a field u(x) kept in the autograd graph
(kanforge/torch/science.py:25-46). Through KAN layers every node of these
graphs is an F, G or P launch of the HIP kernels."""

from __future__ import annotations

from collections.abc import Callable

import torch


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
    """(N,) sum of second derivatives of u = fn(x)."""
    x = x if x.requires_grad else x.detach().requires_grad_()
    g = gradient(fn, x)
    return sum(torch.autograd.grad(g[:, k].sum(), x, create_graph=True)[0][:, k] for k in range(x.shape[1]))
