"""Functions of symbolic edges: an edge fixed to ``c * f(a * x + b) + d``.

A layer stores, per edge, the position of ``f`` in ``NAMES`` (``sym_code``, -1 for a learned
edge) and ``(a, b, c, d)`` (``sym_params``). The names and their order are those of
kanforge/interpret/library.py:34-55, so the codes in saved models mean the same functions in
both packages; the evaluation here is torch code on the layer's device.
"""

from __future__ import annotations

import torch

NAMES = (
    "0", "x", "x^2", "x^3", "x^4", "1/x", "1/x^2", "sqrt", "1/sqrt",
    "exp", "log", "sin", "cos", "tanh", "sigmoid", "gaussian", "abs", "arctan",
)
CODES = {name: code for code, name in enumerate(NAMES)}

# An argument inside every function's domain, given to the functions on the entries of an edge
# list that use another function, so unused branches produce no NaN (in values or gradients).
SAFE_INPUT = 1.0

_TORCH = {
    "0": torch.zeros_like,
    "x": lambda u: u,
    "x^2": lambda u: u * u,
    "x^3": lambda u: u * u * u,
    "x^4": lambda u: (u * u) * (u * u),
    "1/x": torch.reciprocal,
    "1/x^2": lambda u: torch.reciprocal(u * u),
    "sqrt": torch.sqrt,
    "1/sqrt": torch.rsqrt,
    "exp": torch.exp,
    "log": torch.log,
    "sin": torch.sin,
    "cos": torch.cos,
    "tanh": torch.tanh,
    "sigmoid": torch.sigmoid,
    "gaussian": lambda u: torch.exp(-u * u),
    "abs": torch.abs,
    "arctan": torch.atan,
}


def code_of(name: str) -> int:
    if name not in CODES:
        raise ValueError(f"unknown symbolic function {name!r}; available: {list(NAMES)}")
    return CODES[name]


def function(code: int):
    """The torch function of a code."""
    return _TORCH[NAMES[int(code)]]


def evaluate(x_edges: torch.Tensor, codes: torch.Tensor, params: torch.Tensor, present: tuple[int, ...]) -> torch.Tensor:
    """``c * f(a * x + b) + d`` for a list of edges.

    ``x_edges (..., E)`` is each edge's input, ``codes (E,)`` its function, ``params (E, 4)`` its
    ``(a, b, c, d)``; ``present`` lists the distinct codes among ``codes``.
    """
    a, b, c, d = params.unbind(-1)
    u = a * x_edges + b
    out = torch.zeros_like(u)
    for code in present:
        use = codes == code
        val = c * function(code)(torch.where(use, u, torch.full_like(u, SAFE_INPUT))) + d
        out = torch.where(use, val, out)
    return out
