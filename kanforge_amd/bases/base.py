"""The basis contract of the HIP path.

A basis describes the edge functions phi(x) = sum_k c_k B_k(x) of a KAN
layer: its size K, its parameters (``param_specs``) and configuration
(``config``), as in kanforge/bases/base.py:29-136. Evaluation runs on the GPU:
``Basis.derivative(x, m, params)`` on a device tensor launches the HIP feature
kernel (kf_features); there is no host evaluation path.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import numpy as np


@dataclass(frozen=True)
class ParamSpec:
    """Default value of one basis parameter for a single input.

    ``trainable=False`` marks state such as grids (a per-input buffer).
    """

    value: np.ndarray
    trainable: bool = True

    @property
    def shape(self) -> tuple[int, ...]:
        return np.shape(self.value)


BASES: dict[str, type["Basis"]] = {}


class Basis:
    name: str = ""
    local: bool = False

    def __init_subclass__(cls, **kwargs):
        super().__init_subclass__(**kwargs)
        if cls.__dict__.get("name"):
            BASES[cls.name] = cls

    @property
    def size(self) -> int:
        raise NotImplementedError

    @property
    def support(self) -> int:
        return self.size

    def param_specs(self) -> dict[str, ParamSpec]:
        return {}

    def grid_names(self) -> list[str]:
        return [k for k, s in self.param_specs().items() if not s.trainable and k.endswith("grid")]

    def __call__(self, x, params: dict | None = None):
        return self.derivative(x, 0, params)

    def derivative(self, x, order: int = 1, params: dict | None = None):
        """d^order/dx^order of every basis function, ``(..., in, size)``, on the GPU."""
        if order < 0:
            raise ValueError("order must be >= 0")
        from ..torch.kernels import basis_derivative

        return basis_derivative(self, x, int(order), params)

    def host_values(self, x: np.ndarray, params: dict | None = None) -> np.ndarray:
        """Float64 values at host points, for initialisation constants only."""
        raise NotImplementedError

    def config(self) -> dict[str, Any]:
        raise NotImplementedError

    def __repr__(self) -> str:
        args = ", ".join(f"{k}={v!r}" for k, v in self.config().items() if k != "name")
        return f"{type(self).__name__}({args})"

    def __eq__(self, other) -> bool:
        return isinstance(other, Basis) and self.config() == other.config()

    def __hash__(self) -> int:
        return hash(repr(self.config()))

    @classmethod
    def from_config(cls, cfg: dict) -> "Basis":
        cfg = {k: tuple(v) if k == "grid_range" else v for k, v in cfg.items()}
        return cls(**cfg)


def _check_range(grid_range) -> tuple[float, float]:
    lo, hi = float(grid_range[0]), float(grid_range[1])
    if not hi > lo:
        raise ValueError("grid_range must be increasing")
    return lo, hi


def make_basis(spec="bspline", **kwargs) -> Basis:
    """Build a basis from a name, a ``config()`` dict or an existing instance
    (kanforge/bases/base.py:112-128)."""
    if isinstance(spec, Basis):
        if kwargs:
            raise TypeError("kwargs are not allowed with a Basis instance")
        return spec
    if isinstance(spec, dict):
        spec = dict(spec)
        name = spec.pop("name")
        cls = BASES.get(name)
        if cls is None:
            raise ValueError(f"unknown basis {name!r}; available: {sorted(BASES)}")
        return cls.from_config({**spec, **kwargs})
    cls = BASES.get(spec)
    if cls is None:
        raise ValueError(f"unknown basis {spec!r}; available: {sorted(BASES)}")
    return cls(**kwargs)
