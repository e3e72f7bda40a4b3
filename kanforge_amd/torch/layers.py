"""KAN layers whose spline part runs on the HIP kernels.

Same constructor, parameter names, shapes and ``state_dict`` layout as
kanforge/torch/layers.py (KANLinear :28-116, GRKAN :335-363, KAN :366-398),
so checkpoints and ``kanforge.save`` files move between the two unchanged.
The spline branch always takes the fused HIP path (libkfhip.so). The base
branch F.linear(silu(x), W * mask) and the bias join the contractions for
bf16 Chebyshev and cubic B-spline layers with a SiLU base (kf_F_base,
kf_P_base, kf_G_base, where the library takes the shapes); otherwise they
are torch ops on the same device.
"""

from __future__ import annotations

import math
from collections.abc import Callable, Sequence

import numpy as np
import torch
import torch.nn.functional as F
from torch import nn

from .. import grid as grid_tools
from .. import symbolic as sym
from .._layer import basis_param_values, init_stds, resolve_groups
from ..bases import Basis, Rational, make_basis
from ..kernels import plan_for
from ..kernels.plan import AUTO_KINDS, MAX_BASIS
from . import kernels as _kernels

BACKENDS = ("auto", "ops", "kernel")


def _compiling() -> bool:
    return torch.compiler.is_compiling()


class KANLinear(nn.Module):
    """One KAN layer: y_o = sum_i s_oi * phi_oi(x_i) + sum_i w_oi * act(x_i) + b_o.

    Parameters (as in the reference):
      ``coef``           ``(out, in, basis.size)``
      ``base_weight``    ``(out, in)``, absent if ``base_activation`` is None
      ``bias``           ``(out,)``, absent if ``bias=False``
      ``edge_scale``     ``(out, in)``, only with ``edge_scale=True``
      ``basis_<name>``   trainable basis parameters ``(groups, *shape)``
    Buffers: ``basis_<name>`` grids ``(in, *shape)``; ``edge_mask``,
    ``sym_code``, ``sym_params``.

    ``backend``: ``"auto"`` and ``"kernel"`` run the HIP kernels; the
    plain-ops route (``"ops"``) is not part of this build and raises.
    """

    def __init__(
        self,
        in_features: int,
        out_features: int,
        basis: str | dict | Basis = "bspline",
        *,
        bias: bool = True,
        base_activation: Callable[[torch.Tensor], torch.Tensor] | None = F.silu,
        groups: int | None = None,
        edge_scale: bool = False,
        grid_ranges=None,
        coef_init: str = "normal",
        coef_init_std: float = 0.1,
        edge_dropout: float = 0.0,
        backend: str = "auto",
        device=None,
        dtype=None,
    ):
        super().__init__()
        if not 0 <= edge_dropout < 1:
            raise ValueError("edge_dropout must be in [0, 1)")
        factory = {"device": device, "dtype": dtype}
        self.in_features = in_features
        self.out_features = out_features
        self.basis = make_basis(basis)
        self.base_activation = base_activation
        self.groups = resolve_groups(in_features, groups)
        self.coef_init = coef_init
        self.coef_init_std = coef_init_std
        self.edge_dropout = edge_dropout
        if backend not in BACKENDS:
            raise ValueError(f"backend must be one of {BACKENDS}")
        self.backend = backend
        self._grid_ranges = grid_ranges
        self._init_kwargs = {
            "basis": self.basis,
            "bias": bias,
            "base_activation": base_activation,
            "groups": groups,
            "edge_scale": edge_scale,
            "coef_init": coef_init,
            "coef_init_std": coef_init_std,
            "edge_dropout": edge_dropout,
            "backend": backend,
        }
        init_stds(self.basis, in_features, out_features, coef_init, coef_init_std, base_activation is not None)
        self.coef = nn.Parameter(torch.empty(out_features, in_features, self.basis.size, **factory))
        if base_activation is not None:
            self.base_weight = nn.Parameter(torch.empty(out_features, in_features, **factory))
        else:
            self.register_parameter("base_weight", None)
        if bias:
            self.bias = nn.Parameter(torch.empty(out_features, **factory))
        else:
            self.register_parameter("bias", None)
        if edge_scale:
            self.edge_scale = nn.Parameter(torch.empty(out_features, in_features, **factory))
        else:
            self.register_parameter("edge_scale", None)
        self.register_buffer("edge_mask", torch.empty(out_features, in_features, **factory))
        self.register_buffer("sym_code", torch.empty(out_features, in_features, dtype=torch.int32, device=device))
        self.register_buffer("sym_params", torch.empty(out_features, in_features, 4, **factory))
        self._trainable_names: list[str] = []
        self._buffer_names: list[str] = []
        self._state_cache = None
        self._mask_cache = None
        self.reset_parameters()

    # --- parameters -------------------------------------------------------------

    def _set_basis_state(self, trainable: dict, buffers: dict) -> None:
        for name in self._trainable_names + self._buffer_names:
            delattr(self, f"basis_{name}")
        like = {"dtype": self.coef.dtype, "device": self.coef.device}
        for name, value in trainable.items():
            self.register_parameter(f"basis_{name}", nn.Parameter(torch.as_tensor(np.ascontiguousarray(value), **like)))
        for name, value in buffers.items():
            self.register_buffer(f"basis_{name}", torch.as_tensor(np.ascontiguousarray(value), **like))
        self._trainable_names, self._buffer_names = list(trainable), list(buffers)
        self._plan = plan_for(self.basis)
        _check_kernel_limits(self.basis)
        self._plan_key = None if self._plan is None else _kernels.plan_key(self._plan)
        self._state_cache = None

    def reset_parameters(self) -> None:
        coef_std, base_std = init_stds(
            self.basis, self.in_features, self.out_features, self.coef_init, self.coef_init_std, self.base_weight is not None
        )
        nn.init.normal_(self.coef, std=coef_std) if coef_std else nn.init.zeros_(self.coef)
        if self.base_weight is not None:
            if base_std is None:
                nn.init.kaiming_uniform_(self.base_weight, a=math.sqrt(5))
            else:
                nn.init.normal_(self.base_weight, std=base_std)
        if self.bias is not None:
            nn.init.zeros_(self.bias)
        if self.edge_scale is not None:
            nn.init.ones_(self.edge_scale)
        self.edge_mask.fill_(1.0)
        self.sym_code.fill_(-1)
        self.sym_params.zero_()
        self._sym_codes = ()
        self._set_basis_state(*basis_param_values(self.basis, self.groups, self.in_features, self._grid_ranges))

    def basis_params(self) -> dict[str, torch.Tensor]:
        """Basis parameters and buffers expanded to ``(in, *shape)`` (or ``(1, *shape)``)."""
        rep = self.in_features // self.groups
        out = {}
        for name in self._trainable_names:
            p = getattr(self, f"basis_{name}")
            out[name] = p if self.groups in (1, self.in_features) else p.repeat_interleave(rep, dim=0)
        for name in self._buffer_names:
            out[name] = getattr(self, f"basis_{name}")
        return out

    def _mask_is_ones(self) -> bool:
        m = self.edge_mask
        key = (m.data_ptr(), m._version, m.device)
        if self._mask_cache is None or self._mask_cache[0] != key:
            self._mask_cache = (key, bool((m == 1).all()))
        return self._mask_cache[1]

    def effective_coef(self) -> torch.Tensor:
        # under torch.compile the mask is applied without looking at its values
        if self.edge_scale is None and not _compiling() and self._mask_is_ones():
            return self.coef
        scale = self.edge_mask if self.edge_scale is None else self.edge_scale * self.edge_mask
        return self.coef * scale[..., None]

    def effective_base_weight(self) -> torch.Tensor | None:
        if self.base_weight is None:
            return None
        if not _compiling() and self._mask_is_ones():
            return self.base_weight
        return self.base_weight * self.edge_mask

    # --- computation ------------------------------------------------------------

    def _basis_state(self):
        """Device tables of the plan (cached per grid version for B-splines)."""
        plan = self._plan
        if plan.kind == "cheb":
            return None
        if plan.kind == "bspline":
            if _compiling():
                # traced graphs use the tables of the last eager call (built again there when the
                # grid changed); a layer that never ran eagerly builds them now, outside the graph
                if self._state_cache is None:
                    self._state_cache = (None, _kernels.bspline_state(self.basis_grid, self.basis.order))
                return self._state_cache[1]
            grid = self.basis_grid
            key = (grid.data_ptr(), grid._version, grid.device, grid.dtype)
            if self._state_cache is None or self._state_cache[0] != key:
                self._state_cache = (key, _kernels.bspline_state(grid, self.basis.order))
            return self._state_cache[1]
        num, den = self.basis_numerator, self.basis_denominator
        return _kernels.rational_state(num, den, self.in_features // num.shape[0])

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.training and self.edge_dropout > 0:
            edges = self.edge_derivative(x, 0)
            keep = torch.rand_like(edges) >= self.edge_dropout
            y = (edges * keep).sum(-1) / (1 - self.edge_dropout)
            return y if self.bias is None else _kernels.bias_add(y, self.bias)
        if not _compiling():
            self.uses_kernel(x.device)  # raises when the HIP path cannot run
        st = self._basis_state()
        if self._base_fused(x):
            # spline part, SiLU base branch and bias in one contraction (and one backward pass)
            y = _kernels.spline_base_forward(x, self.effective_coef(), self.effective_base_weight(), self.bias, st,
                                             self._plan_key)
            return y + self._symbolic_sum(x) if self._sym_codes else y
        # without a base branch or symbolic part to add after F, the bias rides F's last kernel
        fold_bias = self.bias is not None and self.base_weight is None and not self._sym_codes
        b = self.bias if fold_bias else None
        if self._plan.kind == "rational":
            y = _kernels.spline_forward(x, self.effective_coef(), st, self._plan_key, self.basis_numerator,
                                        self.basis_denominator, bias=b)
        else:
            y = _kernels.spline_forward(x, self.effective_coef(), st, self._plan_key, bias=b)
        if self.base_weight is not None:
            # accumulated into y by the GEMM itself (C = y + act(x) W^T), no separate add (an
            # in-place addmm_ on F's output costs more: its backward copies through the view)
            y2 = torch.addmm(y.reshape(-1, self.out_features), self.base_activation(x).reshape(-1, self.in_features),
                             self.effective_base_weight().t())
            y = y2.reshape(y.shape)
        if self._sym_codes:
            y = y + self._symbolic_sum(x)
        if self.bias is not None and not fold_bias:
            y = _kernels.bias_add(y, self.bias)
        return y

    def _base_fused(self, x: torch.Tensor) -> bool:
        """Whether forward runs the spline part, the SiLU base branch and the bias as one op whose
        kernels fuse the base branch (bf16 Chebyshev and B-spline plans on their contraction
        kernels, float32 B-splines on the sparse route; eager)."""
        if self.base_weight is None or self.base_activation is not F.silu or self._plan.kind not in ("cheb", "bspline"):
            return False
        dt = x.dtype
        if self.coef.dtype != dt or self.base_weight.dtype != dt:
            return False
        if (self.bias is not None and self.bias.dtype != dt) or _compiling() or x.dim() < 1:
            return False
        batch = x.numel() // max(self.in_features, 1)
        return any(_kernels.base_fused(self._plan_key, self._basis_state(), dt, batch, self.in_features, self.out_features))

    def uses_kernel(self, device: torch.device) -> bool:
        """Whether forward runs the fused kernel on ``device`` (always, or an error)."""
        if self.backend == "ops":
            raise RuntimeError("backend='ops' (plain torch ops) is not part of the HIP build; use 'auto' or 'kernel'")
        if self._plan is None:
            raise RuntimeError(f"no fused kernel for this basis: {self.basis!r}")
        if not _kernels.available(device):
            raise RuntimeError(f"no fused kernel for device {device}: the HIP kernels need a ROCm GPU and libkfhip.so")
        if self.backend == "auto" and self._plan.kind not in AUTO_KINDS.get(torch.device(device).type, ()):
            raise RuntimeError(f"no fused kernel for plan kind {self._plan.kind} on {device}")
        return True

    def edge_derivative(self, x: torch.Tensor, order: int = 1) -> torch.Tensor:
        """d^order phi_oi / dx_i^order for every edge, shape ``(..., out, in)``
        (kanforge/torch/layers.py:206-226), through kf_edge_derivative."""
        if order < 0:
            raise ValueError("order must be >= 0")
        self.uses_kernel(x.device)
        bw = self.effective_base_weight()
        other_base = bw is not None and self.base_activation is not F.silu
        if other_base and order > 0:
            raise NotImplementedError("analytic derivatives need base_activation=F.silu or None")
        if self._sym_codes and order > 0:
            raise NotImplementedError("analytic derivatives of symbolic edges are not available; use autograd")
        num = den = None
        if self._plan.kind == "rational":
            num, den = self.basis_numerator, self.basis_denominator
        # the edge kernel evaluates a SiLU base branch itself; another activation is added here
        d = _kernels.edge_derivative(
            x, self.effective_coef(), None if other_base else bw, self._basis_state(), self._plan_key, int(order), num, den
        )
        if other_base:
            d = d + self.base_activation(x).unsqueeze(-2) * bw
        if self._sym_codes:
            d = d + self._symbolic_dense(x)
        return d

    # --- masks and symbolic edges (kanforge/_layer.py:209-272) -------------------------------

    def symbolic_edges(self) -> dict:
        """``{(o, i): (function name, (a, b, c, d))}`` of the edges fixed to a function."""
        code = self.sym_code.detach().cpu().numpy()
        params = self.sym_params.detach().double().cpu().numpy()
        return {(int(o), int(i)): (sym.NAMES[code[o, i]], tuple(float(v) for v in params[o, i])) for o, i in zip(*np.nonzero(code >= 0))}

    @torch.no_grad()
    def fix_symbolic(self, o: int, i: int, name: str, params=(1.0, 0.0, 1.0, 0.0)) -> None:
        """Edge (o, i) becomes ``c * f(a * x + b) + d``; its spline and base parts are masked."""
        code = sym.code_of(name)
        self.edge_mask[o, i] = 0.0
        self.sym_code[o, i] = code
        self.sym_params[o, i] = torch.as_tensor(params, dtype=self.sym_params.dtype)
        self._refresh_symbolic()

    @torch.no_grad()
    def unfix_symbolic(self, o: int, i: int) -> None:
        """Edge (o, i) is the learned edge again (spline and base parts unmasked)."""
        self.edge_mask[o, i] = 1.0
        self.sym_code[o, i] = -1
        self._refresh_symbolic()

    @torch.no_grad()
    def set_edge_mask(self, mask) -> None:
        """0 removes an edge (pruning); symbolic edges stay as they are."""
        self.edge_mask.copy_(torch.as_tensor(np.asarray(mask, dtype=np.float64), dtype=self.edge_mask.dtype))

    def active_edges(self) -> np.ndarray:
        """Boolean ``(out, in)``: learned (unmasked) or symbolic edges."""
        return ((self.edge_mask != 0) | (self.sym_code >= 0)).cpu().numpy()

    def _symbolic_edge_list(self):
        """(out index, in index, code, (a, b, c, d)) of every symbolic edge, cached per buffer version."""
        code, params = self.sym_code, self.sym_params
        key = (code.data_ptr(), code._version, params.data_ptr(), params._version)
        cached = getattr(self, "_sym_cache", None)
        if cached is None or cached[0] != key:
            o_idx, i_idx = torch.nonzero(code >= 0, as_tuple=True)
            cached = (key, (o_idx, i_idx, code[o_idx, i_idx], params[o_idx, i_idx]))
            self._sym_cache = cached
        return cached[1]

    def _symbolic_values(self, x: torch.Tensor) -> torch.Tensor:
        o_idx, i_idx, codes, params = self._symbolic_edge_list()
        return sym.evaluate(x.index_select(-1, i_idx), codes, params.to(x.dtype), self._sym_codes)

    def _symbolic_sum(self, x: torch.Tensor) -> torch.Tensor:
        """``(..., out)``: the symbolic edges summed into their outputs."""
        o_idx = self._symbolic_edge_list()[0]
        v = self._symbolic_values(x)
        return torch.zeros(*x.shape[:-1], self.out_features, dtype=v.dtype, device=v.device).index_add(-1, o_idx, v)

    def _symbolic_dense(self, x: torch.Tensor) -> torch.Tensor:
        """``(..., out, in)``: the symbolic edges' values, zero on the other edges."""
        o_idx, i_idx = self._symbolic_edge_list()[:2]
        v = self._symbolic_values(x)
        flat = torch.zeros(*x.shape[:-1], self.out_features * self.in_features, dtype=v.dtype, device=v.device)
        return flat.index_add(-1, o_idx * self.in_features + i_idx, v).unflatten(-1, (self.out_features, self.in_features))

    # --- state import / export (kanforge.save format) ------------------------------

    @staticmethod
    def _to_numpy(x) -> np.ndarray:
        return x.detach().cpu().double().numpy() if isinstance(x, torch.Tensor) else np.asarray(x)

    def _export_full(self) -> dict:
        named = {**dict(self.named_parameters(recurse=False)), **dict(self.named_buffers(recurse=False))}
        out = {k: self._to_numpy(v) for k, v in named.items()}
        out.update({k: None for k in ("base_weight", "bias", "edge_scale") if getattr(self, k) is None})
        return out

    @torch.no_grad()
    def _import_full(self, state: dict) -> None:
        for name, value in state.items():
            t = getattr(self, name, None)
            if value is None or t is None:
                continue
            if tuple(t.shape) != tuple(np.shape(value)):
                raise ValueError(f"{name}: shape {np.shape(value)} does not fit {tuple(t.shape)}")
            t.copy_(torch.as_tensor(value, dtype=t.dtype, device=t.device))
        self._refresh_symbolic()

    def _refresh_symbolic(self) -> None:
        codes = np.unique(self.sym_code.detach().cpu().numpy().astype(int))
        self._sym_codes = tuple(int(c) for c in codes if c >= 0)

    def _load_from_state_dict(self, *args, **kwargs):
        super()._load_from_state_dict(*args, **kwargs)
        self._refresh_symbolic()

    # --- construction from MLPs (kanforge/torch/layers.py:290-309) ------------------------

    @classmethod
    def from_linear(cls, linear: nn.Linear, activation: Callable = F.silu, basis="bspline", **kwargs) -> "KANLinear":
        """``linear(activation(x))`` as a ``KANLinear``: the activation becomes the base branch
        with the linear's weight and bias, and the spline coefficients start at zero."""
        layer = cls(
            linear.in_features,
            linear.out_features,
            basis,
            bias=linear.bias is not None,
            base_activation=activation,
            coef_init="zero",
            device=linear.weight.device,
            dtype=linear.weight.dtype,
            **kwargs,
        )
        with torch.no_grad():
            layer.base_weight.copy_(linear.weight)
            if linear.bias is not None:
                layer.bias.copy_(linear.bias)
        return layer

    # --- grid update, refinement, basis conversion ----------------------------------------
    #
    # One operation underlies all three tools: snapshot the layer in float64, choose the new
    # basis, its parameters and the sample points, refit every edge function on those points
    # (grid.refit, per-input least squares) and install the result. The refit follows
    # kanforge/_layer.py:116-191 so that a grid change gives the reference's grid and
    # coefficients; parameter shapes can change, so optimizers are re-created afterwards.

    def _snapshot(self) -> "_HostLayer":
        f = self._to_numpy
        return _HostLayer(
            self.in_features,
            self.groups,
            f(self.coef),
            None if self.edge_scale is None else f(self.edge_scale),
            {n: f(getattr(self, f"basis_{n}")) for n in self._trainable_names},
            {n: f(getattr(self, f"basis_{n}")) for n in self._buffer_names},
        )

    @torch.no_grad()
    def _install(self, basis: Basis, coef, edge_scale, trainable: dict, buffers: dict) -> None:
        like = {"dtype": self.coef.dtype, "device": self.coef.device}
        self.basis = basis
        self._init_kwargs["basis"] = basis
        self.coef = nn.Parameter(torch.as_tensor(np.ascontiguousarray(coef), **like))
        if edge_scale is not None:
            self.edge_scale = nn.Parameter(torch.as_tensor(np.ascontiguousarray(edge_scale), **like))
        self._set_basis_state(trainable, buffers)

    def _fit_points(self, x, ranges_of: tuple, n_default: int) -> np.ndarray:
        """The refit's sample points: ``x`` itself, or ``n_default`` points spread over the grid
        ranges of ``ranges_of = (basis, buffers)``."""
        if x is not None:
            return np.asarray(self._to_numpy(x), dtype=np.float64).reshape(-1, self.in_features)
        ranges = grid_tools.grid_ranges(*ranges_of)
        if ranges is None:
            raise ValueError(f"{type(ranges_of[0]).__name__} has no grid: pass samples x")
        return grid_tools.sample_inputs(ranges, n_default)

    def _regrid(self, new_basis: Basis, trainable: dict, buffers: dict, points: np.ndarray, ridge: float) -> None:
        old = self._snapshot()
        coef = grid_tools.refit(
            self.basis, old.per_input(), old.effective_coef(), new_basis, old.per_input(trainable, buffers), points, ridge
        )
        scale = old.edge_scale
        if scale is not None:
            # edge scales are kept; an edge whose scale vanished restarts at scale 1 and the
            # refit goes into its coefficients
            live = np.abs(scale) > 1e-12
            scale = np.where(live, scale, 1.0)
            coef = coef / scale[..., None]
        self._install(new_basis, coef, scale, trainable, buffers)

    def update_grid(self, x, *, margin: float = 0.0, grid_eps: float = 0.02, ridge: float = 0.0) -> None:
        """Adapt every grid to the inputs ``x`` and refit the edge functions on them (pykan's
        update_grid_from_samples; approximate, as a spline on a new grid can only approximate
        the old one)."""
        if x is None:
            raise ValueError("update_grid needs input samples x")
        names = self.basis.grid_names()
        if not names:
            raise TypeError(f"{type(self.basis).__name__} has no grid")
        old = self._snapshot()
        points = self._fit_points(x, (self.basis, old.buffers), 0)
        buffers = {**old.buffers, **{n: grid_tools.adaptive_grid(points, old.buffers[n].shape[-1], margin, grid_eps) for n in names}}
        self._regrid(self.basis, old.trainable, buffers, points, ridge)

    def refine_grid(self, grid_size: int, x=None, *, ridge: float = 0.0) -> None:
        """The same basis on a finer (or coarser) grid; each input's grid keeps its range and
        is resampled to the new number of points."""
        new_basis = make_basis({**self.basis.config(), _resize_key(self.basis): grid_size})
        _check_kernel_limits(new_basis)
        old = self._snapshot()
        trainable, buffers = basis_param_values(new_basis, self.groups, self.in_features)
        for n in new_basis.grid_names():
            if n in old.buffers:
                buffers[n] = grid_tools.resample_grid(old.buffers[n], buffers[n].shape[-1])
        points = self._fit_points(x, (self.basis, old.buffers), 8 * new_basis.size + 64)
        self._regrid(new_basis, trainable, buffers, points, ridge)

    def change_basis(self, basis, x=None, *, ridge: float = 0.0) -> None:
        """Convert to another basis (e.g. B-spline -> Chebyshev) by least squares; without
        ``x`` the fit uses points spread over the current grid ranges (or the new basis'
        ranges), and a new grid inherits each input's range."""
        new_basis = make_basis(basis)
        _check_kernel_limits(new_basis)
        old = self._snapshot()
        old_ranges = grid_tools.grid_ranges(self.basis, old.buffers)
        trainable, buffers = basis_param_values(new_basis, self.groups, self.in_features, old_ranges)
        ranges_of = (self.basis, old.buffers) if old_ranges is not None else (new_basis, buffers)
        points = self._fit_points(x, ranges_of, 8 * max(new_basis.size, self.basis.size) + 64)
        self._regrid(new_basis, trainable, buffers, points, ridge)

    def extra_repr(self) -> str:
        groups = "" if self.groups == self.in_features else f", groups={self.groups}"
        return f"in_features={self.in_features}, out_features={self.out_features}, basis={self.basis!r}{groups}"


class _HostLayer:
    """Float64 NumPy snapshot of what a grid refit reads from a layer."""

    def __init__(self, n_in: int, groups: int, coef, edge_scale, trainable: dict, buffers: dict):
        self.n_in, self.groups = n_in, groups
        self.coef, self.edge_scale = coef, edge_scale
        self.trainable, self.buffers = trainable, buffers

    def effective_coef(self) -> np.ndarray:
        return self.coef if self.edge_scale is None else self.coef * self.edge_scale[..., None]

    def per_input(self, trainable: dict | None = None, buffers: dict | None = None) -> dict:
        """Basis parameters per input: group parameters repeated over their inputs."""
        trainable = self.trainable if trainable is None else trainable
        buffers = self.buffers if buffers is None else buffers
        rep = self.n_in // self.groups
        return {**{k: np.repeat(v, rep, axis=0) for k, v in trainable.items()}, **buffers}


class GRKAN(KANLinear):
    """Group-rational KAN layer of KAT (kanforge/torch/layers.py:335-363)."""

    def __init__(
        self,
        in_features: int,
        out_features: int,
        *,
        groups: int = 8,
        num_degree: int = 5,
        den_degree: int = 4,
        init: str = "gelu",
        bias: bool = True,
        device=None,
        dtype=None,
    ):
        super().__init__(
            in_features,
            out_features,
            Rational(num_degree, den_degree, init),
            bias=bias,
            base_activation=None,
            groups=groups,
            coef_init="variance",
            device=device,
            dtype=dtype,
        )


class KAN(nn.Sequential):
    """Stack of ``KANLinear`` layers (kanforge/torch/layers.py:366-398)."""

    def __init__(self, widths: Sequence[int], basis: str | dict | Basis = "bspline", grid_ranges=None, **layer_kwargs):
        if len(widths) < 2:
            raise ValueError("widths needs at least input and output size")
        super().__init__(
            *(
                KANLinear(a, b, basis, grid_ranges=grid_ranges if k == 0 else None, **layer_kwargs)
                for k, (a, b) in enumerate(zip(widths[:-1], widths[1:]))
            )
        )
        self.widths = list(widths)

    def edge_derivative(self, x: torch.Tensor, order: int = 1) -> list[torch.Tensor]:
        """Per-layer edge derivatives at the activations each layer receives."""
        return [layer.edge_derivative(h, order) for layer, h in layer_inputs(self, x)]

    @torch.no_grad()
    def update_grid(self, x: torch.Tensor, **kwargs) -> None:
        """Update every layer's grid from the activations it receives (pykan)."""
        for layer in self:
            layer.update_grid(x, **kwargs)
            x = layer(x)

    def refine_grid(self, grid_size: int, **kwargs) -> None:
        for layer in self:
            layer.refine_grid(grid_size, **kwargs)


def from_mlp(mlp: nn.Sequential, basis="bspline", **kwargs) -> nn.Sequential:
    """``Linear, act, Linear, act, ..., Linear`` as an equal network (kanforge/torch/layers.py:
    312-328): the first Linear stays and every (activation, Linear) pair becomes a
    ``KANLinear`` whose base branch is that activation."""
    mods = list(mlp)
    if not mods or not isinstance(mods[0], nn.Linear):
        raise ValueError("the MLP must start with nn.Linear")
    out, i = [mods[0]], 1
    while i < len(mods):
        if i + 1 < len(mods) and isinstance(mods[i + 1], nn.Linear) and not isinstance(mods[i], nn.Linear):
            out.append(KANLinear.from_linear(mods[i + 1], mods[i], basis, **kwargs))
            i += 2
        else:
            out.append(mods[i])
            i += 1
    return nn.Sequential(*out)


def _check_kernel_limits(basis: Basis) -> None:
    """The HIP kernels hold at most ``MAX_BASIS`` basis functions per edge (register and LDS tiles
    are sized for it); larger bases are rejected when a layer is built or re-gridded."""
    if basis.size > MAX_BASIS:
        raise ValueError(f"{basis!r} has {basis.size} basis functions per edge; the HIP kernels support at most {MAX_BASIS}")


def _resize_key(basis: Basis) -> str:
    """The config entry that sets a basis' number of grid intervals (kanforge/_layer.py:99-104)."""
    cfg = basis.config()
    for key in ("grid_size", "count", "num_knots"):
        if key in cfg:
            return key
    raise TypeError(f"{type(basis).__name__} has no grid size to refine")


def rebuild_kan(layers: Sequence[KANLinear]) -> KAN:
    """A ``KAN`` made of existing layers."""
    model = KAN.__new__(KAN)
    nn.Sequential.__init__(model, *layers)
    model.widths = [layers[0].in_features] + [layer.out_features for layer in layers]
    return model


def layer_inputs(model: nn.Module, x: torch.Tensor) -> list[tuple[KANLinear, torch.Tensor]]:
    """(KANLinear, the input it receives) for every KAN layer of ``model``
    (kanforge/torch/layers.py:446-467)."""
    out = []

    def walk(m, h):
        if isinstance(m, KANLinear):
            out.append((m, h))
            return m(h)
        if isinstance(m, nn.Sequential):
            for sub in m:
                h = walk(sub, h)
            return h
        return m(h)

    walk(model, x)
    return out
