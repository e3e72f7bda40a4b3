"""PyTorch side of the HIP kernels: launchers and differentiable primitives.

Mirrors kanforge/torch/kernels.py: ``available``, the raw launcher ``_raw``
(kernels.py:39-55), the autograd Functions ``_F``, ``_G``, ``_P`` that close
F/G/P under differentiation (kernels.py:70-128), ``prim_F/prim_G/prim_P``
and ``spline_forward`` (kernels.py:131-150). Every launch goes through the
C ABI of libkfhip.so (include/kfhip.h) on the current HIP stream; there is
no other execution path.

Differences from the reference, by design:
* bfloat16 and float32 run natively (no upcast); accumulation is float32;
* ``w=None`` means ones (no ones tensor is materialised);
* the fold R_m of Chebyshev plans is applied inside the library;
* the rational basis has a plan; its trainable parameters receive
  gradients through ``_F`` (first order).
"""

from __future__ import annotations

import ctypes
import weakref
from functools import lru_cache
from typing import Optional

import numpy as np
import torch

from ..kernels.plan import MAX_ORDER, KernelPlan
from . import _lib

_DTYPES = {torch.float32: _lib.KF_F32, torch.bfloat16: _lib.KF_BF16}
_KINDS = {"cheb": _lib.KF_KIND_CHEB, "bspline": _lib.KF_KIND_BSPLINE, "rational": _lib.KF_KIND_RATIONAL}


_AVAILABLE: dict = {}


def available(device: torch.device) -> bool:
    """True on a ROCm (HIP) device with libkfhip.so loadable (decided once per device: neither
    changes while the process runs)."""
    device = torch.device(device)
    hit = _AVAILABLE.get(device)
    if hit is None:
        hit = device.type == "cuda" and torch.version.hip is not None and torch.cuda.is_available()
        if hit:
            try:
                _lib.load()
            except (RuntimeError, OSError):
                hit = False
        _AVAILABLE[device] = hit
    return hit


def _require_device(t: torch.Tensor) -> None:
    if t.device.type != "cuda" or torch.version.hip is None:
        raise RuntimeError(f"the HIP kernels need a ROCm GPU tensor, got a tensor on {t.device}")


def _dtype_code(dtype: torch.dtype) -> int:
    code = _DTYPES.get(dtype)
    if code is None:
        raise TypeError(f"the HIP kernels compute in float32 or bfloat16, not {dtype}")
    return code


def _ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device):
    """The device's current stream as a hipStream_t (the raw handle, without building a Stream
    object)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(idx))


class _NoContext:
    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_NO_CONTEXT = _NoContext()


def _on(device: torch.device):
    """torch.cuda.device(device), or nothing when it is already the current device."""
    if device.index is None or device.index == torch.cuda.current_device():
        return _NO_CONTEXT
    return torch.cuda.device(device)


# --- basis state ---------------------------------------------------------------


class BasisState:
    """Device tables a plan needs besides x and the coefficients.

    bspline: ``knots`` (in, nk + 2k) and ``knots_cmp`` (in, nk) float32, and ``knots_u`` (in, 2)
    ``(t_0, 1/h)`` when every input's knots are evenly spaced (else None);
    rational: ``num`` (groups, p+1), ``den`` (groups, q) float32 and the group size.
    """

    __slots__ = ("knots", "knots_cmp", "knots_u", "num", "den", "group_size")

    def __init__(self, knots=None, knots_cmp=None, num=None, den=None, group_size=1, knots_u=None):
        self.knots, self.knots_cmp, self.knots_u = knots, knots_cmp, knots_u
        self.num, self.den, self.group_size = num, den, int(group_size)

    def with_params(self, num, den) -> "BasisState":
        return BasisState(self.knots, self.knots_cmp, num, den, self.group_size, self.knots_u)


def bspline_state(grid: torch.Tensor, order: int) -> BasisState:
    """Knot tables of a per-input grid buffer (host float64 preparation)."""
    from ..bases.spline import knot_tables, uniform_table

    g = grid.detach().double().cpu().numpy()
    pad, cmp_ = knot_tables(g, order)
    uni = uniform_table(g, order)
    dev = grid.device
    return BasisState(
        knots=torch.from_numpy(pad).to(dev),
        knots_cmp=torch.from_numpy(cmp_).to(dev),
        knots_u=None if uni is None else torch.from_numpy(uni).to(dev),
    )


# float32 copies of rational parameters, reused while the parameter is the same tensor at the
# same version (one cast per parameter update instead of one per launch)
_F32_COPIES: dict = {}


def _as_f32(t: torch.Tensor) -> torch.Tensor:
    if t.dtype == torch.float32 and t.is_contiguous():
        return t.detach()
    key = (id(t), t.device, t.dtype)
    hit = _F32_COPIES.get(key)
    if hit is not None and hit[0]() is t and hit[1] == t._version:
        return hit[2]
    out = t.detach().float().contiguous()
    if len(_F32_COPIES) >= 64:
        _F32_COPIES.clear()
    _F32_COPIES[key] = (weakref.ref(t), t._version, out)
    return out


def rational_state(num: torch.Tensor, den: torch.Tensor, group_size: int) -> BasisState:
    return BasisState(num=_as_f32(num), den=_as_f32(den), group_size=group_size)


_DESC_CACHE: dict = {}


def _desc(plan: KernelPlan, m: int, st: BasisState | None):
    """(kf_basis struct, keep-alive objects) for derivative order m, cached: the struct holds only
    the plan's constants (the fold of order m) and the state tables' device addresses, so equal
    keys give equal structs."""
    key = (plan, m) if st is None else (
        plan, m, st.group_size,
        *(0 if t is None else t.data_ptr() for t in (st.knots, st.knots_cmp, st.knots_u, st.num, st.den)))
    hit = _DESC_CACHE.get(key)
    if hit is None:
        if len(_DESC_CACHE) > 4096:
            _DESC_CACHE.clear()
        hit = _DESC_CACHE[key] = _make_desc(plan, m, st)
    return hit


def _make_desc(plan: KernelPlan, m: int, st: BasisState | None):
    if m > MAX_ORDER:
        raise NotImplementedError(f"derivative order {m} > {MAX_ORDER} is not compiled into the HIP kernels")
    d = _lib.KfBasis()
    d.kind = _KINDS[plan.kind]
    d.size = plan.size
    keep = []
    if plan.kind == "cheb":
        degree, input_map = plan.consts
        fold, factored = plan.device_fold(m)
        r = np.ascontiguousarray(fold, dtype=np.float32)
        keep.append(r)
        d.order = m
        d.n_t = r.shape[1]
        if input_map == "tanh":
            d.input_map = _lib.KF_MAP_TANH_SQ if factored else _lib.KF_MAP_TANH
        else:
            d.input_map = _lib.KF_MAP_IDENTITY
        d.fold = r.ctypes.data_as(ctypes.c_void_p)
    elif plan.kind == "bspline":
        g, k = plan.consts
        d.order = m
        d.n_t = plan.size
        d.spline_k = k
        d.n_knots = g + 2 * k + 1
        d.knots = st.knots.data_ptr()
        d.knots_cmp = st.knots_cmp.data_ptr()
        d.knots_uniform = None if st.knots_u is None else st.knots_u.data_ptr()
    else:
        p, q = plan.consts
        d.order = m
        d.n_t = 1
        d.num_deg, d.den_deg = p, q
        d.group_size = st.group_size
        d.num = st.num.data_ptr()
        d.den = st.den.data_ptr()
    return d, keep


# --- raw launches (no autograd) ----------------------------------------------------


_WS_BYTES: dict = {}


def _workspace(op: int, desc, dt: int, batch: int, n_in: int, n_out: int, device) -> torch.Tensor | None:
    """A workspace for one call; its size is queried once per (op, descriptor, dtype, shape) (the
    cached entry keeps its descriptor, so a reused id never matches a stale size)."""
    key = (op, id(desc), dt, batch, n_in, n_out)
    hit = _WS_BYTES.get(key)
    if hit is None or hit[0] is not desc:
        if len(_WS_BYTES) > 4096:
            _WS_BYTES.clear()
        hit = _WS_BYTES[key] = (desc, int(_lib.load().kf_workspace_bytes(op, ctypes.byref(desc), dt, batch, n_in, n_out)))
    return torch.empty(max(hit[1], 1), dtype=torch.uint8, device=device)


def _raw(op: str, plan: KernelPlan, m: int, x, a, b, st: BasisState | None, n_out: int, h=None, bias=None,
         bias_grad: bool = False):
    """op F: (x, w, c) -> y (B, out), plus ``bias`` (out) when given (kf_F_bias); G: (x, w, g) ->
    dc (out, in, K), or (dc, sum_b g) with ``bias_grad`` (kf_G_bias); P: (x, g, c) -> p (B, in).

    ``x`` (B, in) and every other array share the dtype of ``x``; ``w`` may be None.
    """
    _require_device(x)
    lib = _lib.load()
    dt = _dtype_code(x.dtype)
    batch, n_in = x.shape
    desc, keep = _desc(plan, m, st)
    dev = x.device
    stream = _stream(dev)
    x = x.contiguous()
    with _on(dev):
        if op == "F":
            w, c = a, b
            w = None if w is None else w.contiguous()
            c = c.contiguous()
            y = torch.empty(batch, n_out, dtype=x.dtype, device=dev)
            ws = _workspace(_lib.KF_OP_F, desc, dt, batch, n_in, n_out, dev)
            if bias is None:
                rc = lib.kf_F(ctypes.byref(desc), dt, batch, n_in, n_out, _ptr(x), _ptr(w), _ptr(c), _ptr(y), _ptr(ws), ws.numel(), stream)
                _lib.check(rc, "kf_F")
            else:
                rc = lib.kf_F_bias(ctypes.byref(desc), dt, batch, n_in, n_out, _ptr(x), _ptr(w), _ptr(c),
                                   _ptr(bias.contiguous()), _ptr(y), _ptr(ws), ws.numel(), stream)
                _lib.check(rc, "kf_F_bias")
            return y
        if op == "G":
            w, g = a, b
            w = None if w is None else w.contiguous()
            g = g.contiguous()
            dc = torch.empty(n_out, n_in, plan.size, dtype=x.dtype, device=dev)
            if bias_grad:
                db = torch.empty(n_out, dtype=x.dtype, device=dev)
                ws = _workspace(_lib.KF_OP_G_BIAS, desc, dt, batch, n_in, n_out, dev)
                rc = lib.kf_G_bias(ctypes.byref(desc), dt, batch, n_in, n_out, _ptr(x), _ptr(g), _ptr(w), _ptr(dc),
                                   _ptr(db), _ptr(ws), ws.numel(), stream)
                _lib.check(rc, "kf_G_bias")
                return dc, db
            ws = _workspace(_lib.KF_OP_G, desc, dt, batch, n_in, n_out, dev)
            rc = lib.kf_G(ctypes.byref(desc), dt, batch, n_in, n_out, _ptr(x), _ptr(g), _ptr(w), _ptr(dc), _ptr(ws), ws.numel(), stream)
            _lib.check(rc, "kf_G")
            return dc
        g, c = a, b
        g, c = g.contiguous(), c.contiguous()
        p = torch.empty(batch, n_in, dtype=x.dtype, device=dev)
        ws = _workspace(_lib.KF_OP_P, desc, dt, batch, n_in, n_out, dev)
        rc = lib.kf_P(ctypes.byref(desc), dt, batch, n_in, n_out, _ptr(x), _ptr(g), _ptr(c), _ptr(p), _ptr(h), _ptr(ws), ws.numel(), stream)
        _lib.check(rc, "kf_P")
        del keep
        return p


def _rational_param_grad(plan, st: BasisState, x, h, w, m: int = 0):
    """(d num, d den) float32 of sum_{b,i} h w phi^(m)(x) for the rational plan."""
    lib = _lib.load()
    desc, keep = _desc(plan, m, st)
    batch, n_in = x.shape
    dev = x.device
    dnum = torch.empty_like(st.num)
    dden = torch.empty_like(st.den)
    nbytes = lib.kf_rational_workspace_bytes(ctypes.byref(desc), batch, n_in)
    ws = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev)
    with _on(dev):
        rc = lib.kf_rational_param_grad(
            ctypes.byref(desc), _dtype_code(x.dtype), batch, n_in, _ptr(x.contiguous()), _ptr(h), _ptr(None if w is None else w.contiguous()),
            _ptr(dnum), _ptr(dden), _ptr(ws), ws.numel(), _stream(dev),
        )
    _lib.check(rc, "kf_rational_param_grad")
    return dnum, dden


# --- custom ops ---------------------------------------------------------------------
#
# Every launch is a torch custom op in the ``kf`` namespace with its autograd formula registered
# (the F/G/P closure of kanforge/torch/kernels.py:70-128) and a fake kernel for shape inference,
# so the layers trace under torch.compile. A plan crosses the op boundary as an exact string key;
# basis tables (B-spline knots, rational parameters) as optional tensors.


_PLAN_KEYS: dict = {}


def plan_key(plan: KernelPlan | str) -> str:
    """Exact text form of a plan (floats in hexadecimal); a key passes through unchanged."""
    if isinstance(plan, str):
        return plan
    key = _PLAN_KEYS.get(plan)
    if key is None:
        consts = ",".join(str(v) for v in plan.consts)
        fold = ",".join(float(v).hex() for v in plan.fold_key)
        key = _PLAN_KEYS[plan] = f"{plan.kind};{consts};{plan.size};{int(plan.grid)};{fold}"
    return key


@lru_cache(maxsize=None)
def plan_of(key: str) -> KernelPlan:
    kind, consts, size, grid, fold = key.split(";")
    parts = consts.split(",")
    if kind == "cheb":
        cst = (int(parts[0]), parts[1])
    else:
        cst = (int(parts[0]), int(parts[1]))
    fk = tuple(float.fromhex(v) for v in fold.split(",")) if fold else ()
    return KernelPlan(kind, cst, int(size), fk, bool(int(grid)))


def _state(knots, knots_cmp, knots_u, num, den, n_in: int) -> BasisState | None:
    if knots is not None:
        return BasisState(knots=knots, knots_cmp=knots_cmp, knots_u=knots_u)
    if num is not None:
        return rational_state(num, den, n_in // num.shape[0])
    return None


def _tables(st: BasisState | None):
    """(knots, knots_cmp, knots_u) of a state, for the op arguments."""
    if st is None or st.knots is None:
        return None, None, None
    return st.knots, st.knots_cmp, st.knots_u


Opt = Optional[torch.Tensor]


def _mul(w, t):
    return t if w is None else w * t


def _plain(t) -> bool:
    """An eager call on a plain device tensor: nothing traces, compiles, fakes or transforms it
    (meta and CPU tensors go to the op: its fake kernel, or its device check)."""
    return (
        type(t) is torch.Tensor
        and t.is_cuda
        and not torch.compiler.is_compiling()
        and torch._C._len_torch_dispatch_stack() == 0
        and not torch._C._is_torch_function_mode_enabled()
        and not torch._C._are_functorch_transforms_active()
    )


class _Entry:
    """How this module calls a kf op. Eager calls on plain tensors run its twin, a
    torch.autograd.Function with the op's implementation and the op's autograd formula (the
    custom-op dispatcher costs more host time per call than a small layer's kernels take);
    traced, compiled and fake-tensor calls run the registered op, so torch.compile and opcheck
    see the ops."""

    def __init__(self, op, impl, setup, backward):
        self.op = op

        # forward(ctx, ...) rather than a separate setup_context: with setup_context, every
        # Function.apply binds its arguments through inspect.signature (tens of microseconds)
        def forward(ctx, *args):
            out = impl(*args)
            setup(ctx, args, out)
            return out

        self.twin = type(
            f"{impl.__name__}_twin",
            (torch.autograd.Function,),
            {"forward": staticmethod(forward), "backward": staticmethod(backward)},
        )

    def __call__(self, *args):
        if _plain(args[0]):
            return self.twin.apply(*args)
        return self.op(*args)


def _F_impl(x: torch.Tensor, w: Opt, c: torch.Tensor, knots: Opt, knots_cmp: Opt, knots_u: Opt, num: Opt, den: Opt, plan: str, m: int) -> torch.Tensor:
    """y[b,o] = sum_{i,k} w[b,i] c[o,i,k] phi_k^(m)(x[b,i])."""
    return _raw("F", plan_of(plan), m, x, w, c, _state(knots, knots_cmp, knots_u, num, den, x.shape[1]), c.shape[0])


op_F = torch.library.custom_op("kf::F", mutates_args=())(_F_impl)


def _G_impl(x: torch.Tensor, g: torch.Tensor, w: Opt, knots: Opt, knots_cmp: Opt, knots_u: Opt, num: Opt, den: Opt, plan: str, m: int) -> torch.Tensor:
    """dc[o,i,k] = sum_b w[b,i] g[b,o] phi_k^(m)(x[b,i])."""
    return _raw("G", plan_of(plan), m, x, w, g, _state(knots, knots_cmp, knots_u, num, den, x.shape[1]), g.shape[1])


op_G = torch.library.custom_op("kf::G", mutates_args=())(_G_impl)


def _P_impl(x: torch.Tensor, g: torch.Tensor, c: torch.Tensor, knots: Opt, knots_cmp: Opt, knots_u: Opt, num: Opt, den: Opt, plan: str, m: int) -> torch.Tensor:
    """p[b,i] = sum_{o,k} g[b,o] c[o,i,k] phi_k^(m)(x[b,i])."""
    return _raw("P", plan_of(plan), m, x, g, c, _state(knots, knots_cmp, knots_u, num, den, x.shape[1]), c.shape[0])


op_P = torch.library.custom_op("kf::P", mutates_args=())(_P_impl)


def _rational_bwd_impl(
    x: torch.Tensor, g: torch.Tensor, c: torch.Tensor, w: Opt, num: torch.Tensor, den: torch.Tensor, plan: str, m: int
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(P_{m+1}(x, g, c), d/dnum, d/dden) of sum_{b,o} g[b,o] F_m(x, c, w)[b,o] for a rational
    plan: one P launch that also writes h = sum_o g c, then the parameter-gradient reduction of
    sum h w phi^(m)."""
    pl = plan_of(plan)
    st = _state(None, None, None, num, den, x.shape[1])
    p1, dnum, dden = _rational_bwd_raw(pl, m, st, x, g, c, w)
    return p1, dnum.to(num.dtype), dden.to(den.dtype)


op_rational_bwd = torch.library.custom_op("kf::rational_bwd", mutates_args=())(_rational_bwd_impl)


def _rational_bwd_raw(pl: KernelPlan, m: int, st: BasisState, x, g, c, w):
    """kf_rational_bwd: (P_{m+1}(x, g, c), float32 d/dnum, d/dden of sum h w phi^(m))."""
    _require_device(x)
    lib = _lib.load()
    desc, keep = _desc(pl, m, st)
    dt = _dtype_code(x.dtype)
    batch, n_in = x.shape
    n_out = c.shape[0]
    x, g, c = x.contiguous(), g.contiguous(), c.contiguous()
    w = None if w is None else w.contiguous()
    p1 = torch.empty_like(x)
    dnum, dden = torch.empty_like(st.num), torch.empty_like(st.den)
    nbytes = lib.kf_rational_bwd_workspace_bytes(ctypes.byref(desc), dt, batch, n_in, n_out)
    ws = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=x.device)
    with _on(x.device):
        rc = lib.kf_rational_bwd(
            ctypes.byref(desc), dt, batch, n_in, n_out, _ptr(x), _ptr(g), _ptr(c), _ptr(w), _ptr(p1), _ptr(dnum),
            _ptr(dden), _ptr(ws), ws.numel(), _stream(x.device),
        )
    _lib.check(rc, "kf_rational_bwd")
    del keep
    return p1, dnum, dden


def _rational_param_grad_impl(x: torch.Tensor, h: torch.Tensor, w: Opt, num: torch.Tensor, den: torch.Tensor, plan: str, m: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(d/dnum, d/dden) of sum_{b,i} h[b,i] w[b,i] phi^(m)(x[b,i]) for a rational plan."""
    st = _state(None, None, None, num, den, x.shape[1])
    dnum, dden = _rational_param_grad(plan_of(plan), st, x, h.float().contiguous(), w, m)
    return dnum.to(num.dtype), dden.to(den.dtype)


op_rational_param_grad = torch.library.custom_op("kf::rational_param_grad", mutates_args=())(_rational_param_grad_impl)


@op_F.register_fake
def _(x, w, c, knots, knots_cmp, knots_u, num, den, plan, m):
    return x.new_empty(x.shape[0], c.shape[0])


@op_G.register_fake
def _(x, g, w, knots, knots_cmp, knots_u, num, den, plan, m):
    return x.new_empty(g.shape[1], x.shape[1], plan_of(plan).size)


@op_P.register_fake
def _(x, g, c, knots, knots_cmp, knots_u, num, den, plan, m):
    return x.new_empty(x.shape)


@op_rational_bwd.register_fake
def _(x, g, c, w, num, den, plan, m):
    return x.new_empty(x.shape), torch.empty_like(num), torch.empty_like(den)


@op_rational_param_grad.register_fake
def _(x, h, w, num, den, plan, m):
    return torch.empty_like(num), torch.empty_like(den)


def _save(ctx, tensors, plan, m):
    ctx.save_for_backward(*tensors)
    ctx.plan, ctx.m = plan, m


def _F_setup(ctx, inputs, output):
    x, w, c, knots, knots_cmp, knots_u, num, den, plan, m = inputs
    _save(ctx, (x, w, c, knots, knots_cmp, knots_u, num, den), plan, m)


def _f_grads(x, w, c, tabs, plan, m, need, gy):
    """(gx, gw, gc, gnum, gden) of sum gy F_m(x, w, c); need = (x, w, c, num, den) flags."""
    gx = gw = gc = gnum = gden = None
    num, den = tabs[3], tabs[4]
    if plan_of(plan).kind == "rational" and (need[3] or need[4]):
        p1, gnum, gden = _RBWD(x, gy, c, w, num, den, plan, m)
        if need[0]:
            # under create_graph the x-gradient stays differentiable through kf::P
            gx = _mul(w, _P(x, gy, c, *tabs, plan, 1) if torch.is_grad_enabled() else p1)
    elif need[0]:
        gx = _mul(w, _P(x, gy, c, *tabs, plan, m + 1))
    if need[2]:
        gc = _G(x, gy, w, *tabs, plan, m)
    if need[1]:
        gw = _P(x, gy, c, *tabs, plan, m)
    return gx, gw, gc, gnum, gden


def _F_backward(ctx, gy):
    x, w, c, knots, knots_cmp, knots_u, num, den = ctx.saved_tensors
    n = ctx.needs_input_grad
    gx, gw, gc, gnum, gden = _f_grads(x, w, c, (knots, knots_cmp, knots_u, num, den), ctx.plan, ctx.m,
                                      (n[0], n[1], n[2], n[6], n[7]), gy.contiguous())
    return gx, gw, gc, None, None, None, gnum, gden, None, None


def _G_setup(ctx, inputs, output):
    x, g, w, knots, knots_cmp, knots_u, num, den, plan, m = inputs
    _save(ctx, (x, g, w, knots, knots_cmp, knots_u, num, den), plan, m)


def _G_backward(ctx, gdc):
    x, g, w, knots, knots_cmp, knots_u, num, den = ctx.saved_tensors
    plan, m = ctx.plan, ctx.m
    need = ctx.needs_input_grad
    gdc = gdc.contiguous()
    tabs = (knots, knots_cmp, knots_u, num, den)
    gx = gnum = gden = None
    if need[6] or need[7]:
        # d<gdc, G_m>/dtheta = sum_{b,i} (sum_o g gdc) w dphi^(m)/dtheta: the h of P(x, g, gdc)
        p1, gnum, gden = _RBWD(x, g, gdc, w, num, den, plan, m)
        if need[0]:
            gx = _mul(w, _P(x, g, gdc, *tabs, plan, m + 1) if torch.is_grad_enabled() else p1)
    elif need[0]:
        gx = _mul(w, _P(x, g, gdc, *tabs, plan, m + 1))
    gg = _F(x, w, gdc, *tabs, plan, m) if need[1] else None
    gw = _P(x, g, gdc, *tabs, plan, m) if need[2] else None
    return gx, gg, gw, None, None, None, gnum, gden, None, None


def _P_setup(ctx, inputs, output):
    x, g, c, knots, knots_cmp, knots_u, num, den, plan, m = inputs
    _save(ctx, (x, g, c, knots, knots_cmp, knots_u, num, den), plan, m)


def _P_backward(ctx, gp):
    x, g, c, knots, knots_cmp, knots_u, num, den = ctx.saved_tensors
    plan, m = ctx.plan, ctx.m
    need = ctx.needs_input_grad
    gp = gp.contiguous()
    tabs = (knots, knots_cmp, knots_u, num, den)
    gx = gnum = gden = None
    if need[6] or need[7]:
        # d<gp, P_m>/dtheta = sum_{b,i} gp (sum_o g c) dphi^(m)/dtheta: P(x, g, c)'s h, weight gp
        p1, gnum, gden = _RBWD(x, g, c, gp, num, den, plan, m)
        if need[0]:
            gx = gp * (_P(x, g, c, *tabs, plan, m + 1) if torch.is_grad_enabled() else p1)
    elif need[0]:
        gx = gp * _P(x, g, c, *tabs, plan, m + 1)
    gg = _F(x, gp, c, *tabs, plan, m) if need[1] else None
    gc = _G(x, g, gp, *tabs, plan, m) if need[2] else None
    return gx, gg, gc, None, None, None, gnum, gden, None, None


def _no_second_order(ctx, *grads):
    raise NotImplementedError("gradients of the rational parameter gradients themselves (third order in the "
                              "parameters) are not compiled into the HIP kernels")


def _no_ctx(ctx, inputs, output):
    pass


op_F.register_autograd(_F_backward, setup_context=_F_setup)
op_G.register_autograd(_G_backward, setup_context=_G_setup)
op_P.register_autograd(_P_backward, setup_context=_P_setup)
op_rational_bwd.register_autograd(_no_second_order, setup_context=_no_ctx)
op_rational_param_grad.register_autograd(_no_second_order, setup_context=_no_ctx)


def _rat(st: BasisState | None, num, den):
    """The rational parameter tensors an op receives: the caller's (so gradients reach them) or
    the state's float32 copies."""
    if st is None or st.num is None:
        return None, None
    return (st.num if num is None else num), (st.den if den is None else den)


def prim_F(x, c, w, st, plan, m=0, num=None, den=None):
    num, den = _rat(st, num, den)
    return _F(x, w, c, *_tables(st), num, den, plan_key(plan), m)


def prim_G(x, g, w, st, plan, m=0, num=None, den=None):
    num, den = _rat(st, num, den)
    return _G(x, g, w, *_tables(st), num, den, plan_key(plan), m)


def prim_P(x, g, c, st, plan, m=0, num=None, den=None):
    num, den = _rat(st, num, den)
    return _P(x, g, c, *_tables(st), num, den, plan_key(plan), m)


def spline_forward(x: torch.Tensor, coef: torch.Tensor, st: BasisState | None, plan: KernelPlan | str, num=None, den=None,
                   bias: torch.Tensor | None = None) -> torch.Tensor:
    """sum_{i,k} coef[o,i,k] phi_k(x[..., i]) (+ bias[o]) through the HIP F kernel.

    Computes in the coefficients' dtype (float32 or bfloat16) and returns ``x.dtype``; a bias in
    that dtype rides F's last kernel (kf_F_bias), one in another dtype is added afterwards.
    """
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    if x2.dtype != coef.dtype:
        x2 = x2.to(coef.dtype)
    if bias is not None and bias.dtype == coef.dtype and x.dtype == coef.dtype:
        nr, dr = _rat(st, num, den)
        y = _F_BIAS(x2, None, coef, bias, *_tables(st), nr, dr, plan_key(plan), 0)
        return y.reshape(*lead, coef.shape[0])
    y = prim_F(x2, coef, None, st, plan, 0, num, den)
    y = y.to(x.dtype).reshape(*lead, coef.shape[0])
    return y if bias is None else bias_add(y, bias)


# --- basis values and edge derivatives ---------------------------------------------


def _features_raw(plan, m, st, x2: torch.Tensor) -> torch.Tensor:
    _require_device(x2)
    lib = _lib.load()
    desc, keep = _desc(plan, m, st)
    batch, n_in = x2.shape
    out = torch.empty(batch, n_in, plan.size, dtype=x2.dtype, device=x2.device)
    with _on(x2.device):
        rc = lib.kf_features(ctypes.byref(desc), _dtype_code(x2.dtype), batch, n_in, _ptr(x2), _ptr(out), _stream(x2.device))
    _lib.check(rc, "kf_features")
    return out


def _features_impl(x: torch.Tensor, knots: Opt, knots_cmp: Opt, knots_u: Opt, num: Opt, den: Opt, plan: str, m: int) -> torch.Tensor:
    """phi_k^(m)(x[b,i]), (B, in, K)."""
    return _features_raw(plan_of(plan), m, _state(knots, knots_cmp, knots_u, num, den, x.shape[1]), x.contiguous())


op_features = torch.library.custom_op("kf::features", mutates_args=())(_features_impl)


@op_features.register_fake
def _(x, knots, knots_cmp, knots_u, num, den, plan, m):
    return x.new_empty(x.shape[0], x.shape[1], plan_of(plan).size)


def _features_setup(ctx, inputs, output):
    x, knots, knots_cmp, knots_u, num, den, plan, m = inputs
    _save(ctx, (x, knots, knots_cmp, knots_u, num, den), plan, m)


def _features_backward(ctx, gphi):
    x, knots, knots_cmp, knots_u, num, den = ctx.saved_tensors
    plan, m = ctx.plan, ctx.m
    need = ctx.needs_input_grad
    gx = gnum = gden = None
    if need[0]:
        gx = (gphi * _FEAT(x, knots, knots_cmp, knots_u, num, den, plan, m + 1)).sum(-1)
    if need[4] or need[5]:
        gnum, gden = _rational_grads_of(plan, x, gphi[..., 0], m, num, den)
    return gx, None, None, None, gnum, gden, None, None


op_features.register_autograd(_features_backward, setup_context=_features_setup)


def _column_sums_impl(g: torch.Tensor) -> torch.Tensor:
    """sum over the rows of g (rows, n), float32 accumulation, g's dtype (kf_column_sums)."""
    _require_device(g)
    g = g.contiguous()
    rows, n = g.shape
    lib = _lib.load()
    out = torch.empty(n, dtype=g.dtype, device=g.device)
    nbytes = lib.kf_column_sums_workspace_bytes(rows, n)
    ws = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=g.device)
    with _on(g.device):
        rc = lib.kf_column_sums(_dtype_code(g.dtype), rows, n, _ptr(g), _ptr(out), _ptr(ws), ws.numel(), _stream(g.device))
    _lib.check(rc, "kf_column_sums")
    return out


op_column_sums = torch.library.custom_op("kf::column_sums", mutates_args=())(_column_sums_impl)


@op_column_sums.register_fake
def _(g):
    return g.new_empty(g.shape[1])


def _colsum_setup(ctx, inputs, output):
    ctx.rows = inputs[0].shape[0]


def _colsum_backward(ctx, gout):
    return gout.unsqueeze(0).expand(ctx.rows, -1) if ctx.needs_input_grad[0] else None


op_column_sums.register_autograd(_colsum_backward, setup_context=_colsum_setup)


def _bias_add_impl(y: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """y + bias over the last dimension; its bias gradient runs on kf_column_sums."""
    return y + bias


op_bias_add = torch.library.custom_op("kf::bias_add", mutates_args=())(_bias_add_impl)


@op_bias_add.register_fake
def _(y, bias):
    return torch.empty_like(y)


def _bias_setup(ctx, inputs, output):
    ctx.bias_dtype = inputs[1].dtype


def _bias_backward(ctx, gy):
    gb = None
    if ctx.needs_input_grad[1]:
        gb = _COLSUM(gy.reshape(-1, gy.shape[-1])).to(ctx.bias_dtype)
    return gy, gb


op_bias_add.register_autograd(_bias_backward, setup_context=_bias_setup)


def _silu_taylor_impl(h: torch.Tensor, hp: torch.Tensor, S: Opt) -> tuple[torch.Tensor, torch.Tensor]:
    """(A, sq) of the SiLU base branch's second-order Taylor terms (kf_silu_taylor): for h (B, n),
    hp (D, B, n), S (B, n) or None, sq = sum_d hp_d^2 and the stacked GEMM operand
    A = [silu(h); silu'(h) hp_d ...; silu''(h) sq + silu'(h) S] ((D + 2) B, n)."""
    _require_device(h)
    D, B, n = hp.shape
    h, hp = h.contiguous(), hp.contiguous()
    S = None if S is None else S.contiguous()
    A = torch.empty((D + 2) * B, n, dtype=h.dtype, device=h.device)
    sq = torch.empty_like(h)
    with _on(h.device):
        rc = _lib.load().kf_silu_taylor(_dtype_code(h.dtype), D, B, n, _ptr(h), _ptr(hp), _ptr(S), _ptr(A), _ptr(sq),
                                        _stream(h.device))
    _lib.check(rc, "kf_silu_taylor")
    return A, sq


op_silu_taylor = torch.library.custom_op("kf::silu_taylor", mutates_args=())(_silu_taylor_impl)


@op_silu_taylor.register_fake
def _(h, hp, S):
    D, B, n = hp.shape
    return h.new_empty((D + 2) * B, n), torch.empty_like(h)


def _silu_taylor_setup(ctx, inputs, output):
    h, hp, S = inputs
    ctx.save_for_backward(h, hp, S, output[1])


def _silu_taylor_backward(ctx, gA, gsq):
    """Derivatives of A and sq through silu^(m), m <= 3, in closed form (s = sigmoid(h)):
    d1 = s (1 + h (1 - s)), d2 = s (1 - s) (2 + h (1 - 2 s)),
    d3 = s (1 - s) (3 (1 - 2 s) + h (1 - 6 s + 6 s^2))."""
    h, hp, S, sq = ctx.saved_tensors
    D, B, n = hp.shape
    f = torch.float32
    x, hpf = h.to(f), hp.to(f)
    s = torch.sigmoid(x)
    d1 = s * (1 + x * (1 - s))
    d2 = s * (1 - s) * (2 + x * (1 - 2 * s))
    d3 = s * (1 - s) * (3 * (1 - 2 * s) + x * (1 - 6 * s + 6 * s * s))
    gA = gA.to(f)
    g0, g1, g2 = gA[:B], gA[B:(D + 1) * B].reshape(D, B, n), gA[(D + 1) * B:]
    sqf = sq.to(f)
    dh = g0 * d1 + (g1 * hpf).sum(0) * d2 + g2 * (d3 * sqf)
    if S is not None:
        dh = dh + g2 * d2 * S.to(f)
    gq = g2 * d2 if gsq is None else g2 * d2 + gsq.to(f)
    dhp = g1 * d1 + 2 * gq * hpf
    dS = None if S is None else (g2 * d1).to(S.dtype)
    return dh.to(h.dtype), dhp.to(hp.dtype), dS


op_silu_taylor.register_autograd(_silu_taylor_backward, setup_context=_silu_taylor_setup)


def silu_taylor(h: torch.Tensor, hp: torch.Tensor, S: torch.Tensor | None) -> tuple[torch.Tensor, torch.Tensor]:
    """kf::silu_taylor (see its implementation): the SiLU base branch's Taylor operands."""
    return _SILU_T(h, hp, S)


BIAS_OP_MIN_ELEMENTS = 1 << 20  # below this a plain add costs less (one op dispatch fewer)


def bias_add(y: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """The layer's bias add: y + bias; for large outputs the bias gradient runs on
    kf_column_sums (torch's reduction over the rows is several times slower there)."""
    if y.numel() < BIAS_OP_MIN_ELEMENTS:
        return y + bias
    return _BIAS(y, bias)


def _rational_grads_of(plan, x2, h, m, num, den):
    """d/d(num, den) of sum_{b,i} h[b,i] phi^(m)(x[b,i]) for a rational plan."""
    return _RPGRAD(x2, h.float().contiguous(), None, num, den, plan, m)


def basis_derivative(basis, x: torch.Tensor, m: int, params: dict | None) -> torch.Tensor:
    """Basis.derivative on a device tensor: ``(..., in, K)`` through kf_features."""
    from ..kernels.plan import plan_for

    if not isinstance(x, torch.Tensor):
        raise TypeError("basis evaluation runs on the GPU: pass a torch tensor on a ROCm device")
    _require_device(x)
    plan = plan_for(basis)
    if plan is None:
        raise RuntimeError(f"no HIP kernel for {basis!r}")
    st = state_from_params(plan, basis, params, x)
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    if x2.dtype not in _DTYPES:
        x2 = x2.float()
    num = den = None
    if plan.kind == "rational":
        num, den = st.num, st.den
        if params is not None and isinstance(params.get("numerator"), torch.Tensor):
            # the (rows, p+1) / (rows, q) views the state was built from, so gradients reach the caller's tensors
            num, den = params["numerator"], params["denominator"]
            if num.dim() == 1:
                num, den = num[None], den[None]
    out = _FEAT(x2, *_tables(st), num, den, plan_key(plan), m)
    return out.to(x.dtype).reshape(*lead, x.shape[-1], plan.size)


def state_from_params(plan, basis, params: dict | None, like: torch.Tensor) -> BasisState | None:
    """BasisState from per-input parameters ``{name: (in or groups, *shape)}`` (or defaults)."""
    n_in = like.shape[-1]
    if plan.kind == "cheb":
        return None
    if plan.kind == "bspline":
        if params is None or "grid" not in params:
            grid = torch.as_tensor(np.broadcast_to(basis.param_specs()["grid"].value, (n_in, basis.grid_size + 1)).copy(), device=like.device)
        else:
            grid = torch.as_tensor(params["grid"], device=like.device)
            grid = grid.expand(n_in, grid.shape[-1]) if grid.dim() == 1 or grid.shape[0] == 1 else grid
        return bspline_state(grid, basis.order)
    if params is None:
        specs = basis.param_specs()
        num = torch.as_tensor(specs["numerator"].value, device=like.device)[None]
        den = torch.as_tensor(specs["denominator"].value, device=like.device)[None]
    else:
        num = torch.as_tensor(params["numerator"], device=like.device)
        den = torch.as_tensor(params["denominator"], device=like.device)
        if num.dim() == 1:
            num, den = num[None], den[None]
    rows = num.shape[0]
    if n_in % rows:
        raise ValueError(f"rational parameters have {rows} rows, which does not divide {n_in} inputs")
    return rational_state(num, den, n_in // rows)


def _edge_raw(plan, m, st, x2, c, base_w):
    lib = _lib.load()
    desc, keep = _desc(plan, m, st)
    batch, n_in = x2.shape
    n_out = c.shape[0]
    out = torch.empty(batch, n_out, n_in, dtype=x2.dtype, device=x2.device)
    with _on(x2.device):
        rc = lib.kf_edge_derivative(
            ctypes.byref(desc), _dtype_code(x2.dtype), batch, n_in, n_out, _ptr(x2), _ptr(c.contiguous()),
            _ptr(None if base_w is None else base_w.contiguous()), _ptr(out), _stream(x2.device),
        )
    _lib.check(rc, "kf_edge_derivative")
    return out


def _edge_impl(x: torch.Tensor, c: torch.Tensor, base_w: Opt, knots: Opt, knots_cmp: Opt, knots_u: Opt, num: Opt, den: Opt, plan: str, m: int) -> torch.Tensor:
    """d[b,o,i] = sum_k c[o,i,k] phi_k^(m)(x[b,i]) + base_w[o,i] silu^(m)(x[b,i]), (B, out, in)."""
    return _edge_raw(plan_of(plan), m, _state(knots, knots_cmp, knots_u, num, den, x.shape[1]), x.contiguous(), c, base_w)


op_edge = torch.library.custom_op("kf::edge_derivative", mutates_args=())(_edge_impl)


@op_edge.register_fake
def _(x, c, base_w, knots, knots_cmp, knots_u, num, den, plan, m):
    return x.new_empty(x.shape[0], c.shape[0], x.shape[1])


def _edge_setup(ctx, inputs, output):
    x, c, base_w, knots, knots_cmp, knots_u, num, den, plan, m = inputs
    _save(ctx, (x, c, base_w, knots, knots_cmp, knots_u, num, den), plan, m)


def _edge_backward(ctx, gd):
    x, c, base_w, knots, knots_cmp, knots_u, num, den = ctx.saved_tensors
    plan, m = ctx.plan, ctx.m
    need = ctx.needs_input_grad
    gx = gc = gw = gnum = gden = None
    tabs = (knots, knots_cmp, knots_u, num, den)
    if need[0]:
        # d/dx of the edge is the edge derivative of order m+1
        gx = (gd * _EDGE(x, c, base_w, *tabs, plan, m + 1)).sum(1)
    if need[1]:
        phi = _FEAT(x, knots, knots_cmp, knots_u, num, den, plan, m)  # (B, in, K)
        gc = torch.einsum("boi,bik->oik", gd, phi)
    if need[2] and base_w is not None:
        gw = torch.einsum("boi,bi->oi", gd, silu_derivative_t(x, m))
    if need[6] or need[7]:
        # one feature per edge: sum_o gd[b,o,i] c[o,i,0] multiplies phi^(m)(x[b,i])
        h = torch.einsum("boi,oi->bi", gd.float(), c[..., 0].float())
        gnum, gden = _rational_grads_of(plan, x, h, m, num, den)
    return gx, gc, gw, None, None, None, gnum, gden, None, None


op_edge.register_autograd(_edge_backward, setup_context=_edge_setup)


def silu_derivative_t(x: torch.Tensor, m: int) -> torch.Tensor:
    """d^m/dx^m silu(x) with torch ops (x p_m(s) + m p_{m-1}(s), s = sigmoid(x))."""
    from .._calculus import SIGMOID_FACTOR, chain_polys

    s = torch.sigmoid(x)
    if m == 0:
        return x * s
    polys = chain_polys([0.0, 1.0], SIGMOID_FACTOR, m)

    def hp(c):
        y = torch.zeros_like(s) + float(c[-1])
        for v in reversed(c[:-1]):
            y = y * s + float(v)
        return y

    return x * hp(polys[m]) + m * hp(polys[m - 1])


def edge_derivative(x: torch.Tensor, coef_eff: torch.Tensor, base_w: torch.Tensor | None, st, plan, m: int,
                    num=None, den=None) -> torch.Tensor:
    """(..., out, in) edge derivatives through kf_edge_derivative; a rational plan's ``num``/``den``
    (groups, ...) receive gradients (order 0)."""
    _require_device(x)
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    if x2.dtype != coef_eff.dtype:
        x2 = x2.to(coef_eff.dtype)
    num, den = _rat(st, num, den)
    d = _EDGE(x2, coef_eff, base_w, *_tables(st), num, den, plan_key(plan), m)
    return d.to(x.dtype).reshape(*lead, coef_eff.shape[0], x.shape[-1])


@torch.library.custom_op("kf::bspline_interval", mutates_args=())
def op_bspline_interval(x: torch.Tensor, knots_cmp: torch.Tensor) -> torch.Tensor:
    """int32 interval index of float32 x (B, in) on the comparison knots (in, nk); -1 outside."""
    _require_device(x)
    lib = _lib.load()
    x = x.contiguous().float()
    kc = knots_cmp.contiguous().float()
    out = torch.empty(x.shape, dtype=torch.int32, device=x.device)
    with _on(x.device):
        rc = lib.kf_bspline_interval(x.shape[0], x.shape[1], _ptr(x), _ptr(kc), kc.shape[1], _ptr(out), _stream(x.device))
    _lib.check(rc, "kf_bspline_interval")
    return out


@op_bspline_interval.register_fake
def _(x, knots_cmp):
    return torch.empty(x.shape, dtype=torch.int32, device=x.device)


def bspline_interval(x: torch.Tensor, knots_cmp: torch.Tensor) -> torch.Tensor:
    """int32 interval index of float32 x (B, in) on the comparison knots (in, nk); -1 outside."""
    return op_bspline_interval(x, knots_cmp)


# --- F with the layer's bias -----------------------------------------------------------


def _F_bias_impl(x: torch.Tensor, w: Opt, c: torch.Tensor, bias: torch.Tensor, knots: Opt, knots_cmp: Opt, knots_u: Opt,
                 num: Opt, den: Opt, plan: str, m: int) -> torch.Tensor:
    """y[b,o] = sum_{i,k} w[b,i] c[o,i,k] phi_k^(m)(x[b,i]) + bias[o] (kf_F_bias)."""
    return _raw("F", plan_of(plan), m, x, w, c, _state(knots, knots_cmp, knots_u, num, den, x.shape[1]), c.shape[0],
                bias=bias)


op_F_bias = torch.library.custom_op("kf::F_bias", mutates_args=())(_F_bias_impl)


@op_F_bias.register_fake
def _(x, w, c, bias, knots, knots_cmp, knots_u, num, den, plan, m):
    return x.new_empty(x.shape[0], c.shape[0])


def _F_bias_setup(ctx, inputs, output):
    x, w, c, bias, knots, knots_cmp, knots_u, num, den, plan, m = inputs
    _save(ctx, (x, w, c, knots, knots_cmp, knots_u, num, den), plan, m)
    ctx.bias_dtype = bias.dtype


def _F_bias_backward(ctx, gy):
    x, w, c, knots, knots_cmp, knots_u, num, den = ctx.saved_tensors
    n = ctx.needs_input_grad
    gy = gy.contiguous()
    tabs = (knots, knots_cmp, knots_u, num, den)
    both = n[2] and n[3]  # coefficient and bias gradients: one G launch with the column sums
    gx, gw, gc, gnum, gden = _f_grads(x, w, c, tabs, ctx.plan, ctx.m, (n[0], n[1], n[2] and not both, n[7], n[8]), gy)
    gb = None
    if both:
        gc, gb = _G_BIAS(x, gy, w, *tabs, ctx.plan, ctx.m)
        gb = gb.to(ctx.bias_dtype)
    elif n[3]:
        gb = _COLSUM(gy).to(ctx.bias_dtype)
    return gx, gw, gc, gb, None, None, None, gnum, gden, None, None


op_F_bias.register_autograd(_F_bias_backward, setup_context=_F_bias_setup)


def _G_bias_impl(x: torch.Tensor, g: torch.Tensor, w: Opt, knots: Opt, knots_cmp: Opt, knots_u: Opt, num: Opt, den: Opt,
                 plan: str, m: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(dc, db): G_m(x, g, w) and the column sums of g (kf_G_bias)."""
    return _raw("G", plan_of(plan), m, x, w, g, _state(knots, knots_cmp, knots_u, num, den, x.shape[1]), g.shape[1],
                bias_grad=True)


op_G_bias = torch.library.custom_op("kf::G_bias", mutates_args=())(_G_bias_impl)


@op_G_bias.register_fake
def _(x, g, w, knots, knots_cmp, knots_u, num, den, plan, m):
    return x.new_empty(g.shape[1], x.shape[1], plan_of(plan).size), x.new_empty(g.shape[1])


def _G_bias_backward(ctx, gdc, gdb):
    """G's formula for dc; the column sums send gdb to every row of g."""
    if gdc is None:
        gdc = torch.zeros(ctx.saved_tensors[1].shape[1], ctx.saved_tensors[0].shape[1], plan_of(ctx.plan).size,
                          dtype=ctx.saved_tensors[0].dtype, device=ctx.saved_tensors[0].device)
    res = list(_G_backward(ctx, gdc))
    if gdb is not None and ctx.needs_input_grad[1]:
        g = ctx.saved_tensors[1]
        extra = gdb.to(g.dtype)[None, :].expand(g.shape[0], -1)
        res[1] = extra if res[1] is None else res[1] + extra
    return tuple(res)


op_G_bias.register_autograd(_G_bias_backward, setup_context=_G_setup)


# --- the SiLU base branch and bias fused into the contractions ----------------------
#
# The reference's layer adds F.linear(silu(x), base_weight) and the bias to the spline part
# (kanforge/torch/layers.py:185-191). For bf16 Chebyshev plans kf_F_base runs silu(x) as one more
# feature of the F contraction and folds the bias into its per-output constant, kf_P_base adds
# silu'(x) (g W) in P's epilogue and kf_G_base returns the base weights' and the bias's gradients
# next to the coefficient gradient. bf16 B-splines run silu(x) and the bias as extra feature
# columns of F's GEMM, G as for Chebyshev, and (cubic, 11 basis functions) P with W^T in a spare
# feature slot of its tile; float32 B-splines (the sparse route) take W as one more basis function
# whose feature is silu(x) in F, P and G.

_FUSED: dict = {}


def base_fused(plan: KernelPlan | str, st: BasisState | None, dtype: torch.dtype, batch: int, n_in: int,
               n_out: int) -> tuple[bool, bool, bool]:
    """Whether (kf_F_base, kf_P_base, kf_G_base) take a layer of this plan and these shapes (the
    routes depend on the plan and the shapes, not on the basis tables)."""
    key = (plan_key(plan), dtype, batch, n_in, n_out)
    hit = _FUSED.get(key)
    if hit is None:
        pl = plan_of(key[0])
        hit = (False, False, False)
        if pl.kind in ("cheb", "bspline") and dtype in _DTYPES and batch > 0:
            lib = _lib.load()
            d0, _ = _desc(pl, 0, st)
            d1, _ = _desc(pl, 1, st)
            dt = _DTYPES[dtype]
            q = lambda op, d: lib.kf_base_fused(op, ctypes.byref(d), dt, batch, n_in, n_out) == 1
            hit = (q(_lib.KF_OP_F_BASE, d0), q(_lib.KF_OP_P_BASE, d1), q(_lib.KF_OP_G_BASE, d0))
        if len(_FUSED) > 4096:
            _FUSED.clear()
        _FUSED[key] = hit
    return hit


def _dsilu(x: torch.Tensor) -> torch.Tensor:
    s = torch.sigmoid(x)
    return s * (1 + x * (1 - s))


def _f_base_raw(pl: KernelPlan, st: BasisState | None, x, c, bw, bias) -> torch.Tensor:
    """kf_F_base on contiguous arrays."""
    lib = _lib.load()
    desc, keep = _desc(pl, 0, st)
    batch, n_in = x.shape
    n_out = c.shape[0]
    dev = x.device
    dt = _dtype_code(x.dtype)
    y = torch.empty(batch, n_out, dtype=x.dtype, device=dev)
    ws = _workspace(_lib.KF_OP_F_BASE, desc, dt, batch, n_in, n_out, dev)
    with _on(dev):
        rc = lib.kf_F_base(ctypes.byref(desc), dt, batch, n_in, n_out, _ptr(x), _ptr(c), _ptr(bw), _ptr(bias), _ptr(y),
                           _ptr(ws), ws.numel(), _stream(dev))
    _lib.check(rc, "kf_F_base")
    del keep
    return y


def _F_base_impl(x: torch.Tensor, c: torch.Tensor, bw: torch.Tensor, bias: Opt, knots: Opt, knots_cmp: Opt, knots_u: Opt,
                 plan: str) -> torch.Tensor:
    """y = F_0(x, c) + silu(x) bw^T + bias: the layer's forward with its SiLU base branch (kf_F_base
    where it takes the layer, else kf_F and one GEMM)."""
    _require_device(x)
    pl = plan_of(plan)
    st = _state(knots, knots_cmp, knots_u, None, None, x.shape[1])
    x, c, bw = x.contiguous(), c.contiguous(), bw.contiguous()
    bias = None if bias is None else bias.contiguous()
    if not base_fused(pl, st, x.dtype, x.shape[0], x.shape[1], c.shape[0])[0]:
        y = _raw("F", pl, 0, x, None, c, st, c.shape[0])
        y = torch.addmm(y, torch.nn.functional.silu(x), bw.t())
        return y if bias is None else y.add_(bias)
    return _f_base_raw(pl, st, x, c, bw, bias)


op_F_base = torch.library.custom_op("kf::F_base", mutates_args=())(_F_base_impl)


@op_F_base.register_fake
def _(x, c, bw, bias, knots, knots_cmp, knots_u, plan):
    return x.new_empty(x.shape[0], c.shape[0])


def _p_base_raw(pl: KernelPlan, st: BasisState | None, x, g, c, bw) -> torch.Tensor:
    """kf_P_base (order-1 descriptor) on contiguous arrays."""
    lib = _lib.load()
    desc, keep = _desc(pl, 1, st)
    batch, n_in = x.shape
    n_out = c.shape[0]
    dev = x.device
    dt = _dtype_code(x.dtype)
    p = torch.empty(batch, n_in, dtype=x.dtype, device=dev)
    ws = _workspace(_lib.KF_OP_P_BASE, desc, dt, batch, n_in, n_out, dev)
    with _on(dev):
        rc = lib.kf_P_base(ctypes.byref(desc), dt, batch, n_in, n_out, _ptr(x), _ptr(g), _ptr(c), _ptr(bw), _ptr(p),
                           _ptr(ws), ws.numel(), _stream(dev))
    _lib.check(rc, "kf_P_base")
    del keep
    return p


def _P_base_impl(x: torch.Tensor, g: torch.Tensor, c: torch.Tensor, bw: torch.Tensor, knots: Opt, knots_cmp: Opt,
                 knots_u: Opt, plan: str) -> torch.Tensor:
    """P_1(x, g, c) + silu'(x) (g bw): the layer's input gradient with its SiLU base branch."""
    _require_device(x)
    st = _state(knots, knots_cmp, knots_u, None, None, x.shape[1])
    return _p_base_raw(plan_of(plan), st, x.contiguous(), g.contiguous(), c.contiguous(), bw.contiguous())


op_P_base = torch.library.custom_op("kf::P_base", mutates_args=())(_P_base_impl)


@op_P_base.register_fake
def _(x, g, c, bw, knots, knots_cmp, knots_u, plan):
    return x.new_empty(x.shape)


def _g_base_raw(pl: KernelPlan, st: BasisState | None, x, g, want_c: bool, want_w: bool, want_b: bool):
    """kf_G_base on contiguous arrays: (dc, dW, db), empty where not wanted."""
    lib = _lib.load()
    desc, keep = _desc(pl, 0, st)
    batch, n_in = x.shape
    n_out = g.shape[1]
    dev = x.device
    dt = _dtype_code(x.dtype)
    dc = torch.empty((n_out, n_in, pl.size) if want_c else (0,), dtype=x.dtype, device=dev)
    dw = torch.empty((n_out, n_in) if want_w else (0,), dtype=x.dtype, device=dev)
    db = torch.empty((n_out,) if want_b else (0,), dtype=x.dtype, device=dev)
    ws = _workspace(_lib.KF_OP_G_BASE, desc, dt, batch, n_in, n_out, dev)
    with _on(dev):
        rc = lib.kf_G_base(ctypes.byref(desc), dt, batch, n_in, n_out, _ptr(x), _ptr(g), _ptr(dc if want_c else None),
                           _ptr(dw if want_w else None), _ptr(db if want_b else None), _ptr(ws), ws.numel(), _stream(dev))
    _lib.check(rc, "kf_G_base")
    del keep
    return dc, dw, db


def _G_base_impl(x: torch.Tensor, g: torch.Tensor, knots: Opt, knots_cmp: Opt, knots_u: Opt, plan: str, want_c: bool,
                 want_w: bool, want_b: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(G_0(x, g), g^T silu(x), sum_b g): the layer's parameter gradients with its SiLU base branch
    and bias; an output not wanted comes back empty."""
    _require_device(x)
    st = _state(knots, knots_cmp, knots_u, None, None, x.shape[1])
    return _g_base_raw(plan_of(plan), st, x.contiguous(), g.contiguous(), want_c, want_w, want_b)


op_G_base = torch.library.custom_op("kf::G_base", mutates_args=())(_G_base_impl)


@op_G_base.register_fake
def _(x, g, knots, knots_cmp, knots_u, plan, want_c, want_w, want_b):
    n_out, n_in, K = g.shape[1], x.shape[1], plan_of(plan).size
    return (x.new_empty((n_out, n_in, K) if want_c else (0,)), x.new_empty((n_out, n_in) if want_w else (0,)),
            x.new_empty((n_out,) if want_b else (0,)))


def _F_base_setup(ctx, inputs, output):
    x, c, bw, bias, knots, knots_cmp, knots_u, plan = inputs
    ctx.save_for_backward(x, c, bw, knots, knots_cmp, knots_u)
    ctx.plan = plan
    ctx.bias_dtype = None if bias is None else bias.dtype


def _F_base_backward(ctx, gy):
    x, c, bw, knots, knots_cmp, knots_u = ctx.saved_tensors
    plan = ctx.plan
    need = ctx.needs_input_grad
    gy = gy.contiguous()
    gx = gc = gw = gb = None
    tabs = (knots, knots_cmp, knots_u)
    rat = (None, None)
    dims = (x.shape[0], x.shape[1], c.shape[0])
    if torch.is_grad_enabled() or not all(type(d) is int for d in dims):
        # a graph is being built (higher orders), or traced with symbolic shapes: composed ops
        fused = (False, False, False)
    else:
        st = _state(knots, knots_cmp, knots_u, None, None, x.shape[1])
        fused = base_fused(plan, st, x.dtype, *dims)
    if need[0]:
        if fused[1]:
            gx = _P_BASE(x, gy, c, bw, *tabs, plan)
        else:  # differentiable composition (also under create_graph)
            gx = _P(x, gy, c, *tabs, *rat, plan, 1) + _dsilu(x) * (gy @ bw)
    if need[1] or need[2] or need[3]:
        if fused[2]:
            dc, dw, db = _G_BASE(x, gy, *tabs, plan, need[1], need[2], need[3])
            gc, gw, gb = (dc if need[1] else None), (dw if need[2] else None), (db if need[3] else None)
        else:
            gc = _G(x, gy, None, *tabs, *rat, plan, 0) if need[1] else None
            gw = gy.t() @ torch.nn.functional.silu(x) if need[2] else None
            gb = _COLSUM(gy).to(ctx.bias_dtype) if need[3] else None
    return gx, gc, gw, gb, None, None, None, None


op_F_base.register_autograd(_F_base_backward, setup_context=_F_base_setup)


class _Direct:
    """An op without autograd (called inside backward formulas): eager calls on plain tensors run
    its implementation directly, everything else the registered op."""

    def __init__(self, op, impl):
        self.op, self.impl = op, impl

    def __call__(self, *args):
        return self.impl(*args) if _plain(args[0]) else self.op(*args)


def spline_base_forward(x: torch.Tensor, coef: torch.Tensor, base_w: torch.Tensor, bias: torch.Tensor | None,
                        st: BasisState | None, plan: KernelPlan | str) -> torch.Tensor:
    """The layer's spline part, SiLU base branch and bias as one op whose forward and backward use
    the fused entry points where they take the layer; x (..., in), everything in x's dtype.
    Callers check base_fused first."""
    lead = x.shape[:-1]
    y = _F_BASE(x.reshape(-1, x.shape[-1]), coef, base_w, bias, *_tables(st), plan_key(plan))
    return y.reshape(*lead, coef.shape[0])


# --- eager entries (see _Entry) ---------------------------------------------------

_F = _Entry(op_F, _F_impl, _F_setup, _F_backward)
_G = _Entry(op_G, _G_impl, _G_setup, _G_backward)
_P = _Entry(op_P, _P_impl, _P_setup, _P_backward)
_RBWD = _Entry(op_rational_bwd, _rational_bwd_impl, _no_ctx, _no_second_order)
_RPGRAD = _Entry(op_rational_param_grad, _rational_param_grad_impl, _no_ctx, _no_second_order)
_FEAT = _Entry(op_features, _features_impl, _features_setup, _features_backward)
_COLSUM = _Entry(op_column_sums, _column_sums_impl, _colsum_setup, _colsum_backward)
_BIAS = _Entry(op_bias_add, _bias_add_impl, _bias_setup, _bias_backward)
_SILU_T = _Entry(op_silu_taylor, _silu_taylor_impl, _silu_taylor_setup, _silu_taylor_backward)
_EDGE = _Entry(op_edge, _edge_impl, _edge_setup, _edge_backward)
_F_BASE = _Entry(op_F_base, _F_base_impl, _F_base_setup, _F_base_backward)
_P_BASE = _Direct(op_P_base, _P_base_impl)
_G_BASE = _Direct(op_G_base, _G_base_impl)
_F_BIAS = _Entry(op_F_bias, _F_bias_impl, _F_bias_setup, _F_bias_backward)
_G_BIAS = _Entry(op_G_bias, _G_bias_impl, _G_setup, _G_bias_backward)
