"""Torch-CPU restatement of the reference's plain-ops route (the CPU baseline).

TEST INFRASTRUCTURE ONLY: timed by ``bench.py`` as ``cpu_baseline`` (kind
"port") and never called by the product path.

kanforge/torch/layers.py:181-186 computes the spline branch as
``F.linear(basis(x).flatten(-2), coef.flatten(1))`` with the basis tensor
materialised by the Chebyshev recurrence of kanforge/bases/polynomial.py:87-95
(z = tanh x; T_0 = 1, T_1 = z, T_j = 2 z T_{j-1} - T_{j-2}); backward is torch
autograd. The same route for the other workloads: B-splines by Cox-de Boor
(kanforge/bases/spline.py:74-92), group rationals P/(1+|Q|)
(kanforge/bases/rational.py:84-101), the SiLU base branch and bias
(kanforge/torch/layers.py:185-191), edge second derivatives by autograd over the
elementwise basis (kanforge/torch/layers.py:206-226) and the Laplacian by
reverse-over-reverse autograd (kanforge/torch/science.py:25-46).
"""

from __future__ import annotations

import os
import platform
import time

import torch
import torch.nn.functional as F


def chebyshev_basis(x: torch.Tensor, degree: int) -> torch.Tensor:
    z = torch.tanh(x)
    ts = [torch.ones_like(z)]
    if degree >= 1:
        ts.append(z)
    for _ in range(2, degree + 1):
        ts.append(2 * z * ts[-1] - ts[-2])
    return torch.stack(ts, -1)


def kan_step(x: torch.Tensor, coef: torch.Tensor, gy: torch.Tensor, degree: int):
    """Forward + dX + dCoef of the spline branch (no base, no bias)."""
    x = x.detach().requires_grad_()
    coef = coef.detach().requires_grad_()
    y = F.linear(chebyshev_basis(x, degree).flatten(-2), coef.flatten(1))
    gx, gc = torch.autograd.grad(y, [x, coef], gy)
    return y, gx, gc


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def time_chebyshev_step(rows: int, n_in: int, n_out: int, degree: int, dtype: torch.dtype, reps: int = 3, seed: int = 0):
    """Median seconds of one fwd+bwd over ``rows`` samples on the CPU, and the thread count."""
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(seed)
    K = degree + 1
    x = torch.randn(rows, n_in, generator=g).to(dtype)
    coef = (torch.randn(n_out, n_in, K, generator=g) / (n_in * K) ** 0.5).to(dtype)
    gy = torch.randn(rows, n_out, generator=g).to(dtype)
    kan_step(x, coef, gy, degree)  # warm-up
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        kan_step(x, coef, gy, degree)
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], threads


# --------------------------------------------------------------------------
# the other layer workloads (module parameters copied to the CPU)


def bspline_basis_t(x: torch.Tensor, knots: torch.Tensor, k: int) -> torch.Tensor:
    """(B, in, n-1-k) B-splines of degree k, knots (in, n), from half-open indicators."""
    xe = x.unsqueeze(-1)
    t = knots.to(x.dtype)
    b = ((xe >= t[:, :-1]) & (xe < t[:, 1:])).to(x.dtype)
    for q in range(1, k + 1):
        left = (xe - t[:, : -(q + 1)]) / (t[:, q:-1] - t[:, : -(q + 1)])
        right = (t[:, q + 1 :] - xe) / (t[:, q + 1 :] - t[:, 1:-q])
        b = left * b[..., :-1] + right * b[..., 1:]
    return b


def polynomial_basis_t(x: torch.Tensor, cheb: torch.Tensor, input_map: str) -> torch.Tensor:
    """(B, in, size): the family's Chebyshev coefficients ``cheb`` (D+1, size) applied to T_j(z)."""
    z = torch.tanh(x) if input_map == "tanh" else x
    ts = [torch.ones_like(z), z]
    for _ in range(2, cheb.shape[0]):
        ts.append(2 * z * ts[-1] - ts[-2])
    return torch.stack(ts[: cheb.shape[0]], -1) @ cheb.to(x.dtype)


def rational_t(x: torch.Tensor, num: torch.Tensor, den: torch.Tensor) -> torch.Tensor:
    """(B, in) P(x)/(1+|Q(x)|) with group g's coefficients on its in/groups consecutive inputs."""
    B, n_in = x.shape
    groups = num.shape[0]
    xg = x.view(B, groups, n_in // groups)
    P = torch.zeros_like(xg)
    for p in range(num.shape[1] - 1, -1, -1):
        P = P * xg + num[:, p, None].to(x.dtype)
    Q = torch.zeros_like(xg)
    for q in range(den.shape[1] - 1, -1, -1):
        Q = Q * xg + den[:, q, None].to(x.dtype)
    return (P / (1 + (Q * xg).abs())).view(B, n_in)


class CpuLayer:
    """A KAN layer's parameters on the CPU and its plain-ops forward."""

    def __init__(self, layer, dtype: torch.dtype):
        from oracle.kan64 import extend_grid

        def cpu(t):
            return None if t is None else t.detach().to("cpu", dtype).clone().requires_grad_()

        self.kind = type(layer.basis).__name__
        self.coef = cpu(layer.coef)
        self.base_weight = cpu(layer.base_weight)
        self.bias = cpu(layer.bias)
        if self.kind == "BSpline":
            g = layer.basis_grid.detach().double().cpu().numpy()
            self.k = layer.basis.order
            self.knots = torch.from_numpy(extend_grid(g, self.k)).to(dtype)
        elif hasattr(layer, "basis_numerator"):
            self.kind = "rational"
            self.num = cpu(layer.basis_numerator)
            self.den = cpu(layer.basis_denominator)
        else:
            self.cheb = torch.from_numpy(layer.basis._cheb).to(dtype)
            self.input_map = layer.basis.input_map

    def params(self):
        extra = [self.num, self.den] if self.kind == "rational" else []
        return [p for p in (self.coef, self.base_weight, self.bias, *extra) if p is not None]

    def basis(self, x):
        if self.kind == "BSpline":
            return bspline_basis_t(x, self.knots, self.k)
        if self.kind == "rational":
            return rational_t(x, self.num, self.den).unsqueeze(-1)
        return polynomial_basis_t(x, self.cheb, self.input_map)

    def __call__(self, x):
        y = F.linear(self.basis(x).flatten(-2), self.coef.flatten(1))
        if self.base_weight is not None:
            y = y + F.linear(F.silu(x), self.base_weight)
        if self.bias is not None:
            y = y + self.bias
        return y

    def edge_second(self, x):
        """(B, out, in) d2/dx2 of every edge's function, by autograd over the elementwise basis."""
        xr = x.detach().requires_grad_()
        phi = self.basis(xr)
        d2 = []
        for k in range(phi.shape[-1]):
            (g1,) = torch.autograd.grad(phi[..., k].sum(), xr, create_graph=True)
            (g2,) = torch.autograd.grad(g1.sum(), xr, retain_graph=True)
            d2.append(g2)
        out = torch.einsum("bik,oik->boi", torch.stack(d2, -1), self.coef.detach())
        if self.base_weight is not None:
            (s1,) = torch.autograd.grad(F.silu(xr).sum(), xr, create_graph=True)
            (s2,) = torch.autograd.grad(s1.sum(), xr)
            out = out + s2[:, None, :] * self.base_weight.detach()[None]
        return out


def _median_time(fn, reps: int = 3):
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    torch.set_num_threads(threads)
    fn()  # warm-up
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], threads


def time_train_step(layers, x: torch.Tensor, gy: torch.Tensor, reps: int = 3):
    """Median seconds of forward + backward (input and every parameter) through the CPU layers."""
    xr = x.detach().requires_grad_()
    params = [xr] + [p for layer in layers for p in layer.params()]

    def step():
        h = xr
        for layer in layers:
            h = layer(h)
        return torch.autograd.grad(h, params, gy)

    return _median_time(step, reps)


def time_edge_step(layers, x: torch.Tensor, reps: int = 3):
    """Median seconds of every layer's (B, out, in) second derivatives at its own input."""

    def step():
        h = x.detach()
        outs = []
        for layer in layers:
            outs.append(layer.edge_second(h))
            with torch.no_grad():
                h = layer(h)
        return outs

    return _median_time(step, reps)


def time_laplacian_step(layers, x: torch.Tensor, reps: int = 3):
    """Median seconds of the Laplacian of the scalar network output, reverse over reverse."""

    def step():
        xr = x.detach().requires_grad_()
        u = xr
        for layer in layers:
            u = layer(u)
        (g,) = torch.autograd.grad(u.sum(), xr, create_graph=True)
        return sum(torch.autograd.grad(g[:, d].sum(), xr, retain_graph=True)[0][:, d] for d in range(x.shape[1]))

    return _median_time(step, reps)


def cpu_isa() -> str:
    """The vector and matrix extensions the host CPU reports (flags of /proc/cpuinfo)."""
    want = ("avx2", "avx512f", "avx512_bf16", "avx512_fp16", "amx_bf16", "amx_tile", "amx_int8")
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    have = set(line.split(":", 1)[1].split())
                    return " ".join(w for w in want if w in have) or "none of " + " ".join(want)
    except OSError:
        pass
    return "unknown"
