"""Torch-CPU restatement of the reference's plain-ops route (the CPU baseline).

TEST INFRASTRUCTURE ONLY: timed by ``bench.py`` as ``cpu_baseline`` (kind
"port") and never called by the product path.

kanforge/torch/layers.py:181-186 computes the spline branch as
``F.linear(basis(x).flatten(-2), coef.flatten(1))`` with the basis tensor
materialised by the Chebyshev recurrence of kanforge/bases/polynomial.py:87-95
(z = tanh x; T_0 = 1, T_1 = z, T_j = 2 z T_{j-1} - T_{j-2}); backward is torch
autograd.
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
