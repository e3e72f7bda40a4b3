"""Headline benchmark: KANLinear 768 -> 3072, Chebyshev(8) (K=9, tanh squash),
bfloat16 with float32 accumulation, batch 8192; one step = forward + dX + dCoef
(the F_0, P_1 and G_0 launches of the HIP path). Prints one JSON line.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu]

Inputs are seeded synthetic tensors resident in HBM before timing starts:
x ~ N(0, 1) (seed 0), coef ~ N(0, 1/(768*9)) (seed 1), upstream gradient
gy ~ N(0, 1) (seed 3). Algorithmic work per step is 3 contractions of
2*B*in*K*out FLOP = 1.0437 TFLOP. The line also carries ``with_base``: the
same step for the layer's defaults (SiLU base branch and bias on, 1.160 TFLOP).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

B, IN, OUT, DEGREE = 8192, 768, 3072, 8
K = DEGREE + 1
FLOP_PER_CONTRACTION = 2.0 * B * IN * K * OUT
STEP_FLOP = 3 * FLOP_PER_CONTRACTION
PEAK_BF16 = 2.5e15  # MI355X dense bf16 MFMA, FLOP/s


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-base", action="store_true", help="skip the default-layer (base branch on) leg")
    return ap.parse_args()


class EntryTimer:
    """HIP events around every F/G/P entry point, on the launch stream."""

    def __init__(self):
        self.active = False
        self.events = {"F": [], "G": [], "P": []}

    def wrap(self, raw):
        def timed(op, *args, **kwargs):
            if not self.active:
                return raw(op, *args, **kwargs)
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record()
            out = raw(op, *args, **kwargs)
            e.record()
            self.events[op].append((s, e))
            return out

        return timed

    def mean_ms(self):
        return {op: (sum(s.elapsed_time(e) for s, e in ev) / len(ev) if ev else 0.0) for op, ev in self.events.items()}


TRAFFIC_FILE = os.path.join("profiles", "kanlinear_768x3072_cheb8_bf16_hbm_traffic.md")


def measured_traffic(entry):
    """HBM bytes per launch of one entry point, from the committed counter summary
    (FETCH_SIZE and WRITE_SIZE passes scaled by a plain copy's readings); None if absent."""
    try:
        lines = open(os.path.join(ROOT, TRAFFIC_FILE)).read().splitlines()
    except OSError:
        return None
    for line in lines:
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) == 4 and cells[0] == entry:
            try:
                return float(cells[3])
            except ValueError:
                return None
    return None


def cpu_baseline():
    from oracle.torch_cpu import cpu_model, time_chebyshev_step

    rows = int(os.environ.get("KF_CPU_ROWS", "1024"))
    t, threads = time_chebyshev_step(rows, IN, OUT, DEGREE, torch.bfloat16)
    t32, _ = time_chebyshev_step(rows, IN, OUT, DEGREE, torch.float32)
    return {
        "value": rows / t,
        "unit": "samples/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{rows} of the {B} rows, same layer shape, bf16 torch-CPU plain route (basis tensor + F.linear + autograd), median of 3 after 1 warm-up",
        "tflops": 3 * 2.0 * rows * IN * K * OUT / t / 1e12,
        "value_fp32": rows / t32,
        "cpu": cpu_model(),
    }


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build runs on a single MI355X (no multi-GPU path); use --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)

    import kanforge_amd as kf
    from kanforge_amd.torch import KANLinear
    from kanforge_amd.torch import kernels as kmod

    timer = EntryTimer()
    kmod._raw = timer.wrap(kmod._raw)

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    layer = KANLinear(IN, OUT, kf.Chebyshev(DEGREE), base_activation=None, bias=False, device=dev, dtype=torch.bfloat16)
    gen = torch.Generator().manual_seed(1)
    with torch.no_grad():
        layer.coef.copy_((torch.randn(OUT, IN, K, generator=gen) / math.sqrt(IN * K)).to(torch.bfloat16))
    x = torch.randn(B, IN, generator=torch.Generator().manual_seed(0)).to(dev, torch.bfloat16).requires_grad_()
    gy = torch.randn(B, OUT, generator=torch.Generator().manual_seed(3)).to(dev, torch.bfloat16)

    def step():
        y = layer(x)
        return torch.autograd.grad(y, [x, layer.coef], gy)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    timer.active = True
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    timer.active = False

    ms = elapsed / args.steps * 1e3
    per_op = timer.mean_ms()

    with_base = None
    if not args.no_base:
        # the default layer (SiLU base branch and bias on): the same step plus the base GEMMs
        # (2 * B * in * out per contraction, forward, dX and dW: 0.116 TFLOP more)
        base = KANLinear(IN, OUT, kf.Chebyshev(DEGREE), device=dev, dtype=torch.bfloat16)
        with torch.no_grad():
            base.coef.copy_(layer.coef)

        def step_base():
            y = base(x)
            return torch.autograd.grad(y, [x, base.coef, base.base_weight, base.bias], gy)

        for _ in range(args.warmup):
            step_base()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for _ in range(args.steps):
            step_base()
        torch.cuda.synchronize()
        ms_base = (time.perf_counter() - t1) / args.steps * 1e3
        with_base = {
            "layer": "KANLinear(768, 3072, Chebyshev(8)) defaults: SiLU base branch, bias",
            "ms_per_step": ms_base,
            "value": B / (ms_base * 1e-3),
            "tflops": (STEP_FLOP + 3 * 2.0 * B * IN * OUT) / (ms_base * 1e-3) / 1e12,
        }
    dominant = max(per_op, key=per_op.get)
    achieved = FLOP_PER_CONTRACTION / (per_op[dominant] * 1e-3) / 1e12
    out = {
        "metric": "KANLinear fwd+bwd samples/sec and TFLOP/s (% MFMA peak) at 768->3072",
        "value": B / (ms * 1e-3),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "KANLinear 768->3072 Chebyshev(8) tanh, bf16 x/coef, fp32 accumulate, batch 8192, forward + dX + dCoef",
            "batch": B,
            "in_features": IN,
            "out_features": OUT,
            "basis": "chebyshev(degree=8)",
            "base_activation": None,
            "bias": False,
            "seeds": {"x": 0, "coef": 1, "gy": 3},
            "coef_init": "N(0, 1/(768*9)) (variance)",
        },
        "tflops": STEP_FLOP / (ms * 1e-3) / 1e12,
        "frac_of_bf16_peak": STEP_FLOP / (ms * 1e-3) / PEAK_BF16,
        "per_entry_ms": per_op,
        "with_base": with_base,
        "roofline": {
            "bound": "mfma",
            "kernel": f"kf_{dominant}",
            "achieved": achieved,
            "peak": PEAK_BF16 / 1e12,
            "unit": "TFLOP/s",
            "frac": achieved * 1e12 / PEAK_BF16,
            "traffic": measured_traffic(f"kf_{dominant}"),
            "traffic_unit": "bytes per launch",
            "traffic_source": TRAFFIC_FILE,
        },
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
