"""Headline benchmark: KANLinear 768 -> 3072, Chebyshev(8) (K=9, tanh squash),
bfloat16 with float32 accumulation, batch 8192; one step = forward + dX + dCoef
(the F_0, P_1 and G_0 launches of the HIP path). Prints one JSON line.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu] [--no-base]
    python bench.py --workload {bspline_ffn,grkan_ffn,pinn_edge,pinn_laplacian,kan64,all}

The second form times the other layer shapes instead of the headline, one JSON
line each (whole-step throughput and HIP-event means per entry point).

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
    ap.add_argument(
        "--workload",
        default="cheb768",
        choices=["cheb768", *WORKLOADS, "all"],
        help="cheb768 (default) is the headline line; the others time the remaining layer shapes one line each",
    )
    return ap.parse_args()


class EntryTimer:
    """HIP events around every F/G/P entry point, on the launch stream."""

    def __init__(self):
        self.active = False
        self.events = {"F": [], "G": [], "P": []}

    def wrap(self, raw, label=None):
        def timed(*args, **kwargs):
            if not self.active:
                return raw(*args, **kwargs)
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record()
            out = raw(*args, **kwargs)
            e.record()
            self.events.setdefault(label or args[0], []).append((s, e))
            return out

        return timed

    def mean_ms(self):
        return {op: (sum(s.elapsed_time(e) for s, e in ev) / len(ev) if ev else 0.0) for op, ev in self.events.items()}

    def count(self):
        return {op: len(ev) for op, ev in self.events.items()}


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


def mfma_probe(dev, iters=4000, blocks=512):
    """Sustained bf16 MFMA rate of this card (kf_probe_mfma): back-to-back 32x32x16 MFMAs on
    pseudo-random operands, rotating through eight register sets ("changing") or one ("fixed"),
    two waves per SIMD; with the shader clock the probe's waves ran at."""
    import ctypes

    from kanforge_amd.torch import _lib

    lib = _lib.load()
    out = torch.empty(blocks * 256 * 3, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev)
    res = {}
    for label, rotate in (("changing", 1), ("fixed", 0)):
        for _ in range(2):  # warm-up launch, then the timed one
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record(stream)
            rc = lib.kf_probe_mfma(blocks, iters, rotate, ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(stream.cuda_stream))
            e.record(stream)
            _lib.check(rc, "kf_probe_mfma")
        torch.cuda.synchronize()
        ms = s.elapsed_time(e)
        flop = blocks * 4 * iters * 8 * 2.0 * 32 * 32 * 16
        t = out.view(blocks, 256, 3)[:, 0, 1:].double().cpu()
        clock = (t[:, 0] / (t[:, 1] / 1e8)).median().item()
        res[label] = {"tflops": flop / (ms * 1e-3) / 1e12, "frac_of_peak": flop / (ms * 1e-3) / PEAK_BF16, "clock_ghz": clock / 1e9}
    return res


def _timed(step, steps, warmup, timer):
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    timer.active = True
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    timer.active = False
    return (time.perf_counter() - t0) / steps * 1e3


def _randn(shape, seed, scale=1.0):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)) * scale


def wl_bspline_ffn(dev):
    """kanify'd GPT-2-small FFN: KANLinear 768->3072 then 3072->768, B-spline grid 8 order 3
    (K=11), layer defaults (SiLU base, bias), bf16, 8 x 2048 tokens, forward + backward."""
    import kanforge_amd as kf
    from kanforge_amd.torch.transformer import KANFFN

    tok, dim, hid, k = 8 * 2048, 768, 3072, 11
    ffn = KANFFN(dim, hid, kind="kan", basis=kf.BSpline(8, 3)).to(dev, torch.bfloat16)
    with torch.no_grad():
        ffn.fc1.coef.copy_(_randn(ffn.fc1.coef.shape, 1, 1 / math.sqrt(dim * k)))
        ffn.fc2.coef.copy_(_randn(ffn.fc2.coef.shape, 1, 1 / math.sqrt(hid * k)))
    x = _randn((8, 2048, dim), 0).to(dev, torch.bfloat16).requires_grad_()
    gy = _randn((8, 2048, dim), 3).to(dev, torch.bfloat16)
    params = [x, *ffn.parameters()]

    def step():
        return torch.autograd.grad(ffn(x), params, gy)

    per_contraction = 2.0 * tok * dim * k * hid
    return step, tok, "tokens/s", 6 * per_contraction + 6 * 2.0 * tok * dim * hid, per_contraction, "bf16"


def wl_grkan_ffn(dev):
    """GR-KAN FFN 768->3072->768, 8 groups, rational P degree 5 / Q degree 4, bf16,
    16 x 1024 tokens, P/Q ~ N(0, 0.1), forward + backward."""
    from kanforge_amd.torch.transformer import KANFFN

    tok, dim, hid = 16 * 1024, 768, 3072
    ffn = KANFFN(dim, hid, kind="grkan", groups=8).to(dev, torch.bfloat16)
    with torch.no_grad():
        for i, layer in enumerate((ffn.fc1, ffn.fc2)):
            layer.basis_numerator.copy_(_randn(layer.basis_numerator.shape, 2 + 2 * i, math.sqrt(0.1)))
            layer.basis_denominator.copy_(_randn(layer.basis_denominator.shape, 3 + 2 * i, math.sqrt(0.1)))
    x = _randn((16, 1024, dim), 0).to(dev, torch.bfloat16).requires_grad_()
    gy = _randn((16, 1024, dim), 3).to(dev, torch.bfloat16)
    params = [x, *ffn.parameters()]

    def step():
        return torch.autograd.grad(ffn(x), params, gy)

    per_gemm = 2.0 * tok * dim * hid
    return step, tok, "tokens/s", 6 * per_gemm, per_gemm, "bf16"


def _pinn_model(dev):
    import kanforge_amd as kf
    from kanforge_amd.torch import KAN

    model = KAN([2, 64, 64, 1], kf.Jacobi(6, 0.5, 0.5, input_map="tanh")).to(dev)
    with torch.no_grad():
        for i, layer in enumerate(model):
            layer.coef.copy_(_randn(layer.coef.shape, 1 + i, 1 / math.sqrt(layer.in_features * 7)))
    x = (torch.rand(65536, 2, generator=torch.Generator().manual_seed(0)) * 2 - 1).to(dev)
    return model, x


def wl_pinn_edge(dev):
    """PINN KAN [2, 64, 64, 1] Jacobi(6, 1/2, 1/2) tanh, fp32, 65536 points x ~ U(-1, 1)^2:
    KAN.edge_derivative(x, 2), every layer's (points, out, in) second derivatives."""
    model, x = _pinn_model(dev)

    def step():
        with torch.no_grad():
            return model.edge_derivative(x, 2)

    n = x.shape[0]
    out_bytes = 4.0 * n * (64 * 2 + 64 * 64 + 1 * 64)
    in_bytes = 4.0 * n * (2 + 64 + 64)
    return step, n, "points/s", None, out_bytes + in_bytes, "f32"


def wl_pinn_laplacian(dev):
    """The same PINN network: the chained Laplacian d2u/dx0^2 + d2u/dx1^2 over the
    network by reverse-over-reverse autograd through the F/G/P closure."""
    from kanforge_amd.torch import laplacian

    model, x = _pinn_model(dev)

    def step():
        return laplacian(model, x)

    n = x.shape[0]
    layer_pass = 2.0 * n * 7 * (2 * 64 + 64 * 64 + 64)
    return step, n, "points/s", None, layer_pass, "f32"


def wl_kan64(dev):
    """KANLinear 64->64 B-spline (grid 5, order 3, K=8) on [-1, 1], SiLU base, fp32,
    batch 4096, x ~ U(-1, 1), coef ~ N(0, 1/(64*8)), forward + backward."""
    import kanforge_amd as kf
    from kanforge_amd.torch import KANLinear

    layer = KANLinear(64, 64, kf.BSpline(5, 3)).to(dev)
    with torch.no_grad():
        layer.coef.copy_(_randn(layer.coef.shape, 1, 1 / math.sqrt(64 * 8)))
    x = (torch.rand(4096, 64, generator=torch.Generator().manual_seed(0)) * 2 - 1).to(dev).requires_grad_()
    gy = _randn((4096, 64), 3).to(dev)
    params = [x, *layer.parameters()]

    def step():
        return torch.autograd.grad(layer(x), params, gy)

    per_contraction = 2.0 * 4096 * 64 * 8 * 64
    return step, 4096, "samples/s", 3 * per_contraction + 3 * 2.0 * 4096 * 64 * 64, per_contraction, "f32"


WORKLOADS = {
    "bspline_ffn": wl_bspline_ffn,
    "grkan_ffn": wl_grkan_ffn,
    "pinn_edge": wl_pinn_edge,
    "pinn_laplacian": wl_pinn_laplacian,
    "kan64": wl_kan64,
}


def run_workload(name, args, dev):
    """One JSON line for a non-headline layer shape: whole-step throughput plus HIP-event
    means of every entry point it calls (F, G, P, edge, features)."""
    from kanforge_amd.torch import kernels as kmod

    timer = EntryTimer()
    timer.events = {}
    orig = kmod._raw, kmod._edge_raw, kmod._features_raw
    kmod._raw = timer.wrap(orig[0])
    kmod._edge_raw = timer.wrap(orig[1], "edge")
    kmod._features_raw = timer.wrap(orig[2], "features")
    try:
        step, units, unit, step_flop, per_launch, dtype = WORKLOADS[name](dev)
        ms = _timed(step, args.steps, args.warmup, timer)
    finally:
        kmod._raw, kmod._edge_raw, kmod._features_raw = orig
    per_op, calls = timer.mean_ms(), timer.count()
    line = {
        "metric": f"{name} throughput",
        "value": units / (ms * 1e-3),
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "dtype": dtype,
        "data": "synthetic",
        "config": {"workload": WORKLOADS[name].__doc__.split("\n\n")[0].replace("\n", " ").strip()},
        "per_entry_ms": per_op,
        "calls_per_step": {k: v / args.steps for k, v in calls.items()},
    }
    if step_flop is not None:
        line["tflops"] = step_flop / (ms * 1e-3) / 1e12
        line["frac_of_bf16_peak" if dtype == "bf16" else "frac_of_fp32_peak"] = (
            step_flop / (ms * 1e-3) / (PEAK_BF16 if dtype == "bf16" else 157.3e12)
        )
    if name == "pinn_edge":
        line["hbm_gbs"] = per_launch / (ms * 1e-3) / 1e9
        line["frac_of_hbm_peak"] = per_launch / (ms * 1e-3) / 8.0e12
    elif name == "pinn_laplacian":
        line["layer_pass_gflop"] = per_launch / 1e9
    return line


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build runs on a single MI355X (no multi-GPU path); use --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.workload != "cheb768":
        for name in WORKLOADS if args.workload == "all" else [args.workload]:
            print(json.dumps(run_workload(name, args, dev)), flush=True)
        return

    import kanforge_amd as kf
    from kanforge_amd.torch import KANLinear
    from kanforge_amd.torch import kernels as kmod

    timer = EntryTimer()
    kmod._raw = timer.wrap(kmod._raw)

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
    out["mfma_probe"] = mfma_probe(dev)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
