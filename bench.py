"""Headline benchmark: KANLinear 768 -> 3072, Chebyshev(8) (K=9, tanh squash),
bfloat16 with float32 accumulation, batch 8192; one step = forward + dX + dCoef
(the F_0, P_1 and G_0 launches of the HIP path). Prints one JSON line.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu] [--no-base] [--no-workloads]
    python bench.py --workload {kan64,grkan_ffn,pinn_edge,pinn_laplacian,bspline_ffn,lut_kan64,all}
    python bench.py --workload NAME --only {F,G,P,edge,...} --steps N

The headline line carries a ``workloads`` object with one entry per other layer
shape (KANLinear 64->64 B-spline fp32, GR-KAN FFN, PINN edge derivatives, PINN
Laplacian, B-spline FFN, lookup-table inference of the 64->64 layer): step time,
throughput, the roofline of the entry
point with the most GPU time (per-call algorithmic FLOP and bytes over HIP-event
durations; bound by whichever of MFMA and HBM time is larger) and a torch-CPU
baseline on a stated sample. The second form prints those lines on their own.
The third form is for counter runs: one step records the calls of one entry
point, a one-block probe kernel marks the end of that step in the dispatch
trace, then only those calls are replayed.

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


def with_base_leg(layer, x, gy, args, dev) -> dict:
    """The headline layer with its defaults (SiLU base branch and bias on): the same step plus the
    base branch's three products (2 B in out FLOP each: forward, dX and dW, 0.116 TFLOP more),
    fused into the contractions where the kernels take the layer."""
    import kanforge_amd as kf
    from kanforge_amd.torch import KANLinear
    from kanforge_amd.torch import kernels as K

    base = KANLinear(IN, OUT, kf.Chebyshev(DEGREE), device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        base.coef.copy_(layer.coef)

    def step_base():
        y = base(x)
        return torch.autograd.grad(y, [x, base.coef, base.base_weight, base.bias], gy)

    ms_base = _timed(step_base, args.steps, args.warmup)
    return {
        "layer": "KANLinear(768, 3072, Chebyshev(8)) defaults: SiLU base branch, bias",
        "ms_per_step": ms_base,
        "value": B / (ms_base * 1e-3),
        "tflops": (STEP_FLOP + 3 * 2.0 * B * IN * OUT) / (ms_base * 1e-3) / 1e12,
        "fused_entries": dict(zip(("F", "P", "G"), K.base_fused(base._plan_key, None, torch.bfloat16, B, IN, OUT))),
    }


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
        choices=["cheb768", "cheb768_base", *WORKLOADS, "all"],
        help="cheb768 (default) is the headline line; cheb768_base times only its default-layer (SiLU base "
        "branch and bias) leg; the others time the remaining layer shapes one line each",
    )
    ap.add_argument("--no-workloads", action="store_true", help="leave the other layer shapes out of the headline line")
    ap.add_argument("--workload-steps", type=int, default=10, help="timed steps of each other layer shape in the headline line")
    ap.add_argument("--only", choices=["F", "G", "P", "F_base", "P_base", "G_base", "edge", "features", "rational_param_grad",
                                       "rational_bwd", "lut"],
                    help="counter runs: replay only this entry point's calls of one step of --workload")
    return ap.parse_args()


PEAK_FP32 = 157.3e12  # MI355X dense fp32 MFMA, FLOP/s
PEAK_HBM = 8.0e12  # MI355X HBM3E, bytes/s


def _work(label, args):
    """Algorithmic (FLOP, HBM bytes) of one entry-point call: contractions count 2 B in K out
    FLOP (dense over the basis, the reference's convention); bytes count every operand read once
    and every output written once."""
    if label in ("F", "G", "P"):
        _, plan, _m, x, a, b, _st, n_out = args[:8]
        h = args[8] if len(args) > 8 else None
        batch, n_in = x.shape
        es, K = x.element_size(), plan.size
        flops = 2.0 * batch * n_in * K * n_out
        coef = n_out * n_in * K
        if label == "F":
            elems = batch * n_in * (1 + (a is not None)) + coef + batch * n_out
        elif label == "G":
            elems = batch * n_in * (1 + (a is not None)) + batch * n_out + coef
        else:
            elems = 2 * batch * n_in + batch * n_out + coef
        return flops, es * elems + (4.0 * batch * n_in if h is not None else 0.0)
    if label in ("F_base", "P_base", "G_base"):
        # the fused SiLU base branch: one more product of 2 B in out FLOP per contraction
        plan, _st, x, a = args[:4]
        batch, n_in = x.shape
        es, K = x.element_size(), plan.size
        if label == "G_base":
            want_c, want_w, want_b = args[4:7]
            n_out = a.shape[1]
            flops = 2.0 * batch * n_in * n_out * (K * want_c + want_w)
            elems = batch * n_in + batch * n_out + n_out * n_in * (K * want_c + want_w) + n_out * want_b
            return flops, float(es * elems)
        c = a if label == "F_base" else args[4]
        n_out = c.shape[0]
        flops = 2.0 * batch * n_in * (K + 1) * n_out
        coef = n_out * n_in * (K + 1)
        if label == "F_base":
            elems = batch * n_in + coef + n_out + batch * n_out
        else:
            elems = 2 * batch * n_in + batch * n_out + coef
        return flops, float(es * elems)
    if label == "edge":
        plan, _m, _st, x2, c, base_w = args[:6]
        batch, n_in = x2.shape
        n_out, es, K = c.shape[0], x2.element_size(), plan.size
        elems = batch * n_in + n_out * n_in * K + (0 if base_w is None else n_out * n_in) + batch * n_out * n_in
        return 2.0 * batch * n_in * K * n_out, float(es * elems)
    if label == "features":
        plan, _m, _st, x2 = args[:4]
        batch, n_in = x2.shape
        return 0.0, float(x2.element_size() * batch * n_in * (1 + plan.size))
    if label == "lut":
        layer, x = args[:2]
        n_in, _size, n_out = layer.tables.shape
        rows = x.numel() // n_in
        return 3.0 * rows * n_in * n_out, float(4 * rows * (n_in + n_out) + layer.tables.nbytes)
    if label == "rational_bwd":
        _plan, _m, _st, x, g, c = args[:6]
        w = args[6] if len(args) > 6 else None
        batch, n_in = x.shape
        n_out, es = c.shape[0], x.element_size()
        elems = 2 * batch * n_in + batch * n_out + n_out * n_in + (0 if w is None else batch * n_in)
        return 2.0 * batch * n_in * n_out, float(es * elems)
    if label == "rational_param_grad":
        _plan, _st, x, h, w = args[:5]
        n = x.numel()
        return 0.0, float(n * (x.element_size() + 4 + (0 if w is None else w.element_size())))
    return 0.0, 0.0


class EntryTimer:
    """HIP events around every entry-point call, on the launch stream, with each call's
    algorithmic work; ``record`` keeps the calls of one entry for replay."""

    def __init__(self):
        self.active = False
        self.events = {}
        self.record = None  # (label, list) while recording one entry's calls

    def wrap(self, raw, label=None):
        def timed(*args, **kwargs):
            lab = label or args[0]
            if self.record is not None and self.record[0] == lab:
                self.record[1].append((raw, args, kwargs))
            if not self.active:
                return raw(*args, **kwargs)
            stream = torch.cuda.current_stream()
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record(stream)
            out = raw(*args, **kwargs)
            e.record(stream)
            self.events.setdefault(lab, []).append((s, e) + _work(lab, args))
            return out

        return timed

    def mean_ms(self):
        return {op: (sum(ev[0].elapsed_time(ev[1]) for ev in evs) / len(evs) if evs else 0.0) for op, evs in self.events.items()}

    def count(self):
        return {op: len(ev) for op, ev in self.events.items()}

    def totals(self):
        """Per entry: (total ms, total FLOP, total bytes, calls) over the timed region."""
        return {
            op: (sum(ev[0].elapsed_time(ev[1]) for ev in evs), sum(ev[2] for ev in evs), sum(ev[3] for ev in evs), len(evs))
            for op, evs in self.events.items()
        }


STREAM_ENTRIES = ("edge", "features", "rational_param_grad", "lut")  # no contraction on MFMA


def roofline_of(totals, dtype, traffic_file=None):
    """Roofline of the entry point with the most GPU time: for contractions (F, G, P) bound by
    whichever of MFMA time (algorithmic FLOP at the dtype's dense peak) and HBM time (algorithmic
    bytes at 8 TB/s) is larger, for the streaming entries by HBM; achieved = that work over the
    entry's measured time (sums over its calls)."""
    op = max(totals, key=lambda k: totals[k][0])
    ms, flops, nbytes, calls = totals[op]
    peak_f = PEAK_BF16 if dtype == "bf16" else PEAK_FP32
    sec = ms * 1e-3
    if op not in STREAM_ENTRIES and flops / peak_f >= nbytes / PEAK_HBM:
        achieved, peak, unit, bound = flops / sec / 1e12, peak_f / 1e12, "TFLOP/s", "mfma"
    else:
        achieved, peak, unit, bound = nbytes / sec / 1e9, PEAK_HBM / 1e9, "GB/s", "hbm"
    traffic = measured_traffic(f"kf_{op}", traffic_file) if traffic_file else None
    return {
        "bound": bound,
        "kernel": f"kf_{op}",
        "achieved": achieved,
        "peak": peak,
        "unit": unit,
        "frac": achieved / peak,
        "traffic": traffic,
        "traffic_unit": "bytes per launch",
        "traffic_source": traffic_file if traffic is not None else None,
        "launches_per_step": None,
        "algorithmic_flop_per_launch": flops / calls,
        "algorithmic_bytes_per_launch": nbytes / calls,
        "ms_per_launch": ms / calls,
    }


TRAFFIC_FILE = os.path.join("profiles", "kanlinear_768x3072_cheb8_bf16_hbm_traffic.md")


def measured_traffic(entry, path=TRAFFIC_FILE):
    """HBM bytes per launch of one entry point, from a committed counter summary (FETCH_SIZE and
    WRITE_SIZE passes scaled by a plain copy's readings; the per-entry table's last column);
    None if absent."""
    try:
        lines = open(os.path.join(ROOT, path)).read().splitlines()
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


def _timed(step, steps, warmup, timer=None):
    """ms per step over ``steps`` after ``warmup``; with ``timer`` its HIP events record every
    entry-point call of the timed steps (their host cost then inflates the wall time of
    launch-bound steps, so the step time is taken from a run without them)."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    if timer is not None:
        timer.active = True
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    if timer is not None:
        timer.active = False
    return (time.perf_counter() - t0) / steps * 1e3


def _randn(shape, seed, scale=1.0):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)) * scale


def _cpu_rows(default):
    return int(os.environ.get("KF_CPU_ROWS_SCALE", "1") or 1) * default


def _cpu_train(layers, x, gy, rows, unit, what):
    """CPU leg: the torch-CPU plain route on the first ``rows`` rows of the same inputs."""
    from oracle import torch_cpu as tc

    dtype = x.dtype
    cl = [tc.CpuLayer(layer, dtype) for layer in layers]
    xs = x.detach()[:rows].cpu()
    gs = gy.detach()[:rows].cpu()
    t, threads = tc.time_train_step(cl, xs.reshape(-1, xs.shape[-1]), gs.reshape(-1, gs.shape[-1]))
    n = xs.reshape(-1, xs.shape[-1]).shape[0]
    return _cpu_line(n / t, unit, threads, f"{n} rows of the same inputs: {what}, torch-CPU plain route, median of 3 after 1 warm-up")


def _cpu_line(value, unit, threads, sample):
    from oracle.torch_cpu import cpu_isa, cpu_model

    return {"value": value, "unit": unit, "cores": threads, "kind": "port", "sample": sample, "cpu": cpu_model(), "isa": cpu_isa()}


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

    def cpu():
        return _cpu_train([ffn.fc1, ffn.fc2], x.reshape(-1, dim), gy.reshape(-1, dim), _cpu_rows(1024), "tokens/s", "B-spline FFN fwd+bwd, bf16")

    return step, tok, "tokens/s", "bf16", cpu


def wl_grkan_ffn(dev):
    """GR-KAN FFN 768->3072->768, 8 groups, rational P degree 5 / Q degree 4, bf16,
    16 x 1024 tokens, P/Q ~ N(0, 0.1), forward + backward."""
    from kanforge_amd.torch.transformer import KANFFN

    dim, hid = 768, 3072
    tok = 16 * 1024
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

    def cpu():
        return _cpu_train([ffn.fc1, ffn.fc2], x.reshape(-1, dim), gy.reshape(-1, dim), _cpu_rows(4096), "tokens/s", "GR-KAN FFN fwd+bwd incl. P/Q grads, bf16")

    return step, tok, "tokens/s", "bf16", cpu


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

    def cpu():
        from oracle import torch_cpu as tc

        rows = _cpu_rows(16384)
        t, threads = tc.time_edge_step([tc.CpuLayer(m, torch.float32) for m in model], x[:rows].cpu())
        return _cpu_line(rows / t, "points/s", threads, f"{rows} of the points: every layer's second edge derivatives by autograd over the basis, fp32, torch-CPU plain route, median of 3 after 1 warm-up")

    return step, x.shape[0], "points/s", "f32", cpu


def wl_pinn_laplacian(dev):
    """The same PINN network: the Laplacian d2u/dx0^2 + d2u/dx1^2 of the network output
    (kanforge_amd.torch.laplacian: second-order Taylor terms carried forward through F)."""
    from kanforge_amd.torch import laplacian

    model, x = _pinn_model(dev)

    def step():
        return laplacian(model, x)

    def cpu():
        from oracle import torch_cpu as tc

        rows = _cpu_rows(65536)
        t, threads = tc.time_laplacian_step([tc.CpuLayer(m, torch.float32) for m in model], x[:rows].cpu())
        return _cpu_line(rows / t, "points/s", threads, f"{rows} of the points: Laplacian by reverse-over-reverse autograd, fp32, torch-CPU plain route, median of 3 after 1 warm-up")

    return step, x.shape[0], "points/s", "f32", cpu


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

    def cpu():
        return _cpu_train([layer], x, gy, 4096, "samples/s", "the whole batch, fwd+bwd, fp32")

    return step, 4096, "samples/s", "f32", cpu


def wl_lut_kan64(dev):
    """Lookup-table inference of the KANLinear 64->64 B-spline (grid 5, order 3) layer with SiLU
    base: tables of 256 points per edge over the inputs' range, 65536 rows x ~ U(-1, 1); one step
    evaluates the float32 tables and their int8 quantisation (gather + lerp + sum)."""
    import kanforge_amd as kf
    from kanforge_amd.export import quantize, to_lut
    from kanforge_amd.torch import KANLinear

    layer = KANLinear(64, 64, kf.BSpline(5, 3)).to(dev)
    with torch.no_grad():
        layer.coef.copy_(_randn(layer.coef.shape, 1, 1 / math.sqrt(64 * 8)))
    x = (torch.rand(65536, 64, generator=torch.Generator().manual_seed(0)) * 2 - 1).to(dev)
    lut = to_lut(layer, x, 256)
    q = quantize(lut)

    def step():
        return lut(x), q(x)

    def cpu():
        from oracle import kan64 as o

        rows = _cpu_rows(8192)
        xs = x[:rows].double().cpu().numpy()
        fl, ql = lut.layers[0], q.layers[0]

        def run():
            o.lut_layer(xs, fl.tables, fl.lo, fl.hi, fl.bias, None, fl.slope_lo, fl.slope_hi)
            o.lut_layer(xs, ql.tables, ql.lo, ql.hi, ql.bias, ql.scale, ql.slope_lo, ql.slope_hi)

        run()
        t0 = time.perf_counter()
        run()
        t = time.perf_counter() - t0
        return _cpu_line(rows / t, "rows/s", 1, f"{rows} of the rows, float32 and int8 tables: the NumPy float64 LUT evaluation, one run after 1 warm-up")

    return step, x.shape[0], "rows/s", "f32", cpu


WORKLOADS = {
    "kan64": wl_kan64,
    "grkan_ffn": wl_grkan_ffn,
    "pinn_edge": wl_pinn_edge,
    "pinn_laplacian": wl_pinn_laplacian,
    "bspline_ffn": wl_bspline_ffn,
    "lut_kan64": wl_lut_kan64,
}


def traffic_file(name):
    return os.path.join("profiles", f"{name}_hbm_traffic.md")


def _hook_entries(timer):
    from kanforge_amd.torch import kernels as kmod

    from kanforge_amd.export.lut import LUTLayer

    names = (("_raw", None), ("_edge_raw", "edge"), ("_features_raw", "features"),
             ("_rational_param_grad", "rational_param_grad"), ("_rational_bwd_raw", "rational_bwd"),
             ("_f_base_raw", "F_base"), ("_p_base_raw", "P_base"), ("_g_base_raw", "G_base"))
    orig = {n: getattr(kmod, n) for n, _ in names}
    for n, lab in names:
        setattr(kmod, n, timer.wrap(orig[n], lab))
    lut_call = LUTLayer.__call__
    LUTLayer.__call__ = timer.wrap(lut_call, "lut")

    def unhook():
        for n, f in orig.items():
            setattr(kmod, n, f)
        LUTLayer.__call__ = lut_call

    return unhook


GRAPH_WORKLOADS = ("kan64",)  # launch-bound steps: also timed as one captured HIP graph
# B-spline layers: k + 1 of the K basis values are non-zero at any x (degree 3: 4 of K)
SPARSE_MACS = {"kan64": (4, 8), "bspline_ffn": (4, 11), "lut_kan64": None}


def graph_timing(step, steps, warmup):
    """(ms per replay, check) of the step captured as one HIP graph. Before timing, the graph is
    replayed three times with eager steps in between and every replay's outputs are compared
    with the eager outputs (bitwise: the same kernels run); on a mismatch the graph is not used."""
    torch.cuda.synchronize()
    ref = [t.detach().clone() for t in step()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        if not all(torch.equal(a, b) for a, b in zip(outs, ref)):
            return None, "replay differs from the eager step"
        step()
        torch.cuda.synchronize()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        graph.replay()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps * 1e3, "replays equal the eager step"


def run_workload(name, args, dev, cpu=True):
    """One layer shape: whole-step throughput, HIP-event means of every entry point it calls,
    the roofline of the entry with the most GPU time and the CPU leg."""
    timer = EntryTimer()
    unhook = _hook_entries(timer)
    try:
        step, units, unit, dtype, cpu_leg = WORKLOADS[name](dev)
        _timed(step, args.steps, args.warmup, timer)  # per-entry HIP-event statistics
    finally:
        unhook()
    ms = _timed(step, args.steps, args.warmup)  # the whole step, no event hooks
    per_op, calls, totals = timer.mean_ms(), timer.count(), timer.totals()
    roof = roofline_of(totals, dtype, traffic_file(name))
    roof["launches_per_step"] = calls[roof["kernel"][3:]] / args.steps
    flops = sum(v[1] for v in totals.values()) / args.steps
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
        "contraction_tflops": flops / (ms * 1e-3) / 1e12,
        "roofline": roof,
    }
    if SPARSE_MACS.get(name):
        nz, K = SPARSE_MACS[name]
        line["sparse_mac_fraction"] = nz / K
        line["sparse_note"] = (f"{nz} of K = {K} B-spline values are non-zero per (row, input); the roofline counts "
                               "the dense 2 B in K out FLOP, the reference's convention")
    if name in GRAPH_WORKLOADS:
        gms, check = graph_timing(step, args.steps, args.warmup)
        line["graph"] = {"ms_per_step": gms, "value": None if gms is None else units / (gms * 1e-3), "check": check,
                         "note": "the same step captured once as a HIP graph and replayed (launch-bound layer)"}
    if cpu:
        line["cpu_baseline"] = cpu_leg()
    return line


def run_only(name, entry, args, dev):
    """Counter-run mode: one full step records the calls of ``entry``, a one-block probe kernel
    marks the end of it in the dispatch trace, then only those calls run ``args.steps`` times."""
    import ctypes

    from kanforge_amd.torch import _lib

    timer = EntryTimer()
    rec = []
    timer.record = (entry, rec)
    unhook = _hook_entries(timer)
    try:
        step, *_ = WORKLOADS[name](dev) if name != "cheb768" else (headline_step(dev),)
        step()
    finally:
        unhook()
    torch.cuda.synchronize()
    lib = _lib.load()
    mark = torch.empty(256 * 3, dtype=torch.float32, device=dev)
    _lib.check(lib.kf_probe_mfma(1, 1, 0, ctypes.c_void_p(mark.data_ptr()), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "marker")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        for fn, a, kw in rec:
            fn(*a, **kw)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    return {"workload": name, "entry": entry, "calls_per_replay": len(rec), "replays": args.steps, "ms_per_replay": ms}


def headline_layer(dev):
    import kanforge_amd as kf
    from kanforge_amd.torch import KANLinear

    layer = KANLinear(IN, OUT, kf.Chebyshev(DEGREE), base_activation=None, bias=False, device=dev, dtype=torch.bfloat16)
    gen = torch.Generator().manual_seed(1)
    with torch.no_grad():
        layer.coef.copy_((torch.randn(OUT, IN, K, generator=gen) / math.sqrt(IN * K)).to(torch.bfloat16))
    x = torch.randn(B, IN, generator=torch.Generator().manual_seed(0)).to(dev, torch.bfloat16).requires_grad_()
    gy = torch.randn(B, OUT, generator=torch.Generator().manual_seed(3)).to(dev, torch.bfloat16)
    return layer, x, gy


def headline_step(dev):
    layer, x, gy = headline_layer(dev)

    def step():
        y = layer(x)
        return torch.autograd.grad(y, [x, layer.coef], gy)

    return step


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
    if args.only:
        print(json.dumps(run_only(args.workload, args.only, args, dev)), flush=True)
        return
    if args.workload not in ("cheb768", "cheb768_base"):
        for name in WORKLOADS if args.workload == "all" else [args.workload]:
            print(json.dumps(run_workload(name, args, dev, cpu=not args.no_cpu)), flush=True)
        return

    timer = EntryTimer()
    layer, x, gy = headline_layer(dev)
    if args.workload == "cheb768_base":
        print(json.dumps(with_base_leg(layer, x, gy, args, dev)), flush=True)
        return
    unhook = _hook_entries(timer)

    def step():
        y = layer(x)
        return torch.autograd.grad(y, [x, layer.coef], gy)

    _timed(step, args.steps, args.warmup, timer)  # per-entry HIP-event statistics
    unhook()
    ms = _timed(step, args.steps, args.warmup)  # the whole step, no event hooks
    per_op = timer.mean_ms()

    with_base = None
    if not args.no_base:
        with_base = with_base_leg(layer, x, gy, args, dev)
        with_base["ratio_to_pure_step"] = with_base["ms_per_step"] / ms
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
    if not args.no_workloads:
        sub = argparse.Namespace(steps=args.workload_steps, warmup=3)
        out["workloads"] = {}
        for name in WORKLOADS:
            line = run_workload(name, sub, dev, cpu=not args.no_cpu)
            keep = ("value", "unit", "dtype", "ms_per_step", "steps", "config", "per_entry_ms", "calls_per_step",
                    "contraction_tflops", "roofline", "graph", "sparse_mac_fraction", "cpu_baseline")
            out["workloads"][name] = {k: line[k] for k in keep if k in line}
            torch.cuda.empty_cache()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
