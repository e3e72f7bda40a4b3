"""kf_F_noalloc: the F entry point without a workspace argument, its scratch in the library's
static device array. Called through the C ABI, it must give exactly kf_F's result (same kernels,
same inputs), on two calls in a row with the second on smaller shapes (the scratch keeps the first
call's contents), and reject shapes whose scratch exceeds the array."""

import ctypes
import math

import numpy as np
import pytest
import torch

import kanforge_amd as kf
from kanforge_amd.kernels import plan_for
from kanforge_amd.torch import _lib
from kanforge_amd.torch import kernels as K

pytestmark = pytest.mark.gpu
DEV = "cuda"


def f_noalloc(plan, st, x, w, c, n_out):
    lib = _lib.load()
    desc, keep = K._desc(plan, 0, st)
    y = torch.empty(x.shape[0], n_out, dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        rc = lib.kf_F_noalloc(
            ctypes.byref(desc), K._dtype_code(x.dtype), x.shape[0], x.shape[1], n_out,
            K._ptr(x), K._ptr(w), K._ptr(c), K._ptr(y), K._stream(x.device),
        )
    _lib.check(rc, "kf_F_noalloc")
    return y


def operands(basis, dtype, B, IN, OUT, weighted, seed):
    g = torch.Generator().manual_seed(seed)
    plan = plan_for(basis)
    x = (torch.rand(B, IN, generator=g) * 2 - 1).to(DEV, dtype)
    c = (torch.randn(OUT, IN, basis.size, generator=g) / math.sqrt(IN * basis.size)).to(DEV, dtype)
    w = (torch.rand(B, IN, generator=g) + 0.5).to(DEV, dtype) if weighted else None
    st = None
    if plan.kind == "bspline":
        grid = torch.as_tensor(np.broadcast_to(np.linspace(-1, 1, basis.grid_size + 1), (IN, basis.grid_size + 1)).copy(), device=DEV)
        st = K.bspline_state(grid, basis.order)
    return plan, st, x, w, c


@pytest.mark.parametrize(
    "basis,dtype,weighted,big,small",
    [
        (kf.Chebyshev(8), torch.bfloat16, False, (2048, 768, 3072), (300, 96, 200)),
        (kf.Chebyshev(8), torch.bfloat16, True, (1024, 768, 1024), (77, 40, 33)),
        (kf.BSpline(5, 3), torch.float32, False, (4096, 64, 64), (500, 24, 19)),
        (kf.Jacobi(6, 0.5, 0.5), torch.float32, True, (8192, 64, 64), (128, 2, 64)),
    ],
    ids=["cheb8-bf16", "cheb8-bf16-weighted", "bspline53-f32", "jacobi6-f32-weighted"],
)
def test_noalloc_F_equals_F_on_two_calls(basis, dtype, weighted, big, small):
    for seed, (B, IN, OUT) in enumerate((big, small)):
        plan, st, x, w, c = operands(basis, dtype, B, IN, OUT, weighted, seed)
        print(f"kf_F_noalloc {basis!r} {dtype} w={weighted} shape {(B, IN, OUT)}", flush=True)
        got = f_noalloc(plan, st, x, w, c, OUT)
        want = K._raw("F", plan, 0, x, w, c, st, OUT)
        torch.cuda.synchronize()
        assert torch.isfinite(want).all()
        assert torch.equal(got, want)


def test_noalloc_F_rejects_shapes_beyond_the_scratch():
    plan, st, x, w, c = operands(kf.Chebyshev(8), torch.bfloat16, 8192, 768, 4096, True, 0)
    lib = _lib.load()
    desc, keep = K._desc(plan, 0, st)
    y = torch.empty(8192, 4096, dtype=torch.bfloat16, device=DEV)
    rc = lib.kf_F_noalloc(ctypes.byref(desc), _lib.KF_BF16, 8192, 768, 4096, K._ptr(x), K._ptr(w), K._ptr(c), K._ptr(y), K._stream(x.device))
    assert rc == _lib.KF_EWORKSPACE
    assert b"static scratch" in lib.kf_last_error()
