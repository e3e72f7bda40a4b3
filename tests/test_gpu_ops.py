"""The torch custom-op boundary on the GPU: torch.library.opcheck of every kf:: op (schema,
autograd registration, fake kernels, AOT dispatch), and torch.compile(fullgraph=True) of
KANLinear forward + backward giving the eager results."""

import math

import numpy as np
import pytest
import torch

import kanforge_amd as kf
from kanforge_amd.kernels import plan_for
from kanforge_amd.torch import GRKAN, KANLinear
from kanforge_amd.torch import kernels as K

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _operands(basis, B=37, IN=12, OUT=9, seed=0, grad=True):
    g = torch.Generator().manual_seed(seed)
    plan = plan_for(basis)
    x = (torch.rand(B, IN, generator=g) * 1.6 - 0.8).to(DEV).requires_grad_(grad)
    c = (torch.randn(OUT, IN, basis.size, generator=g) / math.sqrt(IN * basis.size)).to(DEV).requires_grad_(grad)
    gy = torch.randn(B, OUT, generator=g).to(DEV).requires_grad_(grad)
    w = (torch.rand(B, IN, generator=g) + 0.5).to(DEV).requires_grad_(grad)
    kn = kc = ku = num = den = None
    if plan.kind == "bspline":
        grid = torch.linspace(-1, 1, basis.grid_size + 1, dtype=torch.float64).expand(IN, -1).contiguous().to(DEV)
        st = K.bspline_state(grid, basis.order)
        kn, kc, ku = st.knots, st.knots_cmp, st.knots_u
    if plan.kind == "rational":
        groups = 4
        num = (torch.tensor(basis.param_specs()["numerator"].value, dtype=torch.float32)[None].repeat(groups, 1)
               + 0.05 * torch.randn(groups, basis.num_degree + 1, generator=g)).to(DEV).requires_grad_(grad)
        den = (torch.tensor(basis.param_specs()["denominator"].value, dtype=torch.float32)[None].repeat(groups, 1)
               + 0.05 * torch.randn(groups, basis.den_degree, generator=g)).to(DEV).requires_grad_(grad)
    return K.plan_key(plan), x, c, gy, w, (kn, kc, ku, num, den)


BASES = {"cheb8": kf.Chebyshev(8), "jacobi6": kf.Jacobi(6, 0.5, 0.5), "bspline53": kf.BSpline(5, 3), "rational": kf.Rational(5, 4)}


@pytest.mark.parametrize("name", list(BASES))
def test_opcheck_F_G_P(name):
    key, x, c, gy, w, tabs = _operands(BASES[name])
    rational = tabs[3] is not None
    # rational parameters receive gradients through F at order 0; P and G take them as constants
    fixed = tabs if not rational else (tabs[0], tabs[1], tabs[2], tabs[3].detach(), tabs[4].detach())
    for m in (0, 1):
        torch.library.opcheck(torch.ops.kf.F.default, (x, w, c, *(fixed if m else tabs), key, m))
        torch.library.opcheck(torch.ops.kf.P.default, (x, gy, c, *fixed, key, m))
        torch.library.opcheck(torch.ops.kf.G.default, (x, gy, w, *fixed, key, m))


@pytest.mark.parametrize("name", list(BASES))
def test_opcheck_edge_and_features(name):
    key, x, c, gy, w, tabs = _operands(BASES[name])
    bw = (0.1 * torch.randn(c.shape[:2], generator=torch.Generator().manual_seed(5))).to(DEV).requires_grad_()
    torch.library.opcheck(torch.ops.kf.edge_derivative.default, (x, c, bw, *tabs, key, 0))
    torch.library.opcheck(torch.ops.kf.features.default, (x, *tabs, key, 0))
    if tabs[3] is None:
        torch.library.opcheck(torch.ops.kf.edge_derivative.default, (x, c, bw, *tabs, key, 2))


def test_opcheck_rational_ops_and_interval():
    key, x, c, gy, w, tabs = _operands(BASES["rational"], grad=False)
    h = torch.randn(x.shape, device=DEV)
    for m in (0, 1):
        torch.library.opcheck(torch.ops.kf.rational_bwd.default, (x, gy, c, None, tabs[3], tabs[4], key, m))
        torch.library.opcheck(torch.ops.kf.rational_param_grad.default, (x, h, w, tabs[3], tabs[4], key, m))
    bkey, bx, _, _, _, btabs = _operands(BASES["bspline53"], grad=False)
    torch.library.opcheck(torch.ops.kf.bspline_interval.default, (bx, btabs[1]))


@pytest.mark.parametrize("kind", ["cheb8", "bspline83"])
def test_opcheck_fused_base_ops(kind):
    """kf::F_base (with its autograd formula), kf::P_base and kf::G_base on shapes every fused
    entry takes: Chebyshev(8) with 128 G tiles, cubic B-splines on 8 intervals."""
    basis = kf.Chebyshev(8) if kind == "cheb8" else kf.BSpline(8, 3)
    B, IN, OUT = 64, (3072 if kind == "cheb8" else 96), (384 if kind == "cheb8" else 64)
    key, x, c, gy, _w, tabs = _operands(basis, B=B, IN=IN, OUT=OUT, grad=False)
    st = None if kind == "cheb8" else K.BasisState(knots=tabs[0], knots_cmp=tabs[1], knots_u=tabs[2])
    assert K.base_fused(key, st, torch.bfloat16, B, IN, OUT) == (True, True, True)
    bf = torch.bfloat16
    g = torch.Generator().manual_seed(5)
    x, c, gy = x.to(bf), c.to(bf), gy.to(bf)
    bw = (torch.randn(OUT, IN, generator=g) / math.sqrt(IN)).to(DEV, bf)
    bias = torch.randn(OUT, generator=g).to(DEV, bf)
    t3 = tabs[:3]
    # bf16 with static shapes (the traced backward takes the same fused kernels as eager); with
    # symbolic shapes the traced backward composes kf::P, kf::G and torch ops, whose bf16 rounding
    # differs from the fused epilogue's, so the dynamic-shape gradient check runs in float32
    # (composed on both sides)
    static = ("test_schema", "test_autograd_registration", "test_faketensor", "test_aot_dispatch_static")
    req = [t.detach().requires_grad_() for t in (x, c, bw, bias)]
    torch.library.opcheck(torch.ops.kf.F_base.default, (*req, *t3, key), test_utils=static)
    torch.library.opcheck(torch.ops.kf.F_base.default, (req[0], req[1], req[2], None, *t3, key), test_utils=static)
    r32 = [t.detach().float().requires_grad_() for t in (x, c, bw, bias)]
    torch.library.opcheck(torch.ops.kf.F_base.default, (*r32, *t3, key))
    torch.library.opcheck(torch.ops.kf.P_base.default, (x, gy, c, bw, *t3, key))
    torch.library.opcheck(torch.ops.kf.G_base.default, (x, gy, *t3, key, True, True, True))
    torch.library.opcheck(torch.ops.kf.G_base.default, (x, gy, *t3, key, False, True, False))


@pytest.mark.parametrize("name", ["cheb8", "bspline53", "rational"])
def test_opcheck_F_bias_and_G_bias(name):
    key, x, c, gy, w, tabs = _operands(BASES[name])
    bias = torch.randn(c.shape[0], device=DEV).requires_grad_()
    torch.library.opcheck(torch.ops.kf.F_bias.default, (x, None, c, bias, *tabs, key, 0))
    torch.library.opcheck(torch.ops.kf.G_bias.default, (x, gy, None, *tabs, key, 0))


def _grads(layer, x, gy):
    params = [p for p in layer.parameters()]
    y = layer(x)
    return [y] + list(torch.autograd.grad(y, [x] + params, gy))


@pytest.mark.parametrize(
    "make,dtype",
    [
        (lambda: KANLinear(96, 80, kf.Chebyshev(8), base_activation=None, bias=False), torch.bfloat16),
        (lambda: KANLinear(96, 80, kf.Chebyshev(8)), torch.bfloat16),
        (lambda: KANLinear(64, 48, kf.BSpline(5, 3)), torch.float32),
        (lambda: GRKAN(64, 48, groups=8), torch.float32),
    ],
    ids=["cheb8-bf16", "cheb8-bf16-base", "bspline53-f32-base", "grkan-f32"],
)
def test_compiled_layer_forward_backward_matches_eager(make, dtype):
    torch.manual_seed(0)
    layer = make().to(DEV, dtype)
    x = (torch.rand(256, layer.in_features, device=DEV) * 1.6 - 0.8).to(dtype).requires_grad_()
    gy = torch.randn(256, layer.out_features, device=DEV).to(dtype)
    want = _grads(layer, x, gy)
    torch._dynamo.reset()
    compiled = torch.compile(layer, fullgraph=True)
    y = compiled(x)
    got = [y] + list(torch.autograd.grad(y, [x] + list(layer.parameters()), gy))
    assert len(got) == len(want)
    for a, b in zip(got, want):
        if getattr(layer, "base_weight", None) is not None:
            # compiled graphs take the composed base branch (kf::F, hipBLASLt, torch ops), eager
            # the fused entries: the same sums in another order (and, in bf16, rounded twice)
            err = ((a.float() - b.float()).abs().max() / b.float().abs().max()).item()
            assert err <= (2e-2 if dtype == torch.bfloat16 else 1e-5), err
        else:
            torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("shape", [(16384, 768), (1000, 77), (3, 4096), (0, 5), (37, 8)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_column_sums_and_bias_add(shape, dtype):
    """kf_column_sums against a float64 sum (bias gradients), including ragged and empty shapes
    and a misaligned view; the bias-add op's gradients and opcheck."""
    g = torch.randn(shape, generator=torch.Generator().manual_seed(1)).to(DEV, dtype)
    got = torch.ops.kf.column_sums(g).double().cpu()
    want = g.double().cpu().sum(0)
    scale = max(1.0, float(want.abs().max())) if want.numel() else 1.0
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-5
    assert float((got - want).abs().max() if want.numel() else 0.0) <= tol * scale
    if shape[0] > 1 and shape[1] > 1:
        view = g[:, 1:]  # rows not 16-byte aligned
        np.testing.assert_allclose(torch.ops.kf.column_sums(view.contiguous()).double().cpu(), view.double().cpu().sum(0),
                                   atol=tol * scale)
        y = torch.randn(shape, device=DEV, dtype=dtype, requires_grad=True)
        b = torch.randn(shape[1], device=DEV, dtype=dtype, requires_grad=True)
        out = torch.ops.kf.bias_add(y, b)
        out.backward(g)
        assert torch.equal(y.grad, g)
        np.testing.assert_allclose(b.grad.double().cpu(), want, atol=tol * scale)
        torch.library.opcheck(torch.ops.kf.column_sums.default, (g,))
        torch.library.opcheck(torch.ops.kf.bias_add.default, (y.detach().requires_grad_(), b.detach().requires_grad_()))


@pytest.mark.parametrize("with_S", [False, True])
def test_silu_taylor_values_and_gradients(with_S):
    """kf::silu_taylor against the oracle's SiLU derivatives, and its closed-form backward against
    autograd through the same terms written with torch ops (float32)."""
    from oracle import kan64 as o

    D, B, n = 2, 300, 17
    gen = torch.Generator().manual_seed(4)
    h = (torch.randn(B, n, generator=gen) * 2).to(DEV).requires_grad_()
    hp = torch.randn(D, B, n, generator=gen).to(DEV).requires_grad_()
    S = torch.randn(B, n, generator=gen).to(DEV).requires_grad_() if with_S else None
    A, sq = torch.ops.kf.silu_taylor(h, hp, S)
    hn, hpn = h.detach().double().cpu().numpy(), hp.detach().double().cpu().numpy()
    d0, d1, d2 = (o.silu_derivative(hn, m) for m in (0, 1, 2))
    sqn = (hpn ** 2).sum(0)
    Sn = S.detach().double().cpu().numpy() if with_S else 0.0
    want = np.concatenate([d0, (d1 * hpn).reshape(D * B, n), d2 * sqn + d1 * Sn], 0)
    assert o.normwise_err(A.detach().double().cpu().numpy(), want) <= 1e-5
    assert o.normwise_err(sq.detach().double().cpu().numpy(), sqn) <= 1e-6
    gA = torch.randn(A.shape, generator=gen).to(DEV)
    gq = torch.randn(sq.shape, generator=gen).to(DEV)
    inputs = [h, hp] + ([S] if with_S else [])
    got = torch.autograd.grad((A * gA).sum() + (sq * gq).sum(), inputs)

    def ref(h, hp, S):
        s = torch.sigmoid(h)
        r1 = s * (1 + h * (1 - s))
        r2 = s * (1 - s) * (2 + h * (1 - 2 * s))
        q = (hp * hp).sum(0)
        last = r2 * q + (0 if S is None else r1 * S)
        return torch.cat([h * s, (r1 * hp).reshape(D * B, n), last], 0), q

    Ar, qr = ref(h, hp, S)
    want_g = torch.autograd.grad((Ar * gA).sum() + (qr * gq).sum(), inputs)
    for a, b in zip(got, want_g):
        assert o.normwise_err(a.double().cpu().numpy(), b.double().cpu().numpy()) <= 1e-5
    torch.library.opcheck(torch.ops.kf.silu_taylor.default, (h, hp, S))
