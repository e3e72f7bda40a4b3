"""The headline shape, KANLinear 768 -> 3072 Chebyshev(8) tanh, bf16, batch 8192,
on the HIP path: forward y, dX and dCoef through the layer and autograd (the
F_0, P_1 and G_0 launches the benchmark times) against a plain PyTorch float32
reference of the same op on the GPU (features by the Chebyshev recurrence,
contractions by torch.matmul), plus size-independent identities that tie the
three primitives together:
  adjoint   <F_0(x, c), g> = <c, G_0(x, g)>
  checksum  sum_b P_1(x, g, c)[b, i] = sum_{o,k} c[o, i, k] G_1(x, g)[o, i, k]
Tolerance: bfloat16 normwise 2e-2 (max|d| / max|ref|), as for the small cases.
"""

import math

import numpy as np
import pytest
import torch

import kanforge_amd as kf
from kanforge_amd.torch import KANLinear
from kanforge_amd.torch import kernels as K

pytestmark = pytest.mark.gpu
B, IN, OUT, DEG = 8192, 768, 3072, 8
KB = DEG + 1
TOL = 2e-2


@pytest.fixture(scope="module")
def headline():
    dev = torch.device("cuda")
    layer = KANLinear(IN, OUT, kf.Chebyshev(DEG), base_activation=None, bias=False, device=dev, dtype=torch.bfloat16)
    gen = torch.Generator().manual_seed(1)
    with torch.no_grad():
        layer.coef.copy_((torch.randn(OUT, IN, KB, generator=gen) / math.sqrt(IN * KB)).to(torch.bfloat16))
    x = torch.randn(B, IN, generator=torch.Generator().manual_seed(0)).to(dev, torch.bfloat16).requires_grad_()
    gy = torch.randn(B, OUT, generator=torch.Generator().manual_seed(3)).to(dev, torch.bfloat16)
    y = layer(x)
    dx, dc = torch.autograd.grad(y, [x, layer.coef], gy)
    torch.cuda.synchronize()
    return layer, x.detach(), gy, y.detach(), dx, dc


def features_f32(x, a):
    """Chebyshev features of tanh(x) and their x-derivatives, float32: (B, IN, K) each."""
    z = torch.tanh(x.float())
    t = [torch.ones_like(z), z]
    dt = [torch.zeros_like(z), torch.ones_like(z)]
    for j in range(2, KB):
        t.append(2 * z * t[j - 1] - t[j - 2])
        dt.append(2 * t[j - 1] + 2 * z * dt[j - 1] - dt[j - 2])
    T = torch.stack(t, -1)
    dT = torch.stack(dt, -1) * (1 - z * z).unsqueeze(-1)  # d/dx = (1 - z^2) d/dz
    return T @ a, dT @ a


def normwise(got, want):
    return ((got.float() - want).abs().max() / want.abs().max()).item()


def test_headline_step_matches_float32_reference(headline):
    layer, x, gy, y, dx, dc = headline
    a = torch.as_tensor(np.asarray(layer.basis._cheb), dtype=torch.float32, device=x.device)
    phi, dphi = features_f32(x, a)
    c2 = layer.coef.detach().float().reshape(OUT, IN * KB)
    g32 = gy.float()
    y_ref = torch.matmul(phi.reshape(B, IN * KB), c2.t().contiguous())
    dc_ref = torch.matmul(g32.t().contiguous(), phi.reshape(B, IN * KB)).reshape(OUT, IN, KB)
    dx_ref = (torch.matmul(g32, c2).reshape(B, IN, KB) * dphi).sum(-1)
    assert y.shape == (B, OUT) and dx.shape == (B, IN) and dc.shape == (OUT, IN, KB)
    assert normwise(y, y_ref) < TOL
    assert normwise(dx, dx_ref) < TOL
    assert normwise(dc, dc_ref) < TOL
    assert torch.isfinite(y).all() and torch.isfinite(dx).all() and torch.isfinite(dc).all()


def test_headline_adjoint_identity(headline):
    layer, x, gy, y, dx, dc = headline
    lhs = (y.double() * gy.double()).sum().item()
    rhs = (layer.coef.detach().double() * dc.double()).sum().item()
    scale = (y.double() * gy.double()).abs().sum().item()
    assert abs(lhs - rhs) < 1e-3 * scale


def test_headline_dx_checksum_against_first_order_G(headline):
    layer, x, gy, y, dx, dc = headline
    plan = layer._plan
    c = layer.coef.detach()
    p1 = K.prim_P(x, gy, c, None, plan, 1)
    g1 = K.prim_G(x, gy, None, None, plan, 1)
    torch.cuda.synchronize()
    lhs = p1.double().sum(0)
    rhs = (c.double() * g1.double()).sum((0, 2))
    assert ((lhs - rhs).abs().max() / rhs.abs().max()).item() < TOL
    assert normwise(dx, p1.float()) < 1e-6  # the layer's dX is the P_1 launch itself
