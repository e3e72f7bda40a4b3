"""Kernel plans of the HIP path (see ``plan``).

The spline part of a layer, y[b,o] = sum_{i,k} c[o,i,k] phi_k(x[b,i]), is
computed by three primitives closed under differentiation
(kanforge/kernels/__init__.py:1-13):

  F_m(x, c, w)[b,o]   = sum_{i,k} w[b,i] c[o,i,k] phi_k^(m)(x[b,i])
  G_m(x, g, w)[o,i,k] = sum_b     w[b,i] g[b,o]   phi_k^(m)(x[b,i])
  P_m(x, g, c)[b,i]   = sum_{o,k} g[b,o] c[o,i,k] phi_k^(m)(x[b,i])

  dF/dc = G_m, dF/dw = P_m, dF/dx = w * P_{m+1}   (and alike for G and P)
"""

from .plan import AUTO_KINDS, KernelPlan, plan_for

__all__ = ["AUTO_KINDS", "KernelPlan", "plan_for"]
