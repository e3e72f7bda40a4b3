// Device-side building blocks of the fused KAN kernels for gfx950 (CDNA4):
// element types, MFMA wrappers, and the per-input basis feature generators.
//
// Feature generators evaluate, in float32 registers, what the reference's
// bases compute in float64:
//   Chebyshev features T_j(g(x)), g = tanh | identity   kanforge/bases/polynomial.py:87-106
//   B-splines and their derivatives                     kanforge/bases/spline.py:74-92
//   rational P/(1+|Q|) and its derivatives              kanforge/bases/rational.py:84-101
//   d^m silu                                            kanforge/_calculus.py:90-96
#pragma once

#include <type_traits>

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kfhip.h"

namespace kf {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Launch-time copy of kf_basis; passed by value as a kernel argument.
struct KBasis {
  int kind, K, n_t, order, input_map;
  int spline_k, n_knots;
  int num_deg, den_deg, group_size;
  const float* knots;
  const float* knots_cmp;
  const float* num;
  const float* den;
  const float* knots_uniform;        // (t_0, 1 / h) per input when every input's knots are even
  float fold[KF_MAX_K * KF_MAX_NT];  // R_m, K x n_t row-major (cheb)
};

// ---------------------------------------------------------------------------
// element conversion

template <typename T>
__device__ __forceinline__ float to_f32(T v);
template <>
__device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f32<bf16>(bf16 v) { return (float)v; }

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float v) { return (bf16)v; }  // round to nearest even

// ---------------------------------------------------------------------------
// scalar math

// tanh(x) = sign(x) (1 - e^{-2|x|}) / (1 + e^{-2|x|}); absolute error a few
// float32 ulps of 1, the quantity the features need (T_j(z) is bounded by 1).
__device__ __forceinline__ float fast_tanh(float x) {
  float t = __expf(-2.0f * fabsf(x));
  float r = (1.0f - t) * __frcp_rn(1.0f + t);
  return copysignf(r, x);
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }
// silu(x) = x s and silu'(x) = s (1 + x (1 - s)), s = sigmoid(x)
__device__ __forceinline__ float silu_f(float x) { return x * sigmoidf_(x); }
__device__ __forceinline__ float dsilu_f(float x) {
  const float s = sigmoidf_(x);
  return s * fmaf(x, 1.f - s, 1.f);
}

// d^m/dx^m silu(x) = x p_m(s) + m p_{m-1}(s), s = sigmoid(x), where
// p_0 = s and p_{j+1} = p_j'(s) (s - s^2). The polynomial coefficients are
// generated on the fly (m <= 8).
__device__ inline float silu_derivative(float x, int m) {
  float s = sigmoidf_(x);
  if (m == 0) return x * s;
  // coefficients of p_j in powers of s, degree j+1
  float p[11], q[11];
  for (int a = 0; a < 11; ++a) p[a] = 0.f;
  p[1] = 1.f;  // p_0 = s
  float prev_val = 0.f, cur_val = s;
  for (int j = 1; j <= m; ++j) {
    // q = p' * (s - s^2): p' has coefficients (a+1) p[a+1]
    for (int a = 0; a < 11; ++a) q[a] = 0.f;
    for (int a = 0; a + 1 < 11; ++a) {
      float d = (a + 1) * p[a + 1];  // coefficient of s^a in p'
      if (a + 1 < 11) q[a + 1] += d;
      if (a + 2 < 11) q[a + 2] -= d;
    }
    for (int a = 0; a < 11; ++a) p[a] = q[a];
    prev_val = cur_val;
    float v = 0.f;
    for (int a = 10; a >= 0; --a) v = v * s + p[a];
    cur_val = v;
  }
  return x * cur_val + (float)m * prev_val;
}

// ---------------------------------------------------------------------------
// Chebyshev features: T[j] = w * T_j(g(x)), j < n_t (n_t <= NT).
// The three-term recurrence is linear, so scaling T_0 and T_1 by w scales
// every feature by w.

__device__ __forceinline__ float cheb_map(float x, int input_map) {
  return input_map != KF_MAP_IDENTITY ? fast_tanh(x) : x;
}
// Weight of the kernel features of one element: w, times (1 - z^2) for KF_MAP_TANH_SQ.
__device__ __forceinline__ float cheb_weight(float z, float w, int input_map) {
  return input_map == KF_MAP_TANH_SQ ? w * fmaf(-z, z, 1.f) : w;
}

template <int NT>
__device__ __forceinline__ void cheb_features(float z, float w, int n_t, float* T) {
  float z2 = 2.0f * z;
  T[0] = w;
  if (NT > 1) T[1] = w * z;
#pragma unroll
  for (int j = 2; j < NT; ++j) T[j] = j < n_t ? fmaf(z2, T[j - 1], -T[j - 2]) : 0.f;
}

// phi_k^(m) = sum_j fold[k][j] T_j  (fold = R_m of the plan)
template <int KM, int NT>
__device__ __forceinline__ void cheb_folded(const KBasis& b, const float* T, float* phi) {
#pragma unroll
  for (int k = 0; k < KM; ++k) {
    float acc = 0.f;
    if (k < b.K) {
#pragma unroll
      for (int j = 0; j < NT; ++j)
        if (j < b.n_t) acc = fmaf(b.fold[k * KF_MAX_NT + j], T[j], acc);
    }
    phi[k] = acc;
  }
}

// sum_q p[q * stride] for q < nz, added in q order; the loads eight at a time in flight
__device__ __forceinline__ float slice_sum(const float* __restrict__ p, size_t stride, int nz) {
  float s = 0.f;
  int q = 0;
  for (; q + 8 <= nz; q += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = p[(size_t)(q + u) * stride];
#pragma unroll
    for (int u = 0; u < 8; ++u) s += v[u];
  }
  for (; q < nz; ++q) s += p[(size_t)q * stride];
  return s;
}

// ---------------------------------------------------------------------------
// B-splines. Knot vector of input i: t_0 .. t_{n_knots-1} (real), stored with
// spline_k padding knots per side: kp[r] = t_{r - spline_k}.

// Interval j with t_j <= x < t_{j+1}, or -1: count of comparison knots <= x, minus one.
// The knots are read eight at a time with independent loads (one round trip per
// eight knots instead of one per knot); knots past n_knots are not read.
__device__ __forceinline__ int bspline_interval(float x, const float* kc, int n_knots) {
  int cnt = 0;
  for (int r0 = 0; r0 < n_knots; r0 += 8) {
    float kv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) kv[u] = r0 + u < n_knots ? kc[r0 + u] : __builtin_inff();
#pragma unroll
    for (int u = 0; u < 8; ++u) cnt += (r0 + u < n_knots && x >= kv[u]) ? 1 : 0;
  }
  int j = cnt - 1;
  return (j >= 0 && j <= n_knots - 2) ? j : -1;
}

// Support of the B-spline features at x for degree KD: the interval j (t_j <= x < t_{j+1}) and
// the KD + 1 splines that can be non-zero there, N[r] = w d^m/dx^m B_{KD, j-KD+r}(x), first index
// base = j - KD (indices outside [0, K) belong to no basis function and are dropped by callers).
// Returns 1 for that case, 0 when every feature is zero (x outside [t_0, t_last), or m > KD),
// 2 when x is not finite: every feature is NaN, as the float64 recurrence's (x - t) * 0 gives.
// kc: the input's n_knots comparison knots (each float64 knot rounded up to float32, so x >= kc[r]
// is exactly x >= t_r); kp0: its n_knots + 2 KD padded knots (global memory, or a copy in LDS);
// t0, ih: (t_0, 1/h) when the input's knots are evenly spaced by h, ih == 0 otherwise.
// The derivative order M is a template argument here (bspline_support below dispatches on m), so
// the recurrence's Cox-de Boor / derivative choice is made at compile time.
// EVEN: the caller guarantees even knots (ih != 0) and nk >= 4, and only that path is compiled.
template <int KD, int M, bool EVEN = false>
__device__ inline int bspline_support_m(float x, float w, const float* kc, const float* kp0, float t0, float ih,
                                        int nk, int& base, float (&N)[KD + 1]) {
  constexpr int deg = KD - M;
  const bool fin = __builtin_isfinite(x);
  if constexpr (M > KD) {
    return fin ? 0 : 2;  // every derivative of order > KD is zero
  } else {
    if (EVEN || (ih != 0.f && nk >= 4)) {
      // even knots, without branches on x: the affine estimate e is off by at most one, so with e
      // clamped to [1, nk - 3] the four knots around it decide j in one round of independent
      // reads, j = e - 1 + [x >= kc[e]] + [x >= kc[e + 1]] whenever kc[e - 1] <= x < kc[e + 2]
      // (the search is the fallback that never runs for even knots). x outside the knots or not
      // finite runs the same instructions on clamped indices; the status discards the values.
      // (bitwise & and |: no short-circuit branches around the reads)
      const float kfirst = kc[0], klast = kc[nk - 1];
      const bool inr = fin & (x >= kfirst) & (x < klast);
      const float ef = fminf(fmaxf(floorf((x - t0) * ih), 1.f), (float)(nk - 3));
      const int e = (int)ef;
      const float k0 = kc[e - 1], k1 = kc[e], k2 = kc[e + 1], k3 = kc[e + 2];
      int j = e - 1 + (x >= k1 ? 1 : 0) + (x >= k2 ? 1 : 0);
      if (inr & ((x < k0) | (x >= k3))) j = bspline_interval(x, kc, nk);
      // every knot difference is a whole number of steps: with u = (x - t_j) / h and s = j-q+r,
      // (x - t_s) / (t_{s+q} - t_s) = (u + q - r) / q, (t_{s+q+1} - x) / (t_{s+q+1} - t_{s+1}) = (r + 1 - u) / q,
      // and a derivative step is (left - right) / h; Cox-de Boor to degree KD - M, then M
      // derivative steps, N[r] = B_{q, j-q+r} after step q. B_{q-1,j-q} and B_{q-1,j+1} are zero
      // (and the factors multiplying them finite), so the end terms r = 0 and r = q have one product.
      const float u = (x - kp0[j + KD]) * ih;
#pragma unroll
      for (int r = 0; r <= KD; ++r) N[r] = r == 0 ? 1.f : 0.f;
#pragma unroll
      for (int q = 1; q <= KD; ++q) {
        float nn[KD + 1];
        const float iq = 1.f / (float)q;
#pragma unroll
        for (int r = 0; r <= KD; ++r) {
          if (r > q) nn[r] = 0.f;
          else if (q <= deg) {
            if (r == 0) nn[r] = (1.f - u) * N[0] * iq;
            else if (r == q) nn[r] = u * N[r - 1] * iq;
            else nn[r] = ((u + (float)(q - r)) * N[r - 1] + ((float)(r + 1) - u) * N[r]) * iq;
          } else {
            if (r == 0) nn[r] = -N[0] * ih;
            else if (r == q) nn[r] = N[r - 1] * ih;
            else nn[r] = (N[r - 1] - N[r]) * ih;
          }
        }
#pragma unroll
        for (int r = 0; r <= KD; ++r) N[r] = nn[r];
      }
#pragma unroll
      for (int r = 0; r <= KD; ++r) N[r] *= w;
      base = j - KD;
      return inr ? 1 : (fin ? 0 : 2);
    }
    if constexpr (EVEN) return 0;  // not reached
    if (!fin) return 2;
    if (x < kc[0] || x >= kc[nk - 1]) return 0;
    const int j = bspline_interval(x, kc, nk);
    // general knots: L[r] = t_{j-KD+r}, r = 0..2KD+1 (kp[r'] = t_{r'-KD}, so t_{j-KD+r} = kp[j+r]);
    // the zero end terms are kept: with repeated knots their 0 / 0 gives NaN, as the dense
    // recurrence does
    const float* kp = kp0 + j;
    float L[2 * KD + 2];
#pragma unroll
    for (int r = 0; r < 2 * KD + 2; ++r) L[r] = kp[r];
#pragma unroll
    for (int r = 0; r <= KD; ++r) N[r] = r == 0 ? 1.f : 0.f;
#pragma unroll
    for (int q = 1; q <= KD; ++q) {
      float nn[KD + 1];
#pragma unroll
      for (int r = 0; r <= KD; ++r) {
        if (r > q) {
          nn[r] = 0.f;
          continue;
        }
        const float ts = L[KD - q + r], ts1 = L[KD - q + r + 1], tsq = L[KD + r], tsq1 = L[KD + r + 1];
        const float left = (r >= 1) ? N[r - 1] : 0.f;   // B_{q-1,s}
        const float right = (r <= q - 1) ? N[r] : 0.f;  // B_{q-1,s+1}
        // knot spans divide through the fast reciprocal (<= 2 ulp): an IEEE division costs a
        // dozen instructions and there are two per term
        if (q <= deg)  // Cox-de Boor
          nn[r] = __fdividef(x - ts, tsq - ts) * left + __fdividef(tsq1 - x, tsq1 - ts1) * right;
        else  // derivative step
          nn[r] = (float)q * (__fdividef(left, tsq - ts) - __fdividef(right, tsq1 - ts1));
      }
#pragma unroll
      for (int r = 0; r <= KD; ++r) N[r] = nn[r];
    }
#pragma unroll
    for (int r = 0; r <= KD; ++r) N[r] *= w;
    base = j - KD;
    return 1;
  }
}

// f(std::integral_constant<int, M>) for the derivative order m: M = m for m <= KD, KD + 1 above
// (every feature zero). Hot kernels take the order out of their element loops with it.
template <int KD, int M = 0, typename F>
__device__ __forceinline__ void with_spline_order(int m, F&& f) {
  if constexpr (M > KD) {
    f(std::integral_constant<int, KD + 1>{});
  } else {
    if (m == M) f(std::integral_constant<int, M>{});
    else with_spline_order<KD, M + 1>(m, static_cast<F&&>(f));
  }
}

template <int KD, int M = 0>
__device__ __forceinline__ int bspline_support_dispatch(int m, float x, float w, const float* kc, const float* kp0,
                                                        float t0, float ih, int nk, int& base, float (&N)[KD + 1]) {
  if constexpr (M > KD) {
    return __builtin_isfinite(x) ? 0 : 2;  // m > KD: every derivative is zero
  } else {
    if (m == M) return bspline_support_m<KD, M>(x, w, kc, kp0, t0, ih, nk, base, N);
    return bspline_support_dispatch<KD, M + 1>(m, x, w, kc, kp0, t0, ih, nk, base, N);
  }
}

// bspline_support_m for the basis' derivative order b.order (a launch-uniform branch)
template <int KD>
__device__ __forceinline__ int bspline_support(float x, float w, const float* kc, const float* kp0, float t0, float ih,
                                               const KBasis& b, int& base, float (&N)[KD + 1]) {
  return bspline_support_dispatch<KD>(b.order, x, w, kc, kp0, t0, ih, b.n_knots, base, N);
}

// (t_0, 1/h) of input i, or ih = 0 when the knots are not evenly spaced
__device__ __forceinline__ void bspline_affine(const KBasis& b, int i, float& t0, float& ih) {
  if (b.knots_uniform) {
    t0 = b.knots_uniform[2 * i];
    ih = b.knots_uniform[2 * i + 1];
  } else {
    t0 = 0.f;
    ih = 0.f;
  }
}

// phi[s] = w * d^m/dx^m B_{KD,s}(x) for s < KM (zeros past K = n_knots - 1 - KD) from the support.
template <int KM, int KD>
__device__ inline void bspline_features_rows(float x, float w, const float* kc, const float* kp0, float t0, float ih,
                                             const KBasis& b, float* phi) {
  int base = 0;
  float N[KD + 1];
  const int st = bspline_support<KD>(x, w, kc, kp0, t0, ih, b, base, N);
#pragma unroll
  for (int s = 0; s < KM; ++s) {
    const int r = s - base;
    float v = 0.f;
#pragma unroll
    for (int rr = 0; rr <= KD; ++rr) v = (rr == r) ? N[rr] : v;
    phi[s] = (s < b.K) ? (st == 1 ? v : (st == 2 ? __builtin_nanf("") : 0.f)) : 0.f;
  }
}

template <int KM, int KD>
__device__ inline void bspline_features(float x, float w, int i, const KBasis& b, float* phi) {
  const int nk = b.n_knots;
  float t0, ih;
  bspline_affine(b, i, t0, ih);
  bspline_features_rows<KM, KD>(x, w, b.knots_cmp + (size_t)i * nk, b.knots + (size_t)i * (nk + 2 * KD), t0, ih, b,
                                phi);
}

// ---------------------------------------------------------------------------
// Rational P/(1+|Q|) and derivatives by the quotient rule
//   out_n = (P^(n) - sum_{k=1..n} C(n,k) D^(k) out_{n-k}) / D,  D^(k) = sign(Q) Q^(k) for k >= 1.

// Evaluates sum_{p >= j} c_p p!/(p-j)! x^(p-j) for the polynomial with coefficients
// c_p = coef[p - first] (p = first .. first+n-1).
__device__ inline float poly_dj(const float* coef, int n, int first, int j, float x) {
  int hi = first + n - 1;  // highest power
  if (hi < j) return 0.f;
  float acc = 0.f;
  for (int p = hi; p >= j; --p) {
    float c = (p >= first) ? coef[p - first] : 0.f;
    float f = c;
    for (int t = 0; t < j; ++t) f *= (float)(p - t);
    acc = fmaf(acc, x, f);
  }
  return acc;
}

__device__ inline float binom(int n, int k) {
  float r = 1.f;
  for (int t = 1; t <= k; ++t) r = r * (float)(n - k + t) / (float)t;
  return r;
}

// d^m/dx^m of P/(1+|Q|), m <= 8
// The same recursion with the degrees fixed at compile time: the group's
// coefficients live in registers, every polynomial and derivative is straight
// Horner code (derivatives by differentiating the register coefficients in
// place), and the orders 0..MAXM are unrolled with m selecting the result.
template <int NP, int NQ, int MAXM>
__device__ inline float rational_feature_fixed(float x, const float* __restrict__ a, const float* __restrict__ c,
                                               int m) {
  float dp[NP], dq[NQ + 1];  // P = sum_p dp[p] x^p; Q = sum_{q >= 1} dq[q] x^q
#pragma unroll
  for (int p = 0; p < NP; ++p) dp[p] = a[p];
  dq[0] = 0.f;
#pragma unroll
  for (int q = 1; q <= NQ; ++q) dq[q] = c[q - 1];
  float Pd[MAXM + 1], Qd[MAXM + 1];
#pragma unroll
  for (int n = 0; n <= MAXM; ++n) {
    float hp = 0.f, hq = 0.f;
#pragma unroll
    for (int p = NP - 1; p >= 0; --p) hp = fmaf(hp, x, dp[p]);
#pragma unroll
    for (int q = NQ; q >= 0; --q) hq = fmaf(hq, x, dq[q]);
    Pd[n] = hp;
    Qd[n] = hq;
#pragma unroll
    for (int p = 0; p + 1 < NP; ++p) dp[p] = (float)(p + 1) * dp[p + 1];
    dp[NP - 1] = 0.f;
#pragma unroll
    for (int q = 0; q < NQ; ++q) dq[q] = (float)(q + 1) * dq[q + 1];
    dq[NQ] = 0.f;
  }
  const float sgn = (Qd[0] > 0.f) ? 1.f : ((Qd[0] < 0.f) ? -1.f : 0.f);
  const float invD = 1.f / (1.f + fabsf(Qd[0]));
  float out[MAXM + 1];
  out[0] = Pd[0] * invD;
  float res = out[0];
#pragma unroll
  for (int n = 1; n <= MAXM; ++n) {
    float acc = Pd[n];
    float bc = 1.f;  // binomial C(n, k), built incrementally
#pragma unroll
    for (int k = 1; k <= n; ++k) {
      bc = bc * (float)(n - k + 1) / (float)k;
      acc -= bc * sgn * Qd[k] * out[n - k];
    }
    out[n] = acc * invD;
    res = (n == m) ? out[n] : res;
  }
  return res;
}

__device__ inline float rational_feature(float x, int i, const KBasis& b, int m) {
  const int g = i / b.group_size;
  const float* a = b.num + (size_t)g * (b.num_deg + 1);
  const float* c = b.den + (size_t)g * b.den_deg;
  // the GR-KAN degrees (P 5, Q 4) up to order 4 take the unrolled register path
  if (b.num_deg == 5 && b.den_deg == 4 && m <= 4) return rational_feature_fixed<6, 4, 4>(x, a, c, m);
  float out[9];
  float Q0 = poly_dj(c, b.den_deg, 1, 0, x);
  float sgn = (Q0 > 0.f) ? 1.f : ((Q0 < 0.f) ? -1.f : 0.f);
  float D0 = 1.f + fabsf(Q0);
  float invD = 1.f / D0;
  out[0] = poly_dj(a, b.num_deg + 1, 0, 0, x) * invD;
  for (int n = 1; n <= m && n <= 8; ++n) {
    float acc = poly_dj(a, b.num_deg + 1, 0, n, x);
    for (int k = 1; k <= n; ++k) acc -= binom(n, k) * sgn * poly_dj(c, b.den_deg, 1, k, x) * out[n - k];
    out[n] = acc * invD;
  }
  return out[m < 8 ? m : 8];
}

// Degree dispatch with the knot rows of input i given (degrees 0..5 are compiled).
template <int KM>
__device__ inline void bspline_dispatch_rows(float x, float w, const float* kc, const float* kp0, const KBasis& b,
                                             float* phi, int i) {
  float t0, ih;
  bspline_affine(b, i, t0, ih);
  switch (b.spline_k) {
    case 0: bspline_features_rows<KM, 0>(x, w, kc, kp0, t0, ih, b, phi); break;
    case 1: bspline_features_rows<KM, 1>(x, w, kc, kp0, t0, ih, b, phi); break;
    case 2: bspline_features_rows<KM, 2>(x, w, kc, kp0, t0, ih, b, phi); break;
    case 3: bspline_features_rows<KM, 3>(x, w, kc, kp0, t0, ih, b, phi); break;
    case 4: bspline_features_rows<KM, 4>(x, w, kc, kp0, t0, ih, b, phi); break;
    default: bspline_features_rows<KM, 5>(x, w, kc, kp0, t0, ih, b, phi); break;
  }
}

// Copies the knot rows of inputs i0 .. i0 + n - 1 (zeros past IN) into LDS:
// kc[il * nk + r], kp[il * (nk + 2k) + r]. Every thread of the block calls it;
// the caller synchronises before reading.
// Knot rows of inputs i0 .. i0 + n - 1 into LDS: kc (n x n_knots comparison knots) and kp
// (n x (n_knots + 2 k) padded knots); rows past IN are zeros. The rows of consecutive inputs are
// one contiguous run in each table, and both tables are one index range e < n_kc + n_kp here.
// knot_rows_load issues the first U x blockDim elements' loads (addresses clamped into the
// existing rows, so no branches: they are in flight together, and the caller can put more loads
// behind them); knot_rows_store writes them and stages what remains.
struct KnotRange {
  int n_kc, n_kp, kc_last, kp_last;  // last: index of the last existing element (-1: none)
  const float *kcg, *kpg;
};
__device__ __forceinline__ KnotRange knot_range(const KBasis& b, int i0, int n, int IN) {
  const int nk = b.n_knots, np = nk + 2 * b.spline_k;
  const int rows = IN - i0 < n ? (IN - i0 < 0 ? 0 : IN - i0) : n;
  return {n * nk, n * np, rows * nk - 1, rows * np - 1, b.knots_cmp + (size_t)i0 * nk, b.knots + (size_t)i0 * np};
}
template <int U>
__device__ __forceinline__ void knot_rows_load(const KnotRange& r, int e0, float (&v)[U]) {
  if (r.kc_last < 0) return;  // a tile past the last input (padded widths): zeros only
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int e = e0 + u * blockDim.x, ep = e - r.n_kc;
    const float* src = e < r.n_kc ? r.kcg + (e < r.kc_last ? e : r.kc_last)
                                  : r.kpg + (ep < 0 ? 0 : (ep < r.kp_last ? ep : r.kp_last));
    v[u] = *src;
  }
}
template <int U>
__device__ __forceinline__ void knot_rows_put(const KnotRange& r, int e0, const float (&v)[U], float* kc, float* kp) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int e = e0 + u * blockDim.x, ep = e - r.n_kc;
    if (e < r.n_kc) kc[e] = e <= r.kc_last ? v[u] : 0.f;
    else if (ep < r.n_kp) kp[ep] = ep <= r.kp_last ? v[u] : 0.f;
  }
}
template <int U>
__device__ inline void knot_rows_store(const KnotRange& r, const float (&v)[U], float* kc, float* kp) {
  knot_rows_put<U>(r, threadIdx.x, v, kc, kp);
  for (int e0 = threadIdx.x + U * blockDim.x; e0 < r.n_kc + r.n_kp; e0 += U * blockDim.x) {
    float w[U];
    knot_rows_load<U>(r, e0, w);
    knot_rows_put<U>(r, e0, w, kc, kp);
  }
}
__device__ inline void stage_knot_rows(const KBasis& b, int i0, int n, int IN, float* kc, float* kp) {
  const KnotRange r = knot_range(b, i0, n, IN);
  float v[4];
  knot_rows_load<4>(r, threadIdx.x, v);
  knot_rows_store<4>(r, v, kc, kp);
}
__device__ __forceinline__ int knot_lds_floats(const KBasis& b, int n) {
  return n * (2 * b.n_knots + 2 * b.spline_k);
}

// Degree dispatch (degrees 0..5 are compiled).
template <int KM>
__device__ inline void bspline_dispatch(float x, float w, int i, const KBasis& b, float* phi) {
  switch (b.spline_k) {
    case 0: bspline_features<KM, 0>(x, w, i, b, phi); break;
    case 1: bspline_features<KM, 1>(x, w, i, b, phi); break;
    case 2: bspline_features<KM, 2>(x, w, i, b, phi); break;
    case 3: bspline_features<KM, 3>(x, w, i, b, phi); break;
    case 4: bspline_features<KM, 4>(x, w, i, b, phi); break;
    default: bspline_features<KM, 5>(x, w, i, b, phi); break;
  }
}

// ---------------------------------------------------------------------------
// All K features of order b.order (fold applied for cheb): the generic
// generator used where every feature of one element is needed at once.
template <int KM, int NT>
__device__ inline void basis_features(float x, float w, int i, const KBasis& b, float* phi) {
  if (b.kind == KF_KIND_CHEB) {
    float T[NT];
    const float z = cheb_map(x, b.input_map);
    cheb_features<NT>(z, cheb_weight(z, w, b.input_map), b.n_t, T);
    cheb_folded<KM, NT>(b, T, phi);
  } else if (b.kind == KF_KIND_BSPLINE) {
    bspline_dispatch<KM>(x, w, i, b, phi);
  } else {
#pragma unroll
    for (int s = 0; s < KM; ++s) phi[s] = 0.f;
    phi[0] = w * rational_feature(x, i, b, b.order);
  }
}

// Kernel features (what the F and G contractions consume): for cheb the
// unfolded T_j (n_t of them), otherwise the K basis derivatives.
template <int NT>
__device__ inline void kernel_features(float x, float w, int i, const KBasis& b, float* f) {
  if (b.kind == KF_KIND_CHEB) {
    const float z = cheb_map(x, b.input_map);
    cheb_features<NT>(z, cheb_weight(z, w, b.input_map), b.n_t, f);
  } else if (b.kind == KF_KIND_BSPLINE) {
    bspline_dispatch<NT>(x, w, i, b, f);
  } else {
#pragma unroll
    for (int s = 0; s < NT; ++s) f[s] = 0.f;
    f[0] = w * rational_feature(x, i, b, b.order);
  }
}

// kernel_features with the basis kind fixed at compile time: a kernel that
// evaluates features next to live accumulators only carries the code (and
// the registers) of its own kind.
template <int KIND, int NT>
__device__ __forceinline__ void kind_features(float x, float w, int i, const KBasis& b, float* f) {
  if constexpr (KIND == KF_KIND_CHEB) {
    const float z = cheb_map(x, b.input_map);
    cheb_features<NT>(z, cheb_weight(z, w, b.input_map), b.n_t, f);
  } else if constexpr (KIND == KF_KIND_BSPLINE) {
    bspline_dispatch<NT>(x, w, i, b, f);
  } else {
#pragma unroll
    for (int s = 0; s < NT; ++s) f[s] = 0.f;
    f[0] = w * rational_feature(x, i, b, b.order);
  }
}

}  // namespace kf
