// Elementwise group-rational kernels of the bf16 GEMM routes (GR-KAN, P 5 / Q 4):
//   rational_map_kernel    out[b][i] = w[b][i] phi^(M)(x[b][i])  (or H[b][i] phi^(M)(x[b][i]))
//   rational_map_t_kernel  out[i][b] = w[b][i] phi^(M)(x[b][i])  transposed, rows zero-padded to BP
// phi = P/(1+|Q|) with the coefficients of input i's group (kanforge/bases/rational.py:84-101).
// Eight consecutive inputs per thread (16-byte loads and stores); a group spans a multiple of
// eight inputs, so a thread's coefficients are one group's, held in registers.
#pragma once

#include "kf_kernels.h"

namespace kf {

// phi^(M)(x) of P (NP coefficients) over 1 + |Q| (NQ coefficients, Q = sum_q c[q-1] x^q) by
// Horner and the quotient rule, with only the derivative orders up to M evaluated.
template <int NP, int NQ, int M>
__device__ __forceinline__ float rational_order(float x, const float (&a)[NP], const float (&c)[NQ]) {
  float dp[NP], dq[NQ + 1];
#pragma unroll
  for (int p = 0; p < NP; ++p) dp[p] = a[p];
  dq[0] = 0.f;
#pragma unroll
  for (int q = 1; q <= NQ; ++q) dq[q] = c[q - 1];
  float Pd[M + 1], Qd[M + 1];
#pragma unroll
  for (int n = 0; n <= M; ++n) {
    float hp = 0.f, hq = 0.f;
#pragma unroll
    for (int p = NP - 1; p >= 0; --p) hp = fmaf(hp, x, dp[p]);
#pragma unroll
    for (int q = NQ; q >= 0; --q) hq = fmaf(hq, x, dq[q]);
    Pd[n] = hp;
    Qd[n] = hq;
    if (n < M) {
#pragma unroll
      for (int p = 0; p + 1 < NP; ++p) dp[p] = (float)(p + 1) * dp[p + 1];
      dp[NP - 1] = 0.f;
#pragma unroll
      for (int q = 0; q < NQ; ++q) dq[q] = (float)(q + 1) * dq[q + 1];
      dq[NQ] = 0.f;
    }
  }
  const float sgn = (Qd[0] > 0.f) ? 1.f : ((Qd[0] < 0.f) ? -1.f : 0.f);
  const float invD = 1.f / (1.f + fabsf(Qd[0]));
  float out[M + 1];
  out[0] = Pd[0] * invD;
#pragma unroll
  for (int n = 1; n <= M; ++n) {
    float acc = Pd[n];
    float bc = 1.f;
#pragma unroll
    for (int k = 1; k <= n; ++k) {
      bc = bc * (float)(n - k + 1) / (float)k;
      acc -= bc * sgn * Qd[k] * out[n - k];
    }
    out[n] = acc * invD;
  }
  return out[M];
}

template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    const u32x4 r = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v[2 * q] = __uint_as_float(r[q] << 16);
      v[2 * q + 1] = __uint_as_float(r[q] & 0xffff0000u);
    }
  } else {
    const f32x4 r0 = *reinterpret_cast<const f32x4*>(p), r1 = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v[q] = r0[q];
      v[4 + q] = r1[q];
    }
  }
}

template <typename T>
__device__ __forceinline__ void store8(T* p, const float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    *reinterpret_cast<u32x4*>(p) = pack16<bf16>(v);
  } else {
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
  }
}

// out = scale * phi^(M)(x) with scale = w (T, may be NULL) or H (float, may be NULL); B x IN,
// IN % 8 == 0, group_size % 8 == 0, rows 16-byte aligned.
template <typename T, typename TO, int M>
__global__ __launch_bounds__(256) void rational_map_kernel(KBasis bs, int B, int IN, const T* __restrict__ x,
                                                           const T* __restrict__ w, const float* __restrict__ hsc,
                                                           TO* __restrict__ out) {
  constexpr int NP = 6, NQ = 4;
  const long n8 = (long)B * (IN / 8);
  for (long e = blockIdx.x * 256L + threadIdx.x; e < n8; e += (long)gridDim.x * 256) {
    const int b = (int)(e / (IN / 8)), i0 = (int)(e % (IN / 8)) * 8;
    const int g = i0 / bs.group_size;
    float a[NP], c[NQ];
#pragma unroll
    for (int p = 0; p < NP; ++p) a[p] = bs.num[g * NP + p];
#pragma unroll
    for (int q = 0; q < NQ; ++q) c[q] = bs.den[g * NQ + q];
    const size_t off = (size_t)b * IN + i0;
    float xv[8], sc[8], v[8];
    load8<T>(x + off, xv);
    if (w) load8<T>(w + off, sc);
    if (hsc) load8<float>(hsc + off, sc);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      v[q] = rational_order<NP, NQ, M>(xv[q], a, c);
      if (w || hsc) v[q] *= sc[q];
    }
    store8<TO>(out + off, v);
  }
}

// out[i][b] = w[b][i] phi^(M)(x[b][i]) for 64 x 64 tiles of (batch, inputs); rows b >= B of the
// output (up to BP, a multiple of 64) are zeros. IN % 64 == 0.
template <typename T, int M>
__global__ __launch_bounds__(256) void rational_map_t_kernel(KBasis bs, int B, int IN, int BP, const T* __restrict__ x,
                                                             const T* __restrict__ w, T* __restrict__ out) {
  constexpr int NP = 6, NQ = 4;
  __shared__ float tile[64][65];
  const int b0 = blockIdx.y * 64, i0 = blockIdx.x * 64;
  const int t = threadIdx.x;
  // read: thread t handles rows r = t / 8 and r + 32, inputs 8 (t % 8) .. +7 (one group)
  const int ic = (t % 8) * 8;
  const int g = (i0 + ic) / bs.group_size;
  float a[NP], c[NQ];
#pragma unroll
  for (int p = 0; p < NP; ++p) a[p] = bs.num[g * NP + p];
#pragma unroll
  for (int q = 0; q < NQ; ++q) c[q] = bs.den[g * NQ + q];
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int r = t / 8 + 32 * half, b = b0 + r;
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (b < B) {
      const size_t off = (size_t)b * IN + i0 + ic;
      float xv[8], sc[8];
      load8<T>(x + off, xv);
      if (w) load8<T>(w + off, sc);
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        v[q] = rational_order<NP, NQ, M>(xv[q], a, c);
        if (w) v[q] *= sc[q];
      }
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) tile[r][ic + q] = v[q];
  }
  __syncthreads();
  // write: output row i (64 batch values) in 8 chunks of 8; thread t writes rows t / 8 and + 32
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int il = t / 8 + 32 * half, bc = (t % 8) * 8;
    float v[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] = tile[bc + q][il];
    store8<T>(out + (size_t)(i0 + il) * BP + b0 + bc, v);
  }
}

// Partial sums, per (group, chunk of RROWS rows), of the gradients of
//   sum_{b,i} h[b,i] w[b,i] phi(x[b,i])
// with respect to the group's numerator a_0..a_5 (x^p / D) and denominator b_1..b_4
// (-P sign(Q) x^q / D^2), D = 1 + |Q|: part[(chunk * groups + g) * 10 + q]. Eight consecutive
// inputs per thread (16-byte loads of x, w and h); group_size % 8 == 0.
template <typename T, int RROWS>
__global__ __launch_bounds__(256) void rational_grad_fast(KBasis bs, int B, int IN, const T* __restrict__ x,
                                                          const float* __restrict__ hbuf, const T* __restrict__ w,
                                                          float* __restrict__ part) {
  constexpr int NP = 6, NQ = 4, NPAR = NP + NQ;
  const int g = blockIdx.x, chunk = blockIdx.y, gs = bs.group_size;
  float a[NP], c[NQ];
#pragma unroll
  for (int p = 0; p < NP; ++p) a[p] = bs.num[g * NP + p];
#pragma unroll
  for (int q = 0; q < NQ; ++q) c[q] = bs.den[g * NQ + q];
  float acc[NPAR];
#pragma unroll
  for (int q = 0; q < NPAR; ++q) acc[q] = 0.f;
  const int per_row = gs / 8;
  const int n = RROWS * per_row;
  for (int e = threadIdx.x; e < n; e += 256) {
    const int r = e / per_row, b = chunk * RROWS + r;
    if (b >= B) break;  // rows grow with e
    const size_t off = (size_t)b * IN + g * gs + (e % per_row) * 8;
    float xv[8], hv[8], wv[8];
    load8<T>(x + off, xv);
    load8<float>(hbuf + off, hv);
    if (w) load8<T>(w + off, wv);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float xx = xv[k], hh = w ? hv[k] * wv[k] : hv[k];
      float P = 0.f, Q = 0.f;
#pragma unroll
      for (int p = NP - 1; p >= 0; --p) P = fmaf(P, xx, a[p]);
#pragma unroll
      for (int q = NQ - 1; q >= 0; --q) Q = fmaf(Q, xx, c[q]);
      Q *= xx;
      const float sgn = (Q > 0.f) ? 1.f : ((Q < 0.f) ? -1.f : 0.f);
      const float invD = 1.f / (1.f + fabsf(Q));
      const float hd = hh * invD, hq = -hh * P * sgn * invD * invD;
      float xp = 1.f;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        if (p < NQ) acc[NP + p] = fmaf(hq, xp * xx, acc[NP + p]);
        acc[p] = fmaf(hd, xp, acc[p]);
        xp *= xx;
      }
    }
  }
  // block sums: wave reductions through LDS, one slot per (wave, parameter)
  __shared__ float red[4][NPAR];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int q = 0; q < NPAR; ++q) {
    float v = acc[q];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    if (lane == 0) red[wave][q] = v;
  }
  __syncthreads();
  if (threadIdx.x < NPAR)
    part[((size_t)chunk * gridDim.x + g) * NPAR + threadIdx.x] =
        red[0][threadIdx.x] + red[1][threadIdx.x] + red[2][threadIdx.x] + red[3][threadIdx.x];
}

// Fused rational backward at order 0 (GR-KAN degrees): one pass over x, H (float32 or bf16) and w writes
// p[b,i] = H[b,i] phi'(x[b,i]) (the input gradient) and, per (group, chunk of RROWS rows), the
// partial sums of H w dphi/dtheta (as rational_grad_fast). Eight consecutive inputs per thread.
template <typename T, typename TH, int RROWS>
__global__ __launch_bounds__(256) void rational_bwd_fast(KBasis bs, int B, int IN, const T* __restrict__ x,
                                                         const TH* __restrict__ hbuf, const T* __restrict__ w,
                                                         T* __restrict__ p, float* __restrict__ part) {
  constexpr int NP = 6, NQ = 4, NPAR = NP + NQ;
  const int g = blockIdx.x, chunk = blockIdx.y, gs = bs.group_size;
  float a[NP], c[NQ];
#pragma unroll
  for (int q = 0; q < NP; ++q) a[q] = bs.num[g * NP + q];
#pragma unroll
  for (int q = 0; q < NQ; ++q) c[q] = bs.den[g * NQ + q];
  float acc[NPAR];
#pragma unroll
  for (int q = 0; q < NPAR; ++q) acc[q] = 0.f;
  const int per_row = gs / 8;
  const int n = RROWS * per_row;
  for (int e = threadIdx.x; e < n; e += 256) {
    const int r = e / per_row, b = chunk * RROWS + r;
    if (b >= B) break;  // rows grow with e
    const size_t off = (size_t)b * IN + g * gs + (e % per_row) * 8;
    float xv[8], hv[8], wv[8], pv[8];
    load8<T>(x + off, xv);
    load8<TH>(hbuf + off, hv);
    if (w) load8<T>(w + off, wv);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float xx = xv[k];
      // P, P' and q, q' (Q = x q) by simultaneous Horner; phi = P / D, D = 1 + |Q|,
      // phi' = (P' - phi sign(Q) Q') / D with one reciprocal shared by every term
      float P = a[NP - 1], dP = 0.f;
#pragma unroll
      for (int q = NP - 2; q >= 0; --q) {
        dP = fmaf(dP, xx, P);
        P = fmaf(P, xx, a[q]);
      }
      float qq = c[NQ - 1], dq = 0.f;
#pragma unroll
      for (int q = NQ - 2; q >= 0; --q) {
        dq = fmaf(dq, xx, qq);
        qq = fmaf(qq, xx, c[q]);
      }
      const float Q = xx * qq, dQ = fmaf(xx, dq, qq);
      const float sgn = (Q > 0.f) ? 1.f : ((Q < 0.f) ? -1.f : 0.f);
      const float invD = __builtin_amdgcn_rcpf(1.f + fabsf(Q));
      const float phi = P * invD;
      pv[k] = hv[k] * ((dP - phi * sgn * dQ) * invD);
      const float hh = w ? hv[k] * wv[k] : hv[k];
      const float hd = hh * invD, hq = -hd * phi * sgn;
      float xp = 1.f;
#pragma unroll
      for (int q = 0; q < NP; ++q) {
        if (q < NQ) acc[NP + q] = fmaf(hq, xp * xx, acc[NP + q]);
        acc[q] = fmaf(hd, xp, acc[q]);
        xp *= xx;
      }
    }
    store8<T>(p + off, pv);
  }
  __shared__ float red[4][NPAR];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int q = 0; q < NPAR; ++q) {
    float v = acc[q];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    if (lane == 0) red[wave][q] = v;
  }
  __syncthreads();
  if (threadIdx.x < NPAR)
    part[((size_t)chunk * gridDim.x + g) * NPAR + threadIdx.x] =
        red[0][threadIdx.x] + red[1][threadIdx.x] + red[2][threadIdx.x] + red[3][threadIdx.x];
}

// Partial sums, per (group, chunk of RROWS rows), of the gradients of
//   sum_{b,i} h[b,i] w[b,i] phi^(M)(x[b,i])          (M >= 1, GR-KAN degrees P 5 / Q 4)
// with respect to the group's a_0..a_5 and b_1..b_4: forward-mode derivatives of the quotient
// recursion out_n = (P_n - sum_{k=1..n} C(n,k) D_k out_{n-k}) / D_0, D_0 = 1 + |Q|,
// D_k = sign(Q) Q^(k); a parameter of P enters through P_n = d^n/dx^n x^p, one of Q through
// D_0 (sign(Q) x^(q+1)) and D_k (sign(Q) d^k/dx^k x^(q+1)). part[(chunk * groups + g) * 10 + j].
template <typename T, int M, int RROWS>
__global__ __launch_bounds__(256) void rational_grad_order(KBasis bs, int B, int IN, const T* __restrict__ x,
                                                           const float* __restrict__ hbuf, const T* __restrict__ w,
                                                           float* __restrict__ part) {
  constexpr int NP = 6, NQ = 4, NPAR = NP + NQ, NX = NP + NQ + 1;
  const int g = blockIdx.x, chunk = blockIdx.y, gs = bs.group_size;
  float a[NP], c[NQ];
#pragma unroll
  for (int p = 0; p < NP; ++p) a[p] = bs.num[g * NP + p];
#pragma unroll
  for (int q = 0; q < NQ; ++q) c[q] = bs.den[g * NQ + q];
  float acc[NPAR];
#pragma unroll
  for (int j = 0; j < NPAR; ++j) acc[j] = 0.f;
  const int n = RROWS * gs;
  for (int e = threadIdx.x; e < n; e += 256) {
    const int r = e / gs, b = chunk * RROWS + r;
    if (b >= B) break;  // rows grow with e
    const size_t off = (size_t)b * IN + g * gs + (e - r * gs);
    const float xv = to_f32(x[off]);
    const float hv = hbuf[off] * (w ? to_f32(w[off]) : 1.f);
    float xp[NX];  // x^0 .. x^(NP + NQ)
    xp[0] = 1.f;
#pragma unroll
    for (int k = 1; k < NX; ++k) xp[k] = xp[k - 1] * xv;
    // derivatives 0..M of P and Q at x
    float Pd[M + 1], Qd[M + 1];
#pragma unroll
    for (int d = 0; d <= M; ++d) {
      float sp = 0.f, sq = 0.f;
#pragma unroll
      for (int p = d; p < NP; ++p) {
        float f = 1.f;
#pragma unroll
        for (int t = 0; t < d; ++t) f *= (float)(p - t);
        sp = fmaf(a[p] * f, xp[p - d], sp);
      }
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const int pw = q + 1;
        if (pw < d) continue;
        float f = 1.f;
#pragma unroll
        for (int t = 0; t < d; ++t) f *= (float)(pw - t);
        sq = fmaf(c[q] * f, xp[pw - d], sq);
      }
      Pd[d] = sp;
      Qd[d] = sq;
    }
    const float sgn = (Qd[0] > 0.f) ? 1.f : ((Qd[0] < 0.f) ? -1.f : 0.f);
    float D[M + 1], out[M + 1];
    D[0] = 1.f + fabsf(Qd[0]);
#pragma unroll
    for (int k = 1; k <= M; ++k) D[k] = sgn * Qd[k];
    const float iD = 1.f / D[0];
#pragma unroll
    for (int d = 0; d <= M; ++d) {
      float v = Pd[d];
      float bc = 1.f;
#pragma unroll
      for (int k = 1; k <= d; ++k) {
        bc = bc * (float)(d - k + 1) / (float)k;
        v -= bc * D[k] * out[d - k];
      }
      out[d] = v * iD;
    }
#pragma unroll
    for (int j = 0; j < NPAR; ++j) {
      float dP[M + 1], dD[M + 1], dO[M + 1];
#pragma unroll
      for (int d = 0; d <= M; ++d) {
        dP[d] = 0.f;
        dD[d] = 0.f;
      }
      if (j < NP) {  // a_j: d^d/dx^d x^j
#pragma unroll
        for (int d = 0; d <= M; ++d) {
          if (j < d) continue;
          float f = 1.f;
#pragma unroll
          for (int t = 0; t < d; ++t) f *= (float)(j - t);
          dP[d] = f * xp[j - d];
        }
      } else {  // b_(q+1): x^(q+1) in Q
        const int pw = j - NP + 1;
#pragma unroll
        for (int d = 0; d <= M; ++d) {
          if (pw < d) continue;
          float f = 1.f;
#pragma unroll
          for (int t = 0; t < d; ++t) f *= (float)(pw - t);
          dD[d] = sgn * f * xp[pw - d];
        }
      }
#pragma unroll
      for (int d = 0; d <= M; ++d) {
        float v = dP[d] - dD[0] * out[d];
        float bc = 1.f;
#pragma unroll
        for (int k = 1; k <= d; ++k) {
          bc = bc * (float)(d - k + 1) / (float)k;
          v -= bc * (dD[k] * out[d - k] + D[k] * dO[d - k]);
        }
        dO[d] = v * iD;
      }
      acc[j] = fmaf(hv, dO[M], acc[j]);
    }
  }
  __shared__ float red[4][NPAR];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int j = 0; j < NPAR; ++j) {
    float v = acc[j];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    if (lane == 0) red[wave][j] = v;
  }
  __syncthreads();
  if (threadIdx.x < NPAR)
    part[((size_t)chunk * gridDim.x + g) * NPAR + threadIdx.x] =
        red[0][threadIdx.x] + red[1][threadIdx.x] + red[2][threadIdx.x] + red[3][threadIdx.x];
}

// Whether the rational fast kernels apply: GR-KAN degrees, groups and rows of whole 8-input runs.
inline bool rational_fast(const KBasis& kb, long n_in) {
  return kb.kind == KF_KIND_RATIONAL && kb.num_deg == 5 && kb.den_deg == 4 && kb.group_size % 8 == 0 && n_in % 8 == 0;
}

}  // namespace kf
