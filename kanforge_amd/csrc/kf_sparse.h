// Sparse B-spline contractions: at any x only the k + 1 splines of its interval are non-zero, so
// F, P and G multiply k + 1 coefficients per (row, input) instead of K (the reference's dense
// route, kanforge/torch/layers.py:181-186 over kanforge/bases/spline.py:74-92, counts all K).
//
//   F: y[b, o]      = sum_i sum_r V[b, i, r] c[o, i, s0[b, i] + r]
//   P: p[b, i]      = sum_r V[b, i, r] sum_o g[b, o] c[o, i, s0[b, i] + r]
//   G: dc[o, i, k] += g[b, o] V[b, i, k - s0[b, i]]        (0 <= k - s0 <= KD)
//
// (s0, V) is the support window of (b, i): bspline_support's KD + 1 values w d^m/dx^m B_{KD, s}
// moved to a start s0 in [0, K - KD - 1] so that every index s0 + r is a basis function (values
// of indices outside [0, K) become zeros). x outside the knots gives V = 0; a non-finite x gives
// V = NaN, and G then poisons all K features of the row as the dense recurrence does.
#pragma once

#include "kf_kernels.h"

namespace kf {

constexpr int kSpKMax = 16;  // basis functions per input (the plan limit)
constexpr int kSpRows = 16;  // F / P: rows per workgroup
constexpr int kSpIC = 8;     // F: inputs per staged coefficient chunk
constexpr int kSpOC = 8;     // P: outputs per staged coefficient chunk
constexpr int kSpLane = 65;  // padded LDS row: 64 lanes + 1 (conflict-free transposing writes)

// Support window of input i at x (see above); returns 2 for a non-finite x, else 1.
template <int KD>
__device__ __forceinline__ int bspline_window(float x, float w, int i, const KBasis& b, int& s0, float (&V)[KD + 1]) {
  const int nk = b.n_knots, K = b.K;
  float t0, ih;
  bspline_affine(b, i, t0, ih);
  float N[KD + 1];
  int base = 0;
  const int st = bspline_support<KD>(x, w, b.knots_cmp + (size_t)i * nk, b.knots + (size_t)i * (nk + 2 * KD), t0, ih,
                                     b, base, N);
  s0 = 0;
  if (st != 1) {
    const float v = st == 2 ? __builtin_nanf("") : 0.f;
#pragma unroll
    for (int r = 0; r <= KD; ++r) V[r] = v;
    return st == 2 ? 2 : 1;
  }
  const int hi = K - KD - 1;
  s0 = base < 0 ? 0 : (base > hi ? hi : base);
  const int sh = s0 - base;  // V[r] = N[r + sh] (|sh| <= KD)
#pragma unroll
  for (int r = 0; r <= KD; ++r) {
    float v = 0.f;
#pragma unroll
    for (int q = 0; q <= KD; ++q) v = (q == r + sh) ? N[q] : v;
    V[r] = v;
  }
  return 1;
}

// F: workgroup = kSpRows rows x 64 outputs, 8 waves (lane = output, wave = rows wave + 8 q).
// The windows of the rows' next 64 inputs are computed once into LDS; the coefficients of kSpIC
// inputs x K x 64 outputs are staged in LDS per chunk, the next chunk's loads in flight (registers)
// while the current one is contracted.
// Base branch (bw given): the base weight W[o, i] is staged as each (o, i)'s basis function K
// (LDS rows KC = K + 1 apart), its feature silu(x) next to the windows; y starts from bias[o]
// when given.
template <typename T, int KD>
__global__ __launch_bounds__(512) void f_sparse_kernel(KBasis bs, int B, int IN, int OUT, const T* __restrict__ x,
                                                       const T* __restrict__ w, const T* __restrict__ c,
                                                       T* __restrict__ y, const T* __restrict__ bw,
                                                       const T* __restrict__ bias) {
  constexpr int NW = 8, RQ = kSpRows / NW, WCH = 64;
  constexpr int PF = (kSpIC * kSpKMax * 64 + 511) / 512;  // staged coefficients per thread, at most
  static_assert(kSpIC == 8, "the base weights of a chunk: one per thread of an output's 8");
  static_assert(WCH % kSpIC == 0 && kSpIC == 8, "windows of whole chunks, read as two int4");
  __shared__ float cs[kSpIC * (kSpKMax + 1)][kSpLane];
  __shared__ __align__(16) int ss[kSpRows][WCH];
  __shared__ float vs[kSpRows][WCH][KD + 1];
  __shared__ float svs[kSpRows][WCH];  // silu(x) of the base branch (KC > K)
  const int K = bs.K;
  const bool base = bw != nullptr;
  const int KC = base ? K + 1 : K;
  const float inv_k = 1.f / (float)K;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b0 = blockIdx.x * kSpRows, o0 = blockIdx.y * 64, o = o0 + lane;
  const int no = OUT - o0 < 64 ? OUT - o0 : 64;
  float acc[RQ];
#pragma unroll
  for (int q = 0; q < RQ; ++q) acc[q] = 0.f;
  float pre[PF], wpre = 0.f;
  // staging map without divisions: output row ol = tid / 8 of the chunk, values r = tid % 8 + 8 u
  // of its contiguous run of ni K coefficients (and, with the base branch, W[ol][i0 + tid % 8])
  const int sol = threadIdx.x >> 3, sr = threadIdx.x & 7;
  // with K a multiple of 4 (float c, 16-byte aligned) each thread moves whole float4s: values
  // r = 4 sr + 32 (u / 4) + u % 4, a quarter of the load instructions; else r = sr + 8 u
  const bool vec4 = std::is_same<T, float>::value && (K & 3) == 0 && (reinterpret_cast<uintptr_t>(c) & 15) == 0;
  static_assert(PF % 4 == 0, "whole float4s per thread");
  auto fetch = [&](int i0) {
    const int ni = IN - i0 < kSpIC ? IN - i0 : kSpIC, per_o = ni * K;
    const T* src = c + ((size_t)(o0 + sol) * IN + i0) * K;
    if (vec4) {
#pragma unroll
      for (int u4 = 0; u4 < PF / 4; ++u4) {
        const int r = 4 * sr + 32 * u4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (sol < no && r < per_o) v = *reinterpret_cast<const float4*>(src + r);
        pre[4 * u4] = v.x, pre[4 * u4 + 1] = v.y, pre[4 * u4 + 2] = v.z, pre[4 * u4 + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int u = 0; u < PF; ++u) {
        const int r = sr + 8 * u;
        pre[u] = (sol < no && r < per_o) ? to_f32(src[r]) : 0.f;
      }
    }
    if (base) wpre = (sol < no && sr < ni) ? to_f32(bw[(size_t)(o0 + sol) * IN + i0 + sr]) : 0.f;
  };
  fetch(0);  // the first chunk's loads in flight while the windows are computed
  for (int w0 = 0; w0 < IN; w0 += WCH) {
    const int nw = IN - w0 < WCH ? IN - w0 : WCH;
    __syncthreads();
    static_assert(kSpRows * WCH % 512 == 0, "whole passes of the workgroup");
    // unrolled: the passes' knot-table reads (x, then the knots around it, then the padded
    // knots) are dependent chains, which the two passes then run side by side
#pragma unroll
    for (int t = 0; t < kSpRows * WCH / 512; ++t) {
      const int e = threadIdx.x + 512 * t;
      const int rr = e / WCH, il = e % WCH, b = b0 + rr, i = w0 + il;
      int s0 = 0;
      float V[KD + 1];
#pragma unroll
      for (int r = 0; r <= KD; ++r) V[r] = 0.f;
      float sv = 0.f;
      if (b < B && il < nw) {
        const size_t off = (size_t)b * IN + i;
        const float xv = to_f32(x[off]);
        bspline_window<KD>(xv, w ? to_f32(w[off]) : 1.f, i, bs, s0, V);
        sv = silu_f(xv);
      }
      ss[rr][il] = s0;
      if (base) svs[rr][il] = sv;
#pragma unroll
      for (int r = 0; r <= KD; ++r) vs[rr][il][r] = V[r];
    }
    for (int i0 = w0; i0 < w0 + nw; i0 += kSpIC) {
      __syncthreads();
#pragma unroll
      for (int u = 0; u < PF; ++u) {
        const int r = vec4 ? 4 * sr + 32 * (u >> 2) + (u & 3) : sr + 8 * u;
        // with the base branch, value r (input r / K, function r % K) goes to row r + r / K;
        // (r + 1/2) / K is at least 1 / (2 K) from an integer, so the float quotient is exact
        const int row = base ? r + (int)(((float)r + 0.5f) * inv_k) : r;
        // the whole chunk's rows, zeros past its ni inputs (fetch leaves them 0), so that the
        // contraction below runs over all kSpIC inputs without a data-dependent exit
        if (r < kSpIC * K) cs[row][sol] = pre[u];
      }
      if (base) cs[sr * KC + K][sol] = wpre;
      __syncthreads();
      // the next chunk, also across windows (they are whole chunks: WCH = 8 kSpIC)
      if (i0 + kSpIC < IN) fetch(i0 + kSpIC);
      const int ib = i0 - w0;
      // the chunk's window starts first, then the contraction: inputs past ni have V = 0 and
      // silu 0 from the window pass (they lie past nw) and zero coefficient rows
      int s0q[RQ][kSpIC];
#pragma unroll
      for (int q = 0; q < RQ; ++q) {
        const int4* sp = reinterpret_cast<const int4*>(&ss[wave + NW * q][ib]);
        const int4 a = sp[0], b = sp[1];
        s0q[q][0] = a.x, s0q[q][1] = a.y, s0q[q][2] = a.z, s0q[q][3] = a.w;
        s0q[q][4] = b.x, s0q[q][5] = b.y, s0q[q][6] = b.z, s0q[q][7] = b.w;
      }
#pragma unroll
      for (int il = 0; il < kSpIC; ++il) {
#pragma unroll
        for (int q = 0; q < RQ; ++q) {
          const int rr = wave + NW * q;
          const int row = il * KC + s0q[q][il];
#pragma unroll
          for (int r = 0; r <= KD; ++r) acc[q] = fmaf(vs[rr][ib + il][r], cs[row + r][lane], acc[q]);
          if (base) acc[q] = fmaf(svs[rr][ib + il], cs[il * KC + K][lane], acc[q]);
        }
      }
    }
  }
  if (lane < no) {
    const float bo = bias ? to_f32(bias[o]) : 0.f;
#pragma unroll
    for (int q = 0; q < RQ; ++q) {
      const int b = b0 + wave + NW * q;
      if (b < B) y[(size_t)b * OUT + o] = from_f32<T>(acc[q] + bo);
    }
  }
}

// P: workgroup = kSpRows rows x 64 inputs, 8 waves (lane = input, wave = rows wave + 8 q); each
// lane keeps its rows' windows in registers; the coefficients of kSpOC outputs x K x 64 inputs and
// the rows' g values are staged in LDS per chunk (next chunk prefetched into registers);
// h_r = sum_o g c[o, i, s0 + r], then p = sum_r V_r h_r.
// Base branch (bw given): W[o, i] is staged as each (o, i)'s basis function K (LDS rows KC = K + 1
// apart); hb = sum_o g W accumulates next to h and p gets silu'(x) hb.
template <typename T, int KD>
__global__ __launch_bounds__(512, 4) void p_sparse_kernel(KBasis bs, int B, int IN, int OUT, const T* __restrict__ x,
                                                       const T* __restrict__ g, const T* __restrict__ c,
                                                       T* __restrict__ p, const T* __restrict__ bw) {
  constexpr int NW = 8, RQ = kSpRows / NW;
  constexpr int PF = kSpKMax + 1;  // one (output, input)'s K coefficients and W per thread (kSpOC = NW)
  static_assert(kSpOC == NW, "P stages one output per wave");
  // rows of 64: a wave writes one row at a time, and reads rows that differ per lane (each
  // lane's own window), which a 64-float stride keeps on distinct banks
  __shared__ float cs[kSpOC * (kSpKMax + 1)][64];
  __shared__ float gs[kSpRows][kSpOC];
  const int K = bs.K;
  const bool base = bw != nullptr;
  const int KC = base ? K + 1 : K;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b0 = blockIdx.x * kSpRows, i0 = blockIdx.y * 64, i = i0 + lane;
  const int ni = IN - i0 < 64 ? IN - i0 : 64;
  float pre[PF], gpre = 0.f;
  // staging map without divisions: thread (ol = wave, il = lane) moves the K coefficients of
  // (oc0 + ol, i0 + il)
  // whole float4s of the K coefficients when K is a multiple of 4 (float c, 16-byte aligned):
  // every lane reads its own run, so a quarter of the load instructions
  const bool vec4 = std::is_same<T, float>::value && (K & 3) == 0 && (reinterpret_cast<uintptr_t>(c) & 15) == 0;
  auto fetch = [&](int oc0) {
    const int no = OUT - oc0 < kSpOC ? OUT - oc0 : kSpOC;
    const size_t oi = (size_t)(oc0 + wave) * IN + i0 + lane;
    const T* src = c + oi * K;
    const bool in = wave < no && lane < ni;
    const float wv = (in && base) ? to_f32(bw[oi]) : 0.f;
    if (vec4) {
#pragma unroll
      for (int u4 = 0; u4 < (PF + 3) / 4; ++u4) {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (in && 4 * u4 < K) v = *reinterpret_cast<const float4*>(src + 4 * u4);
        const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (4 * u4 + q < PF) pre[4 * u4 + q] = 4 * u4 + q < K ? vv[q] : (4 * u4 + q == K ? wv : 0.f);
      }
    } else {
#pragma unroll
      for (int u = 0; u < PF; ++u) pre[u] = (in && u < K) ? to_f32(src[u]) : (u == K ? wv : 0.f);
    }
    if (threadIdx.x < kSpRows * kSpOC) {
      const int rr = threadIdx.x / kSpOC, ol = threadIdx.x % kSpOC, b = b0 + rr;
      gpre = (b < B && ol < no) ? to_f32(g[(size_t)b * OUT + oc0 + ol]) : 0.f;
    }
  };
  fetch(0);  // the first chunk's loads in flight while the windows are computed
  int s0[RQ];
  float V[RQ][KD + 1], h[RQ][KD + 1], hb[RQ], xq[RQ];
#pragma unroll
  for (int q = 0; q < RQ; ++q) {
    const int b = b0 + wave + NW * q;
    s0[q] = 0;
    hb[q] = xq[q] = 0.f;
#pragma unroll
    for (int r = 0; r <= KD; ++r) V[q][r] = h[q][r] = 0.f;
    if (b < B && lane < ni) {
      xq[q] = to_f32(x[(size_t)b * IN + i]);
      bspline_window<KD>(xq[q], 1.f, i, bs, s0[q], V[q]);
    }
  }
  for (int oc0 = 0; oc0 < OUT; oc0 += kSpOC) {
    const int no = OUT - oc0 < kSpOC ? OUT - oc0 : kSpOC;
    __syncthreads();
#pragma unroll
    for (int u = 0; u < PF; ++u)
      if (wave < no && u < KC) cs[wave * KC + u][lane] = pre[u];
    if (threadIdx.x < kSpRows * kSpOC) gs[threadIdx.x / kSpOC][threadIdx.x % kSpOC] = gpre;
    __syncthreads();
    if (oc0 + kSpOC < OUT) fetch(oc0 + kSpOC);
    if (lane < ni) {
#pragma unroll
      for (int ol = 0; ol < kSpOC; ++ol) {
        if (ol >= no) break;
#pragma unroll
        for (int q = 0; q < RQ; ++q) {
          const float gv = gs[wave + NW * q][ol];
          const int row = ol * KC + s0[q];
#pragma unroll
          for (int r = 0; r <= KD; ++r) h[q][r] = fmaf(gv, cs[row + r][lane], h[q][r]);
          if (base) hb[q] = fmaf(gv, cs[ol * KC + K][lane], hb[q]);
        }
      }
    }
  }
  if (lane < ni) {
#pragma unroll
    for (int q = 0; q < RQ; ++q) {
      const int b = b0 + wave + NW * q;
      float acc = 0.f;
#pragma unroll
      for (int r = 0; r <= KD; ++r) acc = fmaf(V[q][r], h[q][r], acc);
      if (base) acc = fmaf(dsilu_f(xq[q]), hb[q], acc);
      if (b < B) p[(size_t)b * IN + i] = from_f32<T>(acc);
    }
  }
}

// P for small layers (in and out <= 128, K [+ 1] <= 12): a workgroup = kSmRows rows x 64 inputs
// (lanes) whose 8 waves split the outputs. Each lane holds the coefficients of its 8 (output,
// input) pairs of the current 64-wide output group in registers (one load per group, in flight
// during the window pass; lanes read neighbouring inputs' runs); the rows' derivative windows sit
// in LDS as dense rows of KM features (zeros outside the window; with the base branch, silu'(x)
// as function K), and the waves' partial sums are added in wave order at the end. Dense over the
// features (KM + 1 FMAs per row, input and output instead of k + 2), for one window pass and two
// barriers per 64 outputs instead of eight staged chunks. (The same shape for F, lanes =
// outputs, reads rows IN K apart per lane, 64 cache lines per load, and lost to the staged F.)
constexpr int kSmRows = 16;
// dense-row stride in floats: whole float4s, and not a multiple of 8, so that the per-lane rows
// of P's reads (one row per lane, 16 bytes at a time) fall on distinct banks
template <int KM>
struct SmPad {
  static constexpr int q = (KM + 3) / 4 * 4;
  static constexpr int value = q % 8 == 0 ? q + 4 : q;
};

// the dense row of one (row, input): V at s0 .. s0 + KD, extra at K when with_extra, else zeros
template <int KD, int KP>
__device__ __forceinline__ void sm_dense_row(float* dst, int K, int s0, const float (&V)[KD + 1], bool with_extra,
                                             float extra) {
#pragma unroll
  for (int k4 = 0; k4 < KP / 4; ++k4) {
    float v4[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int k = 4 * k4 + u;
      float v = 0.f;
#pragma unroll
      for (int r = 0; r <= KD; ++r) v = (k == s0 + r) ? V[r] : v;
      v4[u] = k < K ? v : (with_extra && k == K ? extra : 0.f);
    }
    reinterpret_cast<float4*>(dst)[k4] = make_float4(v4[0], v4[1], v4[2], v4[3]);
  }
}

template <typename T, int KD, int KM>
__global__ __launch_bounds__(512) void p_small_kernel(KBasis bs, int B, int IN, int OUT, const T* __restrict__ x,
                                                      const T* __restrict__ g, const T* __restrict__ c,
                                                      T* __restrict__ p, const T* __restrict__ bw) {
  constexpr int NW = 8, R = kSmRows, KP = SmPad<KM>::value, OCH = 64, OPW = OCH / NW;
  constexpr int PH = R * 64 * KP, RED = NW * R * 64;
  __shared__ __align__(16) float lds[PH > RED ? PH : RED];
  __shared__ __align__(16) float gs[R * OCH];
  const int K = bs.K;
  const bool base = bw != nullptr;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b0 = blockIdx.x * R, i0 = blockIdx.y * 64, i = i0 + lane;
  float cr[OPW][KM];
  // whole float4s of each (o, i)'s K coefficients when K is a multiple of 4 and c is 16-byte
  // aligned (a quarter of the load instructions; every lane reads its own run)
  const bool vec4 = std::is_same<T, float>::value && (K & 3) == 0 && (reinterpret_cast<uintptr_t>(c) & 15) == 0;
  auto load_coef = [&](int o0) {
#pragma unroll
    for (int j = 0; j < OPW; ++j) {
      const int o = o0 + wave * OPW + j;
      const bool in = i < IN && o < OUT;
      const size_t oi = (size_t)o * IN + i;
      const float wv = (in && base) ? to_f32(bw[oi]) : 0.f;
      if (vec4) {
#pragma unroll
        for (int k4 = 0; k4 < (KM + 3) / 4; ++k4) {
          float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
          if (in && 4 * k4 < K) v = *reinterpret_cast<const float4*>(c + oi * K + 4 * k4);
          const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int u = 0; u < 4; ++u)
            if (4 * k4 + u < KM) cr[j][4 * k4 + u] = 4 * k4 + u < K ? vv[u] : (4 * k4 + u == K ? wv : 0.f);
        }
      } else {
#pragma unroll
        for (int k = 0; k < KM; ++k) cr[j][k] = (in && k < K) ? to_f32(c[oi * K + k]) : (k == K ? wv : 0.f);
      }
    }
  };
  load_coef(0);  // in flight during the window pass
#pragma unroll
  for (int t = 0; t < R * 64 / 512; ++t) {  // unrolled: the passes' dependent knot reads side by side
    const int e = threadIdx.x + 512 * t;
    const int rr = e / 64, il = e % 64, b = b0 + rr, ii = i0 + il;
    int s0 = 0;
    float V[KD + 1];
#pragma unroll
    for (int r = 0; r <= KD; ++r) V[r] = 0.f;
    float sd = 0.f;
    if (b < B && ii < IN) {
      const float xv = to_f32(x[(size_t)b * IN + ii]);
      bspline_window<KD>(xv, 1.f, ii, bs, s0, V);
      sd = dsilu_f(xv);
    }
    sm_dense_row<KD, KP>(lds + (size_t)e * KP, K, s0, V, base, sd);
  }
  float acc[R];
#pragma unroll
  for (int q = 0; q < R; ++q) acc[q] = 0.f;
  for (int o0 = 0; o0 < OUT; o0 += OCH) {
    if (o0 > 0) load_coef(o0);
    __syncthreads();  // the windows are written; the previous group's g readers are done
    for (int e = threadIdx.x; e < R * OCH; e += 512) {
      const int rr = e / OCH, ol = e % OCH, b = b0 + rr, o = o0 + ol;
      gs[e] = (b < B && o < OUT) ? to_f32(g[(size_t)b * OUT + o]) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < R; ++q) {
      const float4* ph = reinterpret_cast<const float4*>(lds + (size_t)(q * 64 + lane) * KP);
      float f[(KM + 3) / 4 * 4];
#pragma unroll
      for (int k4 = 0; k4 < (KM + 3) / 4; ++k4) {
        const float4 v = ph[k4];
        f[4 * k4] = v.x;
        f[4 * k4 + 1] = v.y;
        f[4 * k4 + 2] = v.z;
        f[4 * k4 + 3] = v.w;
      }
      float a = acc[q];
#pragma unroll
      for (int j = 0; j < OPW; ++j) {
        float t = 0.f;
#pragma unroll
        for (int k = 0; k < KM; ++k) t = fmaf(f[k], cr[j][k], t);
        a = fmaf(gs[q * OCH + wave * OPW + j], t, a);
      }
      acc[q] = a;
    }
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < R; ++q) lds[(wave * R + q) * 64 + lane] = acc[q];
  __syncthreads();
  for (int e = threadIdx.x; e < R * 64; e += 512) {
    const int q = e / 64, l = e % 64, b = b0 + q, ii = i0 + l;
    if (b < B && ii < IN) {
      float sum = 0.f;
#pragma unroll
      for (int v = 0; v < NW; ++v) sum += lds[(v * R + q) * 64 + l];
      p[(size_t)b * IN + ii] = from_f32<T>(sum);
    }
  }
}

// G partial sums over a slice of rows: workgroup = 4 inputs (one per wave) x 64 outputs (lane)
// x rows [z RS, (z + 1) RS); part[z][i][k][o] (float, K per (i, o)). For 64 rows at a time each
// lane turns its row's window into the row's KM features (zeros outside the window, all NaN for a
// non-finite x) in the wave's LDS slot; every row then costs KM broadcast reads and KM FMAs per
// lane, with the loads of sixteen rows' g in flight at once.
// Base branch (KO = K + 1 <= KM): feature K is silu(x), so part holds K + 1 sums per (o, i), the
// last the base weight's gradient; with bpart, the lanes of input 0 also sum g over the slice's
// rows into bpart[z][o] (the bias gradient's slice partials).
template <typename T, int KD, int KM>
__global__ __launch_bounds__(256) void g_sparse_kernel(KBasis bs, int B, int IN, int OUT, int RS,
                                                       const T* __restrict__ x, const T* __restrict__ g,
                                                       const T* __restrict__ w, float* __restrict__ part, int KO,
                                                       float* __restrict__ bpart) {
  __shared__ float phi[4][64][KM];
  const int K = bs.K;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = blockIdx.x * 4 + wave, o = blockIdx.y * 64 + lane;
  const bool live = i < IN && o < OUT;
  const int z = blockIdx.z, r0 = z * RS, r1 = min(B, r0 + RS);
  const bool bsum = bpart != nullptr && i == 0;
  float acc[KM], bacc = 0.f;
#pragma unroll
  for (int k = 0; k < KM; ++k) acc[k] = 0.f;
  for (int bb = r0; bb < r1; bb += 64) {
    const int nb = r1 - bb < 64 ? r1 - bb : 64;
    __syncthreads();
    {
      int s0 = 0;
      float V[KD + 1];
#pragma unroll
      for (int r = 0; r <= KD; ++r) V[r] = 0.f;
      bool nan = false;
      float sv = 0.f;
      if (lane < nb && i < IN) {
        const size_t off = (size_t)(bb + lane) * IN + i;
        const float xv = to_f32(x[off]);
        nan = bspline_window<KD>(xv, w ? to_f32(w[off]) : 1.f, i, bs, s0, V) == 2;
        sv = silu_f(xv);
      }
#pragma unroll
      for (int k = 0; k < KM; ++k) {
        float v = 0.f;
#pragma unroll
        for (int r = 0; r <= KD; ++r) v = (k == s0 + r) ? V[r] : v;
        v = nan ? V[0] : v;
        phi[wave][lane][k] = k < K ? v : (k == K && KO > K ? sv : 0.f);
      }
    }
    __syncthreads();
    if (live) {
      for (int j0 = 0; j0 < nb; j0 += 16) {
        float gb[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) gb[u] = j0 + u < nb ? to_f32(g[(size_t)(bb + j0 + u) * OUT + o]) : 0.f;
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          if (j0 + u >= nb) break;
#pragma unroll
          for (int k = 0; k < KM; ++k) acc[k] = fmaf(gb[u], phi[wave][j0 + u][k], acc[k]);
          if (bsum) bacc += gb[u];
        }
      }
    }
  }
  if (live) {
    // part[z][i][k][o]: a wave's 64 lanes (outputs) store 256 contiguous bytes per k
    float* dst = part + ((size_t)z * IN + i) * KO * OUT + o;
#pragma unroll
    for (int k = 0; k < KM; ++k)
      if (k < KO) dst[(size_t)k * OUT] = acc[k];
    if (bsum) bpart[(size_t)z * OUT + o] = bacc;
  }
}

// G's slice partials part[z][i][k][o] (KO sums per (input, output), outputs contiguous) summed in
// slice order (deterministic): dc[o][i][k] for k < K and, with KO = K + 1, dw[o][i] for k = K;
// with db, db[o] = sum_z bpart[z][o]. dc or dw may be NULL. Reads run along the partials' layout;
// each sum is written once, to its place in dc.
template <typename T>
__global__ __launch_bounds__(256) void g_sparse_reduce(int nz, int IN, int OUT, int K, int KO,
                                                       const float* __restrict__ part, T* __restrict__ dc,
                                                       T* __restrict__ dw, const float* __restrict__ bpart,
                                                       T* __restrict__ db) {
  const long n = (long)IN * KO * OUT, n_all = n + (db ? OUT : 0);
  for (long e = blockIdx.x * 256L + threadIdx.x; e < n_all; e += (long)gridDim.x * 256) {
    if (e >= n) {
      const int o = (int)(e - n);
      db[o] = from_f32<T>(slice_sum(bpart + o, (size_t)OUT, nz));
      continue;
    }
    const float s = slice_sum(part + e, (size_t)n, nz);
    const long t = e / OUT;
    const int o = (int)(e - t * OUT), i = (int)(t / KO), k = (int)(t - (long)i * KO);
    const size_t oi = (size_t)o * IN + i;
    if (k < K) {
      if (dc) dc[oi * K + k] = from_f32<T>(s);
    } else if (dw) {
      dw[oi] = from_f32<T>(s);
    }
  }
}

}  // namespace kf
