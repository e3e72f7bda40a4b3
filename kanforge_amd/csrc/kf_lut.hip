// Lookup-table inference (kanforge/export/lut.py:70-89): every edge of a layer tabulated at
// `size` uniform points over its input's range [lo, hi],
//   t = (x - lo) / step,  tc = clip(t, 0, size - 1),  j = min(floor(tc), size - 2),  f = tc - j
//   y[b, o] = bias[o] + scale[o] * sum_i (T[i, j, o] + f (T[i, j + 1, o] - T[i, j, o]))
//             + sum_i (min(t, 0) slope_lo[i, o] + max(t - (size - 1), 0) slope_hi[i, o])
// (scale omitted for float tables; the slope terms only with linear extrapolation).
//
// One lane per (row, run of V outputs): a wave holds 64 / OW rows of OW lanes (OW a power of two
// covering the row's runs, at most 64; wider layers take slices along grid.y). V fills a 16-byte
// load (4 float, 8 int16, 16 int8 entries) when n_out is a multiple of it, else V = 1. Every lane
// of a row computes the row's (j, f) itself (one instruction for all lanes, so nothing is shared)
// and gathers its runs of T[i, j, :] and T[i, j + 1, :]. The end slopes are read only for inputs
// outside [lo, hi]. Tables are float32, int8 or int16 (in, size, out).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kf_abi.h"

namespace {

using namespace kfabi;

// V consecutive outputs of one table row as floats (one 16-byte load when V * sizeof(TT) == 16)
template <typename TT, int V>
__device__ __forceinline__ void load_run(const TT* p, float (&v)[V]) {
  if constexpr (V * sizeof(TT) == 16) {
    const uint4 r = *reinterpret_cast<const uint4*>(p);
    const TT* e = reinterpret_cast<const TT*>(&r);
#pragma unroll
    for (int q = 0; q < V; ++q) v[q] = (float)e[q];
  } else {
#pragma unroll
    for (int q = 0; q < V; ++q) v[q] = (float)p[q];
  }
}

// lane = (row r = lane / OW, output run oq = lane % OW) of V outputs o = (blockIdx.y OW + oq) V ..
template <typename TT, int OW, int V>
__global__ __launch_bounds__(256) void lut_kernel(int B, int IN, int S, int OUT, const float* __restrict__ x,
                                                  const TT* __restrict__ tab, const float* __restrict__ lo,
                                                  const float* __restrict__ inv_step, const float* __restrict__ bias,
                                                  const float* __restrict__ scale, const float* __restrict__ slo,
                                                  const float* __restrict__ shi, float* __restrict__ y) {
  constexpr int R = 64 / OW;
  const int lane = threadIdx.x & 63;
  const long wave = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const long b = wave * R + lane / OW;
  const int o = (blockIdx.y * OW + lane % OW) * V;
  if (b >= B || o >= OUT) return;  // no cross-lane work follows; OUT % V == 0 when V > 1
  const float top = (float)(S - 1);
  const size_t so = (size_t)S * OUT;
  const float* xr = x + (size_t)b * IN;
  float acc[V], ext[V];
#pragma unroll
  for (int q = 0; q < V; ++q) acc[q] = ext[q] = 0.f;
#pragma unroll 4
  for (int i = 0; i < IN; ++i) {
    const float t = (xr[i] - lo[i]) * inv_step[i];
    const float tc = fminf(fmaxf(t, 0.f), top);
    const float jf = fminf(floorf(tc), top - 1.f);
    const float f = tc - jf;
    const TT* row = tab + i * so + (size_t)(int)jf * OUT + o;
    float t0[V], t1[V];
    load_run<TT, V>(row, t0);
    load_run<TT, V>(row + OUT, t1);
#pragma unroll
    for (int q = 0; q < V; ++q) acc[q] += fmaf(f, t1[q] - t0[q], t0[q]);
    if (slo && (t < 0.f || t > top)) {
      const float below = fminf(t, 0.f), above = fmaxf(t - top, 0.f);
#pragma unroll
      for (int q = 0; q < V; ++q)
        ext[q] += below * slo[(size_t)i * OUT + o + q] + above * shi[(size_t)i * OUT + o + q];
    }
  }
#pragma unroll
  for (int q = 0; q < V; ++q)
    y[(size_t)b * OUT + o + q] = (scale ? acc[q] * scale[o + q] : acc[q]) + bias[o + q] + ext[q];
}

template <typename TT, int OW, int V>
void launch_lut_ow(int64_t B, int64_t IN, int64_t S, int64_t OUT, const float* x, const void* tab, const float* lo,
                   const float* inv_step, const float* bias, const float* scale, const float* slo, const float* shi,
                   float* y, hipStream_t s) {
  constexpr int R = 64 / OW;
  const int64_t waves = (B + R - 1) / R;
  const dim3 grid((unsigned)((waves + 3) / 4), (unsigned)((OUT + OW * V - 1) / (OW * V)));
  hipLaunchKernelGGL((lut_kernel<TT, OW, V>), grid, dim3(256), 0, s, (int)B, (int)IN, (int)S, (int)OUT, x,
                     (const TT*)tab, lo, inv_step, bias, scale, slo, shi, y);
}

// OW = lanes per row: the power of two covering the row's output runs, at most 64
template <typename TT, int V>
void launch_lut_v(int64_t B, int64_t IN, int64_t S, int64_t OUT, const float* x, const void* tab, const float* lo,
                  const float* inv_step, const float* bias, const float* scale, const float* slo, const float* shi,
                  float* y, hipStream_t s) {
  const int64_t runs = (OUT + V - 1) / V;
  if (runs <= 1) launch_lut_ow<TT, 1, V>(B, IN, S, OUT, x, tab, lo, inv_step, bias, scale, slo, shi, y, s);
  else if (runs <= 2) launch_lut_ow<TT, 2, V>(B, IN, S, OUT, x, tab, lo, inv_step, bias, scale, slo, shi, y, s);
  else if (runs <= 4) launch_lut_ow<TT, 4, V>(B, IN, S, OUT, x, tab, lo, inv_step, bias, scale, slo, shi, y, s);
  else if (runs <= 8) launch_lut_ow<TT, 8, V>(B, IN, S, OUT, x, tab, lo, inv_step, bias, scale, slo, shi, y, s);
  else if (runs <= 16) launch_lut_ow<TT, 16, V>(B, IN, S, OUT, x, tab, lo, inv_step, bias, scale, slo, shi, y, s);
  else if (runs <= 32) launch_lut_ow<TT, 32, V>(B, IN, S, OUT, x, tab, lo, inv_step, bias, scale, slo, shi, y, s);
  else launch_lut_ow<TT, 64, V>(B, IN, S, OUT, x, tab, lo, inv_step, bias, scale, slo, shi, y, s);
}

// 16-byte runs of outputs when the rows allow them (n_out a multiple of the run, tables 16-byte
// aligned), else one output per lane
template <typename TT>
int launch_lut(int64_t B, int64_t IN, int64_t S, int64_t OUT, const float* x, const void* tab, const float* lo,
               const float* inv_step, const float* bias, const float* scale, const float* slo, const float* shi,
               float* y, hipStream_t s) {
  constexpr int V = 16 / sizeof(TT);
  if (OUT % V == 0 && (reinterpret_cast<uintptr_t>(tab) & 15) == 0)
    launch_lut_v<TT, V>(B, IN, S, OUT, x, tab, lo, inv_step, bias, scale, slo, shi, y, s);
  else
    launch_lut_v<TT, 1>(B, IN, S, OUT, x, tab, lo, inv_step, bias, scale, slo, shi, y, s);
  return check_launch("LUT");
}

}  // namespace

extern "C" int kf_lut_forward(int table_dtype, int64_t batch, int64_t n_in, int64_t size, int64_t n_out, const float* x,
                              const void* tables, const float* lo, const float* inv_step, const float* bias,
                              const float* scale, const float* slope_lo, const float* slope_hi, float* y,
                              void* stream) {
  g_err.clear();
  if (batch < 0 || n_in < 0 || n_out < 0) return fail(KF_EINVAL, "kf_lut_forward: negative shape");
  if (size < 2) return fail(KF_EINVAL, "kf_lut_forward: tables need at least 2 points (size %lld)", (long long)size);
  if (batch == 0 || n_out == 0) return KF_OK;
  if (batch > INT32_MAX || n_in > INT32_MAX || n_out > INT32_MAX || size > INT32_MAX)
    return fail(KF_EINVAL, "kf_lut_forward: shape too large");
  if (!x || !tables || !lo || !inv_step || !bias || !y) return fail(KF_EINVAL, "kf_lut_forward: NULL array");
  if ((slope_lo == nullptr) != (slope_hi == nullptr))
    return fail(KF_EINVAL, "kf_lut_forward: slope_lo and slope_hi are given together or not at all");
  const bool quant = table_dtype == KF_I8 || table_dtype == KF_I16;
  if (quant != (scale != nullptr))
    return fail(KF_EINVAL, "kf_lut_forward: integer tables need a scale, float tables take none");
  hipStream_t s = (hipStream_t)stream;
  switch (table_dtype) {
    case KF_F32: return launch_lut<float>(batch, n_in, size, n_out, x, tables, lo, inv_step, bias, scale, slope_lo, slope_hi, y, s);
    case KF_I8: return launch_lut<int8_t>(batch, n_in, size, n_out, x, tables, lo, inv_step, bias, scale, slope_lo, slope_hi, y, s);
    case KF_I16: return launch_lut<int16_t>(batch, n_in, size, n_out, x, tables, lo, inv_step, bias, scale, slope_lo, slope_hi, y, s);
    default: return fail(KF_EUNSUPPORTED, "kf_lut_forward: table dtype %d is not float32, int8 or int16", table_dtype);
  }
}
