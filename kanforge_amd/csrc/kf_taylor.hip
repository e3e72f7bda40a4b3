// Second-order Taylor terms of the SiLU base branch for the forward-mode Laplacian of a KAN chain
// (what reverse-over-reverse autograd computes through kanforge/torch/science.py:25-46 and the
// base branch of kanforge/torch/layers.py:183-184). For a layer input h (B, n) with first
// derivatives hp (D, B, n) along the D input dimensions and second-derivative sum S (B, n):
//   sq            = sum_d hp_d^2
//   A[0:B]        = silu(h)
//   A[B + d B ..] = silu'(h) hp_d                          (d < D)
//   A[(D+1) B ..] = silu''(h) sq + silu'(h) S               (S may be NULL: zero)
// so the base branch of (h, h', S) is one GEMM A W^T. One thread per (row, input) element,
// every output coalesced along the inputs.
#include <hip/hip_runtime.h>

#include "kf_abi.h"

namespace {

using namespace kfabi;

template <typename T>
__global__ __launch_bounds__(256) void silu_taylor_kernel(int D, long BN, const T* __restrict__ h,
                                                          const T* __restrict__ hp, const T* __restrict__ S,
                                                          T* __restrict__ A, T* __restrict__ sq) {
  for (long e = blockIdx.x * 256L + threadIdx.x; e < BN; e += (long)gridDim.x * 256) {
    const float x = to_f32(h[e]);
    const float s = 1.f / (1.f + __expf(-x));
    const float d1 = s * (1.f + x * (1.f - s));
    const float d2 = s * (1.f - s) * (2.f + x * (1.f - 2.f * s));
    float q = 0.f;
    A[e] = from_f32<T>(x * s);
    for (int d = 0; d < D; ++d) {
      const float v = to_f32(hp[(size_t)d * BN + e]);
      q = fmaf(v, v, q);
      A[(size_t)(d + 1) * BN + e] = from_f32<T>(d1 * v);
    }
    const float sv = S ? to_f32(S[e]) : 0.f;
    A[(size_t)(D + 1) * BN + e] = from_f32<T>(fmaf(d2, q, d1 * sv));
    sq[e] = from_f32<T>(q);
  }
}

}  // namespace

extern "C" int kf_silu_taylor(int dtype, int64_t D, int64_t batch, int64_t n, const void* h, const void* hp,
                              const void* S, void* A, void* sq, void* stream) {
  g_err.clear();
  if (D < 0 || batch < 0 || n < 0) return fail(KF_EINVAL, "kf_silu_taylor: negative shape");
  const long BN = (long)(batch * n);
  if (BN == 0) return KF_OK;
  if (!h || !A || !sq || (D > 0 && !hp)) return fail(KF_EINVAL, "kf_silu_taylor: NULL array");
  long blocks = (BN + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == KF_BF16)
    hipLaunchKernelGGL(silu_taylor_kernel<bf16>, dim3((unsigned)blocks), dim3(256), 0, s, (int)D, BN, (const bf16*)h,
                       (const bf16*)hp, (const bf16*)S, (bf16*)A, (bf16*)sq);
  else if (dtype == KF_F32)
    hipLaunchKernelGGL(silu_taylor_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, s, (int)D, BN, (const float*)h,
                       (const float*)hp, (const float*)S, (float*)A, (float*)sq);
  else
    return fail(KF_EUNSUPPORTED, "kf_silu_taylor: dtype %d", dtype);
  return check_launch("silu taylor");
}
