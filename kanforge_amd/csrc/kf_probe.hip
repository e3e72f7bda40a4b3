// Sustained bf16 MFMA rate of the card (kf_probe_mfma in include/kfhip.h): the ceiling against
// which the contraction kernels' rates are read. Every wave runs back-to-back
// v_mfma_f32_32x32x16_bf16 on four independent accumulators, with operands taken in rotation
// from eight register sets filled with pseudo-random bf16 values (changing operands, as in a
// real contraction, draw more power than a loop on fixed registers and so lower the clock).
// Each workgroup also records the shader-clock cycles and the 100 MHz real-time ticks its first
// wave spent, from which the host reads the clock the probe ran at.
#include <cstdint>

#include "kf_device.h"
#include "kfhip.h"

namespace {

using kf::bf16;
using kf::bf16x8;
typedef float f32x16p __attribute__((ext_vector_type(16)));
constexpr int kSets = 8;

__device__ inline uint32_t mix(uint32_t v) {
  v ^= v >> 16;
  v *= 0x7feb352du;
  v ^= v >> 15;
  v *= 0x846ca68bu;
  v ^= v >> 16;
  return v;
}

template <bool ROTATE>
__global__ __launch_bounds__(256) void mfma_probe_kernel(int iters, float* __restrict__ out) {
  const uint32_t tid = blockIdx.x * 256u + threadIdx.x;
  bf16x8 a[kSets], b[kSets];
#pragma unroll
  for (int s = 0; s < kSets; ++s)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      // bf16 bit patterns with exponents near 1.0 and random mantissas and signs
      const uint32_t r = mix(tid * 131u + s * 17u + e);
      const uint16_t pa = (uint16_t)(0x3f00u | (r & 0x80ffu)), pb = (uint16_t)(0x3f00u | ((r >> 16) & 0x80ffu));
      a[s][e] = __builtin_bit_cast(bf16, pa);
      b[s][e] = __builtin_bit_cast(bf16, pb);
    }
  f32x16p acc0 = {}, acc1 = {}, acc2 = {}, acc3 = {};
  const uint64_t c0 = __builtin_readcyclecounter();
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int s = 0; s < kSets; s += 4) {
      const int s1 = ROTATE ? s + 1 : 0, s2 = ROTATE ? s + 2 : 0, s3 = ROTATE ? s + 3 : 0, s0 = ROTATE ? s : 0;
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[s0], b[s1], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[s1], b[s2], acc1, 0, 0, 0);
      acc2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[s2], b[s3], acc2, 0, 0, 0);
      acc3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[s3], b[s0], acc3, 0, 0, 0);
    }
  }
  const uint64_t c1 = __builtin_readcyclecounter();
  const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
  float sum = 0.f;
#pragma unroll
  for (int q = 0; q < 16; ++q) sum += acc0[q] + acc1[q] + acc2[q] + acc3[q];
  // one vector store per lane: the checksum keeps the MFMAs live; lane 0 of the block also
  // stores the timing of its wave
  float* o = out + (size_t)blockIdx.x * 256 * 3;
  o[threadIdx.x * 3 + 0] = sum;
  o[threadIdx.x * 3 + 1] = threadIdx.x == 0 ? (float)(c1 - c0) : 0.f;
  o[threadIdx.x * 3 + 2] = threadIdx.x == 0 ? (float)(t1 - t0) : 0.f;
}

}  // namespace

extern "C" int kf_probe_mfma(int blocks, int iters, int rotate, float* out, void* stream) {
  if (blocks < 1 || iters < 1 || !out) return KF_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  if (rotate)
    hipLaunchKernelGGL(mfma_probe_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, s, iters, out);
  else
    hipLaunchKernelGGL(mfma_probe_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, s, iters, out);
  return hipGetLastError() == hipSuccess ? KF_OK : KF_ELAUNCH;
}
