// Column sums out[n] = sum_b g[b, n]: the bias gradient of y + bias (what autograd computes for
// the bias add of kanforge/torch/layers.py:189-190). Slabs of rows are summed per run of 8 columns
// into float32 partials (16-byte row loads, 8 row lanes per workgroup), then the slabs
// (deterministic: fixed lane and slab order).
#include <hip/hip_runtime.h>

#include "kf_abi.h"
#include "kf_rational.h"

namespace {

using namespace kfabi;

// Stage 1: workgroup = 32 runs of V columns (V = 8 with 16-byte row loads, else 1) x 8 row
// lanes over a slab of rows; the row lanes meet in LDS and part[slab][column] is written.
template <typename T, int V>
__global__ __launch_bounds__(256) void colsum_partial(int rows, int n, int rs, const T* __restrict__ g,
                                                      float* __restrict__ part) {
  __shared__ float red[8][32][V + 1];
  const int run = threadIdx.x & 31, rl = threadIdx.x >> 5;
  const int slab = blockIdx.y, r0 = slab * rs, r1 = min(rows, r0 + rs);
  const int c = (blockIdx.x * 32 + run) * V;
  float s[V];
#pragma unroll
  for (int q = 0; q < V; ++q) s[q] = 0.f;
  if (c < n) {
#pragma unroll 4
    for (int r = r0 + rl; r < r1; r += 8) {
      if constexpr (V == 8) {
        float v[8];
        load8<T>(g + (size_t)r * n + c, v);
#pragma unroll
        for (int q = 0; q < 8; ++q) s[q] += v[q];
      } else {
        s[0] += to_f32(g[(size_t)r * n + c]);
      }
    }
  }
#pragma unroll
  for (int q = 0; q < V; ++q) red[rl][run][q] = s[q];
  __syncthreads();
  if (rl == 0 && c < n) {
#pragma unroll
    for (int q = 0; q < V; ++q) {
      float t = 0.f;
#pragma unroll
      for (int l = 0; l < 8; ++l) t += red[l][run][q];
      part[(size_t)slab * n + c + q] = t;
    }
  }
}

// Stage 2: 64 columns x 4 slab lanes per workgroup, the lanes meet in LDS (fixed order).
template <typename T>
__global__ __launch_bounds__(256) void colsum_final(int n, int slabs, const float* __restrict__ part, T* __restrict__ out) {
  __shared__ float red[4][64];
  const int cl = threadIdx.x & 63, j = threadIdx.x >> 6, c = blockIdx.x * 64 + cl;
  float s = 0.f;
  if (c < n) {
#pragma unroll 4
    for (int z = j; z < slabs; z += 4) s += part[(size_t)z * n + c];
  }
  red[j][cl] = s;
  __syncthreads();
  if (j == 0 && c < n) out[c] = from_f32<T>(red[0][cl] + red[1][cl] + red[2][cl] + red[3][cl]);
}

struct Slabs {
  int gx, slabs, rs;
};
// about 512 workgroups in stage 1, slabs of at least 64 rows
Slabs plan_slabs(int64_t rows, int64_t n, bool vec) {
  Slabs p;
  p.gx = (int)(((vec ? (n + 7) / 8 : n) + 31) / 32);
  long slabs = (512 + p.gx - 1) / p.gx;
  const long most = (rows + 63) / 64;
  if (slabs > most) slabs = most;
  if (slabs < 1) slabs = 1;
  p.rs = (int)((rows + slabs - 1) / slabs);
  p.slabs = (int)((rows + p.rs - 1) / p.rs);
  return p;
}

template <typename T>
int run_colsum(int64_t rows, int64_t n, const void* g, void* out, void* ws, hipStream_t s) {
  const bool vec = n % 8 == 0 && aligned16(g);
  const Slabs p = plan_slabs(rows, n, vec);
  if (vec)
    hipLaunchKernelGGL((colsum_partial<T, 8>), dim3((unsigned)p.gx, (unsigned)p.slabs), dim3(256), 0, s, (int)rows,
                       (int)n, p.rs, (const T*)g, (float*)ws);
  else
    hipLaunchKernelGGL((colsum_partial<T, 1>), dim3((unsigned)p.gx, (unsigned)p.slabs), dim3(256), 0, s, (int)rows,
                       (int)n, p.rs, (const T*)g, (float*)ws);
  int rc = check_launch("column sums");
  if (rc) return rc;
  hipLaunchKernelGGL(colsum_final<T>, dim3((unsigned)((n + 63) / 64)), dim3(256), 0, s, (int)n, p.slabs,
                     (const float*)ws, (T*)out);
  return check_launch("column sums final");
}

}  // namespace

extern "C" {

size_t kf_column_sums_workspace_bytes(int64_t rows, int64_t n) {
  if (rows <= 0 || n <= 0) return 0;
  const Slabs p = plan_slabs(rows, n, n % 8 == 0);
  const Slabs q = plan_slabs(rows, n, false);
  const int slabs = p.slabs > q.slabs ? p.slabs : q.slabs;
  return align256((size_t)slabs * n * sizeof(float));
}

int kf_column_sums(int dtype, int64_t rows, int64_t n, const void* g, void* out, void* workspace,
                   size_t workspace_bytes, void* stream) {
  g_err.clear();
  if (rows < 0 || n < 0) return fail(KF_EINVAL, "kf_column_sums: negative shape");
  if (rows > INT32_MAX || n > INT32_MAX) return fail(KF_EINVAL, "kf_column_sums: shape too large");
  if (dtype != KF_F32 && dtype != KF_BF16) return fail(KF_EUNSUPPORTED, "kf_column_sums: dtype %d", dtype);
  if (n == 0) return KF_OK;
  if (!out) return fail(KF_EINVAL, "kf_column_sums: NULL output");
  hipStream_t s = (hipStream_t)stream;
  if (rows == 0) return dtype == KF_BF16 ? zero_fill<bf16>(out, (long)n, s) : zero_fill<float>(out, (long)n, s);
  if (!g) return fail(KF_EINVAL, "kf_column_sums: NULL array");
  const size_t need = kf_column_sums_workspace_bytes(rows, n);
  if (!workspace || workspace_bytes < need)
    return fail(KF_EWORKSPACE, "kf_column_sums: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  if (dtype == KF_BF16) return run_colsum<bf16>(rows, n, g, out, workspace, s);
  return run_colsum<float>(rows, n, g, out, workspace, s);
}

}  // extern "C"
