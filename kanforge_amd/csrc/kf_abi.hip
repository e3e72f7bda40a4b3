// extern "C" entry points of libkfhip.so (declared in include/kfhip.h) other than F, G and P:
// the library's error state, workspace sizing, basis features, edge derivatives, interval
// search and the rational parameter gradients. kf_abi_f.hip, kf_abi_g.hip and kf_abi_p.hip hold
// the three contractions.
#include "kf_abi.h"
#include "kf_rational.h"

using namespace kfabi;

namespace kfabi {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

constexpr int kLdsCeiling = 160 * 1024;
std::mutex g_lds_mutex;
std::set<std::pair<int, const void*>> g_lds_raised;

bool reserve_lds(const void* kern, size_t lds) {
  if (lds <= 65536) return true;
  if (lds > (size_t)kLdsCeiling) return false;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  std::lock_guard<std::mutex> lock(g_lds_mutex);
  if (g_lds_raised.count({dev, kern})) return true;
  if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsCeiling) != hipSuccess) return false;
  g_lds_raised.insert({dev, kern});
  return true;
}

}  // namespace kfabi

namespace {

template <typename T, int KM>
void launch_edge_t(const KBasis& kb, int64_t batch, int64_t n_in, int64_t n_out, const void* x, const void* c,
                   const void* bw, void* out, hipStream_t s) {
  if constexpr (sizeof(T) == 4) {
    // wide float32 layers: 16-byte stores of 4 consecutive inputs
    if (n_in >= 32 && n_in % 4 == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0) {
      dim3 grid((unsigned)((n_in + 31) / 32), (unsigned)((batch + 31) / 32));
      hipLaunchKernelGGL((edge4_kernel<KM>), grid, dim3(kThreads), 0, s, kb, (int)batch, (int)n_in, (int)n_out,
                         (const float*)x, (const float*)c, (const float*)bw, (float*)out);
      return;
    }
  }
  constexpr int ROWS = KM <= 8 ? 32 : 16;  // edge_kernel's block: ROWS rows x IW inputs
  int iw = 32;
  while (iw / 2 >= n_in && iw > 1) iw /= 2;  // narrow layers: the power of two >= n_in
  dim3 grid((unsigned)((n_in + iw - 1) / iw), (unsigned)((batch + ROWS - 1) / ROWS));
  hipLaunchKernelGGL((edge_kernel<T, KM>), grid, dim3(kThreads), 0, s, kb, (int)batch, (int)n_in, (int)n_out, iw,
                     (const T*)x, (const T*)c, (const T*)bw, (T*)out);
}

template <typename T>
int run_edge(const KBasis& kb, int64_t batch, int64_t n_in, int64_t n_out, const void* x, const void* c,
             const void* bw, void* out, hipStream_t s) {
  switch (nt_bucket(kb.K)) {
    case 4: launch_edge_t<T, 4>(kb, batch, n_in, n_out, x, c, bw, out, s); break;
    case 8: launch_edge_t<T, 8>(kb, batch, n_in, n_out, x, c, bw, out, s); break;
    case 12: launch_edge_t<T, 12>(kb, batch, n_in, n_out, x, c, bw, out, s); break;
    default: launch_edge_t<T, 16>(kb, batch, n_in, n_out, x, c, bw, out, s); break;
  }
  return check_launch("edge_derivative");
}

}  // namespace

extern "C" {

const char* kf_last_error(void) { return g_err.c_str(); }

const char* kf_version(void) { return "kfhip 0.1.0 gfx950"; }

size_t kf_workspace_bytes(int op, const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out) {
  if (validate_common(b, dtype, batch, n_in, n_out)) return 0;
  switch (op) {
    case KF_OP_F: {  // weighted or not (the unweighted register-A layout differs)
      const size_t a = ws_f(b, dtype, batch, n_in, n_out, true).total, u = ws_f(b, dtype, batch, n_in, n_out, false).total;
      return a > u ? a : u;
    }
    case KF_OP_P: return ws_p(b, dtype, batch, n_in, n_out).total;
    case KF_OP_G: {  // weighted or not (unweighted Chebyshev plans take T_0 out)
      const size_t a = ws_g(b, dtype, batch, n_in, n_out, true).total, u = ws_g(b, dtype, batch, n_in, n_out, false).total;
      return a > u ? a : u;
    }
    case KF_OP_G_BIAS: {
      const size_t a = ws_g_bias(b, dtype, batch, n_in, n_out, true).total, u = ws_g_bias(b, dtype, batch, n_in, n_out, false).total;
      return a > u ? a : u;
    }
    case KF_OP_F_BASE:
      if (!f_base_route(b, dtype, batch, n_in, n_out)) return 0;
      if (bspline_sparse(b, dtype)) return ws_base_sparse(op, b, dtype, batch, n_in, n_out);
      return b->kind == KF_KIND_BSPLINE ? ws_f_base_bspline(b, dtype, batch, n_in, n_out).total
                                        : ws_f(b, dtype, batch, n_in, n_out, false, true).total;
    case KF_OP_P_BASE:
      if (!p_base_route(b, dtype, batch, n_in, n_out)) return 0;
      return bspline_sparse(b, dtype) ? ws_base_sparse(op, b, dtype, batch, n_in, n_out)
                                      : ws_p_base(b, dtype, batch, n_in, n_out).total;
    case KF_OP_G_BASE:
      if (!g_base_route(b, dtype, batch, n_in, n_out)) return 0;
      return bspline_sparse(b, dtype) ? ws_base_sparse(op, b, dtype, batch, n_in, n_out)
                                      : ws_g_base(b, dtype, batch, n_in, n_out).total;
    default: return 0;
  }
}

int kf_base_fused(int op, const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out) {
  g_err.clear();
  int rc = validate_common(b, dtype, batch, n_in, n_out);
  if (rc) return rc;
  if (batch <= 0 || n_in <= 0 || n_out <= 0) return 0;
  switch (op) {
    case KF_OP_F_BASE: return f_base_route(b, dtype, batch, n_in, n_out) ? 1 : 0;
    case KF_OP_P_BASE: return p_base_route(b, dtype, batch, n_in, n_out) ? 1 : 0;
    case KF_OP_G_BASE: return g_base_route(b, dtype, batch, n_in, n_out) ? 1 : 0;
    default: return fail(KF_EINVAL, "kf_base_fused: op %d is not one of KF_OP_F_BASE, KF_OP_P_BASE, KF_OP_G_BASE", op);
  }
}

int kf_features(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, const void* x, void* out, void* stream) {
  g_err.clear();
  int rc = validate_common(b, dtype, batch, n_in, 0);
  if (rc) return rc;
  if (batch == 0 || n_in == 0) return KF_OK;
  if (!x || !out) return fail(KF_EINVAL, "kf_features: NULL array");
  KBasis kb = to_kbasis(b);
  hipStream_t s = (hipStream_t)stream;
  const long K = b->size;
  if (dtype == KF_BF16)
    return launch_features<bf16, true>(kb, batch, n_in, batch, n_in, x, out, (long)n_in * K, 1L, K, false, s);
  return launch_features<float, true>(kb, batch, n_in, batch, n_in, x, out, (long)n_in * K, 1L, K, false, s);
}

int kf_edge_derivative(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void* x,
                       const void* c, const void* base_w, void* out, void* stream) {
  g_err.clear();
  int rc = validate_common(b, dtype, batch, n_in, n_out);
  if (rc) return rc;
  if (batch == 0 || n_in == 0 || n_out == 0) return KF_OK;
  if (!x || !c || !out) return fail(KF_EINVAL, "kf_edge_derivative: NULL array");
  KBasis kb = to_kbasis(b);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == KF_BF16) return run_edge<bf16>(kb, batch, n_in, n_out, x, c, base_w, out, s);
  return run_edge<float>(kb, batch, n_in, n_out, x, c, base_w, out, s);
}

int kf_bspline_interval(int64_t batch, int64_t n_in, const float* x, const float* knots_cmp, int32_t n_knots,
                        int32_t* idx, void* stream) {
  g_err.clear();
  if (batch < 0 || n_in < 0) return fail(KF_EINVAL, "negative dimension");
  if (n_knots < 2) return fail(KF_EINVAL, "need at least 2 knots");
  if (batch == 0 || n_in == 0) return KF_OK;
  if (!x || !knots_cmp || !idx) return fail(KF_EINVAL, "kf_bspline_interval: NULL array");
  long n = (long)batch * n_in;
  long blocks = (n + kThreads - 1) / kThreads;
  if (blocks > 65535 * 4) blocks = 65535 * 4;
  hipLaunchKernelGGL(interval_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, (hipStream_t)stream, n, (int)n_in, x,
                     knots_cmp, n_knots, idx);
  return check_launch("bspline_interval");
}

size_t kf_rational_workspace_bytes(const kf_basis* b, int64_t batch, int64_t n_in) {
  if (!b || b->kind != KF_KIND_RATIONAL || b->group_size < 1) return 0;
  const int64_t groups = n_in / b->group_size;
  const int64_t chunks = (batch + kRatRows - 1) / kRatRows;
  return align256((size_t)chunks * groups * (b->num_deg + 1 + b->den_deg) * sizeof(float));
}

int kf_rational_param_grad(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, const void* x, const float* h,
                           const void* w, float* dnum, float* dden, void* workspace, size_t workspace_bytes,
                           void* stream) {
  g_err.clear();
  int rc = validate_common(b, dtype, batch, n_in, 0);
  if (rc) return rc;
  if (b->kind != KF_KIND_RATIONAL) return fail(KF_EINVAL, "kf_rational_param_grad needs the rational kind");
  if (!dnum || !dden) return fail(KF_EINVAL, "kf_rational_param_grad: NULL output");
  hipStream_t s = (hipStream_t)stream;
  const int groups = (int)(n_in / b->group_size);
  const int nP = b->num_deg + 1, nQ = b->den_deg;
  if (batch == 0 || n_in == 0) {
    rc = zero_fill<float>(dnum, (long)groups * nP, s);
    if (rc == KF_OK) rc = zero_fill<float>(dden, (long)groups * nQ, s);
    return rc;
  }
  if (!x || !h) return fail(KF_EINVAL, "kf_rational_param_grad: NULL array");
  size_t need = kf_rational_workspace_bytes(b, batch, n_in);
  if (!workspace || workspace_bytes < need)
    return fail(KF_EWORKSPACE, "kf_rational_param_grad: workspace of %zu bytes needed, %zu given", need,
                workspace_bytes);
  KBasis kb = to_kbasis(b);
  const int chunks = (int)((batch + kRatRows - 1) / kRatRows);
  dim3 grid((unsigned)groups, (unsigned)chunks);
  if (b->order > 0) {  // gradients of the derivative features: GR-KAN degrees, orders 1..3
    if (b->num_deg != 5 || b->den_deg != 4 || b->order > 3)
      return fail(KF_EUNSUPPORTED, "kf_rational_param_grad: order %d needs P 5 / Q 4 and order <= 3", b->order);
    auto go = [&](auto tag) {
      constexpr int M = decltype(tag)::value;
      if (dtype == KF_BF16)
        hipLaunchKernelGGL((rational_grad_order<bf16, M, kRatRows>), grid, dim3(256), 0, s, kb, (int)batch,
                           (int)n_in, (const bf16*)x, h, (const bf16*)w, (float*)workspace);
      else
        hipLaunchKernelGGL((rational_grad_order<float, M, kRatRows>), grid, dim3(256), 0, s, kb, (int)batch,
                           (int)n_in, (const float*)x, h, (const float*)w, (float*)workspace);
      return check_launch("rational_grad_order");
    };
    rc = b->order == 1 ? go(std::integral_constant<int, 1>{})
                       : b->order == 2 ? go(std::integral_constant<int, 2>{}) : go(std::integral_constant<int, 3>{});
    if (rc) return rc;
    hipLaunchKernelGGL(rational_grad_final, dim3(1), dim3(256), 0, s, groups, nP, nQ, chunks,
                       (const float*)workspace, dnum, dden);
    return check_launch("rational_grad_final");
  }
  const bool fast = rational_fast(kb, n_in) && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(h) & 15) == 0 && (!w || (reinterpret_cast<uintptr_t>(w) & 15) == 0);
  if (fast && dtype == KF_BF16)
    hipLaunchKernelGGL((rational_grad_fast<bf16, kRatRows>), grid, dim3(256), 0, s, kb, (int)batch, (int)n_in,
                       (const bf16*)x, h, (const bf16*)w, (float*)workspace);
  else if (fast)
    hipLaunchKernelGGL((rational_grad_fast<float, kRatRows>), grid, dim3(256), 0, s, kb, (int)batch, (int)n_in,
                       (const float*)x, h, (const float*)w, (float*)workspace);
  else if (dtype == KF_BF16)
    hipLaunchKernelGGL(rational_grad_partial<bf16>, grid, dim3(kThreads), 0, s, kb, (int)batch, (int)n_in,
                       (const bf16*)x, h, (const bf16*)w, (float*)workspace);
  else
    hipLaunchKernelGGL(rational_grad_partial<float>, grid, dim3(kThreads), 0, s, kb, (int)batch, (int)n_in,
                       (const float*)x, h, (const float*)w, (float*)workspace);
  rc = check_launch("rational_grad_partial");
  if (rc) return rc;
  hipLaunchKernelGGL(rational_grad_final, dim3(1), dim3(256), 0, s, groups, nP, nQ, chunks,
                     (const float*)workspace, dnum, dden);
  return check_launch("rational_grad_final");
}

}  // extern "C"
