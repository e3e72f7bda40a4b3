// kf_P (include/kfhip.h): the input-gradient contraction's launch configurations, workspace
// carving and dispatch.
#include "kf_abi.h"
#include "kf_rational.h"

using namespace kfabi;

namespace {

template <typename T, int WMW, int WJW, int TM, int FW, int KIND>
int launch_p_kind(const WsP& L, hipStream_t s, const KBasis& kb, int64_t batch, int64_t n_in, int64_t n_out,
                  const void* x, const void* g, const void* cfmt, void* p, float* h) {
  constexpr int BM = WMW * TM * 32, NMAX = WJW * FW * 32, RS = 64 + 16;
  const size_t lds_ops = (size_t)2 * (BM + NMAX) * RS, lds_red = (size_t)WJW * BM * 33 * 4;
  const size_t lds = lds_ops > lds_red ? lds_ops : lds_red;
  auto kern = p_kernel<T, WMW, WJW, TM, FW, KIND>;
  if (!reserve_lds((const void*)kern, lds))
    return fail(KF_ELAUNCH, "P: cannot reserve %zu bytes of LDS", lds);
  const int n_m = (int)((batch + BM - 1) / BM), n_n = (int)(L.INP / 32);
  hipLaunchKernelGGL(kern, dim3(n_m * n_n), dim3(WMW * WJW * 64), lds, s, kb, (int)batch, (int)n_in, (int)n_out,
                     (int)L.INP, (int)L.OUTP, (const T*)x, (const T*)g, (const T*)cfmt, (T*)p, h);
  return check_launch("P");
}

template <typename T, int WMW, int WJW, int TM, int FW>
int launch_p_t(const WsP& L, hipStream_t s, const KBasis& kb, int64_t batch, int64_t n_in, int64_t n_out,
               const void* x, const void* g, const void* cfmt, void* p, float* h) {
  switch (kb.kind) {
    case KF_KIND_CHEB:
      return launch_p_kind<T, WMW, WJW, TM, FW, KF_KIND_CHEB>(L, s, kb, batch, n_in, n_out, x, g, cfmt, p, h);
    case KF_KIND_BSPLINE:
      return launch_p_kind<T, WMW, WJW, TM, FW, KF_KIND_BSPLINE>(L, s, kb, batch, n_in, n_out, x, g, cfmt, p, h);
    default:
      return launch_p_kind<T, WMW, WJW, TM, FW, KF_KIND_RATIONAL>(L, s, kb, batch, n_in, n_out, x, g, cfmt, p, h);
  }
}

template <typename T, int FW, int KIND>
int launch_p_dma_kind(const WsP& L, hipStream_t s, const KBasis& kb, int64_t batch, int64_t n_in, const void* x,
                      const void* g, int gstride, const void* cfmt, void* p, float* h) {
  constexpr int TM = p_dma_tm(FW), BM = 2 * TM * 32;
  const size_t knots = KIND == KF_KIND_BSPLINE ? (size_t)32 * (2 * kb.n_knots + 2 * kb.spline_k) * 4 : 0;
  size_t lds_epi = (size_t)3 * BM * 33 * 4 + knots;
  if (KIND == KF_KIND_BSPLINE) {  // x, knots, then the features of one pass or the group sums
    const size_t fb = (size_t)2 * FW * 64 * 33 * 4, red = (size_t)2 * BM * 33 * 4;
    lds_epi = (size_t)BM * 33 * 4 + knots + (fb > red ? fb : red);
  }
  const size_t lds_ops = (size_t)2 * (BM + 2 * FW * 32) * 128;
  const size_t lds = lds_ops > lds_epi ? lds_ops : lds_epi;
  auto kern = p_dma_kernel<T, TM, FW, KIND>;
  if (!reserve_lds((const void*)kern, lds))
    return fail(KF_ELAUNCH, "P: cannot reserve %zu bytes of LDS", lds);
  constexpr int TI = KIND == KF_KIND_RATIONAL ? 64 * FW : 32;  // inputs per tile (flat for rational)
  if (L.INP % TI) return fail(KF_EINVAL, "P: workspace layout not aligned");
  const int n_m = (int)((batch + BM - 1) / BM), n_n = (int)(L.INP / TI);
  hipLaunchKernelGGL(kern, dim3(n_m * n_n), dim3(256), lds, s, kb, (int)batch, (int)n_in, (int)L.INP, (int)L.OUTP,
                     (const T*)x, (const T*)g, gstride, (const T*)cfmt, (T*)p, h);
  return check_launch("P");
}

template <int KIND, int NF, int TN, int RB, bool BASE = false>
int launch_p8(const WsP& L, hipStream_t s, const KBasis& kb, int64_t batch, int64_t n_in, const void* x, const void* g,
              int gstride, const void* cfmt, void* p, const float* hb = nullptr) {
  constexpr int TI = 128 * TN / NF, RPASS = TN == 2 ? 128 : 64;
  // B-splines: the tile's knot rows and (t_0, 1/h) per input after the sums
  const size_t knots = KIND == KF_KIND_BSPLINE ? (size_t)TI * (2 * kb.n_knots + 2 * kb.spline_k + 2) * 4 : 0;
  const size_t lds_ops = (size_t)2 * (256 + NF * TI) * RB, lds_epi = (size_t)NF * RPASS * (TI + 1) * 4 + knots;
  const size_t lds = lds_ops > lds_epi ? lds_ops : lds_epi;
  // cubic B-splines on even knots (the common case): the support without the general-knot path
  const bool even = KIND == KF_KIND_BSPLINE && kb.knots_uniform && kb.n_knots >= 4;
  auto kern = even ? p8_kernel<KIND, NF, TN, RB, 3, true, BASE> : p8_kernel<KIND, NF, TN, RB, 3, false, BASE>;
  if (BASE && (KIND == KF_KIND_BSPLINE ? kb.K >= NF : !hb))
    return fail(KF_EINVAL, "P: the base term needs a spare feature slot (B-splines) or hb");
  if (L.INP % TI || L.OUTP % (RB / 2)) return fail(KF_EINVAL, "P: workspace layout not aligned");
  if (!reserve_lds((const void*)kern, lds))
    return fail(KF_ELAUNCH, "P: cannot reserve %zu bytes of LDS", lds);
  const int n_m = (int)((batch + 255) / 256), n_n = (int)(L.INP / TI);
  hipLaunchKernelGGL(kern, dim3(n_m * n_n), dim3(512), lds, s, kb, (int)batch, (int)n_in, (int)L.INP, (int)L.OUTP,
                     (const bf16*)x, (const bf16*)g, gstride, (const bf16*)cfmt, (bf16*)p, hb);
  return check_launch("P");
}

template <typename T, int FW>
int launch_p_dma(const WsP& L, hipStream_t s, const KBasis& kb, int64_t batch, int64_t n_in, const void* x,
                 const void* g, int gstride, const void* cfmt, void* p, float* h) {
  switch (kb.kind) {
    case KF_KIND_CHEB:
      return launch_p_dma_kind<T, FW, KF_KIND_CHEB>(L, s, kb, batch, n_in, x, g, gstride, cfmt, p, h);
    case KF_KIND_BSPLINE:
      return launch_p_dma_kind<T, FW, KF_KIND_BSPLINE>(L, s, kb, batch, n_in, x, g, gstride, cfmt, p, h);
    default:
      return launch_p_dma_kind<T, FW, KF_KIND_RATIONAL>(L, s, kb, batch, n_in, x, g, gstride, cfmt, p, h);
  }
}

template <typename T>
int run_P(const KBasis& kb, const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void* x,
          const void* g, const void* c, void* p, float* h, void* ws, hipStream_t s, bool h_only = false,
          bool h_bf16 = false) {
  if constexpr (sizeof(T) == 4)
    if (bspline_sparse(b, dtype)) return launch_p_sparse<T>(kb, b->spline_k, batch, n_in, n_out, x, g, c, p, s);
  WsP L = ws_p(b, dtype, batch, n_in, n_out);
  void* cfmt = ws;
  int rc = launch_permute<T>(kb, n_out, n_in, L.OUTP, L.INP, L.ntb, c, cfmt, kPermFMT, s);
  if (rc) return rc;
  if (p_uses_dma(L.cfg)) {
    const void* ga = g;
    int gstride = (int)n_out;
    if (p_needs_gpad(n_out, dtype) || (reinterpret_cast<uintptr_t>(g) & 15) != 0) {
      if (!L.gpad) return fail(KF_EINVAL, "P: g must be 16-byte aligned");
      void* gp = (char*)ws + L.cfmt;
      long n = (long)batch * L.OUTP;
      long blocks = (n + kThreads - 1) / kThreads;
      if (blocks > 65535 * 4) blocks = 65535 * 4;
      hipLaunchKernelGGL(pad_cols_kernel<T>, dim3((unsigned)blocks), dim3(kThreads), 0, s, (int)batch, (int)n_out,
                         (int)L.OUTP, (const T*)g, (T*)gp);
      rc = check_launch("pad_cols");
      if (rc) return rc;
      ga = gp;
      gstride = (int)L.OUTP;
    }
    if constexpr (sizeof(T) == 2) {
      // GR-KAN degrees in bf16: H = g C^T on the GEMM core (float32, into h when given), then
      // p = H phi^(m)(x)
      if (rational_fast(kb, n_in) && kb.order <= 2 && aligned16(x) && aligned16(p) && aligned16(ga) && gstride % 8 == 0) {
        float* hb = h ? h : (float*)((char*)ws + L.cfmt + L.gpad);
        void* gws = (char*)ws + L.cfmt + L.gpad + L.hbuf;
        // h_only: H alone, in bfloat16 when h_bf16 (the fused backward's operand)
        rc = gemm_nt(batch, n_in, L.OUTP, ga, gstride, cfmt, L.OUTP, hb, n_in, !(h_only && h_bf16), gws, L.gemm, s);
        if (rc || h_only) return rc;
        long blocks = ((long)batch * (n_in / 8) + 255) / 256;
        if (blocks > 65535 * 4) blocks = 65535 * 4;
        auto map = kb.order == 0   ? rational_map_kernel<bf16, bf16, 0>
                   : kb.order == 1 ? rational_map_kernel<bf16, bf16, 1>
                                   : rational_map_kernel<bf16, bf16, 2>;
        hipLaunchKernelGGL(map, dim3((unsigned)blocks), dim3(256), 0, s, kb, (int)batch, (int)n_in, (const bf16*)x,
                           (const bf16*)nullptr, (const float*)hb, (bf16*)p);
        return check_launch("rational dX");
      }
    }
    // 7 or 8 Chebyshev features in bf16: the two-waves-per-SIMD kernel
    if (L.p8 && !h) return launch_p8<KF_KIND_CHEB, 8, 3, 128>(L, s, kb, batch, n_in, x, ga, gstride, cfmt, p);
    // 9 to 12 B-spline features in bf16: the same kernel with 12 feature slots
    if (L.p12 && !h) return launch_p8<KF_KIND_BSPLINE, 12, 3, 128>(L, s, kb, batch, n_in, x, ga, gstride, cfmt, p);
    switch (L.cfg) {
      case 0: return launch_p_dma<T, 2>(L, s, kb, batch, n_in, x, ga, gstride, cfmt, p, h);
      case 1: return launch_p_dma<T, 3>(L, s, kb, batch, n_in, x, ga, gstride, cfmt, p, h);
      case 2: return launch_p_dma<T, 4>(L, s, kb, batch, n_in, x, ga, gstride, cfmt, p, h);
      case 3: return launch_p_dma<T, 5>(L, s, kb, batch, n_in, x, ga, gstride, cfmt, p, h);
      default: return launch_p_dma<T, 6>(L, s, kb, batch, n_in, x, ga, gstride, cfmt, p, h);
    }
  }
  switch (L.cfg) {
    case 3: return launch_p_t<T, 4, 2, 2, 5>(L, s, kb, batch, n_in, n_out, x, g, cfmt, p, h);
    case 4: return launch_p_t<T, 4, 2, 1, 6>(L, s, kb, batch, n_in, n_out, x, g, cfmt, p, h);
    case 5: return launch_p_t<T, 4, 2, 1, 8>(L, s, kb, batch, n_in, n_out, x, g, cfmt, p, h);
    default: return launch_p_t<T, 4, 2, 1, 12>(L, s, kb, batch, n_in, n_out, x, g, cfmt, p, h);
  }
}
constexpr int kRatBwdRows = 64;  // rows per chunk of the fused rational backward

// whether the fused order-0 rational backward applies (the bf16 GEMM route of run_P and the
// eight-input kernels)
bool rational_bwd_fuses(const KBasis& kb, int dtype, int64_t n_in, const void* x, const void* g, const void* w,
                        const void* p) {
  return dtype == KF_BF16 && kb.order == 0 && rational_fast(kb, n_in) && aligned16(x) && aligned16(p) &&
         (!w || aligned16(w)) && p_uses_dma(fw_index(1));
}
// The layer's input gradient with its SiLU base branch: the coefficients folded feature-major
// with W^T as one more row, hb = g W on the GEMM core (float32), then p8_kernel, whose epilogue
// adds silu'(x) hb; B-splines put W^T in the tile's last feature slot instead, so the same GEMM
// yields g W next to the feature sums.
int run_P_base(const KBasis& kb, const kf_basis* b1, int dtype, int64_t batch, int64_t n_in, int64_t n_out,
               const void* x, const void* g, const void* c, const void* bw, void* p, void* ws, hipStream_t s) {
  const WsPB LB = ws_p_base(b1, dtype, batch, n_in, n_out);
  const WsP& L = LB.p;
  char* base = (char*)ws;
  void* cfmt = base;
  float* hb = (float*)(base + LB.cfmt + L.gpad);
  void* gws = base + LB.cfmt + L.gpad + LB.hb;
  // B-splines: the folded features and zero rows up to the last slot, W^T in it; Chebyshev: W^T
  // after the features (the B operand of hb = g W)
  const bool spare = kb.kind == KF_KIND_BSPLINE;
  int rc = launch_permute<bf16>(kb, n_out, n_in, L.OUTP, L.INP, spare ? L.ntb - 1 : L.ntb, c, cfmt, kPermFMT, s, 0,
                                nullptr, bw);
  if (rc) return rc;
  const void* ga = g;
  int gstride = (int)n_out;
  if (p_needs_gpad(n_out, dtype) || (reinterpret_cast<uintptr_t>(g) & 15) != 0) {
    if (!L.gpad) return fail(KF_EINVAL, "kf_P_base: g must be 16-byte aligned");
    void* gp = base + LB.cfmt;
    long n = (long)batch * L.OUTP;
    long blocks = (n + kThreads - 1) / kThreads;
    if (blocks > 65535 * 4) blocks = 65535 * 4;
    hipLaunchKernelGGL(pad_cols_kernel<bf16>, dim3((unsigned)blocks), dim3(kThreads), 0, s, (int)batch, (int)n_out,
                       (int)L.OUTP, (const bf16*)g, (bf16*)gp);
    rc = check_launch("pad_cols");
    if (rc) return rc;
    ga = gp;
    gstride = (int)L.OUTP;
  }
  if (spare) return launch_p8<KF_KIND_BSPLINE, 12, 3, 128, true>(L, s, kb, batch, n_in, x, ga, gstride, cfmt, p);
  const bf16* wt = (const bf16*)cfmt + (size_t)L.ntb * L.INP * L.OUTP;  // W^T (INP, OUTP), zero padded
  rc = gemm_nt(batch, n_in, L.OUTP, ga, gstride, wt, L.OUTP, hb, n_in, true, gws, LB.gemm, s);
  if (rc) return rc;
  return launch_p8<KF_KIND_CHEB, 8, 3, 128, true>(L, s, kb, batch, n_in, x, ga, gstride, cfmt, p, hb);
}

}  // namespace

extern "C" {

size_t kf_rational_bwd_workspace_bytes(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out) {
  if (!b || b->kind != KF_KIND_RATIONAL || b->group_size < 1 || batch < 0 || n_in < 0 || n_out < 0) return 0;
  // parameter partials: the fused kernel's 64-row chunks or the unfused reduction's, whichever is more
  const size_t fused = align256((size_t)((batch + kRatBwdRows - 1) / kRatBwdRows) * (n_in / b->group_size) *
                                (b->num_deg + 1 + b->den_deg) * sizeof(float));
  const size_t plain = kf_rational_workspace_bytes(b, batch, n_in);
  return ws_p(b, dtype, batch, n_in, n_out).total + align256((size_t)batch * n_in * sizeof(float)) +
         (fused > plain ? fused : plain);
}

int kf_rational_bwd(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void* x,
                    const void* g, const void* c, const void* w, void* p, float* dnum, float* dden, void* workspace,
                    size_t workspace_bytes, void* stream) {
  g_err.clear();
  int rc = validate_common(b, dtype, batch, n_in, n_out);
  if (rc) return rc;
  if (b->kind != KF_KIND_RATIONAL) return fail(KF_EINVAL, "kf_rational_bwd needs the rational kind");
  if (!p || !dnum || !dden) return fail(KF_EINVAL, "kf_rational_bwd: NULL output");
  const size_t need = kf_rational_bwd_workspace_bytes(b, dtype, batch, n_in, n_out);
  if (batch > 0 && n_in > 0 && (!workspace || workspace_bytes < need))
    return fail(KF_EWORKSPACE, "kf_rational_bwd: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  if (reinterpret_cast<uintptr_t>(workspace) & 255) return fail(KF_EWORKSPACE, "kf_rational_bwd: workspace must be 256-byte aligned");
  // P at order m + 1 with h = g c^T, then the gradients of sum h w phi^(m)
  kf_basis b1 = *b;
  b1.order = b->order + 1;
  const WsP L = ws_p(b, dtype, batch, n_in, n_out);
  char* base = (char*)workspace;
  float* hb = (float*)(base + L.total);
  void* rws = base + L.total + align256((size_t)batch * n_in * sizeof(float));
  const size_t rbytes = kf_rational_workspace_bytes(b, batch, n_in);
  KBasis kb = to_kbasis(b);
  if (batch > 0 && n_in > 0 && n_out > 0 && x && g && c && rational_bwd_fuses(kb, dtype, n_in, x, g, w, p)) {
    hipStream_t s = (hipStream_t)stream;
    // H = g c^T in bfloat16 (half the traffic of float32 between the GEMM and the fused pass)
    rc = run_P<bf16>(kb, b, dtype, batch, n_in, n_out, x, g, c, p, hb, workspace, s, true, true);
    if (rc) return rc;
    const int groups = (int)(n_in / b->group_size), chunks = (int)((batch + kRatBwdRows - 1) / kRatBwdRows);
    hipLaunchKernelGGL((rational_bwd_fast<bf16, bf16, kRatBwdRows>), dim3((unsigned)groups, (unsigned)chunks), dim3(256),
                       0, s, kb, (int)batch, (int)n_in, (const bf16*)x, (const bf16*)hb, (const bf16*)w, (bf16*)p,
                       (float*)rws);
    rc = check_launch("rational backward");
    if (rc) return rc;
    hipLaunchKernelGGL(rational_grad_final, dim3(1), dim3(256), 0, s, groups, b->num_deg + 1, b->den_deg, chunks,
                       (const float*)rws, dnum, dden);
    return check_launch("rational_grad_final");
  }
  rc = kf_P(&b1, dtype, batch, n_in, n_out, x, g, c, p, hb, workspace, L.total, stream);
  if (rc) return rc;
  return kf_rational_param_grad(b, dtype, batch, n_in, x, hb, w, dnum, dden, rws, rbytes, stream);
}

int kf_P(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void* x, const void* g,
         const void* c, void* p, float* h, void* workspace, size_t workspace_bytes, void* stream) {
  g_err.clear();
  int rc = validate_common(b, dtype, batch, n_in, n_out);
  if (rc) return rc;
  if (batch == 0 || n_in == 0) return KF_OK;
  hipStream_t s = (hipStream_t)stream;
  if (n_out == 0) {
    rc = dtype == KF_BF16 ? zero_fill<bf16>(p, (long)batch * n_in, s) : zero_fill<float>(p, (long)batch * n_in, s);
    if (rc == KF_OK && h) rc = zero_fill<float>(h, (long)batch * n_in, s);
    return rc;
  }
  if (!x || !g || !c || !p) return fail(KF_EINVAL, "kf_P: NULL array");
  if (h && b->kind != KF_KIND_RATIONAL) return fail(KF_EINVAL, "kf_P: h output is for the rational kind");
  size_t need = ws_p(b, dtype, batch, n_in, n_out).total;
  if (!workspace || workspace_bytes < need)
    return fail(KF_EWORKSPACE, "kf_P: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  if (reinterpret_cast<uintptr_t>(workspace) & 255)
    return fail(KF_EWORKSPACE, "kf_P: workspace must be 256-byte aligned");
  KBasis kb = to_kbasis(b);
  if (dtype == KF_BF16) return run_P<bf16>(kb, b, dtype, batch, n_in, n_out, x, g, c, p, h, workspace, s);
  return run_P<float>(kb, b, dtype, batch, n_in, n_out, x, g, c, p, h, workspace, s);
}

int kf_P_base(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void* x, const void* g,
              const void* c, const void* base_w, void* p, void* workspace, size_t workspace_bytes, void* stream) {
  g_err.clear();
  int rc = validate_common(b, dtype, batch, n_in, n_out);
  if (rc) return rc;
  if (batch == 0 || n_in == 0) return KF_OK;
  if (n_out == 0) return fail(KF_EINVAL, "kf_P_base: no outputs");
  if (!x || !g || !c || !base_w || !p) return fail(KF_EINVAL, "kf_P_base: NULL array");
  if (!p_base_route(b, dtype, batch, n_in, n_out))
    return fail(KF_EUNSUPPORTED, "kf_P_base: this layer does not run the fused base branch (kf_base_fused)");
  const bool sparse = bspline_sparse(b, dtype);
  const size_t need = sparse ? ws_base_sparse(KF_OP_P_BASE, b, dtype, batch, n_in, n_out)
                             : ws_p_base(b, dtype, batch, n_in, n_out).total;
  if (need && (!workspace || workspace_bytes < need))
    return fail(KF_EWORKSPACE, "kf_P_base: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  if (need && (reinterpret_cast<uintptr_t>(workspace) & 255))
    return fail(KF_EWORKSPACE, "kf_P_base: workspace must be 256-byte aligned");
  KBasis kb = to_kbasis(b);
  if (sparse)  // float32: W as basis function K of the sparse route
    return launch_p_sparse<float>(kb, b->spline_k, batch, n_in, n_out, x, g, c, p, (hipStream_t)stream, base_w);
  return run_P_base(kb, b, dtype, batch, n_in, n_out, x, g, c, base_w, p, workspace, (hipStream_t)stream);
}

}  // extern "C"
