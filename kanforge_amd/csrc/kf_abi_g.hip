// kf_G (include/kfhip.h): the coefficient-gradient contraction's launch configurations,
// workspace carving and dispatch.
#include "kf_abi.h"
#include "kf_rational.h"

using namespace kfabi;

namespace {

template <typename T, int WMW, int WJW, int TM, int FW, int RB, bool CHEB, bool FLAT = false>
int launch_g_t(const WsG& L, hipStream_t s, const KBasis& kb, int64_t batch, int64_t n_in, int64_t n_out,
               const void* phit, const float* zt, const float* wt, const void* gt, void* dc, float* zpart) {
  constexpr int BM = WMW * TM * 32, NMAX = WJW * FW * 32, RS = RB + 16;
  const size_t lds_ops = (size_t)2 * (BM + NMAX) * RS;
  const size_t lds_red = (size_t)(FLAT ? NMAX / 32 : kb.n_t) * (BM / 2) * 33 * 4;
  const size_t lds = lds_ops > lds_red ? lds_ops : lds_red;
  auto kern = g_kernel<T, WMW, WJW, TM, FW, RB, CHEB, FLAT>;
  if (!reserve_lds((const void*)kern, lds))
    return fail(KF_ELAUNCH, "G: cannot reserve %zu bytes of LDS", lds);
  constexpr int TI = FLAT ? NMAX : 32;
  if (FLAT && L.INP % TI) return fail(KF_EINVAL, "G: workspace layout not aligned");
  const int n_m = (int)(L.OUTP / BM), n_n = (int)((n_in + TI - 1) / TI);
  hipLaunchKernelGGL(kern, dim3(n_m * n_n, L.nz), dim3(WMW * WJW * 64), lds, s, kb, (int)batch, (int)n_in,
                     (int)n_out, (int)L.BP, (int)L.OUTP, (int)L.INP, (const T*)phit, zt, wt, (const T*)gt, (T*)dc,
                     L.nz > 1 ? zpart : nullptr);
  int rc = check_launch("G");
  if (rc || L.nz == 1) return rc;
  // the splits summed into split 0 (coalesced), then the fold from that one slice
  const size_t zstride = (size_t)L.OUTP * L.INP * kb.n_t;
  long blocks = ((long)zstride + kThreads - 1) / kThreads;
  if (blocks > 65535 * 4) blocks = 65535 * 4;
  hipLaunchKernelGGL(g_split_sum, dim3((unsigned)blocks), dim3(kThreads), 0, s, (long)zstride, L.nz, zstride, zpart);
  rc = check_launch("G split sum");
  if (rc) return rc;
  long n = (long)n_out * n_in * kb.K;
  blocks = (n + kThreads - 1) / kThreads;
  if (blocks > 65535 * 4) blocks = 65535 * 4;
  hipLaunchKernelGGL(g_split_reduce<T>, dim3((unsigned)blocks), dim3(kThreads), 0, s, kb, (int)n_out, (int)n_in,
                     (int)L.OUTP, (int)L.INP, 1, (const float*)zpart, (T*)dc);
  return check_launch("G split reduce");
}

template <typename T, bool CHEB>
int launch_g_cfg(const WsG& L, hipStream_t s, const KBasis& kb, int64_t batch, int64_t n_in, int64_t n_out,
                 const void* x, const void* w, const float* zt, const float* wt, const void* gt, void* dc) {
  // x: phiT, w: the split partial sums
  float* zp = (float*)w;
  if (!CHEB && kb.kind == KF_KIND_RATIONAL) {
    if (L.cfg != 0) return fail(KF_EINVAL, "G: rational plans have one feature");
    return launch_g_t<T, 2, 2, 2, 2, 128, false, true>(L, s, kb, batch, n_in, n_out, x, zt, wt, gt, dc, zp);
  }
  switch (L.cfg) {
    case 0: return launch_g_t<T, 2, 2, 2, 2, 128, CHEB>(L, s, kb, batch, n_in, n_out, x, zt, wt, gt, dc, zp);
    case 1: return launch_g_t<T, 2, 2, 2, 3, 128, CHEB>(L, s, kb, batch, n_in, n_out, x, zt, wt, gt, dc, zp);
    case 2: return launch_g_t<T, 2, 2, 2, 4, 128, CHEB>(L, s, kb, batch, n_in, n_out, x, zt, wt, gt, dc, zp);
    case 3: return launch_g_t<T, 2, 2, 2, 5, 128, CHEB>(L, s, kb, batch, n_in, n_out, x, zt, wt, gt, dc, zp);
    case 4: return launch_g_t<T, 2, 2, 2, 6, 128, CHEB>(L, s, kb, batch, n_in, n_out, x, zt, wt, gt, dc, zp);
    case 5: return launch_g_t<T, 2, 2, 1, 8, 64, CHEB>(L, s, kb, batch, n_in, n_out, x, zt, wt, gt, dc, zp);
    default: return launch_g_t<T, 2, 2, 1, 12, 64, CHEB>(L, s, kb, batch, n_in, n_out, x, zt, wt, gt, dc, zp);
  }
}

template <typename T, int TM, int FW, int RB>
int launch_g_ws(const WsG& L, hipStream_t s, const KBasis& kb, int64_t batch, int64_t n_in, int64_t n_out,
                const float* zt, const float* wt, const void* gt, const float* colsum, void* dc) {
  constexpr int BM = 2 * TM * 32, NMAX = 2 * FW * 32, RS = RB + 16;
  const size_t lds_ops = (size_t)2 * (BM + NMAX) * RS, lds_red = (size_t)kb.n_t * (BM / 2) * 33 * 4;
  const size_t lds = lds_ops > lds_red ? lds_ops : lds_red;
  auto kern = L.skip0 ? g_ws_kernel<T, TM, FW, RB, true> : g_ws_kernel<T, TM, FW, RB, false>;
  if (!reserve_lds((const void*)kern, lds))
    return fail(KF_ELAUNCH, "G: cannot reserve %zu bytes of LDS", lds);
  const int n_m = (int)(L.OUTP / BM), n_n = (int)((n_in + 31) / 32);
  hipLaunchKernelGGL(kern, dim3(n_m * n_n), dim3(512), lds, s, kb, (int)batch, (int)n_in, (int)n_out, (int)L.BP,
                     (int)L.OUTP, zt, wt, (const T*)gt, colsum, (T*)dc);
  return check_launch("G");
}

template <bool SKIP0>
int launch_g96(const WsG& L, hipStream_t s, const KBasis& kb, int64_t batch, int64_t n_in, int64_t n_out,
               const float* zt, const float* wt, const void* gt, const float* colsum, void* dc) {
  const size_t lds_ops = (size_t)2 * (192 * 64 + 8 * 48 * 64);
  const size_t lds_red = (size_t)(8 * 32 * 49 + 32) * 4 + (size_t)32 * 48 * kb.K * 2;  // sums, output rows
  const int vout = (n_in * kb.K * 2) % 16 == 0 && aligned16(dc);
  const size_t lds = lds_ops > lds_red ? lds_ops : lds_red;
  auto kern = g96_kernel<SKIP0>;
  if (!reserve_lds((const void*)kern, lds))
    return fail(KF_ELAUNCH, "G: cannot reserve %zu bytes of LDS", lds);
  const int n_m = (int)(L.OUTP / 192), n_n = (int)(L.INP / 48);
  const int skip = SKIP0 ? 1 : 0, n_run = kb.n_t - skip;
  KFoldG fg;
  for (int k = 0; k < KF_MAX_K; ++k) {
    fg.v[k][0] = SKIP0 && k < kb.K ? kb.fold[k * KF_MAX_NT] : 0.f;
    for (int f = 0; f < 8; ++f) fg.v[k][1 + f] = k < kb.K && f < n_run ? kb.fold[k * KF_MAX_NT + f + skip] : 0.f;
  }
  hipLaunchKernelGGL(kern, dim3(n_m * n_n), dim3(512), lds, s, fg, kb.K, n_run, (int)batch, (int)n_in, (int)n_out,
                     (int)L.BP, (int)L.OUTP, (int)L.INP, zt, wt, (const bf16*)gt, colsum, (bf16*)dc, vout);
  return check_launch("G");
}

// G over precomputed B-spline features as p_dma_kernel's flat GEMM (identity fold).
template <typename T>
int launch_g_dma(const WsG& L, hipStream_t s, const KBasis& kb, int64_t n_in, int64_t n_out, const void* gt,
                 const void* phit, void* dc) {
  constexpr int FW = kGdmaFW, TM = p_dma_tm(FW), BM = 2 * TM * 32, EPS = 128 / (int)sizeof(T);
  const size_t lds = (size_t)2 * (BM + 2 * FW * 32) * 128;
  auto kern = p_dma_kernel<T, TM, FW, KF_KIND_BSPLINE, 1>;
  if (L.INP % kGdmaRows || L.BP % EPS || L.BP / EPS < 1) return fail(KF_EINVAL, "G: workspace layout not aligned");
  if (!reserve_lds((const void*)kern, lds))
    return fail(KF_ELAUNCH, "G: cannot reserve %zu bytes of LDS", lds);
  const int n_m = (int)((n_out + BM - 1) / BM), n_n = (int)(kb.n_t * L.INP / kGdmaRows);
  hipLaunchKernelGGL(kern, dim3(n_m * n_n), dim3(256), lds, s, kb, (int)n_out, (int)n_in, (int)L.INP, (int)L.BP,
                     (const T*)nullptr, (const T*)gt, (int)L.BP, (const T*)phit, (T*)dc, (float*)nullptr);
  return check_launch("G");
}

template <typename T>
// dbias (dtype, n_out) or NULL: the column sums of g, taken from the transpose's block partials
// (bias_part / bias_sums: (BP / 64, OUTP) and OUTP floats after G's own workspace, unless the
// Chebyshev layout already has them), which sets *dbias_done; the sparse route sums g per row
// slice beside its partials (bias_part: nz x n_out floats) and sets it too.
int run_G(const KBasis& kb, const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void* x,
          const void* g, const void* w, void* dc, void* ws, hipStream_t s, void* dbias = nullptr,
          float* bias_part = nullptr, float* bias_sums = nullptr, bool* dbias_done = nullptr) {
  if constexpr (sizeof(T) == 4)
    if (bspline_sparse(b, dtype)) {
      const int rc = launch_g_sparse<T>(kb, b->spline_k, batch, n_in, n_out, x, g, w, dc, ws, s, dbias, bias_part);
      if (!rc && dbias && bias_part && dbias_done) *dbias_done = true;
      return rc;
    }
  const bool cheb_kind = kb.kind == KF_KIND_CHEB;
  const bool weighted = features_weighted(b, w);
  WsG L = ws_g(b, dtype, batch, n_in, n_out, weighted);
  const bool cheb = cheb_kind && !L.pre;
  char* base = (char*)ws;
  void* gt = base;
  float* zt = cheb ? (float*)(base + L.gt) : nullptr;
  float* wt = cheb && weighted ? (float*)(base + L.gt + L.zt) : nullptr;
  float* part = L.skip0 ? (float*)(base + L.gt + L.zt + L.wt) : nullptr;
  float* colsum = L.skip0 ? (float*)(base + L.gt + L.zt + L.wt + L.part) : nullptr;
  // the bias gradient from the same partials: the Chebyshev sums (skip0) copy it out, other
  // routes total the partials in a launch of their own
  const bool own_sums = dbias && !L.skip0;
  if (own_sums) part = bias_part;
  if (L.BP % 32 || !aligned16(gt)) return fail(KF_EINVAL, "G: workspace layout not aligned");
  dim3 tg((unsigned)((L.OUTP + 63) / 64), (unsigned)((L.BP + 63) / 64));
  hipLaunchKernelGGL(transpose_kernel<T>, tg, dim3(kThreads), 0, s, (int)batch, (int)n_out, (int)L.BP, (int)L.OUTP,
                     (int)rows_vec<T>(n_out, g), (const T*)g, (T*)gt, part);
  int rc = check_launch("transpose");
  if (rc) return rc;
  if (own_sums) {
    hipLaunchKernelGGL(sum_parts_kernel<T>, dim3((unsigned)((L.OUTP + 7) / 8)), dim3(kThreads), 0, s,
                       (int)((L.BP + 63) / 64), (int)L.OUTP, (const float*)part, bias_sums, (T*)dbias, (int)n_out);
    rc = check_launch("bias gradient");
    if (rc) return rc;
  }
  if (dbias_done) *dbias_done = dbias != nullptr && (own_sums || cheb);
  if (cheb) {
    // block rows past the batch tiles total the column sums of g (skip0 implies cheb)
    const unsigned gx = (unsigned)((L.INP + 63) / 64), sblocks = L.skip0 ? (unsigned)((L.OUTP + 7) / 8) : 0u;
    dim3 zg(gx, (unsigned)((L.BP + 63) / 64) + (sblocks + gx - 1) / gx);
    hipLaunchKernelGGL(zmapT_kernel<T>, zg, dim3(kThreads), (size_t)(wt ? 2 : 1) * 64 * 65 * sizeof(float), s,
                       (int)batch, (int)n_in, (int)L.BP, (int)L.INP, kb.input_map,
                       (int)(rows_vec<T>(n_in, x) && rows_vec<T>(n_in, w)), (const T*)x, (const T*)w, zt, wt,
                       (int)((L.BP + 63) / 64), (int)L.OUTP, part, colsum, (T*)nullptr,
                       (T*)(L.skip0 ? dbias : nullptr), (int)n_out);
    rc = check_launch("zmapT");
    if (rc) return rc;
    if (L.g96) {
      if (L.skip0) return launch_g96<true>(L, s, kb, batch, n_in, n_out, zt, wt, gt, colsum, dc);
      return launch_g96<false>(L, s, kb, batch, n_in, n_out, zt, wt, gt, colsum, dc);
    }
    switch (L.cfg) {
      case 0: return launch_g_ws<T, 2, 2, 128>(L, s, kb, batch, n_in, n_out, zt, wt, gt, colsum, dc);
      case 1: return launch_g_ws<T, 2, 3, 128>(L, s, kb, batch, n_in, n_out, zt, wt, gt, colsum, dc);
      case 2: return launch_g_ws<T, 2, 4, 128>(L, s, kb, batch, n_in, n_out, zt, wt, gt, colsum, dc);
      case 3: return launch_g_ws<T, 2, 5, 128>(L, s, kb, batch, n_in, n_out, zt, wt, gt, colsum, dc);
      case 4: return launch_g_ws<T, 2, 6, 128>(L, s, kb, batch, n_in, n_out, zt, wt, gt, colsum, dc);
      case 5: return launch_g_ws<T, 1, 8, 64>(L, s, kb, batch, n_in, n_out, zt, wt, gt, colsum, dc);
      default: return launch_g_ws<T, 1, 12, 64>(L, s, kb, batch, n_in, n_out, zt, wt, gt, colsum, dc);
    }
  }
  // other kinds: features (times w) precomputed once into phiT[j][INP][BP]
  void* phit = base + L.gt + L.zt + L.wt + L.part + L.colsum;
  if constexpr (sizeof(T) == 2) {
    // GR-KAN degrees in bf16: phi^(m)(x) w transposed to (in, BP), then the GEMM g^T phi over the batch
    if (rational_fast(kb, n_in) && n_in % 64 == 0 && kb.order <= 2 && L.BP % 64 == 0 && aligned16(x) &&
        (!w || aligned16(w))) {
      auto mapt = kb.order == 0 ? rational_map_t_kernel<bf16, 0>
                  : kb.order == 1 ? rational_map_t_kernel<bf16, 1>
                                  : rational_map_t_kernel<bf16, 2>;
      hipLaunchKernelGGL(mapt, dim3((unsigned)(n_in / 64), (unsigned)(L.BP / 64)), dim3(256), 0, s, kb, (int)batch,
                         (int)n_in, (int)L.BP, (const bf16*)x, (const bf16*)w, (bf16*)phit);
      rc = check_launch("rational features (transposed)");
      if (rc) return rc;
      void* gws = (char*)phit + L.phit + L.zpart;
      return gemm_nt(n_out, n_in, L.BP, gt, L.BP, phit, L.BP, dc, n_in, false, gws, L.gemm, s);
    }
  }
  float* zpart = L.nz > 1 ? (float*)((char*)phit + L.phit) : nullptr;
  if constexpr (sizeof(T) == 2) {
    // B-splines in bf16: phiT rows input-major (i K + k), so that dc[o][i][k] is the GEMM
    // g^T phiT^T stored row by row
    if (kb.kind == KF_KIND_BSPLINE && L.BP % 64 == 0 && (n_in * kb.K) % 8 == 0 && aligned16(dc)) {
      rc = launch_features_t<T>(kb, batch, n_in, L.BP, L.INP, x, w, phit, s, 1);
      if (rc) return rc;
      void* gws = (char*)phit + L.phit + L.zpart;
      return gemm_nt(n_out, n_in * kb.K, L.BP, gt, L.BP, phit, L.BP, dc, n_in * kb.K, false, gws, L.gemm, s);
    }
  }
  rc = launch_features_t<T>(kb, batch, n_in, L.BP, L.INP, x, w, phit, s);
  if (rc) return rc;
  if (L.gdma) return launch_g_dma<T>(L, s, kb, n_in, n_out, gt, phit, dc);
  return launch_g_cfg<T, false>(L, s, kb, batch, n_in, n_out, phit, zpart, nullptr, nullptr, gt, dc);
}
// The layer's parameter gradients with its SiLU base branch and bias: the g transpose (with its
// column sums: the T_0 constant and the bias gradient), z^T and silu(x)^T in one prepass, G on
// g96_kernel, and the base weights' gradient gT silu(x)^T on the GEMM core. dc, dbw and dbias may
// each be NULL (not wanted).
// B-splines: the transposed features (input-major rows) and the dc GEMM of kf_G's GEMM-core
// route, with the column sums and silu(x)^T from one extra prepass.
int run_G_base_bspline(const KBasis& kb, const WsGB& LB, int64_t batch, int64_t n_in, int64_t n_out, const void* x,
                       const void* g, void* dc, void* dbw, void* dbias, void* ws, hipStream_t s) {
  const WsG& L = LB.g;
  char* base = (char*)ws;
  void* gt = base;
  void* phit = base + L.gt + L.zt + L.wt + L.part + L.colsum;
  void* gws = (char*)phit + L.phit + L.zpart;
  float* part = (float*)(base + L.total);
  float* colsum = (float*)(base + L.total + LB.part);
  bf16* st = dbw ? (bf16*)(base + L.total + LB.part + LB.colsum) : nullptr;
  void* gws2 = base + L.total + LB.part + LB.colsum + LB.st;
  if (!aligned16(gt) || (dc && !aligned16(dc))) return fail(KF_EINVAL, "kf_G_base: arrays not 16-byte aligned");
  dim3 tg((unsigned)((L.OUTP + 63) / 64), (unsigned)((L.BP + 63) / 64));
  hipLaunchKernelGGL(transpose_kernel<bf16>, tg, dim3(kThreads), 0, s, (int)batch, (int)n_out, (int)L.BP, (int)L.OUTP,
                     (int)rows_vec<bf16>(n_out, g), (const bf16*)g, (bf16*)gt, dbias ? part : nullptr);
  int rc = check_launch("transpose");
  if (rc) return rc;
  if (st || dbias) {
    const unsigned gx = (unsigned)((L.INP + 63) / 64), sblocks = dbias ? (unsigned)((L.OUTP + 7) / 8) : 0u;
    dim3 zg(gx, (unsigned)((L.BP + 63) / 64) + (sblocks + gx - 1) / gx);
    hipLaunchKernelGGL(zmapT_kernel<bf16>, zg, dim3(kThreads), (size_t)2 * 64 * 65 * sizeof(float), s, (int)batch,
                       (int)n_in, (int)L.BP, (int)L.INP, kb.input_map, (int)rows_vec<bf16>(n_in, x), (const bf16*)x,
                       (const bf16*)nullptr, (float*)nullptr, (float*)nullptr, (int)((L.BP + 63) / 64),
                       dbias ? (int)L.OUTP : 0, part, colsum, st, (bf16*)dbias, (int)n_out);
    rc = check_launch("silu transpose");
    if (rc) return rc;
  }
  if (dc) {
    rc = launch_features_t<bf16>(kb, batch, n_in, L.BP, L.INP, x, nullptr, phit, s, 1);
    if (rc) return rc;
    rc = gemm_nt(n_out, n_in * kb.K, L.BP, gt, L.BP, phit, L.BP, dc, n_in * kb.K, false, gws, L.gemm, s);
    if (rc) return rc;
  }
  if (dbw) return gemm_nt(n_out, n_in, L.BP, gt, L.BP, st, L.BP, dbw, n_in, false, gws2, LB.gemm, s);
  return KF_OK;
}

int run_G_base(const KBasis& kb, const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out,
               const void* x, const void* g, void* dc, void* dbw, void* dbias, void* ws, hipStream_t s) {
  const WsGB LB = ws_g_base(b, dtype, batch, n_in, n_out);
  if (kb.kind == KF_KIND_BSPLINE) return run_G_base_bspline(kb, LB, batch, n_in, n_out, x, g, dc, dbw, dbias, ws, s);
  const WsG& L = LB.g;
  char* base = (char*)ws;
  void* gt = base;
  float* zt = (float*)(base + L.gt);
  float* part = (float*)(base + L.gt + L.zt + L.wt);
  float* colsum = (float*)(base + L.gt + L.zt + L.wt + L.part);
  bf16* st = dbw ? (bf16*)(base + L.total + LB.part + LB.colsum) : nullptr;
  void* gws = base + L.total + LB.part + LB.colsum + LB.st;
  if (!L.g96 || !L.skip0 || L.pre || L.BP % 64 || !aligned16(gt)) return fail(KF_EINVAL, "kf_G_base: layer not on g96");
  dim3 tg((unsigned)((L.OUTP + 63) / 64), (unsigned)((L.BP + 63) / 64));
  hipLaunchKernelGGL(transpose_kernel<bf16>, tg, dim3(kThreads), 0, s, (int)batch, (int)n_out, (int)L.BP, (int)L.OUTP,
                     (int)rows_vec<bf16>(n_out, g), (const bf16*)g, (bf16*)gt, part);
  int rc = check_launch("transpose");
  if (rc) return rc;
  const unsigned gx = (unsigned)((L.INP + 63) / 64), sblocks = (unsigned)((L.OUTP + 7) / 8);
  dim3 zg(gx, (unsigned)((L.BP + 63) / 64) + (sblocks + gx - 1) / gx);
  hipLaunchKernelGGL(zmapT_kernel<bf16>, zg, dim3(kThreads), (size_t)(st ? 2 : 1) * 64 * 65 * sizeof(float), s,
                     (int)batch, (int)n_in, (int)L.BP, (int)L.INP, kb.input_map, (int)rows_vec<bf16>(n_in, x),
                     (const bf16*)x, (const bf16*)nullptr, zt, (float*)nullptr, (int)((L.BP + 63) / 64), (int)L.OUTP,
                     part, colsum, st, (bf16*)dbias, (int)n_out);
  rc = check_launch("zmapT");
  if (rc) return rc;
  if (dc) {
    rc = launch_g96<true>(L, s, kb, batch, n_in, n_out, zt, nullptr, gt, colsum, dc);
    if (rc) return rc;
  }
  if (dbw) return gemm_nt(n_out, n_in, L.BP, gt, L.BP, st, L.BP, dbw, n_in, false, gws, LB.gemm, s);
  return KF_OK;
}

}  // namespace

extern "C" {

int kf_G(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void* x, const void* g,
         const void* w, void* dc, void* workspace, size_t workspace_bytes, void* stream) {
  g_err.clear();
  int rc = validate_common(b, dtype, batch, n_in, n_out);
  if (rc) return rc;
  if (n_in == 0 || n_out == 0) return KF_OK;
  hipStream_t s = (hipStream_t)stream;
  const long n = (long)n_out * n_in * b->size;
  if (batch == 0) return dtype == KF_BF16 ? zero_fill<bf16>(dc, n, s) : zero_fill<float>(dc, n, s);
  if (!x || !g || !dc) return fail(KF_EINVAL, "kf_G: NULL array");
  size_t need = ws_g(b, dtype, batch, n_in, n_out, features_weighted(b, w)).total;
  if (!workspace || workspace_bytes < need)
    return fail(KF_EWORKSPACE, "kf_G: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  if (reinterpret_cast<uintptr_t>(workspace) & 255)
    return fail(KF_EWORKSPACE, "kf_G: workspace must be 256-byte aligned");
  KBasis kb = to_kbasis(b);
  if (dtype == KF_BF16) return run_G<bf16>(kb, b, dtype, batch, n_in, n_out, x, g, w, dc, workspace, s);
  return run_G<float>(kb, b, dtype, batch, n_in, n_out, x, g, w, dc, workspace, s);
}

int kf_G_base(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void* x, const void* g,
              void* dc, void* dbase_w, void* dbias, void* workspace, size_t workspace_bytes, void* stream) {
  g_err.clear();
  int rc = validate_common(b, dtype, batch, n_in, n_out);
  if (rc) return rc;
  if (n_in == 0 || n_out == 0) return KF_OK;
  if (batch == 0) return fail(KF_EINVAL, "kf_G_base: empty batch");
  if (!x || !g) return fail(KF_EINVAL, "kf_G_base: NULL array");
  if (!dc && !dbase_w && !dbias) return KF_OK;
  if (!g_base_route(b, dtype, batch, n_in, n_out))
    return fail(KF_EUNSUPPORTED, "kf_G_base: this layer does not run the fused base branch (kf_base_fused)");
  const bool sparse = bspline_sparse(b, dtype);
  const size_t need = sparse ? ws_base_sparse(KF_OP_G_BASE, b, dtype, batch, n_in, n_out)
                             : ws_g_base(b, dtype, batch, n_in, n_out).total;
  if (!workspace || workspace_bytes < need)
    return fail(KF_EWORKSPACE, "kf_G_base: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  if (reinterpret_cast<uintptr_t>(workspace) & 255)
    return fail(KF_EWORKSPACE, "kf_G_base: workspace must be 256-byte aligned");
  KBasis kb = to_kbasis(b);
  if (sparse) {  // float32: silu(x) as basis function K of the sparse G, the bias gradient beside it
    if (dc || dbase_w)
      return launch_g_sparse_base<float>(kb, b->spline_k, batch, n_in, n_out, x, g, dc, dbase_w, dbias, workspace,
                                         (hipStream_t)stream);
    const size_t part = sparse_g_plan(batch, n_in, n_out, kb.K + 1).part;
    return kf_column_sums(dtype, batch, n_out, g, dbias, (char*)workspace + part, need - part, stream);
  }
  return run_G_base(kb, b, dtype, batch, n_in, n_out, x, g, dc, dbase_w, dbias, workspace, (hipStream_t)stream);
}

int kf_G_bias(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void* x, const void* g,
              const void* w, void* dc, void* dbias, void* workspace, size_t workspace_bytes, void* stream) {
  g_err.clear();
  if (!dbias) return kf_G(b, dtype, batch, n_in, n_out, x, g, w, dc, workspace, workspace_bytes, stream);
  int rc = validate_common(b, dtype, batch, n_in, n_out);
  if (rc) return rc;
  if (n_out == 0) return KF_OK;
  hipStream_t s = (hipStream_t)stream;
  if (batch == 0 || n_in == 0) {
    rc = kf_G(b, dtype, batch, n_in, n_out, x, g, w, dc, workspace, workspace_bytes, stream);
    if (rc) return rc;
    if (batch == 0) return dtype == KF_BF16 ? zero_fill<bf16>(dbias, n_out, s) : zero_fill<float>(dbias, n_out, s);
    return kf_column_sums(dtype, batch, n_out, g, dbias, workspace, workspace_bytes, stream);
  }
  if (!x || !g || !dc) return fail(KF_EINVAL, "kf_G_bias: NULL array");
  const bool weighted = features_weighted(b, w);
  const WsGBias L = ws_g_bias(b, dtype, batch, n_in, n_out, weighted);
  if (!workspace || workspace_bytes < L.total)
    return fail(KF_EWORKSPACE, "kf_G_bias: workspace of %zu bytes needed, %zu given", L.total, workspace_bytes);
  if (reinterpret_cast<uintptr_t>(workspace) & 255)
    return fail(KF_EWORKSPACE, "kf_G_bias: workspace must be 256-byte aligned");
  KBasis kb = to_kbasis(b);
  char* extra = (char*)workspace + L.g;
  float* bpart = (float*)extra;
  float* bsums = (float*)(extra + L.part);
  bool done = false;
  rc = dtype == KF_BF16 ? run_G<bf16>(kb, b, dtype, batch, n_in, n_out, x, g, w, dc, workspace, s, dbias, bpart, bsums, &done)
                        : run_G<float>(kb, b, dtype, batch, n_in, n_out, x, g, w, dc, workspace, s, dbias, bpart, bsums, &done);
  if (rc || done) return rc;
  return kf_column_sums(dtype, batch, n_out, g, dbias, extra + L.part + L.sums, L.cws, stream);
}

}  // extern "C"
