// kf_F and kf_F_noalloc (include/kfhip.h): the forward contraction's launch configurations,
// workspace carving and dispatch.
#include "kf_abi.h"
#include "kf_rational.h"

using namespace kfabi;

namespace kf {
// Multiplies precomputed features phi[b][j][i] by w[b][i] (weighted F, non-Chebyshev kinds).
template <typename T>
__global__ __launch_bounds__(kThreads) void scale_phi_kernel(int B, int IN, int n_t, int INP, const T* __restrict__ w,
                                                             T* __restrict__ phi) {
  const long n = (long)B * n_t * INP;
  for (long e = blockIdx.x * (long)kThreads + threadIdx.x; e < n; e += (long)gridDim.x * kThreads) {
    const int i = (int)(e % INP);
    const int b = (int)(e / ((long)n_t * INP));
    if (i < IN) phi[e] = from_f32<T>(to_f32(phi[e]) * to_f32(w[(size_t)b * IN + i]));
  }
}
// y[b][o] += bias[o] (the bias of routes whose last kernel does not take it).
template <typename T>
__global__ __launch_bounds__(kThreads) void bias_rows_kernel(int B, int OUT, const T* __restrict__ bias, T* __restrict__ y) {
  const long n = (long)B * OUT;
  for (long e = blockIdx.x * (long)kThreads + threadIdx.x; e < n; e += (long)gridDim.x * kThreads)
    y[e] = from_f32<T>(to_f32(y[e]) + to_f32(bias[e % OUT]));
}
}  // namespace kf

namespace {


template <typename T, int BM, int BN, int WMW, int WNW, bool CHEB, bool HAS_W>
int launch_f_t(const WsF& L, int64_t batch, int64_t n_out, int n_t, const float* z, const float* wz, const void* cfm,
               const void* phi, void* y, hipStream_t s) {
  constexpr int FPS = sizeof(T) == 2 ? 2 : 1;
  const int n_m = (int)(L.BP / BM), n_n = (int)(L.OUTP / BN);
  const int rs = 32 * (int)sizeof(T) + 16;
  const size_t lds = (size_t)2 * FPS * (BM + BN) * rs;
  auto kern = f_kernel<T, BM, BN, WMW, WNW, FPS, CHEB, HAS_W>;
  if (!reserve_lds((const void*)kern, lds))
    return fail(KF_ELAUNCH, "F: cannot reserve %zu bytes of LDS", lds);
  hipLaunchKernelGGL(kern, dim3(n_m * n_n), dim3(WMW * WNW * 64), lds, s, (int)batch, (int)n_out, (int)L.INP,
                     (int)L.OUTP, n_t, L.n_tp, z, wz, (const T*)cfm, (const T*)phi, (T*)y);
  return check_launch("F");
}

template <bool HAS_W, bool SKIP0, bool BASE = false>
int launch_f_rega(const WsF& L, int64_t batch, int64_t n_out, const float* zc, const float* wc, const void* cfm,
                  const float* ysum, void* y, hipStream_t s) {
  const int n_m = (int)(L.BP / RA_BM), n_n = (int)(L.OUTP / RA_BN);
  // RA_NBUF stage buffers of 2 features, z (and w, or silu(x)) of two chunks
  // (reused by the epilogue's bf16 staging of each wave's output tile: RA_BM rows of
  // RA_BN / RA_WN * 2 + 16 bytes per column group)
  const size_t lds_ops = (size_t)RA_NBUF * 2 * RA_BN * 32 + (size_t)(HAS_W || BASE ? 4 : 2) * RA_BM * 64;
  const size_t lds_epi = (size_t)RA_WN * RA_BM * (RA_BN / RA_WN * 2 + 16);
  const size_t lds = lds_ops > lds_epi ? lds_ops : lds_epi;
  const int vout = n_out % 8 == 0 && aligned16(y);
  constexpr int TNW = RA_TN / RA_WN;
  if (BASE && !(L.n_tp == 9 || (L.n_tp % 2 == 0 && L.n_tp >= 6)))
    return fail(KF_EINVAL, "F: the base feature needs chunks of 9 or an even count >= 6 features");
  auto kern = BASE          ? (L.n_tp == 9 ? f_rega_kernel<HAS_W, 9, RA_TM, TNW, RA_NBUF, SKIP0, RA_WN, RA_NWM, BASE>
                                           : f_rega_kernel<HAS_W, 0, RA_TM, TNW, RA_NBUF, SKIP0, RA_WN, RA_NWM, BASE>)
              : L.n_tp == 9 ? f_rega_kernel<HAS_W, 9, RA_TM, TNW, RA_NBUF, SKIP0, RA_WN, RA_NWM>
              : L.n_tp == 8 ? f_rega_kernel<HAS_W, 8, RA_TM, TNW, RA_NBUF, SKIP0, RA_WN, RA_NWM>
                            : f_rega_kernel<HAS_W, 0, RA_TM, TNW, RA_NBUF, SKIP0, RA_WN, RA_NWM>;
  if (!reserve_lds((const void*)kern, lds))
    return fail(KF_ELAUNCH, "F: cannot reserve %zu bytes of LDS", lds);
  hipLaunchKernelGGL(kern, dim3(n_m * n_n), dim3(64 * RA_NWM * RA_WN), lds, s, (int)batch, (int)n_out, (int)L.OUTP, (int)L.BP,
                     (int)(L.INP / 16), L.n_tp, zc, wc, (const bf16*)cfm, ysum, (bf16*)y, vout);
  return check_launch("F");
}

template <typename T, bool CHEB, bool HAS_W>
int launch_f_cfg(const WsF& L, int64_t batch, int64_t n_out, int n_t, const float* z, const float* wz, const void* cfm,
                 const void* phi, void* y, hipStream_t s) {
  switch (L.cfg) {
    case 0: return launch_f_t<T, 256, 192, 4, 2, CHEB, HAS_W>(L, batch, n_out, n_t, z, wz, cfm, phi, y, s);
    case 1: return launch_f_t<T, 256, 256, 2, 4, CHEB, HAS_W>(L, batch, n_out, n_t, z, wz, cfm, phi, y, s);
    default: return launch_f_t<T, 256, 128, 4, 2, CHEB, HAS_W>(L, batch, n_out, n_t, z, wz, cfm, phi, y, s);
  }
}

// B-spline features into rows ld elements apart (plus the base columns, base_cols > 0):
// 32 inputs x 64 rows per block, knot rows staged once per block
template <typename T>
int launch_phi_block(const KBasis& kb, int64_t batch, int64_t n_in, const void* x, void* phi, long ld, int base_cols,
                     hipStream_t s) {
  const size_t rpb = ((size_t)32 * kb.K * sizeof(T) + 15) / 16 * 16 + 16;
  const size_t plds = 64 * rpb + (size_t)32 * (2 * kb.n_knots + 2 * kb.spline_k) * 4;
  dim3 pg((unsigned)((n_in + 31) / 32), (unsigned)((batch + 63) / 64));
  const bool even = kb.knots_uniform && kb.n_knots >= 4;  // cubic even knots: the common case
  auto kern = kb.spline_k == 0   ? phi_block_kernel<T, 0>
              : kb.spline_k == 1 ? phi_block_kernel<T, 1>
              : kb.spline_k == 2 ? phi_block_kernel<T, 2>
              : kb.spline_k == 3 ? (even ? phi_block_kernel<T, 3, true> : phi_block_kernel<T, 3>)
              : kb.spline_k == 4 ? phi_block_kernel<T, 4>
                                 : phi_block_kernel<T, 5>;
  if (!reserve_lds((const void*)kern, plds)) return fail(KF_ELAUNCH, "F: cannot reserve %zu bytes of LDS", plds);
  hipLaunchKernelGGL(kern, pg, dim3(kThreads), plds, s, kb, (int)batch, (int)n_in, (const T*)x, (T*)phi, ld, base_cols);
  return check_launch("phi_block");
}

template <typename T>
int run_F_dma(const KBasis& kb, int64_t batch, int64_t n_in, int64_t n_out, const void* x, const void* c, void* phi,
              void* y, void* gws, size_t gws_bytes, hipStream_t s, const void* bias = nullptr, bool* bias_done = nullptr) {
  constexpr int FW = kGdmaFW, TM = p_dma_tm(FW), BM = 2 * TM * 32, TI = 2 * FW * 32;
  const long ld = (long)n_in * kb.K;  // Phi row length: the reduction
  if (kb.n_t != kb.K || (ld * (long)sizeof(T)) % 16) return fail(KF_EINVAL, "F: Phi rows not aligned");
  if (kb.kind == KF_KIND_BSPLINE && ld % 8 == 0 && aligned16(phi)) {
    int rc = launch_phi_block<T>(kb, batch, n_in, x, phi, ld, 0, s);
    if (rc) return rc;
  } else if (kb.K == 1) {  // one feature: the plain (B, in) writes are already coalesced
    int rc = launch_features<T, false>(kb, batch, n_in, batch, n_in, x, phi, ld, 1L, 1L, false, s);
    if (rc) return rc;
  } else {
    dim3 pg((unsigned)((n_in + kThreads - 1) / kThreads), (unsigned)(batch < 65535 ? batch : 65535));
    const size_t plds = (size_t)kThreads * kb.K * sizeof(T);
    switch (nt_bucket(kb.n_t)) {
      case 4: hipLaunchKernelGGL((phi_rows_kernel<T, 4>), pg, dim3(kThreads), plds, s, kb, (int)batch, (int)n_in, (const T*)x, (T*)phi); break;
      case 8: hipLaunchKernelGGL((phi_rows_kernel<T, 8>), pg, dim3(kThreads), plds, s, kb, (int)batch, (int)n_in, (const T*)x, (T*)phi); break;
      case 12: hipLaunchKernelGGL((phi_rows_kernel<T, 12>), pg, dim3(kThreads), plds, s, kb, (int)batch, (int)n_in, (const T*)x, (T*)phi); break;
      case 16: hipLaunchKernelGGL((phi_rows_kernel<T, 16>), pg, dim3(kThreads), plds, s, kb, (int)batch, (int)n_in, (const T*)x, (T*)phi); break;
      default: hipLaunchKernelGGL((phi_rows_kernel<T, 24>), pg, dim3(kThreads), plds, s, kb, (int)batch, (int)n_in, (const T*)x, (T*)phi); break;
    }
    int rc = check_launch("phi_rows");
    if (rc) return rc;
  }
  if constexpr (sizeof(T) == 2) {
    if (ld % 64 == 0) {
      if (bias_done) *bias_done = bias != nullptr;
      return gemm_nt(batch, n_out, ld, phi, ld, c, ld, y, n_out, false, gws, gws_bytes, s, bias);
    }
  }
  const size_t lds = (size_t)2 * (BM + TI) * 128;
  auto kern = p_dma_kernel<T, TM, FW, KF_KIND_BSPLINE, 2>;
  if (!reserve_lds((const void*)kern, lds))
    return fail(KF_ELAUNCH, "F: cannot reserve %zu bytes of LDS", lds);
  const int n_m = (int)((batch + BM - 1) / BM), n_n = (int)((n_out + TI - 1) / TI);
  hipLaunchKernelGGL(kern, dim3(n_m * n_n), dim3(256), lds, s, kb, (int)batch, (int)n_out, n_n * TI, (int)ld,
                     (const T*)nullptr, (const T*)phi, (int)ld, (const T*)c, (T*)y, (float*)nullptr);
  return check_launch("F");
}

// Narrow layers (at most 8 outputs, or inputs x basis functions <= 64 with at most 4 inputs):
// row streaming. Chebyshev-family layers with at most 8 outputs and 128 inputs first fold the
// coefficients into the workspace's feature-major block and run one lane per (row, input).
bool f_streams(const KBasis& kb, int64_t n_in, int64_t n_out) {
  return kb.kind != KF_KIND_RATIONAL && (n_out <= 8 || (n_in <= 4 && n_in * kb.K <= 64 && n_in * 16 <= 64));
}

template <typename T, int KM, int L, int NC, int OM>
int launch_f_lanes(const KBasis& kb, int64_t batch, int64_t n_in, int64_t n_out, const void* x, const void* w,
                   const void* cf, void* y, int64_t OUTP, int64_t INP, hipStream_t s) {
  constexpr int R = 64 / L, WPB = kThreads / 64;
  const int64_t waves = (batch + R - 1) / R;
  const int64_t blocks = std::min<int64_t>((waves + WPB - 1) / WPB, 2048);
  hipLaunchKernelGGL((f_lanes_kernel<T, KM, L, NC, OM>), dim3((unsigned)blocks), dim3(kThreads), 0, s, kb, (int)batch,
                     (int)n_in, (int)n_out, (const T*)x, (const T*)w, (const T*)cf, (T*)y, (int)OUTP, (int)INP);
  return check_launch("F lanes");
}

template <typename T, int KM>
int pick_f_lanes(const KBasis& kb, int64_t batch, int64_t n_in, int64_t n_out, const void* x, const void* w,
                 const void* cf, void* y, int64_t OUTP, int64_t INP, hipStream_t s) {
  const auto go = [&](auto l_tag, auto nc_tag) {
    constexpr int L = decltype(l_tag)::value, NC = decltype(nc_tag)::value;
    if (n_out == 1) return launch_f_lanes<T, KM, L, NC, 1>(kb, batch, n_in, n_out, x, w, cf, y, OUTP, INP, s);
    return launch_f_lanes<T, KM, L, NC, 8>(kb, batch, n_in, n_out, x, w, cf, y, OUTP, INP, s);
  };
  using I16 = std::integral_constant<int, 16>;
  using I64 = std::integral_constant<int, 64>;
  using N1 = std::integral_constant<int, 1>;
  using N2 = std::integral_constant<int, 2>;
  if (n_in <= 16) return go(I16{}, N1{});
  if (n_in <= 64) return go(I64{}, N1{});
  return go(I64{}, N2{});
}

// whether the lane kernel takes the layer: registers for NC x OM x KM coefficients per lane
inline bool f_lanes_fit(const KBasis& kb, int64_t n_in, int64_t n_out) {
  if (kb.kind != KF_KIND_CHEB || n_out > 8 || n_in > 128) return false;
  const int km = kb.n_t <= 8 ? 8 : 16;
  const int nc = n_in <= 64 ? 1 : 2, om = n_out == 1 ? 1 : 8;
  return kb.n_t <= 16 && nc * om * km <= 128;
}

template <typename T, int KM>
int launch_f_stream(const KBasis& kb, int64_t batch, int64_t n_in, int64_t n_out, const void* x, const void* w,
                    const void* c, void* y, hipStream_t s) {
  if (n_out <= 8) {
    dim3 grid((unsigned)((batch + kThreads - 1) / kThreads));
    hipLaunchKernelGGL((f_stream_kernel<T, KM>), grid, dim3(kThreads), 0, s, kb, (int)batch, (int)n_in, (int)n_out,
                       (const T*)x, (const T*)w, (const T*)c, (T*)y);
  } else {  // at most 4 inputs (f_streams): rows of 128 x chunks of 64 outputs
    if (n_in > 4) return fail(KF_EINVAL, "F: the wide streaming route takes at most 4 inputs");
    dim3 grid((unsigned)((batch + 127) / 128), (unsigned)((n_out + 63) / 64));
    hipLaunchKernelGGL((f_wide_kernel<T, KM>), grid, dim3(kThreads), 0, s, kb, (int)batch, (int)n_in, (int)n_out,
                       (const T*)x, (const T*)w, (const T*)c, (T*)y);
  }
  return check_launch("F stream");
}

template <typename T>
// bias (dtype, n_out) or NULL: added where the route's last kernel can take it (the register-A
// kernel's per-output constant, the GEMM core's epilogue), which sets *bias_done; otherwise the
// caller adds it.
int run_F(const KBasis& kb, const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void* x,
          const void* w, const void* c, void* y, void* ws, hipStream_t s, const void* bias = nullptr,
          bool* bias_done = nullptr) {
  const bool has_w = w != nullptr;
  const bool cheb = kb.kind == KF_KIND_CHEB;
  const bool weighted = features_weighted(b, w);
  if constexpr (sizeof(T) == 4)
    if (bspline_sparse(b, dtype)) return launch_f_sparse<T>(kb, b->spline_k, batch, n_in, n_out, x, w, c, y, s);
  const WsF LW = ws_f(b, dtype, batch, n_in, n_out, weighted);
  // the folded copy holds n_t features (the workspace is sized for at least n_tp of them)
  const bool lanes_ws = (size_t)kb.n_t * LW.OUTP * LW.INP * elt_size(dtype) <= LW.total;
  if (batch >= 1024 && lanes_ws && f_lanes_fit(kb, n_in, n_out)) {
    const WsF& L = LW;
    int rc = launch_permute<T>(kb, n_out, n_in, L.OUTP, L.INP, kb.n_t, c, ws, kPermFM, s);
    if (rc) return rc;
    if (kb.n_t <= 8) return pick_f_lanes<T, 8>(kb, batch, n_in, n_out, x, w, ws, y, L.OUTP, L.INP, s);
    return pick_f_lanes<T, 16>(kb, batch, n_in, n_out, x, w, ws, y, L.OUTP, L.INP, s);
  }
  if (batch >= 1024 && f_streams(kb, n_in, n_out)) {
    if (kb.K <= 4) return launch_f_stream<T, 4>(kb, batch, n_in, n_out, x, w, c, y, s);
    if (kb.K <= 8) return launch_f_stream<T, 8>(kb, batch, n_in, n_out, x, w, c, y, s);
    if (kb.K <= 12) return launch_f_stream<T, 12>(kb, batch, n_in, n_out, x, w, c, y, s);
    return launch_f_stream<T, 16>(kb, batch, n_in, n_out, x, w, c, y, s);
  }
  WsF L = ws_f(b, dtype, batch, n_in, n_out, weighted);
  char* base = (char*)ws;
  void* cfm = base;
  float* z = (float*)(base + L.cfm);
  float* wz = weighted && cheb ? (float*)(base + L.cfm + L.z) : nullptr;
  void* phi = base + L.cfm + L.z + L.wz;
  if (L.cfg == F_REGA) {
    float* part0 = L.skip0 ? (float*)(base + L.cfm + L.z + L.wz + L.phi) : nullptr;
    float* ysum = L.skip0 ? (float*)(base + L.cfm + L.z + L.wz + L.phi + L.part0) : nullptr;
    int rc = launch_permute<T>(kb, n_out, n_in, L.OUTP, L.INP, L.n_tp, c, cfm, kPermC16, s, L.skip0 ? 1 : 0, part0);
    if (rc) return rc;
    if (L.INP % 16 || L.BP % 32) return fail(KF_EINVAL, "F: workspace layout not aligned");
    long n = (L.INP + 63) / 64 * L.BP * (64 / (16 / (long)sizeof(T)));
    long blocks = (n + kThreads - 1) / kThreads;
    if (blocks > 65535 * 4) blocks = 65535 * 4;
    // the same launch totals the feature-0 partial sums in blocks of its own
    const long sblocks = L.skip0 ? (L.OUTP + 7) / 8 : 0;
    const int vin = rows_vec<T>(n_in, x) && rows_vec<T>(n_in, w);
    hipLaunchKernelGGL(zmapc_kernel<T>, dim3((unsigned)(blocks + sblocks)), dim3(kThreads), 0, s, (int)batch,
                       (int)n_in, (int)L.BP, (int)L.INP, kb.input_map, vin, (const T*)x, (const T*)w, z, wz,
                       (int)blocks, (int)(L.INP / 16), (int)L.OUTP, part0, ysum, 0,
                       (const T*)(L.skip0 ? bias : nullptr), (int)n_out);
    rc = check_launch("zmapc");
    if (rc) return rc;
    if (bias_done) *bias_done = L.skip0 && bias;
    if (weighted) return launch_f_rega<true, false>(L, batch, n_out, z, wz, cfm, nullptr, y, s);
    if (L.skip0) return launch_f_rega<false, true>(L, batch, n_out, z, nullptr, cfm, ysum, y, s);
    return launch_f_rega<false, false>(L, batch, n_out, z, nullptr, cfm, nullptr, y, s);
  }
  // B-spline or rational, unweighted, in K a whole number of 128-byte stages: Phi (B, in K) in the
  // reference's layout, then the flat GEMM Phi c^T on p_dma_kernel (no coefficient permute)
  constexpr int EPS = 128 / (int)sizeof(T);
  const long dma_tiles = ((batch + 255) / 256) * ((n_out + 255) / 256);  // at least half a round of the CUs
  void* gws = base + L.cfm + L.z + L.wz + L.phi + L.part0 + L.ysum;
  if constexpr (sizeof(T) == 2) {
    // GR-KAN degrees in bf16: phi^(m)(x) (times w) in the (B, in) layout, then the GEMM phi c^T
    if (rational_fast(kb, n_in) && n_in % 64 == 0 && kb.order <= 2 && aligned16(x) && aligned16(c) &&
        (!has_w || aligned16(w))) {
      long blocks = ((long)batch * (n_in / 8) + 255) / 256;
      if (blocks > 65535 * 4) blocks = 65535 * 4;
      auto map = kb.order == 0   ? rational_map_kernel<bf16, bf16, 0>
                 : kb.order == 1 ? rational_map_kernel<bf16, bf16, 1>
                                 : rational_map_kernel<bf16, bf16, 2>;
      hipLaunchKernelGGL(map, dim3((unsigned)blocks), dim3(256), 0, s, kb, (int)batch, (int)n_in, (const bf16*)x,
                         (const bf16*)w, (const float*)nullptr, (bf16*)phi);
      int rc = check_launch("rational features");
      if (rc) return rc;
      if (bias_done) *bias_done = bias != nullptr;
      return gemm_nt(batch, n_out, n_in, phi, n_in, c, n_in, y, n_out, false, gws, L.gemm, s, bias);
    }
  }
  const bool identity_fold = kb.kind == KF_KIND_BSPLINE || kb.kind == KF_KIND_RATIONAL;
  const bool gemm_core = sizeof(T) == 2 && (n_in * kb.K) % 64 == 0;  // any tile count: the core splits
  if (identity_fold && !has_w && (n_in * kb.K) % EPS == 0 && aligned16(c) && aligned16(phi) && (dma_tiles >= 128 || gemm_core))
    return run_F_dma<T>(kb, batch, n_in, n_out, x, c, phi, y, gws, L.gemm, s, bias, bias_done);
  int rc = launch_permute<T>(kb, n_out, n_in, L.OUTP, L.INP, L.n_tp, c, cfm, kPermFM, s);
  if (rc) return rc;
  if (cheb) {
    long n = (long)L.BP * L.INP;
    long blocks = (n + kThreads - 1) / kThreads;
    if (blocks > 65535 * 4) blocks = 65535 * 4;
    hipLaunchKernelGGL(zmap_kernel<T>, dim3((unsigned)blocks), dim3(kThreads), 0, s, (int)batch, (int)n_in, (int)L.BP,
                       (int)L.INP, kb.input_map, (const T*)x, (const T*)w, z, wz);
    rc = check_launch("zmap");
    if (rc) return rc;
    if (weighted) return launch_f_cfg<T, true, true>(L, batch, n_out, kb.n_t, z, wz, cfm, nullptr, y, s);
    return launch_f_cfg<T, true, false>(L, batch, n_out, kb.n_t, z, nullptr, cfm, nullptr, y, s);
  }
  // precomputed features phi_fm[b][j][i] (BP, n_t, INP)
  rc = launch_features<T, false>(kb, batch, n_in, L.BP, L.INP, x, phi, (long)L.n_tp * L.INP, (long)L.INP, 1L, false,
                                 s);
  if (rc) return rc;
  if (has_w) {
    long n = (long)batch * L.n_tp * L.INP;
    long blocks = (n + kThreads - 1) / kThreads;
    if (blocks > 65535 * 4) blocks = 65535 * 4;
    if (blocks > 0)
      hipLaunchKernelGGL(scale_phi_kernel<T>, dim3((unsigned)blocks), dim3(kThreads), 0, s, (int)batch, (int)n_in,
                         L.n_tp, (int)L.INP, (const T*)w, (T*)phi);
    rc = check_launch("scale_phi");
    if (rc) return rc;
  }
  return launch_f_cfg<T, false, false>(L, batch, n_out, kb.n_t, nullptr, nullptr, cfm, phi, y, s);
}

// Scratch of kf_F_noalloc: a file-scope device array, so that entry point never allocates. Every
// GPU the library runs on holds its own copy (at its own address) until the process ends. Host
// code never uses the array's name as an address: the address of the current device's copy comes
// from hipGetSymbolAddress, looked up once per device with that device current.
static __device__ __align__(256) unsigned char scratch[KF_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::once_flag g_scratch_once[kMaxDevices];
void* g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];

int scratch_of_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(KF_ELAUNCH, "kf_F_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(KF_EUNSUPPORTED, "kf_F_noalloc: device %d >= %d", dev, kMaxDevices);
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = g_scratch_err[dev] == hipSuccess ? p : nullptr;
  });
  if (g_scratch_err[dev] != hipSuccess || !g_scratch_ptr[dev])
    return fail(KF_ELAUNCH, "kf_F_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                hipGetErrorString(g_scratch_err[dev]));
  *out = g_scratch_ptr[dev];
  return KF_OK;
}
// The layer's forward with its SiLU base branch and bias in the register-A contraction:
// coefficients folded into C16 blocks with the base weights as every chunk's last block, z and
// silu(x) in the chunked layout, the T_0 sums plus the bias as the per-output constant.
int run_F_base(const KBasis& kb, const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out,
               const void* x, const void* c, const void* bw, const void* bias, void* y, void* ws, hipStream_t s) {
  const WsF L = ws_f(b, dtype, batch, n_in, n_out, false, true);
  char* base = (char*)ws;
  void* cfm = base;
  float* z = (float*)(base + L.cfm);
  float* sz = (float*)(base + L.cfm + L.z);
  float* part0 = (float*)(base + L.cfm + L.z + L.wz + L.phi);
  float* ysum = (float*)(base + L.cfm + L.z + L.wz + L.phi + L.part0);
  if (L.cfg != F_REGA || !L.skip0 || L.INP % 16 || L.BP % 32)
    return fail(KF_EINVAL, "kf_F_base: layer not on the register-A route");
  int rc = launch_permute<bf16>(kb, n_out, n_in, L.OUTP, L.INP, L.n_tp - 1, c, cfm, kPermC16, s, 1, part0, bw);
  if (rc) return rc;
  long n = (L.INP + 63) / 64 * L.BP * 8;
  long blocks = (n + kThreads - 1) / kThreads;
  if (blocks > 65535 * 4) blocks = 65535 * 4;
  const long sblocks = (L.OUTP + 7) / 8;
  const int vin = rows_vec<bf16>(n_in, x);
  hipLaunchKernelGGL(zmapc_kernel<bf16>, dim3((unsigned)(blocks + sblocks)), dim3(kThreads), 0, s, (int)batch,
                     (int)n_in, (int)L.BP, (int)L.INP, kb.input_map, vin, (const bf16*)x, (const bf16*)nullptr, z, sz,
                     (int)blocks, (int)(L.INP / 16), (int)L.OUTP, part0, ysum, 1, (const bf16*)bias, (int)n_out);
  rc = check_launch("zmapc");
  if (rc) return rc;
  return launch_f_rega<false, true, true>(L, batch, n_out, z, sz, cfm, ysum, y, s);
}

// B-splines: Phi with silu(x) and zero padding after each row's features, and the coefficients
// with W and zeros after each row's: the base branch is features of the one GEMM-core product,
// whose epilogue adds the bias.
int run_F_base_bspline(const KBasis& kb, const kf_basis* b, int64_t batch, int64_t n_in, int64_t n_out, const void* x,
                       const void* c, const void* bw, const void* bias, void* y, void* ws, hipStream_t s) {
  const WsFB L = ws_f_base_bspline(b, KF_BF16, batch, n_in, n_out);
  char* base = (char*)ws;
  bf16* phi = (bf16*)base;
  bf16* cf = (bf16*)(base + L.phi);
  void* gws = base + L.phi + L.cf;
  if (!aligned16(c) || (n_in * kb.K) % 8) return fail(KF_EINVAL, "kf_F_base: coefficient rows not 16-byte aligned");
  const long n = (long)n_out * (L.ld / 8);
  long blocks = (n + kThreads - 1) / kThreads;
  if (blocks > 65535 * 4) blocks = 65535 * 4;
  hipLaunchKernelGGL(base_coef_kernel<bf16>, dim3((unsigned)blocks), dim3(kThreads), 0, s, (int)n_out, (int)n_in, kb.K,
                     (long)L.ld, (const bf16*)c, (const bf16*)bw, cf);
  int rc = check_launch("base_coef");
  if (rc) return rc;
  rc = launch_phi_block<bf16>(kb, batch, n_in, x, phi, (long)L.ld, (int)(L.ld - n_in * kb.K), s);
  if (rc) return rc;
  return gemm_nt(batch, n_out, L.ld, phi, L.ld, cf, L.ld, y, n_out, false, gws, L.gemm, s, bias);
}

}  // namespace

extern "C" {

int kf_F(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void* x, const void* w,
         const void* c, void* y, void* workspace, size_t workspace_bytes, void* stream) {
  g_err.clear();
  int rc = validate_common(b, dtype, batch, n_in, n_out);
  if (rc) return rc;
  if (batch == 0 || n_out == 0) return KF_OK;
  hipStream_t s = (hipStream_t)stream;
  if (n_in == 0) return dtype == KF_BF16 ? zero_fill<bf16>(y, (long)batch * n_out, s) : zero_fill<float>(y, (long)batch * n_out, s);
  if (!x || !c || !y) return fail(KF_EINVAL, "kf_F: NULL array");
  size_t need = ws_f(b, dtype, batch, n_in, n_out, features_weighted(b, w)).total;
  if (!workspace || workspace_bytes < need)
    return fail(KF_EWORKSPACE, "kf_F: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  if (reinterpret_cast<uintptr_t>(workspace) & 255)
    return fail(KF_EWORKSPACE, "kf_F: workspace must be 256-byte aligned");
  KBasis kb = to_kbasis(b);
  if (dtype == KF_BF16) return run_F<bf16>(kb, b, dtype, batch, n_in, n_out, x, w, c, y, workspace, s);
  return run_F<float>(kb, b, dtype, batch, n_in, n_out, x, w, c, y, workspace, s);
}

int kf_F_noalloc(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void* x,
                 const void* w, const void* c, void* y, void* stream) {
  g_err.clear();
  int rc = validate_common(b, dtype, batch, n_in, n_out);
  if (rc) return rc;
  if (batch == 0 || n_out == 0) return KF_OK;
  hipStream_t s = (hipStream_t)stream;
  if (n_in == 0) return dtype == KF_BF16 ? zero_fill<bf16>(y, (long)batch * n_out, s) : zero_fill<float>(y, (long)batch * n_out, s);
  if (!x || !c || !y) return fail(KF_EINVAL, "kf_F_noalloc: NULL array");
  const size_t need = ws_f(b, dtype, batch, n_in, n_out, features_weighted(b, w)).total;
  if (need > KF_NOALLOC_SCRATCH_BYTES)
    return fail(KF_EWORKSPACE, "kf_F_noalloc: these shapes need %zu bytes of scratch, the static scratch holds %zu",
                need, (size_t)KF_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  rc = scratch_of_current_device(&ws);
  if (rc) return rc;
  KBasis kb = to_kbasis(b);
  if (dtype == KF_BF16) return run_F<bf16>(kb, b, dtype, batch, n_in, n_out, x, w, c, y, ws, s);
  return run_F<float>(kb, b, dtype, batch, n_in, n_out, x, w, c, y, ws, s);
}

int kf_F_base(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void* x, const void* c,
              const void* base_w, const void* bias, void* y, void* workspace, size_t workspace_bytes, void* stream) {
  g_err.clear();
  int rc = validate_common(b, dtype, batch, n_in, n_out);
  if (rc) return rc;
  if (batch == 0 || n_out == 0) return KF_OK;
  if (n_in == 0) return fail(KF_EINVAL, "kf_F_base: no inputs");
  if (!x || !c || !base_w || !y) return fail(KF_EINVAL, "kf_F_base: NULL array");
  if (!f_base_route(b, dtype, batch, n_in, n_out))
    return fail(KF_EUNSUPPORTED, "kf_F_base: this layer does not run the fused base branch (kf_base_fused)");
  const bool sparse = bspline_sparse(b, dtype), spline = b->kind == KF_KIND_BSPLINE;
  const size_t need = sparse   ? ws_base_sparse(KF_OP_F_BASE, b, dtype, batch, n_in, n_out)
                      : spline ? ws_f_base_bspline(b, dtype, batch, n_in, n_out).total
                               : ws_f(b, dtype, batch, n_in, n_out, false, true).total;
  if (need && (!workspace || workspace_bytes < need))
    return fail(KF_EWORKSPACE, "kf_F_base: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  if (need && (reinterpret_cast<uintptr_t>(workspace) & 255))
    return fail(KF_EWORKSPACE, "kf_F_base: workspace must be 256-byte aligned");
  KBasis kb = to_kbasis(b);
  if (sparse)  // float32: W as basis function K of the sparse route, the bias in its stores
    return launch_f_sparse<float>(kb, b->spline_k, batch, n_in, n_out, x, nullptr, c, y, (hipStream_t)stream, base_w,
                                  bias);
  if (spline) return run_F_base_bspline(kb, b, batch, n_in, n_out, x, c, base_w, bias, y, workspace, (hipStream_t)stream);
  return run_F_base(kb, b, dtype, batch, n_in, n_out, x, c, base_w, bias, y, workspace, (hipStream_t)stream);
}

int kf_F_bias(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void* x, const void* w,
              const void* c, const void* bias, void* y, void* workspace, size_t workspace_bytes, void* stream) {
  g_err.clear();
  int rc = validate_common(b, dtype, batch, n_in, n_out);
  if (rc) return rc;
  if (batch == 0 || n_out == 0) return KF_OK;
  hipStream_t s = (hipStream_t)stream;
  if (!y || (n_in > 0 && (!x || !c))) return fail(KF_EINVAL, "kf_F_bias: NULL array");
  bool done = false;
  if (n_in == 0) {
    rc = dtype == KF_BF16 ? zero_fill<bf16>(y, (long)batch * n_out, s) : zero_fill<float>(y, (long)batch * n_out, s);
  } else {
    size_t need = ws_f(b, dtype, batch, n_in, n_out, features_weighted(b, w)).total;
    if (!workspace || workspace_bytes < need)
      return fail(KF_EWORKSPACE, "kf_F_bias: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
    if (reinterpret_cast<uintptr_t>(workspace) & 255)
      return fail(KF_EWORKSPACE, "kf_F_bias: workspace must be 256-byte aligned");
    KBasis kb = to_kbasis(b);
    rc = dtype == KF_BF16 ? run_F<bf16>(kb, b, dtype, batch, n_in, n_out, x, w, c, y, workspace, s, bias, &done)
                          : run_F<float>(kb, b, dtype, batch, n_in, n_out, x, w, c, y, workspace, s, bias, &done);
  }
  if (rc || !bias || done) return rc;
  long n = (long)batch * n_out;
  long blocks = (n + kThreads - 1) / kThreads;
  if (blocks > 65535 * 4) blocks = 65535 * 4;
  if (dtype == KF_BF16)
    hipLaunchKernelGGL(bias_rows_kernel<bf16>, dim3((unsigned)blocks), dim3(kThreads), 0, s, (int)batch, (int)n_out,
                       (const bf16*)bias, (bf16*)y);
  else
    hipLaunchKernelGGL(bias_rows_kernel<float>, dim3((unsigned)blocks), dim3(kThreads), 0, s, (int)batch, (int)n_out,
                       (const float*)bias, (float*)y);
  return check_launch("bias rows");
}

}  // extern "C"
