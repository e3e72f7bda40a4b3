// Host-side helpers shared by the entry points of libkfhip.so (kf_abi*.hip): error reporting,
// argument validation, basis descriptors, workspace layouts and the launchers several entry
// points use.
#pragma once

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <set>
#include <string>
#include <utility>

#include "kf_kernels.h"
#include "kf_sparse.h"

namespace kfabi {

using namespace kf;


extern thread_local std::string g_err;

int fail(int code, const char* fmt, ...);

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(KF_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
  return KF_OK;
}

// The dynamic-LDS ceiling of a kernel above the default 64 KB is raised once per (device, kernel)
// to the whole 160 KB of a CU; launches then pass their actual size. The table of kernels already
// raised is the library's only mutable state besides the scratch addresses, and is guarded.
// Raises a kernel's dynamic-LDS ceiling above the default 64 KB, once per (device, kernel);
// false when the request cannot be met.
bool reserve_lds(const void* kern, size_t lds);

// C = A B^T (+ bias[n]) on the bf16 MFMA GEMM core (kf_gemm_nt.hip): A (M, lda), B (N, ldb) bf16
// with k contiguous, K a multiple of 64, rows 16-byte aligned; C (M, ldc) bf16 or float32; bias
// bf16 (N) or NULL. A split of the reduction needs gemm_nt_workspace(M, N, K) bytes of workspace.
size_t gemm_nt_workspace(long M, long N, long K);
int gemm_nt(long M, long N, long K, const void* A, long lda, const void* B, long ldb, void* C, long ldc, bool out_f32,
            void* ws, size_t ws_bytes, hipStream_t s, const void* bias = nullptr);

inline int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }
inline size_t align256(size_t v) { return (v + 255) & ~size_t(255); }
inline int elt_size(int dtype) { return dtype == KF_BF16 ? 2 : 4; }

// tile constants shared by workspace sizing and launches
constexpr int CHUNK = 32;

inline int validate_basis(const kf_basis* b) {
  if (!b) return fail(KF_EINVAL, "basis descriptor is NULL");
  if (b->size < 1 || b->size > KF_MAX_K) return fail(KF_EINVAL, "basis size %d outside [1, %d]", b->size, KF_MAX_K);
  if (b->order < 0 || b->order > 8) return fail(KF_EUNSUPPORTED, "derivative order %d outside [0, 8]", b->order);
  if (b->n_t < 1 || b->n_t > KF_MAX_NT) return fail(KF_EINVAL, "n_t %d outside [1, %d]", b->n_t, KF_MAX_NT);
  switch (b->kind) {
    case KF_KIND_CHEB:
      if (!b->fold) return fail(KF_EINVAL, "cheb basis needs the fold matrix");
      if (b->input_map != KF_MAP_TANH && b->input_map != KF_MAP_IDENTITY && b->input_map != KF_MAP_TANH_SQ)
        return fail(KF_EINVAL, "unknown input map %d", b->input_map);
      break;
    case KF_KIND_BSPLINE:
      if (b->spline_k < 0 || b->spline_k > 5) return fail(KF_EUNSUPPORTED, "B-spline degree %d outside [0, 5]", b->spline_k);
      if (b->n_knots != b->size + b->spline_k + 1)
        return fail(KF_EINVAL, "n_knots %d != size + degree + 1 = %d", b->n_knots, b->size + b->spline_k + 1);
      if (b->n_t != b->size) return fail(KF_EINVAL, "bspline n_t must equal size");
      if (!b->knots || !b->knots_cmp) return fail(KF_EINVAL, "bspline basis needs knot tables");
      break;
    case KF_KIND_RATIONAL:
      if (b->size != 1 || b->n_t != 1) return fail(KF_EINVAL, "rational basis has size 1");
      if (b->num_deg < 0 || b->den_deg < 1 || b->num_deg + 1 + b->den_deg > kRatMaxParams)
        return fail(KF_EUNSUPPORTED, "rational degrees (%d, %d) unsupported", b->num_deg, b->den_deg);
      if (!b->num || !b->den) return fail(KF_EINVAL, "rational basis needs num/den");
      if (b->group_size < 1) return fail(KF_EINVAL, "group_size must be >= 1");
      break;
    default:
      return fail(KF_EINVAL, "unknown basis kind %d", b->kind);
  }
  return KF_OK;
}

inline int validate_common(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out) {
  int rc = validate_basis(b);
  if (rc) return rc;
  if (dtype != KF_F32 && dtype != KF_BF16) return fail(KF_EINVAL, "unsupported dtype %d", dtype);
  if (batch < 0 || n_in < 0 || n_out < 0) return fail(KF_EINVAL, "negative dimension");
  if (batch > (1LL << 31) - 1024 || n_in > (1 << 24) || n_out > (1 << 24))
    return fail(KF_EINVAL, "dimension too large");
  if (b->kind == KF_KIND_RATIONAL && n_in % b->group_size)
    return fail(KF_EINVAL, "group_size %d does not divide n_in %lld", b->group_size, (long long)n_in);
  return KF_OK;
}

inline KBasis to_kbasis(const kf_basis* b) {
  KBasis k;
  memset(&k, 0, sizeof(k));
  k.kind = b->kind;
  k.K = b->size;
  k.n_t = b->n_t;
  k.order = b->order;
  k.input_map = b->input_map;
  k.spline_k = b->spline_k;
  k.n_knots = b->n_knots;
  k.num_deg = b->num_deg;
  k.den_deg = b->den_deg;
  k.group_size = b->group_size > 0 ? b->group_size : 1;
  k.knots = b->knots;
  k.knots_cmp = b->knots_cmp;
  k.num = b->num;
  k.den = b->den;
  k.knots_uniform = b->kind == KF_KIND_BSPLINE ? b->knots_uniform : nullptr;
  if (b->kind == KF_KIND_CHEB) {
    for (int r = 0; r < b->size; ++r)
      for (int c = 0; c < b->n_t; ++c) k.fold[r * KF_MAX_NT + c] = b->fold[r * b->n_t + c];
  } else {
    for (int r = 0; r < b->size; ++r) k.fold[r * KF_MAX_NT + r] = 1.f;  // identity
  }
  return k;
}

// Whether a call's features carry a per-element weight: an explicit w, or the (1 - z^2) factor of
// a reduced tanh fold. The workspace size checks and the workspace layouts of F and G both use it.
inline bool features_weighted(const kf_basis* b, const void* w) {
  return w != nullptr || (b->kind == KF_KIND_CHEB && b->input_map == KF_MAP_TANH_SQ);
}

inline int nt_bucket(int n) { return n <= 4 ? 4 : n <= 8 ? 8 : n <= 12 ? 12 : n <= 16 ? 16 : 24; }

// F tile configurations: (BM, BN, waves along M, waves along N), 512 threads.
struct FCfg {
  int bm, bn, wm, wn;
};
constexpr FCfg F_CFGS[] = {{256, 192, 4, 2}, {256, 256, 2, 4}, {256, 128, 4, 2}};
constexpr int N_CUS = 256;

// The configuration with the fewest tile-area x dispatch rounds (whole-GPU
// waves of 256 workgroups); ties keep the larger tile.
inline int pick_f_cfg(int64_t batch, int64_t n_out) {
  int best = 0;
  double best_cost = 1e300;
  for (int k = 0; k < 3; ++k) {
    const FCfg& c = F_CFGS[k];
    int64_t tiles = ((batch + c.bm - 1) / c.bm) * ((n_out + c.bn - 1) / c.bn);
    int64_t rounds = (tiles + N_CUS - 1) / N_CUS;
    double cost = (double)rounds * c.bm * c.bn;
    if (cost < best_cost * 0.999) {
      best = k;
      best_cost = cost;
    }
  }
  return best;
}

struct WsF {
  int cfg, n_tp;
  bool skip0;  // register-A kernel without feature 0 (T_0 = 1 folded into a per-output sum)
  int64_t INP, OUTP, BP;
  size_t cfm, z, wz, phi, part0, ysum, gemm, total;
};
// bf16 Chebyshev plans run the register-A F kernel: workgroup tile (128 RA_TM) x
// (32 RA_TN), four waves along the batch times RA_WN along the outputs (wave
// tile (32 RA_TM) x (32 RA_TN / RA_WN)).
constexpr int F_REGA = -1;
constexpr int RA_TM = 1, RA_TN = 6, RA_WN = 1, RA_NWM = 8, RA_BM = 32 * RA_NWM * RA_TM, RA_BN = 32 * RA_TN;
constexpr int RA_NBUF = 4;  // coefficient stage buffers (prefetch distance RA_NBUF - 1 stages)
inline bool f_uses_rega(const kf_basis* b, int dtype) { return b->kind == KF_KIND_CHEB && dtype == KF_BF16; }
// odd feature counts with an unpadded, unrolled variant
inline bool f_rega_unpadded(int n_t, int64_t n_in) { return n_t == 9; }

// base: the fused SiLU base branch (kf_F_base): the register-A kernel's chunks run T_1 ..
// T_{n_t - 1} and silu(x) (n_tp = n_t, silu(x) in the wz buffer).
inline WsF ws_f(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out, bool has_w,
                bool base = false) {
  WsF w;
  const bool rega = f_uses_rega(b, dtype);
  w.cfg = rega ? F_REGA : pick_f_cfg(batch, n_out);
  const int bm = rega ? RA_BM : F_CFGS[w.cfg].bm, bn = rega ? RA_BN : F_CFGS[w.cfg].bn;
  w.INP = round_up(n_in, CHUNK);
  w.OUTP = round_up(n_out, bn);
  w.BP = round_up(batch, bm);
  const int es = elt_size(dtype);
  const bool cheb = b->kind == KF_KIND_CHEB;
  const int fps = dtype == KF_BF16 ? 2 : 1;
  w.skip0 = rega && !has_w && b->n_t >= 2;
  const int n_run = b->n_t - (w.skip0 ? 1 : 0);  // features the contraction runs over
  w.n_tp = rega && f_rega_unpadded(n_run, n_in) ? n_run : (n_run + fps - 1) / fps * fps;
  // the register-A kernel needs chunks of at least RA_NBUF / 2 (and 2) stages
  const int min_tp = RA_NBUF < 4 ? 4 : RA_NBUF;
  if (rega && w.n_tp < min_tp) w.n_tp = min_tp;
  if (base) w.n_tp = n_run + 1;
  w.cfm = align256((size_t)w.n_tp * w.OUTP * w.INP * es);
  w.z = cheb ? align256((size_t)w.BP * w.INP * sizeof(float)) : 0;
  w.wz = cheb && (has_w || base) ? align256((size_t)w.BP * w.INP * sizeof(float)) : 0;
  w.phi = cheb ? 0 : align256((size_t)w.BP * w.n_tp * w.INP * es);
  w.part0 = w.skip0 ? align256((size_t)(w.INP / 16) * w.OUTP * sizeof(float)) : 0;
  w.ysum = w.skip0 ? align256((size_t)w.OUTP * sizeof(float)) : 0;
  // bf16 B-spline and rational plans contract on the GEMM core (split partial sums)
  const bool gemm = dtype == KF_BF16 && !cheb;
  w.gemm = gemm ? gemm_nt_workspace(batch, n_out, n_in * b->size) : 0;
  w.total = w.cfm + w.z + w.wz + w.phi + w.part0 + w.ysum + w.gemm;
  return w;
}
// P / G configurations. The MFMA waves split the features in two groups of
// FW = ceil(n_t / 2) (FW in {2,3,4,5,6,8,12}); TM 32-row tiles per wave keep
// the accumulators at <= 192 registers. P: 4x2 waves (512 threads, 64-byte
// stages); G: warp-specialised for Chebyshev plans (4 MFMA waves + 4
// producer waves, 128-byte stages, 64 from FW = 8), else 2x2 waves.
constexpr int FW_LIST[] = {2, 3, 4, 5, 6, 8, 12};
inline int fw_index(int n_t) {
  const int need = (n_t + 1) / 2;
  for (int k = 0; k < 7; ++k)
    if (FW_LIST[k] >= need) return k;
  return 6;
}
inline int g_tm(int fw) { return fw <= 6 ? 2 : 1; }
inline int g_rb(int fw) { return fw <= 6 ? 128 : 64; }

struct WsP {
  int cfg, ntb;
  bool p8;   // bf16 Chebyshev with 7 or 8 features: p8_kernel (256 x (8 x 48) tiles)
  bool p12;  // bf16 B-splines with 9 to 12 features: p8_kernel with 12 slots (256 x (12 x 32) tiles)
  int64_t INP, OUTP;
  size_t cfmt, gpad, hbuf, gemm, total;
};
// P with FW <= 4 runs the copy kernel (p_dma_kernel; 4 x FW accumulator tiles in AGPRs); it needs
// g with whole 128-byte stages of columns and 16-byte aligned rows, else a zero-padded copy of g
// in the workspace.
inline bool p_uses_dma(int cfg) { return FW_LIST[cfg] <= 6; }
constexpr int p_dma_tm(int fw) { return fw <= 4 ? 4 : 2; }  // row tiles per wave (LDS: two stages fit)
inline int64_t p_stage_cols(int dtype) { return 128 / elt_size(dtype); }
inline bool p_needs_gpad(int64_t n_out, int dtype) { return n_out % p_stage_cols(dtype) != 0; }
inline WsP ws_p(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out) {
  WsP w;
  w.cfg = fw_index(b->n_t);
  w.ntb = 2 * FW_LIST[w.cfg];
  w.p8 = b->kind == KF_KIND_CHEB && dtype == KF_BF16 && w.ntb == 8;
  w.p12 = b->kind == KF_KIND_BSPLINE && dtype == KF_BF16 && w.ntb == 12 && b->spline_k == 3;
  // 96: whole tiles of p8_kernel (48) and p_dma_kernel (32); rational: flat tiles of 2 FW x 32 inputs
  w.INP = round_up(n_in, w.p8 ? 96 : b->kind == KF_KIND_RATIONAL ? 64 * FW_LIST[w.cfg] : 32);
  w.OUTP = round_up(n_out, p_uses_dma(w.cfg) ? p_stage_cols(dtype) : 32);
  w.cfmt = align256((size_t)w.ntb * w.INP * w.OUTP * elt_size(dtype));
  w.gpad = p_uses_dma(w.cfg) && p_needs_gpad(n_out, dtype) ? align256((size_t)batch * w.OUTP * elt_size(dtype)) : 0;
  // bf16 rational plans: H = g C^T on the GEMM core into float32 (the caller's h or hbuf)
  const bool rgemm = dtype == KF_BF16 && b->kind == KF_KIND_RATIONAL;
  w.hbuf = rgemm ? align256((size_t)batch * n_in * sizeof(float)) : 0;
  w.gemm = rgemm ? gemm_nt_workspace(batch, n_in, w.OUTP) : 0;
  w.total = w.cfmt + w.gpad + w.hbuf + w.gemm;
  return w;
}
constexpr size_t kSpGBytes = size_t(256) << 20;  // cap of the sparse G partial sums
// fp32 B-spline layers of degree <= 3 contract over the k + 1 non-zero splines of each (row,
// input): f_sparse_kernel, p_sparse_kernel, g_sparse_kernel (+ g_sparse_reduce)
inline bool bspline_sparse(const kf_basis* b, int dtype) {
  return b->kind == KF_KIND_BSPLINE && dtype == KF_F32 && b->spline_k >= 0 && b->spline_k <= 3 && b->size <= kSpKMax;
}

// G's row slices for the sparse kernels: about 512 workgroups, slices of whole 64-row groups,
// float partial sums capped at kSpGBytes
struct SpG {
  int nz, RS;
  size_t part;
};
inline SpG sparse_g_plan(int64_t batch, int64_t n_in, int64_t n_out, int K) {
  const long base = (long)((n_in + 3) / 4) * (long)((n_out + 63) / 64);
  long nz = (512 + base - 1) / base;
  const long groups = (long)((batch + 63) / 64);
  if (nz > groups) nz = groups;
  const size_t per = (size_t)n_out * n_in * K * sizeof(float);
  if (nz > 1 && (size_t)nz * per > kSpGBytes) nz = (long)(kSpGBytes / per);
  if (nz < 1) nz = 1;
  const long rs = ((batch + nz - 1) / nz + 63) / 64 * 64;
  SpG p;
  p.RS = (int)(rs > 0 ? rs : 64);
  p.nz = (int)((batch + p.RS - 1) / p.RS);
  if (p.nz < 1) p.nz = 1;
  p.part = align256((size_t)p.nz * per);
  return p;
}

struct WsG {
  int cfg;
  bool skip0;  // Chebyshev, unweighted: T_0 = 1 taken out of the contraction (column sums of g)
  bool g96;    // bf16 Chebyshev with at most 8 features run: g96_kernel (192 x 48 x 8 tiles)
  bool pre;    // features precomputed into phiT (other kinds, and Chebyshev plans on small grids)
  bool gdma;   // B-spline without batch splits: p_dma_kernel as the flat GEMM gT x phiT^T
  int nz;      // pre: batch splits of g_kernel (raw sums reduced by g_split_reduce when > 1)
  int64_t OUTP, BP, INP;
  size_t gt, zt, wt, part, colsum, phit, zpart, gemm, total;
};
constexpr size_t kGSplitBytes = size_t(256) << 20;  // cap of the split partial sums
constexpr long kGSplitMax = 64;                      // cap of the batch splits
constexpr int kGdmaFW = 4, kGdmaRows = 2 * kGdmaFW * 32;  // G on p_dma_kernel: phiT rows per tile
// base: kf_G_base (the batch padded to whole 64-row stages of the GEMM core, which contracts
// gT with silu(x)^T over it)
inline WsG ws_g(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out, bool has_w,
                bool base = false) {
  WsG w;
  if (bspline_sparse(b, dtype)) {
    w = WsG{};
    w.total = sparse_g_plan(batch, n_in, n_out, b->size).part;
    return w;
  }
  const bool cheb_kind = b->kind == KF_KIND_CHEB;
  w.skip0 = cheb_kind && !has_w && b->n_t >= 2;
  w.cfg = fw_index(b->n_t - (w.skip0 ? 1 : 0));
  w.g96 = cheb_kind && dtype == KF_BF16 && b->n_t - (w.skip0 ? 1 : 0) <= 8;
  w.pre = !cheb_kind;
  if (cheb_kind) {
    // the Chebyshev kernels keep one workgroup per output tile over the whole batch;
    // with fewer than 128 tiles the batch-split precomputed-feature path fills the chip
    const int fw = FW_LIST[w.cfg];
    const long bm = w.g96 ? 192 : 2 * g_tm(fw) * 32, bn = w.g96 ? 48 : 32;
    const long tiles = (round_up(n_out, bm) / bm) * (round_up(n_in, bn) / bn);
    if (tiles < 128) {
      w.pre = true;
      w.skip0 = w.g96 = false;
      w.cfg = fw_index(b->n_t);
    }
  }
  const int fw = FW_LIST[w.cfg];
  const int bm = w.g96 ? 192 : 2 * g_tm(fw) * 32;
  const int eps = w.g96 ? 32 : g_rb(fw) / elt_size(dtype);
  w.OUTP = round_up(n_out, bm);
  w.BP = round_up(batch, base ? 64 : eps);
  const bool flat = b->kind == KF_KIND_RATIONAL;  // g_kernel's flat tiles: 2 FW x 32 inputs
  w.INP = round_up(n_in, w.g96 ? 48 : flat ? 64 * fw : 32);
  const bool cheb = cheb_kind && !w.pre;
  w.gt = align256((size_t)w.OUTP * w.BP * elt_size(dtype));
  w.zt = cheb ? align256((size_t)w.INP * w.BP * sizeof(float)) : 0;
  w.wt = cheb && has_w ? align256((size_t)w.INP * w.BP * sizeof(float)) : 0;
  w.part = w.skip0 ? align256((size_t)((w.BP + 63) / 64) * w.OUTP * sizeof(float)) : 0;
  w.colsum = w.skip0 ? align256((size_t)w.OUTP * sizeof(float)) : 0;
  w.phit = w.zpart = 0;
  w.nz = 1;
  w.gdma = false;
  if (w.pre) {
    w.phit = align256((size_t)b->n_t * w.INP * w.BP * elt_size(dtype));
    // fewer output tiles than two rounds of the 256 CUs: split the batch
    const long tiles = (long)(w.OUTP / bm) * (w.INP / (flat ? 64 * fw : 32)), stages = w.BP / eps;
    if (tiles < 512) {
      const size_t per = (size_t)w.OUTP * w.INP * b->n_t * sizeof(float);
      long nz = (512 + tiles - 1) / tiles;
      if (nz > kGSplitMax) nz = kGSplitMax;
      if (nz > stages) nz = stages;
      if ((size_t)nz * per > kGSplitBytes) nz = (long)(kGSplitBytes / per);
      w.nz = nz > 1 ? (int)nz : 1;
    }
    w.zpart = w.nz > 1 ? align256((size_t)w.nz * w.OUTP * w.INP * b->n_t * sizeof(float)) : 0;
    // identity fold, one split, stages of 128 bytes (n_t <= 12): flat 256-row tiles of phiT
    w.gdma = b->kind == KF_KIND_BSPLINE && w.nz == 1 && g_rb(fw) == 128;
    if (w.gdma) {
      w.INP = round_up(n_in, kGdmaRows);
      w.phit = align256((size_t)b->n_t * w.INP * w.BP * elt_size(dtype));
    }
  }
  // bf16 rational plans contract on the GEMM core (split partial sums)
  w.gemm = dtype == KF_BF16 && b->kind == KF_KIND_RATIONAL ? gemm_nt_workspace(n_out, n_in, w.BP) : 0;
  if (dtype == KF_BF16 && b->kind == KF_KIND_BSPLINE) w.gemm = gemm_nt_workspace(n_out, n_in * b->size, w.BP);
  w.total = w.gt + w.zt + w.wt + w.part + w.colsum + w.phit + w.zpart + w.gemm;
  return w;
}

// The fused SiLU base branch (kf_F_base, kf_P_base, kf_G_base) rides the bf16 Chebyshev kernels:
// F on the register-A kernel with silu(x) as the last feature of every chunk (T_0 taken out, so
// n_t features a chunk: 9, or an even count of at least 6); layers narrow enough for F's
// streaming routes keep those. P on p8_kernel (the order-1 descriptor), G on g96_kernel.
// bf16 B-splines: F on the GEMM core with silu(x) and a ones column after each row's features;
// cubic with 11 basis functions: P on p8_kernel's 12 feature slots (W^T in the spare one); G on
// the GEMM core (features and silu(x) transposed).
inline bool f_base_route(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out) {
  if (bspline_sparse(b, dtype)) return b->order == 0 && b->size < kSpKMax;  // base weight as basis function K
  if (dtype != KF_BF16 || b->order != 0) return false;
  const bool narrow = n_out <= 8 || (n_in <= 4 && n_in * b->size <= 64 && n_in * 16 <= 64);
  if (batch >= 1024 && narrow) return false;
  if (b->kind == KF_KIND_BSPLINE) return (n_in * b->size) % 8 == 0;
  return f_uses_rega(b, dtype) && (b->n_t == 9 || (b->n_t % 2 == 0 && b->n_t >= 6));
}
// The base entry points on the sparse route (float32 B-splines): F and P stage W next to the
// coefficients themselves (no workspace); G needs its K + 1-feature partial sums and, after them,
// the bias gradient's slice partials (or, for the bias gradient alone, the column-sum kernels'
// scratch).
inline size_t ws_base_sparse(int op, const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out) {
  (void)dtype;
  if (op != KF_OP_G_BASE) return 0;
  const SpG sp = sparse_g_plan(batch, n_in, n_out, b->size + 1);
  const size_t bias = std::max((size_t)sp.nz * n_out * sizeof(float), kf_column_sums_workspace_bytes(batch, n_out));
  return sp.part + align256(bias);
}
// kf_F_base for B-splines: Phi with the base columns (B, ld), [c | W | 0] (OUT, ld) and the GEMM
// core's split partial sums; ld = IN K + IN rounded up to whole 64-element stages
struct WsFB {
  int64_t ld;
  size_t phi, cf, gemm, total;
};
inline WsFB ws_f_base_bspline(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out) {
  WsFB w;
  w.ld = round_up(n_in * b->size + n_in, 64);
  w.phi = align256((size_t)batch * w.ld * elt_size(dtype));
  w.cf = align256((size_t)n_out * w.ld * elt_size(dtype));
  w.gemm = gemm_nt_workspace(batch, n_out, w.ld);
  w.total = w.phi + w.cf + w.gemm;
  return w;
}
inline bool p_base_route(const kf_basis* b1, int dtype, int64_t batch, int64_t n_in, int64_t n_out) {
  if (bspline_sparse(b1, dtype)) return b1->order >= 1 && b1->size < kSpKMax;
  if (dtype != KF_BF16 || b1->order < 1) return false;
  const WsP w = ws_p(b1, dtype, batch, n_in, n_out);
  if (b1->kind == KF_KIND_BSPLINE) return w.p12 && b1->size < 12;
  return b1->kind == KF_KIND_CHEB && w.p8;
}
inline bool g_base_route(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out) {
  if (bspline_sparse(b, dtype)) return b->order == 0 && b->size < kSpKMax;
  if (dtype != KF_BF16 || b->order != 0) return false;
  const WsG w = ws_g(b, dtype, batch, n_in, n_out, false, true);
  // B-splines: features transposed input-major (the GEMM core's route of kf_G)
  if (b->kind == KF_KIND_BSPLINE) return w.pre && w.BP % 64 == 0 && (n_in * b->size) % 8 == 0;
  return b->kind == KF_KIND_CHEB && w.g96 && w.skip0 && !w.pre;
}
// workspace of kf_P_base: P's, one more coefficient row (W^T), hb = g W (float32) and the
// GEMM core's split partial sums
struct WsPB {
  WsP p;
  size_t cfmt, hb, gemm, total;
};
// (B-splines: the spare feature slot holds W^T, no hb)
inline WsPB ws_p_base(const kf_basis* b1, int dtype, int64_t batch, int64_t n_in, int64_t n_out) {
  WsPB w;
  w.p = ws_p(b1, dtype, batch, n_in, n_out);
  const bool spare = b1->kind == KF_KIND_BSPLINE;
  w.cfmt = align256((size_t)(w.p.ntb + (spare ? 0 : 1)) * w.p.INP * w.p.OUTP * elt_size(dtype));
  w.hb = spare ? 0 : align256((size_t)batch * n_in * sizeof(float));
  w.gemm = spare ? 0 : gemm_nt_workspace(batch, n_in, w.p.OUTP);
  w.total = w.cfmt + w.p.gpad + w.hb + w.gemm;
  return w;
}
// workspace of kf_G_base: G's, the column sums of g and their block partials (B-splines; the
// Chebyshev layout has them), silu(x)^T (INP, BP) in bf16 and the GEMM core's partial sums
struct WsGB {
  WsG g;
  size_t part, colsum, st, gemm, total;
};
inline WsGB ws_g_base(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out) {
  WsGB w;
  w.g = ws_g(b, dtype, batch, n_in, n_out, false, true);
  const bool own_sums = !w.g.skip0;
  w.part = own_sums ? align256((size_t)((w.g.BP + 63) / 64) * w.g.OUTP * sizeof(float)) : 0;
  w.colsum = own_sums ? align256((size_t)w.g.OUTP * sizeof(float)) : 0;
  w.st = align256((size_t)w.g.INP * w.g.BP * elt_size(dtype));
  w.gemm = gemm_nt_workspace(n_out, n_in, w.g.BP);
  w.total = w.g.total + w.part + w.colsum + w.st + w.gemm;
  return w;
}

// workspace of kf_G_bias: G's (the larger of its weighted and unweighted layouts), then the
// transpose's block partials and the column sums for the bias gradient, then the column-sum
// kernels' scratch for the routes without a transpose (the sparse ones)
struct WsGBias {
  size_t g, part, sums, cws, total;
};
inline WsGBias ws_g_bias(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out, bool has_w) {
  WsGBias w;
  const WsG L = ws_g(b, dtype, batch, n_in, n_out, has_w);
  w.g = L.total;
  // the transpose's 64-row block partials, or the sparse G's slice partials of sum_b g
  w.part = bspline_sparse(b, dtype)
               ? align256((size_t)sparse_g_plan(batch, n_in, n_out, b->size).nz * n_out * sizeof(float))
               : align256((size_t)((L.BP + 63) / 64) * L.OUTP * sizeof(float));
  w.sums = align256((size_t)L.OUTP * sizeof(float));
  w.cws = align256(kf_column_sums_workspace_bytes(batch, n_out));
  w.total = w.g + w.part + w.sums + w.cws;
  return w;
}

template <typename Fn>
int with_spline_degree(int kd, Fn&& fn) {
  switch (kd) {
    case 0: return fn(std::integral_constant<int, 0>{});
    case 1: return fn(std::integral_constant<int, 1>{});
    case 2: return fn(std::integral_constant<int, 2>{});
    case 3: return fn(std::integral_constant<int, 3>{});
    default: return fail(KF_EINVAL, "sparse B-spline route: degree %d above 3", kd);
  }
}

// The small-layer P's dense feature count for kc = K (+ 1 with the base branch) features, or 0
// where the staged sparse P runs (a side above 128, or more than 12 features)
inline int small_km(int64_t n_in, int64_t n_out, int kc) {
  if (n_in > 128 || n_out > 128) return 0;
  return kc <= 8 ? 8 : kc <= 9 ? 9 : kc <= 12 ? 12 : 0;
}
template <typename Fn>
void with_small_km(int km, Fn&& fn) {
  if (km == 8)
    fn(std::integral_constant<int, 8>{});
  else if (km == 9)
    fn(std::integral_constant<int, 9>{});
  else
    fn(std::integral_constant<int, 12>{});
}

template <typename T>
int launch_f_sparse(const KBasis& kb, int kd, int64_t batch, int64_t n_in, int64_t n_out, const void* x, const void* w,
                    const void* c, void* y, hipStream_t s, const void* bw = nullptr, const void* bias = nullptr) {
  const dim3 grid((unsigned)((batch + kSpRows - 1) / kSpRows), (unsigned)((n_out + 63) / 64));
  if (bw && kb.K + 1 > kSpKMax) return fail(KF_EINVAL, "F sparse: base weight needs K < %d", kSpKMax);
  return with_spline_degree(kd, [&](auto tag) {
    constexpr int KD = decltype(tag)::value;
    hipLaunchKernelGGL((f_sparse_kernel<T, KD>), grid, dim3(512), 0, s, kb, (int)batch, (int)n_in, (int)n_out,
                       (const T*)x, (const T*)w, (const T*)c, (T*)y, (const T*)bw, (const T*)bias);
    return check_launch("F sparse");
  });
}

template <typename T>
int launch_p_sparse(const KBasis& kb, int kd, int64_t batch, int64_t n_in, int64_t n_out, const void* x, const void* g,
                    const void* c, void* p, hipStream_t s, const void* bw = nullptr) {
  const dim3 grid((unsigned)((batch + kSpRows - 1) / kSpRows), (unsigned)((n_in + 63) / 64));
  if (bw && kb.K + 1 > kSpKMax) return fail(KF_EINVAL, "P sparse: base weight needs K < %d", kSpKMax);
  static_assert(kSmRows == kSpRows, "one grid for both P kernels");
  if (const int km = small_km(n_in, n_out, kb.K + (bw ? 1 : 0)))
    return with_spline_degree(kd, [&](auto tag) {
      constexpr int KD = decltype(tag)::value;
      with_small_km(km, [&](auto kmc) {
        constexpr int KM = decltype(kmc)::value;
        hipLaunchKernelGGL((p_small_kernel<T, KD, KM>), grid, dim3(512), 0, s, kb, (int)batch, (int)n_in, (int)n_out,
                           (const T*)x, (const T*)g, (const T*)c, (T*)p, (const T*)bw);
      });
      return check_launch("P small");
    });
  return with_spline_degree(kd, [&](auto tag) {
    constexpr int KD = decltype(tag)::value;
    hipLaunchKernelGGL((p_sparse_kernel<T, KD>), grid, dim3(512), 0, s, kb, (int)batch, (int)n_in, (int)n_out,
                       (const T*)x, (const T*)g, (const T*)c, (T*)p, (const T*)bw);
    return check_launch("P sparse");
  });
}

// g_sparse_kernel with the smallest feature tile KM in {8, 12, 16} that holds ko features
template <typename T>
int launch_g_sparse_kernel(const KBasis& kb, int kd, dim3 grid, int64_t batch, int64_t n_in, int64_t n_out, int rs,
                           const void* x, const void* g, const void* w, float* part, int ko, float* bpart,
                           hipStream_t s) {
  return with_spline_degree(kd, [&](auto tag) {
    constexpr int KD = decltype(tag)::value;
    auto go = [&](auto km) {
      constexpr int KM = decltype(km)::value;
      hipLaunchKernelGGL((g_sparse_kernel<T, KD, KM>), grid, dim3(256), 0, s, kb, (int)batch, (int)n_in, (int)n_out,
                         rs, (const T*)x, (const T*)g, (const T*)w, part, ko, bpart);
    };
    if (ko <= 8)
      go(std::integral_constant<int, 8>{});
    else if (ko <= 12)
      go(std::integral_constant<int, 12>{});
    else
      go(std::integral_constant<int, kSpKMax>{});
    return check_launch("G sparse");
  });
}

// The sparse G; with db, also the bias gradient db = sum_b g from the same pass (the lanes of
// input 0 sum g per slice into bpart, nz x n_out floats, which the reduction totals).
template <typename T>
int launch_g_sparse(const KBasis& kb, int kd, int64_t batch, int64_t n_in, int64_t n_out, const void* x, const void* g,
                    const void* w, void* dc, void* ws, hipStream_t s, void* db = nullptr, float* bpart = nullptr) {
  const SpG sp = sparse_g_plan(batch, n_in, n_out, kb.K);
  const dim3 grid((unsigned)((n_in + 3) / 4), (unsigned)((n_out + 63) / 64), (unsigned)sp.nz);
  if (!db) bpart = nullptr;
  int rc = launch_g_sparse_kernel<T>(kb, kd, grid, batch, n_in, n_out, sp.RS, x, g, w, (float*)ws, kb.K, bpart, s);
  if (rc) return rc;
  const long n = (long)n_out * n_in * kb.K + (bpart ? n_out : 0);
  long blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(g_sparse_reduce<T>, dim3((unsigned)blocks), dim3(256), 0, s, sp.nz, (int)n_in, (int)n_out, kb.K,
                     kb.K, (const float*)ws, (T*)dc, (T*)nullptr, (const float*)bpart, (T*)(bpart ? db : nullptr));
  return check_launch("G sparse reduce");
}

// The sparse G with the base branch's feature silu(x) as basis function K: partials of K + 1 sums
// per (o, i) (plan sparse_g_plan(..., K + 1)) and, with db, the bias gradient's slice partials
// after them (nz x n_out floats at ws + part); the reduction splits them into dc, dw and db.
template <typename T>
int launch_g_sparse_base(const KBasis& kb, int kd, int64_t batch, int64_t n_in, int64_t n_out, const void* x,
                         const void* g, void* dc, void* dw, void* db, void* ws, hipStream_t s) {
  const SpG sp = sparse_g_plan(batch, n_in, n_out, kb.K + 1);
  const dim3 grid((unsigned)((n_in + 3) / 4), (unsigned)((n_out + 63) / 64), (unsigned)sp.nz);
  if (kb.K + 1 > kSpKMax) return fail(KF_EINVAL, "G sparse: base feature needs K < %d", kSpKMax);
  float* bpart = db ? (float*)((char*)ws + sp.part) : nullptr;
  int rc = launch_g_sparse_kernel<T>(kb, kd, grid, batch, n_in, n_out, sp.RS, x, g, nullptr, (float*)ws, kb.K + 1,
                                     bpart, s);
  if (rc) return rc;
  const long n = (long)n_out * n_in * (kb.K + 1) + (db ? n_out : 0);
  long blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(g_sparse_reduce<T>, dim3((unsigned)blocks), dim3(256), 0, s, sp.nz, (int)n_in, (int)n_out, kb.K,
                     kb.K + 1, (const float*)ws, (T*)dc, (T*)dw, (const float*)bpart, (T*)db);
  return check_launch("G sparse reduce");
}


template <typename T>
__global__ void fill_zero_kernel(T* p, long n) {
  for (long e = blockIdx.x * (long)blockDim.x + threadIdx.x; e < n; e += (long)gridDim.x * blockDim.x) p[e] = T(0.f);
}

template <typename T>
int zero_fill(void* p, long n, hipStream_t s) {
  if (n <= 0) return KF_OK;
  long blocks = (n + 255) / 256;
  if (blocks > 65535) blocks = 65535;
  hipLaunchKernelGGL(fill_zero_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, s, (T*)p, n);
  return check_launch("fill");
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// 16-byte loads of rows of n elements of T: rows start aligned when n is a
// multiple of the vector width and the array is
template <typename T>
bool rows_vec(int64_t n, const void* p) {
  return n % (int64_t)(16 / sizeof(T)) == 0 && (p == nullptr || aligned16(p));
}

// permute (and fold) coefficients into a feature-major workspace layout with
// n_feat >= n_t features (zeros past n_t)
template <typename T>
int launch_permute(const KBasis& kb, int64_t n_out, int64_t n_in, int64_t OUTP, int64_t INP, int n_feat, const void* c,
                   void* out, int fmt, hipStream_t s, int j_first = 0, float* part0 = nullptr, const void* bw = nullptr) {
  if (OUTP % 32 || INP % 16 || !aligned16(out)) return fail(KF_EINVAL, "permute: workspace layout not aligned");
  dim3 grid((unsigned)(OUTP / 32), (unsigned)(INP / 16));
  const size_t rows = (size_t)32 * (16 * kb.K + 1), tile = (size_t)(n_feat + j_first + (bw ? 1 : 0)) * 16 * kPermTS;
  const size_t lds = (rows > tile ? rows : tile) * sizeof(float);
  KFoldT ft;
  for (int j = 0; j < KF_MAX_NT; ++j)
    for (int k = 0; k < KF_MAX_K; ++k) ft.v[j][k] = k < kb.K && j < kb.n_t ? kb.fold[k * KF_MAX_NT + j] : 0.f;
  const int vin = n_in % 16 == 0 && rows_vec<T>(n_in * kb.K, c);
  auto pick = [&](auto kb_tag) {
    constexpr int KB = decltype(kb_tag)::value;
    return fmt == kPermFMT ? permute_coef_kernel<T, kPermFMT, KB>
           : fmt == kPermC16 ? permute_coef_kernel<T, kPermC16, KB>
                             : permute_coef_kernel<T, kPermFM, KB>;
  };
  auto kern = kb.K <= 4    ? pick(std::integral_constant<int, 4>())
              : kb.K <= 9  ? pick(std::integral_constant<int, 9>())
              : kb.K <= 12 ? pick(std::integral_constant<int, 12>())
                           : pick(std::integral_constant<int, KF_MAX_K>());
  hipLaunchKernelGGL(kern, grid, dim3(kThreads), lds, s, ft, kb.K, kb.n_t, (int)n_out, (int)n_in, (int)OUTP, (int)INP,
                     n_feat, j_first, vin, (const T*)c, (const T*)bw, (T*)out, part0);
  return check_launch("permute_coef");
}

template <typename T, int NTB, bool FOLDED>
void launch_features_t(const KBasis& kb, int64_t batch, int64_t n_in, int64_t brows, int64_t icols, const void* x,
                       void* out, long sb, long sj, long si, bool b_fastest, hipStream_t s) {
  long n = (long)brows * icols;
  long blocks = (n + kThreads - 1) / kThreads;
  if (blocks > 65535 * 4) blocks = 65535 * 4;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL((features_kernel<T, NTB, FOLDED>), dim3((unsigned)blocks), dim3(kThreads), 0, s, kb, (int)batch,
                     (int)n_in, (int)brows, (int)icols, (const T*)x, (T*)out, sb, sj, si, b_fastest);
}

template <typename T, bool FOLDED>
int launch_features(const KBasis& kb, int64_t batch, int64_t n_in, int64_t brows, int64_t icols, const void* x,
                    void* out, long sb, long sj, long si, bool b_fastest, hipStream_t s) {
  // folded Chebyshev features need max(n_t, K) slots (n_t < K for the (1 - z^2) reduced fold)
  const int nb = nt_bucket(FOLDED ? (kb.kind == KF_KIND_CHEB ? (kb.n_t > kb.K ? kb.n_t : kb.K) : kb.K) : kb.n_t);
  switch (nb) {
    case 4: launch_features_t<T, 4, FOLDED>(kb, batch, n_in, brows, icols, x, out, sb, sj, si, b_fastest, s); break;
    case 8: launch_features_t<T, 8, FOLDED>(kb, batch, n_in, brows, icols, x, out, sb, sj, si, b_fastest, s); break;
    case 12: launch_features_t<T, 12, FOLDED>(kb, batch, n_in, brows, icols, x, out, sb, sj, si, b_fastest, s); break;
    case 16: launch_features_t<T, 16, FOLDED>(kb, batch, n_in, brows, icols, x, out, sb, sj, si, b_fastest, s); break;
    default: launch_features_t<T, 24, FOLDED>(kb, batch, n_in, brows, icols, x, out, sb, sj, si, b_fastest, s); break;
  }
  return check_launch("features");
}

template <typename T, int NTB, int RUN>
int launch_features_t_nb(const KBasis& kb, int64_t batch, int64_t n_in, int64_t BP, int64_t INP, const void* x,
                         const void* w, void* phit, int rows_ij, hipStream_t s) {
  constexpr int BT = RUN / (int)sizeof(T);  // features_t_kernel: 32 inputs x RUN-byte runs of rows
  const size_t knots = kb.kind == KF_KIND_BSPLINE ? (size_t)32 * (2 * kb.n_knots + 2 * kb.spline_k) * 4 : 0;
  const size_t lds = (size_t)kb.n_t * 32 * (RUN + 16) + knots;
  auto kern = features_t_kernel<T, NTB, RUN>;
  if (!reserve_lds((const void*)kern, lds))
    return fail(KF_ELAUNCH, "features: cannot reserve %zu bytes of LDS", lds);
  dim3 grid((unsigned)(INP / 32), (unsigned)((BP + BT - 1) / BT));
  hipLaunchKernelGGL(kern, grid, dim3(kThreads), lds, s, kb, (int)batch, (int)n_in, (int)BP, (int)INP, (const T*)x,
                     (const T*)w, (T*)phit, rows_ij);
  return check_launch("features_t");
}

template <typename T, int KD>
int launch_bspline_t(const KBasis& kb, int64_t batch, int64_t n_in, int64_t BP, int64_t INP, const void* x,
                     const void* w, void* phit, int rows_ij, hipStream_t s) {
  constexpr int RUN = 128, BT = RUN / (int)sizeof(T);
  const size_t lds = (size_t)kb.K * 32 * (RUN + 16) + (size_t)32 * (2 * kb.n_knots + 2 * KD) * 4;
  auto kern = KD == 3 && kb.knots_uniform && kb.n_knots >= 4 ? bspline_t_kernel<T, KD, RUN, true> : bspline_t_kernel<T, KD, RUN>;
  if (!reserve_lds((const void*)kern, lds)) return fail(KF_ELAUNCH, "features: cannot reserve %zu bytes of LDS", lds);
  dim3 grid((unsigned)(INP / 32), (unsigned)((BP + BT - 1) / BT));
  hipLaunchKernelGGL(kern, grid, dim3(kThreads), lds, s, kb, (int)batch, (int)n_in, (int)BP, (int)INP, (const T*)x,
                     (const T*)w, (T*)phit, rows_ij);
  return check_launch("bspline_t");
}

// phiT rows: feature-major (j INP + i), or input-major (i n_t + j, rows_ij)
template <typename T>
int launch_features_t(const KBasis& kb, int64_t batch, int64_t n_in, int64_t BP, int64_t INP, const void* x,
                      const void* w, void* phit, hipStream_t s, int rows_ij = 0) {
  if (INP % 32) return fail(KF_EINVAL, "features_t: padded input count not a multiple of 32");
  if (kb.kind == KF_KIND_BSPLINE) {  // B-splines: supports only, degree compiled in
    switch (kb.spline_k) {
      case 0: return launch_bspline_t<T, 0>(kb, batch, n_in, BP, INP, x, w, phit, rows_ij, s);
      case 1: return launch_bspline_t<T, 1>(kb, batch, n_in, BP, INP, x, w, phit, rows_ij, s);
      case 2: return launch_bspline_t<T, 2>(kb, batch, n_in, BP, INP, x, w, phit, rows_ij, s);
      case 3: return launch_bspline_t<T, 3>(kb, batch, n_in, BP, INP, x, w, phit, rows_ij, s);
      case 4: return launch_bspline_t<T, 4>(kb, batch, n_in, BP, INP, x, w, phit, rows_ij, s);
      default: return launch_bspline_t<T, 5>(kb, batch, n_in, BP, INP, x, w, phit, rows_ij, s);
    }
  }
  if (rows_ij) return fail(KF_EINVAL, "features_t: input-major rows are for B-splines");
  switch (nt_bucket(kb.n_t)) {
    case 4: return launch_features_t_nb<T, 4, 64>(kb, batch, n_in, BP, INP, x, w, phit, 0, s);
    case 8: return launch_features_t_nb<T, 8, 64>(kb, batch, n_in, BP, INP, x, w, phit, 0, s);
    case 12: return launch_features_t_nb<T, 12, 64>(kb, batch, n_in, BP, INP, x, w, phit, 0, s);
    case 16: return launch_features_t_nb<T, 16, 64>(kb, batch, n_in, BP, INP, x, w, phit, 0, s);
    default: return launch_features_t_nb<T, 24, 64>(kb, batch, n_in, BP, INP, x, w, phit, 0, s);
  }
}

}  // namespace kfabi
