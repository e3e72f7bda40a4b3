// extern "C" entry points of libkfhip.so (declared in include/kfhip.h):
// argument validation, workspace carving and kernel dispatch.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <set>
#include <string>
#include <utility>

#include "kf_kernels.h"

using namespace kf;

namespace {

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

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(KF_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
  return KF_OK;
}

// The dynamic-LDS ceiling of a kernel above the default 64 KB is raised once per (device, kernel)
// to the whole 160 KB of a CU; launches then pass their actual size. The table of kernels already
// raised is the library's only mutable state besides the scratch addresses, and is guarded.
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

inline int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }
inline size_t align256(size_t v) { return (v + 255) & ~size_t(255); }
inline int elt_size(int dtype) { return dtype == KF_BF16 ? 2 : 4; }

// tile constants shared by workspace sizing and launches
constexpr int CHUNK = 32;

int validate_basis(const kf_basis* b) {
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

int validate_common(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out) {
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

KBasis to_kbasis(const kf_basis* b) {
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
bool features_weighted(const kf_basis* b, const void* w) {
  return w != nullptr || (b->kind == KF_KIND_CHEB && b->input_map == KF_MAP_TANH_SQ);
}

int nt_bucket(int n) { return n <= 4 ? 4 : n <= 8 ? 8 : n <= 12 ? 12 : n <= 16 ? 16 : 24; }

// F tile configurations: (BM, BN, waves along M, waves along N), 512 threads.
struct FCfg {
  int bm, bn, wm, wn;
};
constexpr FCfg F_CFGS[] = {{256, 192, 4, 2}, {256, 256, 2, 4}, {256, 128, 4, 2}};
constexpr int N_CUS = 256;

// The configuration with the fewest tile-area x dispatch rounds (whole-GPU
// waves of 256 workgroups); ties keep the larger tile.
int pick_f_cfg(int64_t batch, int64_t n_out) {
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
  size_t cfm, z, wz, phi, part0, ysum, total;
};
// bf16 Chebyshev plans run the register-A F kernel: workgroup tile (128 RA_TM) x
// (32 RA_TN), four waves along the batch times RA_WN along the outputs (wave
// tile (32 RA_TM) x (32 RA_TN / RA_WN)).
constexpr int F_REGA = -1;
constexpr int RA_TM = 1, RA_TN = 6, RA_WN = 1, RA_NWM = 8, RA_BM = 32 * RA_NWM * RA_TM, RA_BN = 32 * RA_TN;
constexpr int RA_NBUF = 4;  // coefficient stage buffers (prefetch distance RA_NBUF - 1 stages)
bool f_uses_rega(const kf_basis* b, int dtype) { return b->kind == KF_KIND_CHEB && dtype == KF_BF16; }
// odd feature counts with an unpadded, unrolled variant
bool f_rega_unpadded(int n_t, int64_t n_in) { return n_t == 9; }

WsF ws_f(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out, bool has_w) {
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
  w.cfm = align256((size_t)w.n_tp * w.OUTP * w.INP * es);
  w.z = cheb ? align256((size_t)w.BP * w.INP * sizeof(float)) : 0;
  w.wz = cheb && has_w ? align256((size_t)w.BP * w.INP * sizeof(float)) : 0;
  w.phi = cheb ? 0 : align256((size_t)w.BP * w.n_tp * w.INP * es);
  w.part0 = w.skip0 ? align256((size_t)(w.INP / 16) * w.OUTP * sizeof(float)) : 0;
  w.ysum = w.skip0 ? align256((size_t)w.OUTP * sizeof(float)) : 0;
  w.total = w.cfm + w.z + w.wz + w.phi + w.part0 + w.ysum;
  return w;
}
// P / G configurations. The MFMA waves split the features in two groups of
// FW = ceil(n_t / 2) (FW in {2,3,4,5,6,8,12}); TM 32-row tiles per wave keep
// the accumulators at <= 192 registers. P: 4x2 waves (512 threads, 64-byte
// stages); G: warp-specialised for Chebyshev plans (4 MFMA waves + 4
// producer waves, 128-byte stages, 64 from FW = 8), else 2x2 waves.
constexpr int FW_LIST[] = {2, 3, 4, 5, 6, 8, 12};
int fw_index(int n_t) {
  const int need = (n_t + 1) / 2;
  for (int k = 0; k < 7; ++k)
    if (FW_LIST[k] >= need) return k;
  return 6;
}
int g_tm(int fw) { return fw <= 6 ? 2 : 1; }
int g_rb(int fw) { return fw <= 6 ? 128 : 64; }

struct WsP {
  int cfg, ntb;
  bool p8;  // bf16 Chebyshev with 7 or 8 features: p8_kernel (256 x (8 x 48) tiles)
  int64_t INP, OUTP;
  size_t cfmt, gpad, total;
};
// P with FW <= 4 runs the copy kernel (p_dma_kernel; 4 x FW accumulator tiles in AGPRs); it needs
// g with whole 128-byte stages of columns and 16-byte aligned rows, else a zero-padded copy of g
// in the workspace.
bool p_uses_dma(int cfg) { return FW_LIST[cfg] <= 6; }
constexpr int p_dma_tm(int fw) { return fw <= 4 ? 4 : 2; }  // row tiles per wave (LDS: two stages fit)
int64_t p_stage_cols(int dtype) { return 128 / elt_size(dtype); }
bool p_needs_gpad(int64_t n_out, int dtype) { return n_out % p_stage_cols(dtype) != 0; }
WsP ws_p(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out) {
  WsP w;
  w.cfg = fw_index(b->n_t);
  w.ntb = 2 * FW_LIST[w.cfg];
  w.p8 = b->kind == KF_KIND_CHEB && dtype == KF_BF16 && w.ntb == 8;
  // 96: whole tiles of p8_kernel (48) and p_dma_kernel (32); rational: flat tiles of 2 FW x 32 inputs
  w.INP = round_up(n_in, w.p8 ? 96 : b->kind == KF_KIND_RATIONAL ? 64 * FW_LIST[w.cfg] : 32);
  w.OUTP = round_up(n_out, p_uses_dma(w.cfg) ? p_stage_cols(dtype) : 32);
  w.cfmt = align256((size_t)w.ntb * w.INP * w.OUTP * elt_size(dtype));
  w.gpad = p_uses_dma(w.cfg) && p_needs_gpad(n_out, dtype) ? align256((size_t)batch * w.OUTP * elt_size(dtype)) : 0;
  w.total = w.cfmt + w.gpad;
  return w;
}
struct WsG {
  int cfg;
  bool skip0;  // Chebyshev, unweighted: T_0 = 1 taken out of the contraction (column sums of g)
  bool g96;    // bf16 Chebyshev with at most 8 features run: g96_kernel (192 x 48 x 8 tiles)
  bool pre;    // features precomputed into phiT (other kinds, and Chebyshev plans on small grids)
  bool gdma;   // B-spline without batch splits: p_dma_kernel as the flat GEMM gT x phiT^T
  int nz;      // pre: batch splits of g_kernel (raw sums reduced by g_split_reduce when > 1)
  int64_t OUTP, BP, INP;
  size_t gt, zt, wt, part, colsum, phit, zpart, total;
};
constexpr size_t kGSplitBytes = size_t(256) << 20;  // cap of the split partial sums
constexpr long kGSplitMax = 64;                      // cap of the batch splits
constexpr int kGdmaFW = 4, kGdmaRows = 2 * kGdmaFW * 32;  // G on p_dma_kernel: phiT rows per tile
WsG ws_g(const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out, bool has_w) {
  WsG w;
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
  w.BP = round_up(batch, eps);
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
  w.total = w.gt + w.zt + w.wt + w.part + w.colsum + w.phit + w.zpart;
  return w;
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

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

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
                   void* out, int fmt, hipStream_t s, int j_first = 0, float* part0 = nullptr) {
  if (OUTP % 32 || INP % 16 || !aligned16(out)) return fail(KF_EINVAL, "permute: workspace layout not aligned");
  dim3 grid((unsigned)(OUTP / 32), (unsigned)(INP / 16));
  const size_t rows = (size_t)32 * (16 * kb.K + 1), tile = (size_t)(n_feat + j_first) * 16 * kPermTS;
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
                     n_feat, j_first, vin, (const T*)c, (T*)out, part0);
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

template <typename T, int NTB>
int launch_features_t_nb(const KBasis& kb, int64_t batch, int64_t n_in, int64_t BP, int64_t INP, const void* x,
                         const void* w, void* phit, hipStream_t s) {
  constexpr int BT = 64 / (int)sizeof(T);  // features_t_kernel: 32 inputs x 64-byte runs of rows
  const size_t knots = kb.kind == KF_KIND_BSPLINE ? (size_t)32 * (2 * kb.n_knots + 2 * kb.spline_k) * 4 : 0;
  const size_t lds = (size_t)kb.n_t * 32 * 80 + knots;
  auto kern = features_t_kernel<T, NTB>;
  if (!reserve_lds((const void*)kern, lds))
    return fail(KF_ELAUNCH, "features: cannot reserve %zu bytes of LDS", lds);
  dim3 grid((unsigned)(INP / 32), (unsigned)((BP + BT - 1) / BT));
  hipLaunchKernelGGL(kern, grid, dim3(kThreads), lds, s, kb, (int)batch, (int)n_in, (int)BP, (int)INP, (const T*)x,
                     (const T*)w, (T*)phit);
  return check_launch("features_t");
}

template <typename T>
int launch_features_t(const KBasis& kb, int64_t batch, int64_t n_in, int64_t BP, int64_t INP, const void* x,
                      const void* w, void* phit, hipStream_t s) {
  if (INP % 32) return fail(KF_EINVAL, "features_t: padded input count not a multiple of 32");
  switch (nt_bucket(kb.n_t)) {
    case 4: return launch_features_t_nb<T, 4>(kb, batch, n_in, BP, INP, x, w, phit, s);
    case 8: return launch_features_t_nb<T, 8>(kb, batch, n_in, BP, INP, x, w, phit, s);
    case 12: return launch_features_t_nb<T, 12>(kb, batch, n_in, BP, INP, x, w, phit, s);
    case 16: return launch_features_t_nb<T, 16>(kb, batch, n_in, BP, INP, x, w, phit, s);
    default: return launch_features_t_nb<T, 24>(kb, batch, n_in, BP, INP, x, w, phit, s);
  }
}

}  // namespace

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

template <bool HAS_W, bool SKIP0>
int launch_f_rega(const WsF& L, int64_t batch, int64_t n_out, const float* zc, const float* wc, const void* cfm,
                  const float* ysum, void* y, hipStream_t s) {
  const int n_m = (int)(L.BP / RA_BM), n_n = (int)(L.OUTP / RA_BN);
  // RA_NBUF stage buffers of 2 features, z (and w) of two chunks
  // (reused by the epilogue's bf16 staging of each wave's output tile: RA_BM rows of
  // RA_BN / RA_WN * 2 + 16 bytes per column group)
  const size_t lds_ops = (size_t)RA_NBUF * 2 * RA_BN * 32 + (size_t)(HAS_W ? 4 : 2) * RA_BM * 64;
  const size_t lds_epi = (size_t)RA_WN * RA_BM * (RA_BN / RA_WN * 2 + 16);
  const size_t lds = lds_ops > lds_epi ? lds_ops : lds_epi;
  const int vout = n_out % 8 == 0 && aligned16(y);
  constexpr int TNW = RA_TN / RA_WN;
  auto kern = L.n_tp == 9   ? f_rega_kernel<HAS_W, 9, RA_TM, TNW, RA_NBUF, SKIP0, RA_WN, RA_NWM>
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

template <typename T>
int run_F_dma(const KBasis& kb, int64_t batch, int64_t n_in, int64_t n_out, const void* x, const void* c, void* phi,
              void* y, hipStream_t s) {
  constexpr int FW = kGdmaFW, TM = p_dma_tm(FW), BM = 2 * TM * 32, TI = 2 * FW * 32;
  const long ld = (long)n_in * kb.K;  // Phi row length: the reduction
  if (kb.n_t != kb.K || (ld * (long)sizeof(T)) % 16) return fail(KF_EINVAL, "F: Phi rows not aligned");
  if (kb.K == 1) {  // one feature: the plain (B, in) writes are already coalesced
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
  const size_t lds = (size_t)2 * (BM + TI) * 128;
  auto kern = p_dma_kernel<T, TM, FW, KF_KIND_BSPLINE, 2>;
  if (!reserve_lds((const void*)kern, lds))
    return fail(KF_ELAUNCH, "F: cannot reserve %zu bytes of LDS", lds);
  const int n_m = (int)((batch + BM - 1) / BM), n_n = (int)((n_out + TI - 1) / TI);
  hipLaunchKernelGGL(kern, dim3(n_m * n_n), dim3(256), lds, s, kb, (int)batch, (int)n_out, n_n * TI, (int)ld,
                     (const T*)nullptr, (const T*)phi, (int)ld, (const T*)c, (T*)y, (float*)nullptr);
  return check_launch("F");
}

template <typename T>
int run_F(const KBasis& kb, const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void* x,
          const void* w, const void* c, void* y, void* ws, hipStream_t s) {
  const bool has_w = w != nullptr;
  const bool cheb = kb.kind == KF_KIND_CHEB;
  const bool weighted = features_weighted(b, w);
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
                       (int)blocks, (int)(L.INP / 16), (int)L.OUTP, part0, ysum);
    rc = check_launch("zmapc");
    if (rc) return rc;
    if (weighted) return launch_f_rega<true, false>(L, batch, n_out, z, wz, cfm, nullptr, y, s);
    if (L.skip0) return launch_f_rega<false, true>(L, batch, n_out, z, nullptr, cfm, ysum, y, s);
    return launch_f_rega<false, false>(L, batch, n_out, z, nullptr, cfm, nullptr, y, s);
  }
  // B-spline or rational, unweighted, in K a whole number of 128-byte stages: Phi (B, in K) in the
  // reference's layout, then the flat GEMM Phi c^T on p_dma_kernel (no coefficient permute)
  constexpr int EPS = 128 / (int)sizeof(T);
  const long dma_tiles = ((batch + 255) / 256) * ((n_out + 255) / 256);  // at least half a round of the CUs
  const bool identity_fold = kb.kind == KF_KIND_BSPLINE || kb.kind == KF_KIND_RATIONAL;
  if (identity_fold && !has_w && (n_in * kb.K) % EPS == 0 && aligned16(c) && aligned16(phi) && dma_tiles >= 128)
    return run_F_dma<T>(kb, batch, n_in, n_out, x, c, phi, y, s);
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

template <int TN, int RB>
int launch_p8(const WsP& L, hipStream_t s, const KBasis& kb, int64_t batch, int64_t n_in, const void* x, const void* g,
              int gstride, const void* cfmt, void* p) {
  constexpr int TI = 16 * TN, RPASS = TN == 2 ? 128 : 64;
  const size_t lds_ops = (size_t)2 * (256 + 8 * TI) * RB, lds_epi = (size_t)8 * RPASS * (TI + 1) * 4;
  const size_t lds = lds_ops > lds_epi ? lds_ops : lds_epi;
  auto kern = p8_kernel<KF_KIND_CHEB, TN, RB>;
  if (L.INP % TI || L.OUTP % (RB / 2)) return fail(KF_EINVAL, "P: workspace layout not aligned");
  if (!reserve_lds((const void*)kern, lds))
    return fail(KF_ELAUNCH, "P: cannot reserve %zu bytes of LDS", lds);
  const int n_m = (int)((batch + 255) / 256), n_n = (int)(L.INP / TI);
  hipLaunchKernelGGL(kern, dim3(n_m * n_n), dim3(512), lds, s, kb, (int)batch, (int)n_in, (int)L.INP, (int)L.OUTP,
                     (const bf16*)x, (const bf16*)g, gstride, (const bf16*)cfmt, (bf16*)p);
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
          const void* g, const void* c, void* p, float* h, void* ws, hipStream_t s) {
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
    // 7 or 8 Chebyshev features in bf16: the two-waves-per-SIMD kernel
    if (L.p8 && !h) return launch_p8<3, 128>(L, s, kb, batch, n_in, x, ga, gstride, cfmt, p);
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
int run_G(const KBasis& kb, const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void* x,
          const void* g, const void* w, void* dc, void* ws, hipStream_t s) {
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
  if (L.BP % 32 || !aligned16(gt)) return fail(KF_EINVAL, "G: workspace layout not aligned");
  dim3 tg((unsigned)((L.OUTP + 63) / 64), (unsigned)((L.BP + 63) / 64));
  hipLaunchKernelGGL(transpose_kernel<T>, tg, dim3(kThreads), 0, s, (int)batch, (int)n_out, (int)L.BP, (int)L.OUTP,
                     (int)rows_vec<T>(n_out, g), (const T*)g, (T*)gt, part);
  int rc = check_launch("transpose");
  if (rc) return rc;
  if (cheb) {
    // block rows past the batch tiles total the column sums of g (skip0 implies cheb)
    const unsigned gx = (unsigned)((L.INP + 63) / 64), sblocks = L.skip0 ? (unsigned)((L.OUTP + 7) / 8) : 0u;
    dim3 zg(gx, (unsigned)((L.BP + 63) / 64) + (sblocks + gx - 1) / gx);
    hipLaunchKernelGGL(zmapT_kernel<T>, zg, dim3(kThreads), (size_t)(wt ? 2 : 1) * 64 * 65 * sizeof(float), s,
                       (int)batch, (int)n_in, (int)L.BP, (int)L.INP, kb.input_map,
                       (int)(rows_vec<T>(n_in, x) && rows_vec<T>(n_in, w)), (const T*)x, (const T*)w, zt, wt,
                       (int)((L.BP + 63) / 64), (int)L.OUTP, part, colsum);
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
  float* zpart = L.nz > 1 ? (float*)((char*)phit + L.phit) : nullptr;
  rc = launch_features_t<T>(kb, batch, n_in, L.BP, L.INP, x, w, phit, s);
  if (rc) return rc;
  if (L.gdma) return launch_g_dma<T>(L, s, kb, n_in, n_out, gt, phit, dc);
  return launch_g_cfg<T, false>(L, s, kb, batch, n_in, n_out, phit, zpart, nullptr, nullptr, gt, dc);
}

template <typename T, int KM>
void launch_edge_t(const KBasis& kb, int64_t batch, int64_t n_in, int64_t n_out, const void* x, const void* c,
                   const void* bw, void* out, hipStream_t s) {
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
    default: return 0;
  }
}

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
  if (dtype == KF_BF16)
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
