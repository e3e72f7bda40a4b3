/*
 * kfhip.h — C ABI of the MI355X (gfx950) fused KAN basis kernels.
 *
 * One shared library, libkfhip.so, built from the HIP sources in kanforge_amd/csrc. The
 * entry points below replace the reference's raw launcher
 *   kanforge/torch/kernels.py:39-55   _raw(op, plan, m, x, a, b, grid, n_out, nf)
 *   kanforge/kernels/triton_kernels.py:225-242   launch(op, ...)
 * op "F" -> kf_F, "G" -> kf_G, "P" -> kf_P, plus entry points for what the
 * reference computes with plain ops on this path (basis evaluation,
 * edge_derivative, the group-rational parameter gradients).
 *
 * Conventions
 *  - All array arguments are DEVICE pointers to dense row-major arrays
 *    (no strides); the caller owns every buffer. The library never
 *    allocates, frees or synchronises.
 *  - Work that needs scratch memory takes a caller-provided workspace of at
 *    least kf_workspace_bytes(...) bytes (256-byte aligned); where that size is
 *    0 the workspace may be NULL.
 *  - `stream` is a hipStream_t (passed as void*); every launch is ordered on it.
 *  - Return value: 0 on success, a negative KF_E* code otherwise; the text
 *    of the last error of the calling thread is kf_last_error().
 *  - x, w, coefficients, upstream gradients and outputs of one call share
 *    one dtype (kf_dtype). Accumulation is float32.
 */
#ifndef KFHIP_H
#define KFHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define KF_OK 0
#define KF_EINVAL -1     /* bad argument (shape, null pointer, unsupported combination) */
#define KF_EWORKSPACE -2 /* workspace missing or too small */
#define KF_ELAUNCH -3    /* a HIP launch failed */
#define KF_EUNSUPPORTED -4

/* element types */
#define KF_F32 0
#define KF_BF16 1
#define KF_I8 2  /* lookup tables only */
#define KF_I16 3 /* lookup tables only */

/* basis kinds (kanforge/kernels/plan.py:39-45 KernelPlan.kind, plus rational) */
#define KF_KIND_CHEB 0     /* T_j(g(x)) features, g = tanh or identity; derivatives folded */
#define KF_KIND_BSPLINE 1  /* B-splines on a per-input knot vector; derivative order native */
#define KF_KIND_RATIONAL 2 /* P(x)/(1+|Q(x)|), parameters shared by groups of inputs */

/* input maps of the Chebyshev family (kanforge/bases/polynomial.py:66-85) */
#define KF_MAP_IDENTITY 0
#define KF_MAP_TANH 1
/* tanh map whose kernel features carry the factor (1 - z^2): every x-derivative of f(tanh x)
 * of order m >= 1 is (1 - z^2) q(z) with deg q = deg f + m - 2, so R_m divided by (1 - z^2)
 * needs two features fewer than R_m itself (same values; not a reference map) */
#define KF_MAP_TANH_SQ 2

#define KF_MAX_K 16   /* basis functions per edge */
#define KF_MAX_NT 24  /* kernel features per edge (K + derivative order for tanh maps) */

/*
 * What one input's kernel features are. Mirrors KernelPlan
 * (kanforge/kernels/plan.py:39-72): kind, consts, size, and the fold matrix
 * R_m (plan.py:75-101) that maps kernel features to the m-th derivative of
 * the basis functions.
 *
 *  cheb:     features T_0..T_{n_t-1}(g(x)); `fold` is R_m (size x n_t,
 *            row-major, HOST pointer, copied into the launch) so that
 *            phi_k^(m) = sum_j fold[k][j] T_j.  n_t = size + m (tanh) or size.
 *  bspline:  features are the m-th derivatives of the `size` = G + k
 *            B-splines of degree `spline_k` on per-input knots.
 *            knots:     (n_in, n_knots + 2*spline_k) float32, the real knots
 *                       padded by spline_k strictly increasing knots per side.
 *            knots_cmp: (n_in, n_knots) float32, each real float64 knot
 *                       rounded toward +inf; x >= t64 <=> x >= ceil32(t64) for
 *                       every float32 x, so interval search is exact.
 *  rational: one feature, the m-th derivative of P/(1+|Q|),
 *            P = sum_{j<=num_deg} num[g][j] x^j, Q = sum_{1<=j<=den_deg} den[g][j-1] x^j,
 *            g = input / group_size. num (groups, num_deg+1), den (groups, den_deg),
 *            float32 device arrays.
 */
typedef struct kf_basis {
  int32_t kind;
  int32_t size;      /* K: basis functions per input */
  int32_t order;     /* m: derivative order of the features */
  int32_t n_t;       /* kernel features per input (n_t == size unless cheb+tanh) */
  int32_t input_map; /* cheb */
  int32_t spline_k;  /* bspline degree */
  int32_t n_knots;   /* bspline real knots per input (G + 2k + 1) */
  int32_t num_deg;   /* rational */
  int32_t den_deg;
  int32_t group_size;
  const float *fold;      /* cheb, host */
  const float *knots;     /* bspline, device */
  const float *knots_cmp; /* bspline, device */
  const float *num;       /* rational, device */
  const float *den;       /* rational, device */
  /* bspline, device, optional: (n_in, 2) float32 (t_0, 1 / h) of each input whose real knots are
   * evenly spaced by h (t_0 its first real knot); NULL unless every input's knots are. Only speeds
   * up the kernels: intervals are still decided by knots_cmp, so results keep their semantics. */
  const float *knots_uniform;
} kf_basis;

/* operation ids for kf_workspace_bytes (and kf_base_fused for the *_BASE ids) */
#define KF_OP_F 0
#define KF_OP_G 1
#define KF_OP_P 2
#define KF_OP_F_BASE 3
#define KF_OP_P_BASE 4
#define KF_OP_G_BASE 5
#define KF_OP_G_BIAS 6 /* kf_G_bias (kf_F_bias needs kf_F's workspace, KF_OP_F) */

/*
 * Scratch bytes kf_F / kf_G / kf_P need for these shapes (0 is possible).
 * Replaces nothing in the reference (Triton allocates implicitly).
 */
size_t kf_workspace_bytes(int op, const kf_basis *basis, int dtype, int64_t batch, int64_t n_in, int64_t n_out);

/*
 * y[b,o] = sum_{i,k} w[b,i] c[o,i,k] phi_k^(m)(x[b,i])          (op "F")
 * x (batch, n_in); w (batch, n_in) or NULL for ones; c (n_out, n_in, size);
 * y (batch, n_out).  Replaces _raw("F", ...) (kanforge/torch/kernels.py:77)
 * together with the fold c @ R_m (kanforge/torch/kernels.py:75-76).
 */
int kf_F(const kf_basis *basis, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void *x,
         const void *w, const void *c, void *y, void *workspace, size_t workspace_bytes, void *stream);

/*
 * y[b,o] = F_m(x, w, c)[b,o] + bias[o]: kf_F plus the layer's bias (kanforge/torch/layers.py:
 * 189-190, `y + self.bias`), bias in dtype (n_out) or NULL (then exactly kf_F). Where F's last
 * kernel can take the bias (the register-A Chebyshev kernel's per-output constant, the GEMM
 * core's epilogue: bf16 B-spline and rational routes) it costs no pass of its own; other routes
 * add it in one more pass over y. Same workspace as kf_F.
 */
int kf_F_bias(const kf_basis *basis, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void *x,
              const void *w, const void *c, const void *bias, void *y, void *workspace, size_t workspace_bytes,
              void *stream);

/*
 * kf_F without a workspace argument and without any allocation: the same kernels and result as
 * kf_F, with their scratch in a static device array of KF_NOALLOC_SCRATCH_BYTES that the library
 * holds on every GPU it runs on until the process ends. No counterpart in the reference: it is for
 * callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). Shapes whose F workspace exceeds the scratch are rejected with
 * KF_EWORKSPACE. Every call on one GPU shares that GPU's scratch: calls that overlap on one GPU
 * (on different streams, or from different threads) race; calls ordered on one stream do not.
 */
#define KF_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int kf_F_noalloc(const kf_basis *basis, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void *x,
                 const void *w, const void *c, void *y, void *stream);

/*
 * dc[o,i,k] = sum_b w[b,i] g[b,o] phi_k^(m)(x[b,i])              (op "G")
 * g (batch, n_out); dc (n_out, n_in, size). Replaces _raw("G", ...) and the
 * fold gt @ R_m^T (kanforge/torch/kernels.py:95-98).
 */
int kf_G(const kf_basis *basis, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void *x,
         const void *g, const void *w, void *dc, void *workspace, size_t workspace_bytes, void *stream);

/*
 * kf_G plus the bias gradient dbias[o] = sum_b g[b,o] (dtype, n_out; NULL: exactly kf_G), what
 * autograd computes for `y + self.bias` (kanforge/torch/layers.py:189-190) next to _G. The column
 * sums come from the block partials of G's own transpose of g where its route has one, else from
 * kf_column_sums. Workspace: kf_workspace_bytes(KF_OP_G_BIAS, ...).
 */
int kf_G_bias(const kf_basis *basis, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void *x,
              const void *g, const void *w, void *dc, void *dbias, void *workspace, size_t workspace_bytes,
              void *stream);

/*
 * p[b,i] = sum_{o,k} g[b,o] c[o,i,k] phi_k^(m)(x[b,i])            (op "P")
 * Replaces _raw("P", ...) (kanforge/torch/kernels.py:118). If h is not NULL,
 * also writes h[b,i] = sum_o g[b,o] c[o,i,0] as float32 (rational kind,
 * size 1: the input of kf_rational_param_grad).
 */
int kf_P(const kf_basis *basis, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void *x,
         const void *g, const void *c, void *p, float *h, void *workspace, size_t workspace_bytes, void *stream);

/*
 * The KANLinear layer with its SiLU base branch and bias fused into the contractions: what
 * kanforge/torch/layers.py:185-191 computes as the spline part (_F) plus
 * F.linear(silu(x), base_weight) plus bias, and what autograd then computes for it.
 *
 * kf_base_fused(op, ...) is 1 when the entry point of op (KF_OP_F_BASE, KF_OP_P_BASE,
 * KF_OP_G_BASE) takes the layer, 0 when the caller composes kf_F / kf_P / kf_G with its own base
 * branch instead, negative for an invalid descriptor. It takes bf16 Chebyshev plans on their
 * contraction kernels (F: n_t of 9 or an even count >= 6), bf16 B-spline plans (P: cubic with
 * 11 basis functions) and float32 B-spline plans with fewer than 16 basis functions (the sparse
 * route, base weight as basis function K), not the narrow streaming routes. Workspace:
 * kf_workspace_bytes(KF_OP_*_BASE, ...) (0, workspace may be NULL, for F and P on the sparse
 * route).
 *
 * kf_F_base: y = F_0(x, c) + silu(x) base_w^T + bias, basis of order 0; base_w (n_out, n_in),
 *   bias (n_out) or NULL. silu(x) is one more feature per input in the same contraction (B-splines:
 *   silu(x) and the bias as extra feature columns of the one GEMM).
 * kf_P_base: p = P_m(x, g, c) + silu'(x) * (g base_w), basis of order m >= 1 (the x-gradient's
 *   descriptor, m = 1); g (batch, n_out).
 * kf_G_base: dc = G_0(x, g), dbase_w = g^T silu(x) (n_out, n_in), dbias = sum_b g (n_out),
 *   basis of order 0; each output may be NULL (not wanted).
 */
int kf_base_fused(int op, const kf_basis *basis, int dtype, int64_t batch, int64_t n_in, int64_t n_out);
int kf_F_base(const kf_basis *basis, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void *x,
              const void *c, const void *base_w, const void *bias, void *y, void *workspace, size_t workspace_bytes,
              void *stream);
int kf_P_base(const kf_basis *basis, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void *x,
              const void *g, const void *c, const void *base_w, void *p, void *workspace, size_t workspace_bytes,
              void *stream);
int kf_G_base(const kf_basis *basis, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void *x,
              const void *g, void *dc, void *dbase_w, void *dbias, void *workspace, size_t workspace_bytes,
              void *stream);

/*
 * phi[b,i,k] = phi_k^(m)(x[b,i]), out (batch, n_in, size) in dtype.
 * Replaces Basis.derivative (kanforge/bases/base.py:79-85) for the kinds above.
 */
int kf_features(const kf_basis *basis, int dtype, int64_t batch, int64_t n_in, const void *x, void *out,
                void *stream);

/*
 * d[b,o,i] = sum_k c[o,i,k] phi_k^(m)(x[b,i]) + base_w[o,i] silu^(m)(x[b,i])
 * out (batch, n_out, n_in); base_w may be NULL (no base branch).
 * Replaces KANLinear.edge_derivative (kanforge/torch/layers.py:206-226).
 * `c` holds the basis coefficients (n_out, n_in, size), not a folded copy.
 */
int kf_edge_derivative(const kf_basis *basis, int dtype, int64_t batch, int64_t n_in, int64_t n_out,
                       const void *x, const void *c, const void *base_w, void *out, void *stream);

/*
 * Interval index j with knots[i][j] <= x[b,i] < knots[i][j+1] (float64
 * knots, compared exactly through the ceil32 table), -1 outside.
 * x float32 (batch, n_in); idx int32 (batch, n_in). This is the level-0
 * indicator of kanforge/bases/spline.py:80.
 */
int kf_bspline_interval(int64_t batch, int64_t n_in, const float *x, const float *knots_cmp, int32_t n_knots,
                        int32_t *idx, void *stream);

/*
 * Gradients of sum_{b,i} h[b,i] w[b,i] phi^(m)(x[b,i]) with respect to the
 * rational parameters, m = basis->order (0, or 1..3 for numerator degree 5 and
 * denominator degree 4): dnum (groups, num_deg+1), dden (groups, den_deg),
 * float32, overwritten. h float32 (batch, n_in) from kf_P; w may be NULL.
 * What autograd computes through Rational._eval (kanforge/bases/rational.py:84-101).
 * Needs kf_workspace_bytes-independent scratch: workspace of
 * kf_rational_workspace_bytes(...) bytes.
 */
size_t kf_rational_workspace_bytes(const kf_basis *basis, int64_t batch, int64_t n_in);
int kf_rational_param_grad(const kf_basis *basis, int dtype, int64_t batch, int64_t n_in, const void *x,
                           const float *h, const void *w, float *dnum, float *dden, void *workspace,
                           size_t workspace_bytes, void *stream);

/*
 * The rational part of F's backward in one call: p = P_{m+1}(x, g, c) (the input gradient
 * without w, batch x n_in in dtype) and the gradients of sum_{b,o} g[b,o] F_m(x, c, w)[b,o]
 * with respect to the rational parameters, m = basis->order (dnum, dden float32,
 * overwritten). What autograd computes through Rational._eval inside the reference's
 * _F.backward (kanforge/torch/kernels.py:79-87, kanforge/bases/rational.py:84-101). At m = 0
 * for numerator degree 5 / denominator degree 4 in bf16 it fuses the input gradient and the
 * parameter reduction into one pass over h = g c^T. Workspace of
 * kf_rational_bwd_workspace_bytes(...) bytes, 256-byte aligned.
 */
size_t kf_rational_bwd_workspace_bytes(const kf_basis *basis, int dtype, int64_t batch, int64_t n_in, int64_t n_out);
int kf_rational_bwd(const kf_basis *basis, int dtype, int64_t batch, int64_t n_in, int64_t n_out, const void *x,
                    const void *g, const void *c, const void *w, void *p, float *dnum, float *dden, void *workspace,
                    size_t workspace_bytes, void *stream);

/*
 * out[n] = sum_b g[b, n] for g (rows, n), accumulated in float32, out (n) in dtype: the bias
 * gradient of the layer's bias add (kanforge/torch/layers.py:189-190, where torch autograd sums).
 * Deterministic (slabs of rows summed in order). Workspace of
 * kf_column_sums_workspace_bytes(rows, n) bytes.
 */
size_t kf_column_sums_workspace_bytes(int64_t rows, int64_t n);
int kf_column_sums(int dtype, int64_t rows, int64_t n, const void *g, void *out, void *workspace,
                   size_t workspace_bytes, void *stream);

/*
 * Second-order Taylor terms of the SiLU base branch, for the forward-mode Laplacian of a KAN
 * chain (what reverse-over-reverse autograd computes through kanforge/torch/science.py:25-46 and
 * the base branch of kanforge/torch/layers.py:183-184): for h (batch, n), hp (D, batch, n) and S
 * (batch, n) or NULL, writes sq = sum_d hp_d^2 (batch, n) and the stacked GEMM operand
 * A ((D + 2) batch, n) = [silu(h); silu'(h) hp_d for each d; silu''(h) sq + silu'(h) S].
 */
int kf_silu_taylor(int dtype, int64_t D, int64_t batch, int64_t n, const void *h, const void *hp, const void *S,
                   void *A, void *sq, void *stream);

/*
 * Diagnostics, no reference counterpart: the card's sustained bf16 MFMA rate. Launches `blocks`
 * workgroups of 4 waves, each running iters x 8 v_mfma_f32_32x32x16_bf16 on pseudo-random
 * operands (taken in rotation from eight register sets when `rotate`, else one fixed set).
 * out: device float[blocks * 256 * 3]; per workgroup, lane 0's entries 1 and 2 are the
 * shader-clock cycles and the 100 MHz real-time ticks of its first wave's MFMA loop.
 */
int kf_probe_mfma(int blocks, int iters, int rotate, float *out, void *stream);

/*
 * Lookup-table inference of one tabulated KAN layer. Replaces LUTLayer.__call__
 * (kanforge/export/lut.py:70-89):
 *   t = (x[b,i] - lo[i]) * inv_step[i]   (inv_step = (size - 1) / (hi - lo))
 *   j = min(floor(clip(t, 0, size-1)), size-2),  f = clip(t, 0, size-1) - j
 *   y[b,o] = bias[o] + scale[o] * sum_i (T[i,j,o] + f (T[i,j+1,o] - T[i,j,o]))
 *            + sum_i (min(t,0) slope_lo[i,o] + max(t-(size-1),0) slope_hi[i,o])
 * table_dtype: KF_F32 (scale NULL) or KF_I8 / KF_I16 (scale (n_out), from quantize,
 * kanforge/export/lut.py:175-197); tables (n_in, size, n_out); slope_lo/slope_hi (n_in, n_out)
 * per index step for linear extrapolation, both NULL to hold the end values ("clamp").
 * x (batch, n_in) and y (batch, n_out) float32; lo, inv_step (n_in), bias (n_out) float32.
 * Non-finite t clamps to the ends (x = NaN reads the first entry); size >= 2.
 */
int kf_lut_forward(int table_dtype, int64_t batch, int64_t n_in, int64_t size, int64_t n_out, const float *x,
                   const void *tables, const float *lo, const float *inv_step, const float *bias, const float *scale,
                   const float *slope_lo, const float *slope_hi, float *y, void *stream);

/* Text of the last error on the calling thread ("" if none). */
const char *kf_last_error(void);

/* Library version string, e.g. "kfhip 0.1.0 gfx950". */
const char *kf_version(void);

#ifdef __cplusplus
}
#endif

#endif /* KFHIP_H */
