// Host-side checks of the C ABI (include/kfhip.h) for an AddressSanitizer + UndefinedBehavior
// build of libkfhip's sources: every workspace-size query over the layer shapes the library is
// benchmarked and tested on, and the argument validation of every entry point. Nothing here
// launches a kernel or touches a device, so it runs without a GPU; the sanitizers check the
// host code (descriptor validation, route and tile planning, workspace arithmetic).
//
// Prints "abi host checks: N passed" and exits 0, or lists the failures and exits 1.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "kfhip.h"

namespace {

int g_pass = 0;
std::vector<std::string> g_fail;

void check(bool ok, const std::string& what) {
  if (ok)
    ++g_pass;
  else
    g_fail.push_back(what);
}

// rc must be the error code `code` (any negative code when code == 0) with a message set
void expect_error(const char* what, int rc, int code = 0) {
  const char* msg = kf_last_error();
  const bool has_msg = msg && std::strlen(msg) > 0 && std::strlen(msg) < 4096;
  const bool ok = (code == 0 ? rc < 0 : rc == code) && has_msg;
  check(ok, std::string(what) + ": rc " + std::to_string(rc) + " msg '" + (msg ? msg : "(null)") + "'");
}

float g_host[4096];  // stands in for device tables: nothing below dereferences them on a device

kf_basis cheb(int K, int order, int n_t, int map) {
  kf_basis b{};
  b.kind = KF_KIND_CHEB;
  b.size = K;
  b.order = order;
  b.n_t = n_t;
  b.input_map = map;
  b.fold = g_host;
  return b;
}

kf_basis bspline(int grid, int k, int order, bool even) {
  kf_basis b{};
  b.kind = KF_KIND_BSPLINE;
  b.size = grid + k;
  b.order = order;
  b.n_t = b.size;
  b.spline_k = k;
  b.n_knots = b.size + k + 1;
  b.knots = g_host;
  b.knots_cmp = g_host;
  b.knots_uniform = even ? g_host : nullptr;
  return b;
}

kf_basis rational(int order, int group_size) {
  kf_basis b{};
  b.kind = KF_KIND_RATIONAL;
  b.size = 1;
  b.n_t = 1;
  b.order = order;
  b.num_deg = 5;
  b.den_deg = 4;
  b.group_size = group_size;
  b.num = g_host;
  b.den = g_host;
  return b;
}

struct Shape {
  int64_t batch, n_in, n_out;
};

}  // namespace

int main() {
  // the benchmarked and tested layer shapes, small and ragged ones
  const std::vector<Shape> shapes = {
      {8192, 768, 3072},  {16384, 768, 3072}, {16384, 3072, 768}, {4096, 64, 64},  {65536, 2, 64},
      {196608, 64, 64},   {65536, 64, 1},     {1, 1, 1},          {3, 5, 7},       {1000, 300, 265},
      {257, 129, 65},     {512, 768, 3072},   {512, 3072, 768},   {33, 7, 5},      {4096, 1024, 8},
  };
  std::vector<kf_basis> bases;
  for (int order = 0; order <= 3; ++order) {
    bases.push_back(cheb(9, order, order ? 9 + order - 2 : 9, order ? KF_MAP_TANH_SQ : KF_MAP_TANH));
    bases.push_back(cheb(7, order, 7, KF_MAP_IDENTITY));
    bases.push_back(bspline(8, 3, order, true));
    bases.push_back(bspline(5, 3, order, false));
    bases.push_back(bspline(3, 1, order, true));
  }
  for (const kf_basis& b : bases)
    for (const Shape& s : shapes)
      for (int dtype : {KF_F32, KF_BF16})
        for (int op : {KF_OP_F, KF_OP_G, KF_OP_P, KF_OP_F_BASE, KF_OP_P_BASE, KF_OP_G_BASE, KF_OP_G_BIAS}) {
          const size_t n = kf_workspace_bytes(op, &b, dtype, s.batch, s.n_in, s.n_out);
          check(n < (size_t(1) << 40), "workspace bytes of op " + std::to_string(op) + " kind " +
                                           std::to_string(b.kind) + " shape " + std::to_string(s.batch) + "x" +
                                           std::to_string(s.n_in) + "x" + std::to_string(s.n_out));
        }
  for (const Shape& s : shapes)
    for (int gs : {1, 8, 96, 384})
      if (s.n_in % gs == 0)
        for (int order = 0; order <= 3; ++order)
          for (int dtype : {KF_F32, KF_BF16}) {
            kf_basis b = rational(order, gs);
            for (int op : {KF_OP_F, KF_OP_G, KF_OP_P})
              check(kf_workspace_bytes(op, &b, dtype, s.batch, s.n_in, s.n_out) < (size_t(1) << 40), "rational ws");
            check(kf_rational_workspace_bytes(&b, s.batch, s.n_in) < (size_t(1) << 40), "rational grad ws");
            check(kf_rational_bwd_workspace_bytes(&b, dtype, s.batch, s.n_in, s.n_out) < (size_t(1) << 40),
                  "rational bwd ws");
          }
  for (const Shape& s : shapes) check(kf_column_sums_workspace_bytes(s.batch, s.n_out) < (size_t(1) << 40), "colsum ws");

  // the fused SiLU base branch: routes and their workspaces (a fused op has a workspace)
  for (const kf_basis& b : bases)
    for (const Shape& s : shapes)
      for (int dtype : {KF_F32, KF_BF16})
        for (int op : {KF_OP_F_BASE, KF_OP_P_BASE, KF_OP_G_BASE}) {
          const int r = kf_base_fused(op, &b, dtype, s.batch, s.n_in, s.n_out);
          const size_t n = kf_workspace_bytes(op, &b, dtype, s.batch, s.n_in, s.n_out);
          const bool sparse = dtype == KF_F32 && b.kind == KF_KIND_BSPLINE;  // F and P stage W themselves
          check(r == 0 || (r == 1 && (n > 0 || (sparse && op != KF_OP_G_BASE))),
                "base route " + std::to_string(op) + " reports a workspace");
          check(r == 0 || (dtype == KF_BF16 && (b.kind == KF_KIND_CHEB || b.kind == KF_KIND_BSPLINE)) ||
                    (dtype == KF_F32 && b.kind == KF_KIND_BSPLINE),
                "base route only for bf16 Chebyshev and B-spline layers and float32 B-splines");
        }
  {
    const kf_basis c0 = cheb(9, 0, 9, KF_MAP_TANH), c1 = cheb(9, 1, 8, KF_MAP_TANH_SQ);
    check(kf_base_fused(KF_OP_F_BASE, &c0, KF_BF16, 8192, 768, 3072) == 1, "headline F fused");
    check(kf_base_fused(KF_OP_P_BASE, &c1, KF_BF16, 8192, 768, 3072) == 1, "headline P fused");
    check(kf_base_fused(KF_OP_G_BASE, &c0, KF_BF16, 8192, 768, 3072) == 1, "headline G fused");
    const kf_basis c7 = cheb(7, 0, 7, KF_MAP_TANH);  // 7 features a chunk: not fused
    check(kf_base_fused(KF_OP_F_BASE, &c7, KF_BF16, 8192, 768, 3072) == 0, "7 features not fused");
    check(kf_base_fused(KF_OP_F_BASE, &c0, KF_BF16, 4096, 64, 4) == 0, "narrow layer not fused");
    expect_error("kf_base_fused unknown op", kf_base_fused(KF_OP_F, &c0, KF_BF16, 64, 64, 64), KF_EINVAL);
    const kf_basis s0 = bspline(8, 3, 0, true), s1 = bspline(8, 3, 1, true), s5 = bspline(5, 3, 1, true);
    check(kf_base_fused(KF_OP_P_BASE, &s1, KF_BF16, 16384, 768, 3072) == 1, "B-spline(8, 3) P fused");
    check(kf_base_fused(KF_OP_G_BASE, &s0, KF_BF16, 16384, 768, 3072) == 1, "B-spline(8, 3) G fused");
    check(kf_base_fused(KF_OP_F_BASE, &s0, KF_BF16, 16384, 768, 3072) == 1, "B-spline F fused");
    check(kf_base_fused(KF_OP_F_BASE, &s0, KF_BF16, 4096, 64, 4) == 0, "narrow B-spline layer not fused");
    check(kf_base_fused(KF_OP_P_BASE, &s5, KF_BF16, 16384, 768, 3072) == 0, "B-spline(5, 3) P: no spare slot tile");
    // float32 B-splines: the sparse kernels take W as basis function K
    const kf_basis f0 = bspline(5, 3, 0, false), f1 = bspline(5, 3, 1, false);
    for (int op : {KF_OP_F_BASE, KF_OP_G_BASE})
      check(kf_base_fused(op, &f0, KF_F32, 4096, 64, 64) == 1, "64 -> 64 float32 B-spline fused " + std::to_string(op));
    check(kf_base_fused(KF_OP_P_BASE, &f1, KF_F32, 4096, 64, 64) == 1, "64 -> 64 float32 B-spline P fused");
    check(kf_base_fused(KF_OP_F_BASE, &c0, KF_F32, 4096, 64, 64) == 0, "float32 Chebyshev not fused");
    check(kf_workspace_bytes(KF_OP_G_BASE, &f0, KF_F32, 4096, 64, 64) >
              kf_workspace_bytes(KF_OP_G, &f0, KF_F32, 4096, 64, 64),
          "sparse G_base partials hold K + 1 features");
  }

  // descriptor validation (through kf_F: every entry point validates the same way first)
  float* d = g_host;
  auto F = [&](const kf_basis* b, int dtype, int64_t batch, int64_t n_in, int64_t n_out) {
    return kf_F(b, dtype, batch, n_in, n_out, d, nullptr, d, d, nullptr, 0, nullptr);
  };
  expect_error("NULL descriptor", F(nullptr, KF_F32, 4, 4, 4), KF_EINVAL);
  {
    kf_basis b = cheb(9, 0, 9, KF_MAP_TANH);
    b.size = 0;
    expect_error("size 0", F(&b, KF_F32, 4, 4, 4), KF_EINVAL);
    b.size = KF_MAX_K + 1;
    expect_error("size above the maximum", F(&b, KF_F32, 4, 4, 4), KF_EINVAL);
    b = cheb(9, 9, 9, KF_MAP_TANH);
    expect_error("order 9", F(&b, KF_F32, 4, 4, 4), KF_EUNSUPPORTED);
    b = cheb(9, 0, KF_MAX_NT + 1, KF_MAP_TANH);
    expect_error("n_t above the maximum", F(&b, KF_F32, 4, 4, 4), KF_EINVAL);
    b = cheb(9, 0, 9, 7);
    expect_error("unknown input map", F(&b, KF_F32, 4, 4, 4), KF_EINVAL);
    b = cheb(9, 0, 9, KF_MAP_TANH);
    b.fold = nullptr;
    expect_error("cheb without fold", F(&b, KF_F32, 4, 4, 4), KF_EINVAL);
    b = cheb(9, 0, 9, KF_MAP_TANH);
    b.kind = 9;
    expect_error("unknown kind", F(&b, KF_F32, 4, 4, 4), KF_EINVAL);
  }
  {
    kf_basis b = bspline(8, 3, 0, true);
    b.spline_k = 6;
    expect_error("B-spline degree 6", F(&b, KF_F32, 4, 4, 4), KF_EUNSUPPORTED);
    b = bspline(8, 3, 0, true);
    b.n_knots += 1;
    expect_error("n_knots mismatch", F(&b, KF_F32, 4, 4, 4), KF_EINVAL);
    b = bspline(8, 3, 0, true);
    b.n_t = b.size + 1;
    expect_error("B-spline n_t != size", F(&b, KF_F32, 4, 4, 4), KF_EINVAL);
    b = bspline(8, 3, 0, true);
    b.knots_cmp = nullptr;
    expect_error("B-spline without knot tables", F(&b, KF_F32, 4, 4, 4), KF_EINVAL);
  }
  {
    kf_basis b = rational(0, 4);
    b.size = 2;
    expect_error("rational size 2", F(&b, KF_F32, 4, 8, 4), KF_EINVAL);
    b = rational(0, 4);
    b.den_deg = 0;
    expect_error("rational degree Q 0", F(&b, KF_F32, 4, 8, 4), KF_EUNSUPPORTED);
    b = rational(0, 4);
    b.num_deg = 20;
    expect_error("rational degrees above the parameter limit", F(&b, KF_F32, 4, 8, 4), KF_EUNSUPPORTED);
    b = rational(0, 4);
    b.num = nullptr;
    expect_error("rational without num", F(&b, KF_F32, 4, 8, 4), KF_EINVAL);
    b = rational(0, 0);
    expect_error("group size 0", F(&b, KF_F32, 4, 8, 4), KF_EINVAL);
    b = rational(0, 3);
    expect_error("group size not dividing n_in", F(&b, KF_F32, 4, 8, 4), KF_EINVAL);
  }
  {
    kf_basis b = cheb(9, 0, 9, KF_MAP_TANH);
    expect_error("dtype 5", F(&b, 5, 4, 4, 4), KF_EINVAL);
    expect_error("negative batch", F(&b, KF_F32, -1, 4, 4), KF_EINVAL);
    expect_error("negative n_out", F(&b, KF_F32, 4, 4, -3), KF_EINVAL);
    expect_error("n_in too large", F(&b, KF_F32, 4, int64_t(1) << 25, 4), KF_EINVAL);
    expect_error("batch too large", F(&b, KF_F32, int64_t(1) << 31, 4, 4), KF_EINVAL);
  }

  // arrays and workspaces of each entry point
  kf_basis cb = cheb(9, 0, 9, KF_MAP_TANH), bb = bspline(8, 3, 1, true), rb = rational(0, 8);
  char* misaligned = reinterpret_cast<char*>(g_host) + 1;
  expect_error("kf_F NULL x", kf_F(&cb, KF_BF16, 64, 32, 16, nullptr, nullptr, d, d, d, 1 << 20, nullptr), KF_EINVAL);
  expect_error("kf_F no workspace", kf_F(&cb, KF_BF16, 8192, 768, 3072, d, nullptr, d, d, nullptr, 0, nullptr),
               KF_EWORKSPACE);
  expect_error("kf_F small workspace", kf_F(&bb, KF_BF16, 8192, 768, 3072, d, nullptr, d, d, d, 64, nullptr),
               KF_EWORKSPACE);
  expect_error("kf_F misaligned workspace",
               kf_F(&cb, KF_F32, 8192, 768, 3072, d, nullptr, d, d, misaligned, size_t(1) << 40, nullptr),
               KF_EWORKSPACE);
  expect_error("kf_F_noalloc NULL y", kf_F_noalloc(&cb, KF_F32, 64, 32, 16, d, nullptr, d, nullptr, nullptr),
               KF_EINVAL);
  expect_error("kf_G NULL g", kf_G(&cb, KF_BF16, 64, 32, 16, d, nullptr, nullptr, d, d, 1 << 20, nullptr), KF_EINVAL);
  expect_error("kf_G small workspace", kf_G(&bb, KF_BF16, 16384, 768, 3072, d, d, nullptr, d, d, 64, nullptr),
               KF_EWORKSPACE);
  expect_error("kf_P NULL c", kf_P(&cb, KF_BF16, 64, 32, 16, d, d, nullptr, d, nullptr, d, 1 << 20, nullptr),
               KF_EINVAL);
  expect_error("kf_P h for a non-rational kind", kf_P(&cb, KF_F32, 64, 32, 16, d, d, d, d, g_host, d, 1 << 20, nullptr),
               KF_EINVAL);
  expect_error("kf_P small workspace", kf_P(&rb, KF_BF16, 16384, 3072, 768, d, d, d, d, nullptr, d, 64, nullptr),
               KF_EWORKSPACE);
  expect_error("kf_features NULL out", kf_features(&bb, KF_F32, 64, 32, d, nullptr, nullptr), KF_EINVAL);
  expect_error("kf_edge_derivative NULL c",
               kf_edge_derivative(&cb, KF_F32, 64, 32, 16, d, nullptr, nullptr, d, nullptr), KF_EINVAL);
  expect_error("kf_bspline_interval one knot", kf_bspline_interval(4, 4, d, d, 1, nullptr, nullptr), KF_EINVAL);
  expect_error("kf_bspline_interval negative batch", kf_bspline_interval(-4, 4, d, d, 8, nullptr, nullptr), KF_EINVAL);
  expect_error("kf_rational_param_grad non-rational kind",
               kf_rational_param_grad(&cb, KF_F32, 64, 32, d, d, nullptr, g_host, g_host, d, 1 << 20, nullptr),
               KF_EINVAL);
  expect_error("kf_rational_param_grad NULL outputs",
               kf_rational_param_grad(&rb, KF_F32, 64, 32, d, d, nullptr, nullptr, nullptr, d, 1 << 20, nullptr),
               KF_EINVAL);
  expect_error("kf_rational_bwd NULL p",
               kf_rational_bwd(&rb, KF_BF16, 64, 32, 16, d, d, d, nullptr, nullptr, g_host, g_host, d, 1 << 20, nullptr),
               KF_EINVAL);
  expect_error("kf_rational_bwd small workspace",
               kf_rational_bwd(&rb, KF_BF16, 16384, 3072, 768, d, d, d, nullptr, d, g_host, g_host, d, 64, nullptr),
               KF_EWORKSPACE);
  expect_error("kf_column_sums negative rows", kf_column_sums(KF_F32, -1, 8, d, d, d, 1 << 20, nullptr), KF_EINVAL);
  expect_error("kf_column_sums dtype", kf_column_sums(KF_I8, 8, 8, d, d, d, 1 << 20, nullptr), KF_EUNSUPPORTED);
  expect_error("kf_column_sums small workspace", kf_column_sums(KF_BF16, 16384, 3072, d, d, d, 0, nullptr),
               KF_EWORKSPACE);
  expect_error("kf_silu_taylor NULL hp", kf_silu_taylor(KF_F32, 2, 64, 8, d, nullptr, nullptr, d, d, nullptr),
               KF_EINVAL);
  expect_error("kf_silu_taylor negative D", kf_silu_taylor(KF_F32, -1, 64, 8, d, d, nullptr, d, d, nullptr), KF_EINVAL);
  expect_error("kf_lut_forward one point",
               kf_lut_forward(KF_F32, 64, 8, 1, 8, d, d, d, d, d, nullptr, nullptr, nullptr, d, nullptr), KF_EINVAL);
  expect_error("kf_lut_forward int8 without scale",
               kf_lut_forward(KF_I8, 64, 8, 16, 8, d, d, d, d, d, nullptr, nullptr, nullptr, d, nullptr), KF_EINVAL);
  expect_error("kf_lut_forward one slope table",
               kf_lut_forward(KF_F32, 64, 8, 16, 8, d, d, d, d, d, nullptr, d, nullptr, d, nullptr), KF_EINVAL);
  expect_error("kf_lut_forward table dtype",
               kf_lut_forward(KF_BF16, 64, 8, 16, 8, d, d, d, d, d, nullptr, nullptr, nullptr, d, nullptr),
               KF_EUNSUPPORTED);

  {
    const kf_basis c0 = cheb(9, 0, 9, KF_MAP_TANH), c1 = cheb(9, 1, 8, KF_MAP_TANH_SQ);
    expect_error("kf_F_base NULL base_w",
                 kf_F_base(&c0, KF_BF16, 8192, 768, 3072, d, d, nullptr, nullptr, d, d, 1 << 30, nullptr), KF_EINVAL);
    expect_error("kf_F_base float32", kf_F_base(&c0, KF_F32, 8192, 768, 3072, d, d, d, nullptr, d, d, 1 << 30, nullptr),
                 KF_EUNSUPPORTED);
    expect_error("kf_F_base order 1", kf_F_base(&c1, KF_BF16, 8192, 768, 3072, d, d, d, nullptr, d, d, 1 << 30, nullptr),
                 KF_EUNSUPPORTED);
    expect_error("kf_F_base small workspace",
                 kf_F_base(&c0, KF_BF16, 8192, 768, 3072, d, d, d, nullptr, d, d, 64, nullptr), KF_EWORKSPACE);
    expect_error("kf_P_base order 0", kf_P_base(&c0, KF_BF16, 8192, 768, 3072, d, d, d, d, d, d, 1 << 30, nullptr),
                 KF_EUNSUPPORTED);
    expect_error("kf_P_base NULL g", kf_P_base(&c1, KF_BF16, 8192, 768, 3072, d, nullptr, d, d, d, d, 1 << 30, nullptr),
                 KF_EINVAL);
    expect_error("kf_P_base no workspace", kf_P_base(&c1, KF_BF16, 8192, 768, 3072, d, d, d, d, d, nullptr, 0, nullptr),
                 KF_EWORKSPACE);
    expect_error("kf_G_base small workspace",
                 kf_G_base(&c0, KF_BF16, 8192, 768, 3072, d, d, d, d, d, d, 256, nullptr), KF_EWORKSPACE);
    expect_error("kf_G_base empty batch", kf_G_base(&c0, KF_BF16, 0, 768, 3072, d, d, d, d, d, d, 256, nullptr),
                 KF_EINVAL);
    expect_error("kf_G_base small layer", kf_G_base(&c0, KF_BF16, 64, 48, 192, d, d, d, d, d, d, 1 << 30, nullptr),
                 KF_EUNSUPPORTED);
    check(kf_G_base(&c0, KF_BF16, 64, 48, 192, d, d, nullptr, nullptr, nullptr, nullptr, 0, nullptr) == KF_OK,
          "G_base with nothing wanted");
  }

  {
    const kf_basis c0 = cheb(9, 0, 9, KF_MAP_TANH);
    expect_error("kf_F_bias NULL y", kf_F_bias(&c0, KF_BF16, 64, 32, 16, d, nullptr, d, d, nullptr, d, 1 << 20, nullptr),
                 KF_EINVAL);
    expect_error("kf_F_bias small workspace",
                 kf_F_bias(&c0, KF_BF16, 8192, 768, 3072, d, nullptr, d, d, d, d, 64, nullptr), KF_EWORKSPACE);
    check(kf_F_bias(&c0, KF_F32, 0, 4, 4, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0, nullptr) == KF_OK,
          "empty F_bias");
    expect_error("kf_G_bias NULL dc", kf_G_bias(&c0, KF_BF16, 64, 32, 16, d, d, nullptr, nullptr, d, d, 1 << 20, nullptr),
                 KF_EINVAL);
    expect_error("kf_G_bias small workspace",
                 kf_G_bias(&c0, KF_BF16, 8192, 768, 3072, d, d, nullptr, d, d, d, 256, nullptr), KF_EWORKSPACE);
  }

  // empty calls succeed without touching a device
  check(kf_F(&cb, KF_F32, 0, 4, 4, nullptr, nullptr, nullptr, nullptr, nullptr, 0, nullptr) == KF_OK, "empty F");
  check(kf_G(&cb, KF_F32, 4, 0, 4, nullptr, nullptr, nullptr, nullptr, nullptr, 0, nullptr) == KF_OK, "empty G");
  check(kf_P(&cb, KF_F32, 0, 4, 4, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0, nullptr) == KF_OK,
        "empty P");
  check(std::strlen(kf_version()) > 0, "version string");

  if (!g_fail.empty()) {
    for (const std::string& f : g_fail) std::printf("FAILED %s\n", f.c_str());
    std::printf("abi host checks: %d passed, %zu failed\n", g_pass, g_fail.size());
    return 1;
  }
  std::printf("abi host checks: %d passed\n", g_pass);
  return 0;
}
