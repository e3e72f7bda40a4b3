// MFMA tile primitives shared by the F, G and P contractions (gfx950).
//
// Every contraction is staged as "k-groups" of 64 bytes of the reduction
// dimension: 32 bf16 or 16 float32 values. Operand tiles live in LDS with the
// reduction dimension contiguous; each lane reads 16 bytes per fragment:
//   lane l supplies row (l % 16) and reduction elements [h*E, h*E+E) of the
//   k-group, h = l / 16, E = 16 / sizeof(T).
// bf16: one v_mfma_f32_16x16x32_bf16 per k-group and 16x16 tile.
// f32 : four v_mfma_f32_16x16x4_f32; instruction q takes element q of each
//       lane's four, so lanes h = 0..3 contribute reduction elements 4h+q.
// A and B use the same element-to-lane assignment, so the sum runs over the
// whole k-group. The accumulator of a 16x16 tile holds, in lane l,
// D[4*(l/16) + r][l % 16], r = 0..3 (checked on gfx950 hardware).
#pragma once

#include "kf_device.h"

namespace kf {

template <typename T>
struct KG {
  static constexpr int elems = 64 / sizeof(T);  // reduction elements per k-group
  static constexpr int per_lane = 16 / sizeof(T);
};

template <typename T>
__device__ __forceinline__ void mma(f32x4& acc, const u32x4& a, const u32x4& b);

template <>
__device__ __forceinline__ void mma<bf16>(f32x4& acc, const u32x4& a, const u32x4& b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), acc, 0,
                                                 0, 0);
}

template <>
__device__ __forceinline__ void mma<float>(f32x4& acc, const u32x4& a, const u32x4& b) {
  const f32x4 af = __builtin_bit_cast(f32x4, a);
  const f32x4 bf = __builtin_bit_cast(f32x4, b);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af[0], bf[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af[1], bf[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af[2], bf[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af[3], bf[3], acc, 0, 0, 0);
}

__device__ __forceinline__ u32x4 lds_read16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void lds_write16(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }

// Pack 16 bytes worth of float values into T elements.
template <typename T>
__device__ __forceinline__ u32x4 pack16(const float* v);
template <>
__device__ __forceinline__ u32x4 pack16<bf16>(const float* v) {
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (bf16)v[e];
  return __builtin_bit_cast(u32x4, r);
}
template <>
__device__ __forceinline__ u32x4 pack16<float>(const float* v) {
  f32x4 r = {v[0], v[1], v[2], v[3]};
  return __builtin_bit_cast(u32x4, r);
}

// Unpack 16 bytes of T elements into float values.
template <typename T>
__device__ __forceinline__ void unpack16(const u32x4& u, float* v);
template <>
__device__ __forceinline__ void unpack16<bf16>(const u32x4& u, float* v) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[2 * e] = __uint_as_float(u[e] << 16);
    v[2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u);
  }
}
template <>
__device__ __forceinline__ void unpack16<float>(const u32x4& u, float* v) {
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = __uint_as_float(u[e]);
}

// Load 16 bytes from global memory; `ok` false gives zeros.
__device__ __forceinline__ u32x4 gload16(const void* p, bool ok) {
  u32x4 z = {0u, 0u, 0u, 0u};
  return ok ? *reinterpret_cast<const u32x4*>(p) : z;
}

// gload16 without a branch: the load always runs, from p when ok and from the valid 16-byte aligned
// address safe otherwise, and the value is replaced by zeros when !ok. A predicated load compiles
// to a branch whose body waits for the load, which serialises a thread's loads; these stay in
// flight together.
__device__ __forceinline__ u32x4 gload16s(const void* p, bool ok, const void* safe) {
  const u32x4 v = *reinterpret_cast<const u32x4*>(ok ? p : safe);
  const u32x4 z = {0u, 0u, 0u, 0u};
  return ok ? v : z;
}

__device__ __forceinline__ void gstore16(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }

}  // namespace kf

namespace kf {

typedef float f32x16 __attribute__((ext_vector_type(16)));

// 32x32 tiles. A 16-byte lane fragment covers 32 bytes of the reduction
// dimension across the two lane halves h = lane / 32:
//   bf16: one v_mfma_f32_32x32x16_bf16 (lane supplies 8 consecutive elements);
//   f32 : four v_mfma_f32_32x32x2_f32; instruction q takes element q of each
//         lane, so lane halves contribute elements q and 4 + q.
// Accumulator element r of lane l is D[(r%4) + 8*(r/4) + 4*(l/32)][l % 32].
template <typename T>
__device__ __forceinline__ void mma32(f32x16& acc, const u32x4& a, const u32x4& b);

template <>
__device__ __forceinline__ void mma32<bf16>(f32x16& acc, const u32x4& a, const u32x4& b) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), acc, 0,
                                                 0, 0);
}

template <>
__device__ __forceinline__ void mma32<float>(f32x16& acc, const u32x4& a, const u32x4& b) {
  const f32x4 af = __builtin_bit_cast(f32x4, a);
  const f32x4 bf = __builtin_bit_cast(f32x4, b);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(af[0], bf[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(af[1], bf[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(af[2], bf[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(af[3], bf[3], acc, 0, 0, 0);
}

__device__ __forceinline__ int acc_row(int r, int lane) { return (r & 3) + 8 * (r >> 2) + 4 * (lane >> 5); }

// Workgroup index -> (m tile, n tile), XCD aware: hardware dispatches
// consecutive workgroups round-robin over the 8 XCDs, so workgroup g runs
// on XCD g % 8. Each XCD is given a contiguous range of the row-major tile
// order, so the tiles sharing operand panels meet in the same L2.
__device__ __forceinline__ void xcd_tile(int g, int n_m, int n_n, int& tm, int& tn) {
  const int total = n_m * n_n;
  int logical = g;
  if (total % 8 == 0) logical = (g % 8) * (total / 8) + g / 8;
  tm = logical / n_n;
  tn = logical % n_n;
}

// Grouped variant: inside each XCD's contiguous range, tiles run in groups
// of GM m-tiles x every n-tile, m fastest, so the workgroups resident on one
// XCD at a time share both operand panels in its L2 (GM m-panels and about
// 32 / GM n-panels instead of 1 x 32 or 32 x 1).
__device__ __forceinline__ void xcd_tile_grouped(int g, int n_m, int n_n, int GM, int& tm, int& tn) {
  const int total = n_m * n_n;
  int logical = g;
  if (total % 8 == 0) logical = (g % 8) * (total / 8) + g / 8;
  const int per_group = GM * n_n;
  const int first_m = (logical / per_group) * GM;
  const int gm = n_m - first_m < GM ? n_m - first_m : GM;
  const int r = logical % per_group;
  tm = first_m + r % gm;
  tn = r / gm;
}

}  // namespace kf
