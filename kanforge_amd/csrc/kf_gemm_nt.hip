// Plain bf16 GEMM with both operands contiguous along the reduction ("NT"):
//   C[m][n] = sum_k A[m][k] B[n][k]       A (M, lda), B (N, ldb) row-major, float32 accumulate,
// the contraction core of the routes whose features are precomputed (B-spline and rational F and
// G, rational P). Declared in kf_abi.h (gemm_nt, gemm_nt_workspace).
//
// Workgroup tile 256 x BN (BN = 128 TN), 8 waves, two per SIMD: wave (wm, wn) = (wave & 1,
// wave >> 1) owns rows 128 wm .. +127 and columns 32 TN wn .. +32 TN - 1 (4 x TN accumulator tiles
// of v_mfma_f32_32x32x16_bf16). A stage is RB bytes of k for the tile's 256 A rows and BN B rows,
// copied global -> LDS by all waves (direct copies, no VGPRs) into a ring of NBUF buffers
// (prefetch distance NBUF - 1), one barrier per stage; rows are dense with their 16-byte chunks
// XOR-swizzled by low row bits, so the fragment reads are free of bank conflicts. Rows past M or
// N repeat the last row (never stored). A split of the reduction (gridDim.y > 1) writes float32
// partial tiles, summed in split order by gemm_split_reduce (deterministic).
// Epilogue in passes of 64 rows through LDS, 16-byte stores where rows are aligned. An optional
// bias (bf16, one per column n) is added where the final sums are stored (the epilogue without a
// split, else the reductions).
#include "kf_abi.h"

using namespace kfabi;

namespace {

template <int TN, int RB, int NBUF, bool OUT_F32>
__global__ __launch_bounds__(512) void gemm_nt_kernel(int M, int N, int S, int s_per_split, const bf16* __restrict__ A,
                                                      long lda, const bf16* __restrict__ B, long ldb, void* __restrict__ C,
                                                      long ldc, long split_stride, int vout, int tile0, int compact,
                                                      const bf16* __restrict__ bias) {
  constexpr int BM = 256, BN = 128 * TN, SA = BM * RB, SS = (BM + BN) * RB, NBLK = SS / 1024, BPW = NBLK / 8;
  constexpr int CPR = RB / 16, RPB = 1024 / RB, KS = RB / 32, EPS = RB / 2;
  constexpr int RPASS = 64, RP = BN + 4;
  static_assert(RB == 64 || RB == 128, "64- or 128-byte stage rows");
  static_assert(BPW * 8 == NBLK, "copy blocks divide over the waves");
  static_assert(NBUF >= 2 && NBUF * SS <= 160 * 1024 && (RPASS * RP + BN) * 4 <= 160 * 1024,
                "stages and epilogue fit in LDS");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

  const int n_m = (M + BM - 1) / BM, n_n = (N + BN - 1) / BN;
  int tm_, tn_;
  xcd_tile_grouped(tile0 + blockIdx.x, n_m, n_n, 8, tm_, tn_);
  const int m0 = tm_ * BM, n0 = tn_ * BN;
  const int z = blockIdx.y;
  const int s_begin = z * s_per_split, s_end = s_begin + s_per_split < S ? s_begin + s_per_split : S;
  const int n_st = s_end - s_begin;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int h = lane >> 5, l32 = lane & 31;
  auto swz = [](int row) { return RB == 64 ? (row >> 2) & 3 : (row >> 1) & 7; };

  f32x16 acc[4][TN];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][t][r] = 0.f;

  // copy block k of this wave: RPB rows of the stage; lane l fills LDS chunk l % CPR of row
  // l / CPR with global chunk (l % CPR) ^ swz(row)
  const bf16* src[BPW];
#pragma unroll
  for (int k = 0; k < BPW; ++k) {
    const int row = (BPW * wave + k) * RPB + lane / CPR;
    const int c = (lane % CPR) ^ swz(row);
    if (row < BM) {
      const int m = m0 + row < M ? m0 + row : M - 1;
      src[k] = A + (size_t)m * lda + c * 8;
    } else {
      const int n = n0 + row - BM < N ? n0 + row - BM : N - 1;
      src[k] = B + (size_t)n * ldb + c * 8;
    }
  }
  auto copy_stage = [&](int st) {  // st relative to s_begin
    unsigned char* dst = smem + (st % NBUF) * SS + BPW * wave * 1024;
    const size_t koff = (size_t)(s_begin + st) * EPS;
#pragma unroll
    for (int k = 0; k < BPW; ++k) lds_dma16(src[k] + koff, dst + k * 1024);
  };
  const int sw = swz(l32);
  auto mma_stage = [&](int st) {
    const unsigned char* base = smem + (st % NBUF) * SS;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int co = 16 * ((2 * ks + h) ^ sw);
      u32x4 fa[4], fb[TN];
#pragma unroll
      for (int a = 0; a < 4; ++a) fa[a] = lds_read16(base + (wm * 128 + a * 32 + l32) * RB + co);
#pragma unroll
      for (int t = 0; t < TN; ++t) fb[t] = lds_read16(base + SA + ((TN * wn + t) * 32 + l32) * RB + co);
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int t = 0; t < TN; ++t) mma32<bf16>(acc[a][t], fa[a], fb[t]);
    }
  };

  for (int st = 0; st < NBUF - 1 && st < n_st; ++st) copy_stage(st);
  for (int s = 0; s < n_st; ++s) {
    // this wave's copies of stage s landed (the NBUF - 2 newer groups may still be in flight),
    // and its reads of stage s - 1, whose buffer is refilled below, returned
    if (s + NBUF - 1 <= n_st)
      vmem_wait<(NBUF - 2) * BPW>();
    else
      vmem_wait<0>();
    lds_wait();
    __builtin_amdgcn_s_barrier();
    if (s + NBUF - 1 < n_st) copy_stage(s + NBUF - 1);
    mma_stage(s);
  }
  vmem_wait<0>();
  lds_wait();

  // epilogue: passes of RPASS rows, accumulators -> LDS -> global
  float* red = reinterpret_cast<float*>(smem);  // [RPASS][RP], then the tile's bias [BN]
  float* bsh = red + RPASS * RP;
  const bool add_bias = bias && gridDim.y == 1 && !compact;  // final sums only
  constexpr int CH = OUT_F32 ? 4 : 8;            // elements per 16-byte chunk
  // compact: this workgroup's whole BM x BN float32 tile at (z gridDim.x + blockIdx.x) BM BN
  char* cbase = compact ? reinterpret_cast<char*>(C) + ((size_t)z * gridDim.x + blockIdx.x) * BM * BN * 4
                        : reinterpret_cast<char*>(C) + (size_t)z * split_stride * (OUT_F32 ? 4 : 2);
#pragma unroll
  for (int ps = 0; ps < BM / RPASS; ++ps) {
    __syncthreads();
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      if ((wm * 128 + a * 32) / RPASS != ps) continue;
      const int rbase = (wm * 128 + a * 32) % RPASS;
#pragma unroll
      for (int t = 0; t < TN; ++t) {
        const int col = (TN * wn + t) * 32 + l32;
#pragma unroll
        for (int r = 0; r < 16; ++r) red[(rbase + acc_row(r, lane)) * RP + col] = acc[a][t][r];
      }
    }
    // the tile's bias columns, once (after the first barrier: no wave still reads a stage there)
    if (add_bias && ps == 0)
      for (int t = tid; t < BN; t += 512) bsh[t] = n0 + t < N ? to_f32(bias[n0 + t]) : 0.f;
    __syncthreads();
    for (int e = tid; e < RPASS * (BN / CH); e += 512) {
      const int row = e / (BN / CH), ch = e % (BN / CH);
      const int m = m0 + ps * RPASS + row, n = n0 + ch * CH;
      const float* v = red + row * RP + ch * CH;
      if (OUT_F32 && compact) {
        gstore16(reinterpret_cast<float*>(cbase) + (size_t)(ps * RPASS + row) * BN + ch * CH,
                 __builtin_bit_cast(u32x4, f32x4{v[0], v[1], v[2], v[3]}));
        continue;
      }
      if (m >= M || n >= N) continue;
      float val[CH];
#pragma unroll
      for (int q = 0; q < CH; ++q) val[q] = v[q] + (add_bias ? bsh[ch * CH + q] : 0.f);
      if (OUT_F32) {
        float* dst = reinterpret_cast<float*>(cbase) + (size_t)m * ldc + n;
        if (vout && n + CH <= N) {
          gstore16(dst, __builtin_bit_cast(u32x4, f32x4{val[0], val[1], val[2], val[3]}));
        } else {
#pragma unroll
          for (int q = 0; q < CH; ++q)
            if (n + q < N) dst[q] = val[q];
        }
      } else {
        bf16* dst = reinterpret_cast<bf16*>(cbase) + (size_t)m * ldc + n;
        if (vout && n + CH <= N) {
          gstore16(dst, pack16<bf16>(val));
        } else {
#pragma unroll
          for (int q = 0; q < CH; ++q)
            if (n + q < N) dst[q] = from_f32<bf16>(val[q]);
        }
      }
    }
  }
}

// C[m][n] = sum over the splits z (in order) of part[z][m][n] (float32, row pitch N), converted to
// the output dtype; four consecutive columns per thread. With N % 4 == 0 (the partials are 256-byte
// aligned) every split is one 16-byte load and the loop over z has no branches, so its loads are
// in flight together; other widths read the four columns with clamped addresses and mask them.
// VST: C rows take one 8-byte (bf16) or 16-byte (float32) store per thread.
template <bool OUT_F32>
__global__ __launch_bounds__(256) void gemm_split_reduce(int M, int N, int nz, const float* __restrict__ part,
                                                         void* __restrict__ C, long ldc, int vst,
                                                         const bf16* __restrict__ bias) {
  const int n4 = (N + 3) / 4;
  const long total = (long)M * n4;
  const size_t zs = (size_t)M * N;
  for (long e = blockIdx.x * 256L + threadIdx.x; e < total; e += (long)gridDim.x * 256) {
    const int m = (int)(e / n4), n = (int)(e - (long)m * n4) * 4;
    const float* p = part + (size_t)m * N + n;
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    if (N % 4 == 0) {
#pragma unroll 4
      for (int z = 0; z < nz; ++z) {
        const float4 v = *reinterpret_cast<const float4*>(p + z * zs);
        s[0] += v.x;
        s[1] += v.y;
        s[2] += v.z;
        s[3] += v.w;
      }
    } else {
      int off[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) off[q] = n + q < N ? q : N - 1 - n;
#pragma unroll 2
      for (int z = 0; z < nz; ++z)
#pragma unroll
        for (int q = 0; q < 4; ++q) s[q] += p[z * zs + off[q]];
    }
    if (bias) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (n + q < N) s[q] += to_f32(bias[n + q]);
    }
    if (vst && n + 4 <= N) {
      if (OUT_F32) {
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(C) + (size_t)m * ldc + n) = float4{s[0], s[1], s[2], s[3]};
      } else {
        const bf16 o[4] = {from_f32<bf16>(s[0]), from_f32<bf16>(s[1]), from_f32<bf16>(s[2]), from_f32<bf16>(s[3])};
        *reinterpret_cast<uint2*>(reinterpret_cast<bf16*>(C) + (size_t)m * ldc + n) = __builtin_bit_cast(uint2, o);
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (n + q >= N) break;
        if (OUT_F32)
          reinterpret_cast<float*>(C)[(size_t)m * ldc + n + q] = s[q];
        else
          reinterpret_cast<bf16*>(C)[(size_t)m * ldc + n + q] = from_f32<bf16>(s[q]);
      }
    }
  }
}

// The tail tiles of a tail split: tile t of the launch that started at logical tile tile0 holds
// nz compact float32 partials part[z][t][256][BN]; C gets their sum in split order (deterministic)
// at the tile's place, rows and columns past M and N dropped. blockIdx.y = t.
template <bool OUT_F32>
__global__ __launch_bounds__(256) void gemm_tail_reduce(int M, int N, int n_m, int n_n, int tile0, int n_tail, int nz,
                                                        int BN, const float* __restrict__ part, void* __restrict__ C,
                                                        long ldc, int vst, const bf16* __restrict__ bias) {
  int tm, tn;
  xcd_tile_grouped(tile0 + blockIdx.y, n_m, n_n, 8, tm, tn);
  const int m0 = tm * 256, n0 = tn * BN, c4 = BN / 4;
  const size_t tsz = (size_t)256 * BN;
  for (int e = blockIdx.x * 256 + threadIdx.x; e < 256 * c4; e += gridDim.x * 256) {
    const int r = e / c4, c = (e - r * c4) * 4, m = m0 + r, n = n0 + c;
    if (m >= M || n >= N) continue;
    const float* p = part + (size_t)blockIdx.y * tsz + (size_t)r * BN + c;
    float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
    for (int z = 0; z < nz; ++z) {
      const float4 v = *reinterpret_cast<const float4*>(p + (size_t)z * n_tail * tsz);
      s[0] += v.x;
      s[1] += v.y;
      s[2] += v.z;
      s[3] += v.w;
    }
    if (bias) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (n + q < N) s[q] += to_f32(bias[n + q]);
    }
    if (vst && n + 4 <= N) {
      if (OUT_F32) {
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(C) + (size_t)m * ldc + n) = float4{s[0], s[1], s[2], s[3]};
      } else {
        const bf16 o[4] = {from_f32<bf16>(s[0]), from_f32<bf16>(s[1]), from_f32<bf16>(s[2]), from_f32<bf16>(s[3])};
        *reinterpret_cast<uint2*>(reinterpret_cast<bf16*>(C) + (size_t)m * ldc + n) = __builtin_bit_cast(uint2, o);
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (n + q >= N) break;
        if (OUT_F32)
          reinterpret_cast<float*>(C)[(size_t)m * ldc + n + q] = s[q];
        else
          reinterpret_cast<bf16*>(C)[(size_t)m * ldc + n + q] = from_f32<bf16>(s[q]);
      }
    }
  }
}

struct GemmCfg {
  int tn, nz;
  int tail_nz = 0;  // > 0: tail split (whole rounds of tiles over the full reduction, the rest split)
  long full = 0, rem = 0;  // tail split: tiles of the whole rounds, tail tiles
};

// Tile width and reduction split with the least modelled time: whole rounds of 256 workgroups,
// each stage of a 256 x 128 TN tile at ~4.7 TFLOP/s per CU (the core's measured rate; 15 % less
// for TN = 1, whose waves read 5 fragments per 4 MFMAs), plus the float32 partial sums of a split
// written and read back at ~5 TB/s. The tail split runs the tiles of whole rounds over the full
// reduction and splits only the remaining tiles, so a tile count just past a multiple of 256
// does not cost another whole round (plus ~5 us for its two extra launches). Narrow tiles
// (TN = 1) fill the chip without a split where N is small.
GemmCfg pick_gemm(long M, long N, long S) {
  GemmCfg best{3, 1};
  double best_t = 1e300;
  for (int tn : {3, 2, 1}) {
    const long tiles = ((M + 255) / 256) * ((N + 128 * tn - 1) / (128 * tn));
    const double t_stage = 256.0 * 128 * tn * 64 * 2 / (tn == 1 ? 4.0e12 : 4.7e12);
    for (int nz : {1, 2, 3, 4, 6, 8, 10, 12, 16, 24, 32}) {
      if (nz > S) break;
      const long wg = tiles * nz, rounds = (wg + 255) / 256, s_per = (S + nz - 1) / nz;
      double t = (double)rounds * s_per * t_stage;
      if (nz > 1) t += (double)nz * M * N * 8.0 / 5e12;
      if (t < best_t * 0.98) {
        best_t = t;
        best = {tn, nz};
      }
    }
    const long full = tiles / 256 * 256, rem = tiles - full;
    if (full == 0 || rem == 0) continue;
    for (int tz : {2, 4, 8, 16, 32}) {
      if (tz > S || rem * tz > 256) break;
      const double t = (double)(full / 256) * S * t_stage + (double)((S + tz - 1) / tz) * t_stage +
                       (double)tz * rem * 256 * 128 * tn * 8.0 / 5e12 + 5e-6;
      if (t < best_t * 0.98) {
        best_t = t;
        best = {tn, 1, tz, full, rem};
      }
    }
  }
  return best;
}

template <int TN, int RB, int NBUF, bool OUT_F32>
int launch_gemm(int M, int N, int S, int nz, const bf16* A, long lda, const bf16* B, long ldb, void* C, long ldc,
                long split_stride, int vout, hipStream_t s, long tile0 = 0, long n_tiles = -1, int compact = 0,
                const bf16* bias = nullptr) {
  constexpr int SS = (256 + 128 * TN) * RB, EPI = 64 * (128 * TN + 4) * 4 + 128 * TN * 4;
  constexpr size_t lds = (size_t)NBUF * SS > (size_t)EPI ? (size_t)NBUF * SS : (size_t)EPI;
  auto kern = gemm_nt_kernel<TN, RB, NBUF, OUT_F32>;
  if (!reserve_lds((const void*)kern, lds)) return fail(KF_ELAUNCH, "gemm: cannot reserve %zu bytes of LDS", lds);
  const int n_m = (M + 255) / 256, n_n = (N + 128 * TN - 1) / (128 * TN);
  if (n_tiles < 0) n_tiles = (long)n_m * n_n;
  const int s_per = (S + nz - 1) / nz;
  hipLaunchKernelGGL(kern, dim3((unsigned)n_tiles, (unsigned)nz), dim3(512), lds, s, M, N, S, s_per, A, lda, B, ldb,
                     C, ldc, split_stride, vout, (int)tile0, compact, bias);
  return check_launch("gemm_nt");
}

// Tail split: the whole rounds into C, the tail tiles' compact partials into ws, their sum into C.
template <int TN>
int launch_gemm_tail(const GemmCfg& c, int M, int N, int S, const bf16* A, long lda, const bf16* B, long ldb, void* C,
                     long ldc, bool out_f32, void* ws, hipStream_t s, const bf16* bias) {
  const int CH = out_f32 ? 4 : 8;
  const int vout = ldc % CH == 0 && aligned16(C);
  int rc = out_f32 ? launch_gemm<TN, 128, 2, true>(M, N, S, 1, A, lda, B, ldb, C, ldc, 0, vout, s, 0, c.full, 0, bias)
                   : launch_gemm<TN, 128, 2, false>(M, N, S, 1, A, lda, B, ldb, C, ldc, 0, vout, s, 0, c.full, 0, bias);
  if (rc) return rc;
  rc = launch_gemm<TN, 128, 2, true>(M, N, S, c.tail_nz, A, lda, B, ldb, ws, 0, 0, 1, s, c.full, c.rem, 1);
  if (rc) return rc;
  const int n_m = (M + 255) / 256, n_n = (N + 128 * TN - 1) / (128 * TN), BN = 128 * TN;
  const int vst = ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(C) & (out_f32 ? 15 : 7)) == 0;
  const dim3 grid(16, (unsigned)c.rem);
  if (out_f32)
    hipLaunchKernelGGL(gemm_tail_reduce<true>, grid, dim3(256), 0, s, M, N, n_m, n_n, (int)c.full, (int)c.rem,
                       c.tail_nz, BN, (const float*)ws, C, ldc, vst, bias);
  else
    hipLaunchKernelGGL(gemm_tail_reduce<false>, grid, dim3(256), 0, s, M, N, n_m, n_n, (int)c.full, (int)c.rem,
                       c.tail_nz, BN, (const float*)ws, C, ldc, vst, bias);
  return check_launch("gemm tail reduce");
}

size_t split_bytes(const GemmCfg& c, long M, long N) {
  if (c.tail_nz) return (size_t)c.tail_nz * c.rem * 256 * 128 * c.tn * sizeof(float);
  return c.nz > 1 ? (size_t)c.nz * M * N * sizeof(float) : 0;
}

}  // namespace

namespace kfabi {

size_t gemm_nt_workspace(long M, long N, long K) {
  if (K % 64 != 0) return 0;
  const size_t b = split_bytes(pick_gemm(M, N, K / 64), M, N);
  return b ? align256(b) : 0;
}

int gemm_nt(long M, long N, long K, const void* A, long lda, const void* B, long ldb, void* C, long ldc, bool out_f32,
            void* ws, size_t ws_bytes, hipStream_t s, const void* bias_v) {
  const bf16* bias = (const bf16*)bias_v;
  if (M <= 0 || N <= 0) return KF_OK;
  if (K % 64 || lda % 8 || ldb % 8 || !aligned16(A) || !aligned16(B) || K > lda || K > ldb)
    return fail(KF_EINVAL, "gemm: operands must be 16-byte aligned with whole 64-element stages");
  if (M > (1L << 30) || N > (1L << 30)) return fail(KF_EINVAL, "gemm: dimension too large");
  const int S = (int)(K / 64);
  const GemmCfg c = pick_gemm(M, N, S);
  const int CH = out_f32 ? 4 : 8;
  if (c.tail_nz) {
    const size_t need = split_bytes(c, M, N);
    if (!ws || ws_bytes < need || !aligned16(ws)) return fail(KF_EWORKSPACE, "gemm: split workspace of %zu bytes needed", need);
    return c.tn == 3   ? launch_gemm_tail<3>(c, (int)M, (int)N, S, (const bf16*)A, lda, (const bf16*)B, ldb, C, ldc, out_f32, ws, s, bias)
           : c.tn == 2 ? launch_gemm_tail<2>(c, (int)M, (int)N, S, (const bf16*)A, lda, (const bf16*)B, ldb, C, ldc, out_f32, ws, s, bias)
                       : launch_gemm_tail<1>(c, (int)M, (int)N, S, (const bf16*)A, lda, (const bf16*)B, ldb, C, ldc, out_f32, ws, s, bias);
  }
  if (c.nz == 1) {
    const int vout = ldc % CH == 0 && aligned16(C);
    if (out_f32)
      return c.tn == 3   ? launch_gemm<3, 128, 2, true>((int)M, (int)N, S, 1, (const bf16*)A, lda, (const bf16*)B, ldb, C, ldc, 0, vout, s, 0, -1, 0, bias)
             : c.tn == 2 ? launch_gemm<2, 128, 2, true>((int)M, (int)N, S, 1, (const bf16*)A, lda, (const bf16*)B, ldb, C, ldc, 0, vout, s, 0, -1, 0, bias)
                         : launch_gemm<1, 128, 2, true>((int)M, (int)N, S, 1, (const bf16*)A, lda, (const bf16*)B, ldb, C, ldc, 0, vout, s, 0, -1, 0, bias);
    return c.tn == 3   ? launch_gemm<3, 128, 2, false>((int)M, (int)N, S, 1, (const bf16*)A, lda, (const bf16*)B, ldb, C, ldc, 0, vout, s, 0, -1, 0, bias)
           : c.tn == 2 ? launch_gemm<2, 128, 2, false>((int)M, (int)N, S, 1, (const bf16*)A, lda, (const bf16*)B, ldb, C, ldc, 0, vout, s, 0, -1, 0, bias)
                       : launch_gemm<1, 128, 2, false>((int)M, (int)N, S, 1, (const bf16*)A, lda, (const bf16*)B, ldb, C, ldc, 0, vout, s, 0, -1, 0, bias);
  }
  const size_t need = (size_t)c.nz * M * N * sizeof(float);
  if (!ws || ws_bytes < need || !aligned16(ws)) return fail(KF_EWORKSPACE, "gemm: split workspace of %zu bytes needed", need);
  const int vout = N % 4 == 0;
  int rc = c.tn == 3   ? launch_gemm<3, 128, 2, true>((int)M, (int)N, S, c.nz, (const bf16*)A, lda, (const bf16*)B, ldb, ws, N, (long)M * N, vout, s)
           : c.tn == 2 ? launch_gemm<2, 128, 2, true>((int)M, (int)N, S, c.nz, (const bf16*)A, lda, (const bf16*)B, ldb, ws, N, (long)M * N, vout, s)
                       : launch_gemm<1, 128, 2, true>((int)M, (int)N, S, c.nz, (const bf16*)A, lda, (const bf16*)B, ldb, ws, N, (long)M * N, vout, s);
  if (rc) return rc;
  long blocks = ((long)M * ((N + 3) / 4) + 255) / 256;
  if (blocks > 65535 * 4) blocks = 65535 * 4;
  // whole 4-column stores: rows start 8- (bf16) or 16-byte (float32) aligned
  const int vst = ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(C) & (out_f32 ? 15 : 7)) == 0;
  if (out_f32)
    hipLaunchKernelGGL(gemm_split_reduce<true>, dim3((unsigned)blocks), dim3(256), 0, s, (int)M, (int)N, c.nz, (const float*)ws, C, ldc, vst, bias);
  else
    hipLaunchKernelGGL(gemm_split_reduce<false>, dim3((unsigned)blocks), dim3(256), 0, s, (int)M, (int)N, c.nz, (const float*)ws, C, ldc, vst, bias);
  return check_launch("gemm split reduce");
}

}  // namespace kfabi
