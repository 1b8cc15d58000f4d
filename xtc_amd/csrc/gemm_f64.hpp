// SPDX-License-Identifier: BSD-3-Clause
// fp64 GEMM / implicit-GEMM conv2d on gfx950 MFMA (v_mfma_f64_16x16x4_f64):
//   C[M,N] (fp64) = epilogue( sum_k A[M,K] * B[K,N] ), all operands fp64
// the float64 case of XTCOperMatmul / XTCOperConv2D
// (src/xtc/graphs/xtc/operators.py:159-347), which the reference's MLIR
// backend lowers for f32 and f64 alike (src/xtc/backends/mlir/MlirOps.py:
// 194-195, 234, 339): linalg.fill(0) then accumulate, beta = 0.
//
// Structure (per workgroup = one BM x BN output tile, WGM x WGN waves, each
// owning (BM/WGM) x (BN/WGN) of 16x16 MFMA tiles with fp64 accumulators):
//   * K is walked in 16-deep slabs through two LDS buffers; the global loads
//     of slab t+1 (16-byte chunks = 2 doubles) go to registers before the
//     MFMAs of slab t and to the other buffer after them: one barrier per
//     slab.  fp64 MFMAs take 64 cycles per 16x16x4 step on a SIMD, so a
//     register-staged double buffer keeps the matrix core busy; no LDS DMA
//     is needed at this rate.
//   * A is stored row-major [BM][16 + 2] (144-byte rows: the 16 lanes of a
//     lane group read 16-byte chunks of 16 rows on distinct banks), B
//     row-major [16][BN + 8] (two k-rows 32 dwords apart modulo the banks).
//   * The MFMA's 4 k-slots are taken in a permuted order: within an 8-deep
//     chunk c of the slab, lane group g supplies k = 8c + 2g + s on MFMA
//     step s (s = 0, 1), so one ds_read_b128 gives a lane both of its A
//     values for the chunk; B is read as one double per lane per step with
//     the same k.  Every k of the slab is taken exactly once.
//   * MFMA operands: lane (l16, g) holds A[row l16][k_g] and B[k_g][col l16];
//     result register r of lane (l16, g) is row 4r + g of column l16 (the
//     fp64 16x16x4 result interleaves rows over the lane groups, unlike the
//     fp32 16x16x4 result, whose lane group g holds rows 4g .. 4g+3).
//   * Conv (CONV = true): A is the implicit im2col view of an NHWC input,
//     RSCF weights; the pad of a pad producer is folded into the loader
//     (out-of-image taps read pad_value).  C must be even (a 16-byte chunk
//     never crosses a tap).
//   * Epilogue: bias[N] and relu (max(x, threshold), NaN kept) fused; split-K
//     (blockIdx.z) stores fp64 partial tiles with 8-byte agent-scope atomic
//     stores, and the last workgroup to arrive at the tile's counter sums
//     them in split order (splitk.hpp's protocol, fp64 partials).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "splitk.hpp"

namespace xtc_hip {

typedef double f64x4 __attribute__((ext_vector_type(4)));
typedef double f64x2 __attribute__((ext_vector_type(2)));

struct GemmArgs64 {
  const double* A;     // [M][lda] (matrix) or NHWC input (conv)
  const double* B;     // [K][ldb]
  double* C;           // [M][ldc]
  const double* bias;  // [N] or null
  double* partial;     // split-K workspace [splits][M][N] or null
  unsigned* counters;  // split-K arrival counters [tiles_m * tiles_n], zero between launches
  int M, N, K;
  int lda, ldb, ldc;
  int k_per_split;     // multiple of 16
  int relu;
  double relu_threshold;
  int tiles_m, tiles_n;
  int group_m;
  int xcd_remap;
  int cH, cW, cC;      // conv: input spatial dims / channels (unpadded)
  int cOH, cOW;
  int cS;
  int cSH, cSW;
  int cPH, cPW;
  double pad_value;
};

namespace f64k {

// block id -> (tile row, tile column): contiguous tile ranges per XCD, then
// raster groups of group_m tile rows (the mapping of gemm.hpp's tile_coords)
__device__ __forceinline__ void tile_of(const GemmArgs64& a, int& tm, int& tn) {
  const int nb = a.tiles_m * a.tiles_n;
  int bid = blockIdx.x;
  if (a.xcd_remap && (nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
  const int per_group = a.group_m * a.tiles_n;
  const int group = bid / per_group;
  const int first_m = group * a.group_m;
  const int gsize = min(a.tiles_m - first_m, a.group_m);
  const int in_group = bid - group * per_group;
  tm = first_m + in_group % gsize;
  tn = in_group / gsize;
}

__device__ __forceinline__ void store_partial(double* p, double v) {
  __hip_atomic_store(reinterpret_cast<unsigned long long*>(p), (unsigned long long)__double_as_longlong(v),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ double load_partial(const double* p) {
  return __longlong_as_double((long long)__hip_atomic_load(
      reinterpret_cast<unsigned long long*>(const_cast<double*>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

}  // namespace f64k

template <int BM, int BN, int WGM, int WGN, bool CONV>
__global__ void __attribute__((amdgpu_flat_work_group_size(WGM * WGN * 64, WGM * WGN * 64)))
gemm_f64_kernel(GemmArgs64 args) {
  constexpr int BK = 16;
  constexpr int NT = WGM * WGN * 64;
  constexpr int WTM = BM / WGM, WTN = BN / WGN;
  constexpr int TM = WTM / 16, TN = WTN / 16;
  constexpr int AST = BK + 2;  // doubles per A row in LDS
  constexpr int BST = BN + 8;  // doubles per B row in LDS
  constexpr int A_ELEMS = BM * AST, B_ELEMS = BK * BST;
  constexpr int STAGE = A_ELEMS + B_ELEMS;
  constexpr int A_CHUNKS = BM * (BK / 2), B_CHUNKS = BK * (BN / 2);  // 16-byte chunks
  constexpr int A_PER_T = (A_CHUNKS + NT - 1) / NT, B_PER_T = (B_CHUNKS + NT - 1) / NT;
  static_assert(BM % (16 * WGM) == 0 && BN % (16 * WGN) == 0, "wave tile");
  static_assert(A_CHUNKS % NT == 0 || A_CHUNKS < NT, "A tile must split evenly over threads");
  static_assert(B_CHUNKS % NT == 0 || B_CHUNKS < NT, "B tile must split evenly over threads");

  __shared__ __attribute__((aligned(16))) double smem[2 * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int l16 = lane & 15, g = lane >> 4;

  int tile_m, tile_n;
  f64k::tile_of(args, tile_m, tile_n);
  const int m0 = tile_m * BM, n0 = tile_n * BN;
  const int split = blockIdx.z;
  const int k_begin = split * args.k_per_split;
  const int k_end = min(args.K, k_begin + args.k_per_split);
  const int nk = (k_end - k_begin + BK - 1) / BK;

  // ---- per-thread A chunk coordinates (fixed over the K walk)
  int a_row[A_PER_T], a_col[A_PER_T], a_base[A_PER_T], a_ih0[A_PER_T], a_iw0[A_PER_T];
  bool a_ok[A_PER_T], a_mine[A_PER_T];
#pragma unroll
  for (int i = 0; i < A_PER_T; ++i) {
    int c = tid + i * NT;
    a_mine[i] = A_CHUNKS % NT == 0 || c < A_CHUNKS;
    if (!a_mine[i]) c = 0;
    a_row[i] = c / (BK / 2);
    a_col[i] = (c % (BK / 2)) * 2;
    const int m = m0 + a_row[i];
    a_ok[i] = a_mine[i] && m < args.M;
    if constexpr (CONV) {
      const int mm = a_ok[i] ? m : 0;
      const int ow = mm % args.cOW;
      const int t = mm / args.cOW;
      const int oh = t % args.cOH;
      a_base[i] = (t / args.cOH) * args.cH;
      a_ih0[i] = oh * args.cSH - args.cPH;
      a_iw0[i] = ow * args.cSW - args.cPW;
    } else {
      a_base[i] = m * args.lda;
      a_ih0[i] = a_iw0[i] = 0;
    }
  }

  f64x2 areg[A_PER_T], breg[B_PER_T];
  const f64x2 zero2 = {0.0, 0.0};
  const f64x2 pad2 = {args.pad_value, args.pad_value};
  const bool tap_slabs = CONV && args.cC % BK == 0;

  auto load = [&](int kt) {
    int slab_r = 0, slab_s = 0, slab_c = 0;
    if constexpr (CONV) {
      if (tap_slabs) {
        const int rs = kt / args.cC;
        slab_c = kt - rs * args.cC;
        slab_s = rs % args.cS;
        slab_r = rs / args.cS;
      }
    }
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int k = kt + a_col[i];
      const bool ok = a_ok[i] && k < k_end;
      if constexpr (CONV) {
        int c, s, r;
        if (tap_slabs) {
          c = slab_c + a_col[i];
          s = slab_s;
          r = slab_r;
        } else {
          c = k % args.cC;
          const int rs = k / args.cC;
          s = rs % args.cS;
          r = rs / args.cS;
        }
        const int ih = a_ih0[i] + r, iw = a_iw0[i] + s;
        const bool inb = ok && ih >= 0 && ih < args.cH && iw >= 0 && iw < args.cW;
        areg[i] = inb ? *(const f64x2*)(args.A + ((size_t)(a_base[i] + ih) * args.cW + iw) * args.cC + c)
                      : (ok ? pad2 : zero2);
      } else {
        areg[i] = ok ? *(const f64x2*)(args.A + (size_t)a_base[i] + k) : zero2;
      }
    }
#pragma unroll
    for (int i = 0; i < B_PER_T; ++i) {
      const int c = tid + i * NT;
      const bool mine = B_CHUNKS % NT == 0 || c < B_CHUNKS;
      const int kr = c / (BN / 2);
      const int n = n0 + (c % (BN / 2)) * 2;
      const int k = kt + kr;
      breg[i] = mine && k < k_end && n < args.N ? *(const f64x2*)(args.B + (size_t)k * args.ldb + n) : zero2;
    }
  };

  auto store = [&](double* st) {
    double* As = st;
    double* Bs = st + A_ELEMS;
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i)
      if (a_mine[i]) *(f64x2*)(As + a_row[i] * AST + a_col[i]) = areg[i];
#pragma unroll
    for (int i = 0; i < B_PER_T; ++i) {
      const int c = tid + i * NT;
      if (!(B_CHUNKS % NT == 0 || c < B_CHUNKS)) continue;
      *(f64x2*)(Bs + (c / (BN / 2)) * BST + (c % (BN / 2)) * 2) = breg[i];
    }
  };

  f64x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f64x4{0.0, 0.0, 0.0, 0.0};

  const int wrow = wm * WTM, wcol = wn * WTN;
  auto compute = [&](const double* st) {
    const double* As = st;
    const double* Bs = st + A_ELEMS;
#pragma unroll
    for (int c = 0; c < BK / 8; ++c) {
      f64x2 af[TM];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = *(const f64x2*)(As + (wrow + i * 16 + l16) * AST + c * 8 + 2 * g);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        double bf[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) bf[j] = Bs[(c * 8 + 2 * g + s) * BST + wcol + j * 16 + l16];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(af[i][s], bf[j], acc[i][j], 0, 0, 0);
      }
    }
  };

  if (nk > 0) {
    load(k_begin);
    store(smem);
    __syncthreads();
    for (int it = 0; it < nk; ++it) {
      double* cur = smem + (it & 1) * STAGE;
      double* nxt = smem + ((it & 1) ^ 1) * STAGE;
      if (it + 1 < nk) load(k_begin + (it + 1) * BK);
      compute(cur);
      if (it + 1 < nk) store(nxt);
      __syncthreads();
    }
  }

  // ---- epilogue: register r of the lane is row wrow + 16 i + 4 r + g of column wcol + 16 j + l16
  const bool to_partial = args.partial != nullptr;
  double* out = to_partial ? args.partial + (size_t)split * args.M * args.N : args.C;
  const int ldo = to_partial ? args.N : args.ldc;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int col = n0 + wcol + j * 16 + l16;
    if (col >= args.N) continue;
    const double bv = (!to_partial && args.bias) ? args.bias[col] : 0.0;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wrow + i * 16 + 4 * r + g;
        if (row >= args.M) continue;
        double v = acc[i][j][r];
        if (to_partial) {
          f64k::store_partial(out + (size_t)row * ldo + col, v);
        } else {
          v += bv;
          if (args.relu && v < args.relu_threshold) v = args.relu_threshold;
          out[(size_t)row * ldo + col] = v;
        }
      }
    }
  }
  if (to_partial && splitk_arrive(args.counters + tile_m * args.tiles_n + tile_n, (int)gridDim.z)) {
    const size_t plane = (size_t)args.M * args.N;
    const int splits = (int)gridDim.z;
    for (int idx = tid; idx < BM * BN; idx += NT) {
      const int m = m0 + idx / BN, n = n0 + idx % BN;
      if (m >= args.M || n >= args.N) continue;
      double v = 0.0;
      for (int s = 0; s < splits; ++s) v += f64k::load_partial(args.partial + s * plane + (size_t)m * args.N + n);
      if (args.bias) v += args.bias[n];
      if (args.relu && v < args.relu_threshold) v = args.relu_threshold;
      args.C[(size_t)m * args.ldc + n] = v;
    }
    splitk_release(args.counters + tile_m * args.tiles_n + tile_n);
  }
}

}  // namespace xtc_hip
