// SPDX-License-Identifier: BSD-3-Clause
// fp32 GEMM for small aligned shapes on gfx950, split-K inside a workgroup:
//   C[M,N] = epilogue( A[M,K] @ B[K,N] ), fp32 row-major,
// with M % 32 == 0, N % 32 == 0, K % (16 S) == 0, lda % 4 == 0 and A 16-byte
// aligned.
//
// It implements the one-wave 32x32 tile (2x2 v_mfma_f32_16x16x4_f32 tiles
// per wave) with split-K S <= 8.  The generic kernel (gemm.hpp) runs that
// tile as S workgroups of one wave over the grid, each writing a partial
// plane, and the last of them to arrive sums the planes.  For a small GEMM
// (512^3: 16 MFMA k-chunks per split) that walk is all latency: register
// staged slabs, a barrier per slab, a global round trip for the partials.
// Here the S splits of a tile are the S waves of one workgroup:
//   * wave q walks K range [q K/S, (q+1) K/S) in 16-deep chunks, loading its
//     operands straight from global memory into a ring of R chunks of
//     registers (no LDS, no barrier), R chunks ahead of the MFMAs; the
//     compiler's own vmcnt waits order each chunk's loads before its use.
//     R is the kernel's pipeline depth (2, 4 or 8).  At 512^3 with S = 4
//     (8 chunks per wave) R = 2 and 4 run within 3 % of each other and R = 8
//     is 20 % slower: every wave's full set of loads in flight at once
//     delays each wave's first chunk.  An empty kernel of the same grid
//     takes 2.4 us back to back, the MFMAs 1.7 us of the remaining ~3 us;
//   * per chunk a lane loads A[m][k .. k+3] (one 16-byte load per 16 rows,
//     k = 16 c + 4 g) and B[k + s][n] for s = 0..3 (four 4-byte loads per 16
//     columns), and issues 16 MFMAs: MFMA k index g at step s is physical
//     k = 16 c + 4 g + s, as in gemm.hpp;
//   * the S partial tiles meet in LDS; the first min(S, 4) waves then sum
//     the tile's four 16x16 quarters over the splits in split order,
//     starting from +0.0, and apply bias and relu.
// Per split, the MFMA sequence of every accumulator is the generic kernel's
// (chunk by chunk, s = 0..3), and the partials are summed in the same order,
// so the results are bit-identical to the generic split-K path.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemm.hpp"

namespace xtc_hip {

namespace splitwave {
typedef float f32x4 __attribute__((ext_vector_type(4)));
}  // namespace splitwave

// S splits (waves), R chunks of operands in flight per wave
template <int S, int R>
__global__ void __attribute__((amdgpu_flat_work_group_size(S * 64, S * 64))) gemm_f32_splitwave(GemmArgs args) {
  using namespace splitwave;
  static_assert(S >= 2 && S <= 8, "splits");
  static_assert(R >= 1 && R <= 16, "ring depth");
  constexpr int R_ = R;
  __shared__ f32x4 red[S][2][2][64];  // partial tiles, [split][i][j][lane]

  const int lane = threadIdx.x & 63;
  const int q = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15;
  const int g = lane >> 4;

  int tile_m, tile_n;
  tile_coords(args, tile_m, tile_n);
  const int m0 = tile_m * 32;
  const int n0 = tile_n * 32;
  const int kq = args.K / S;
  const int nch = kq / 16;
  const int kb = q * kq;

  const float* A = (const float*)args.A;
  const float* B = (const float*)args.B;
  // lane's A rows m0 + 16 i + l16 at k = kb + 16 c + 4 g; B rows kb + 16 c + 4 g + s at n0 + 16 j + l16
  const float* a_ptr = A + (size_t)(m0 + l16) * args.lda + kb + 4 * g;
  const size_t a_i = (size_t)16 * args.lda;
  const float* b_ptr = B + (size_t)(kb + 4 * g) * args.ldb + n0 + l16;
  const size_t b_s = (size_t)args.ldb;

  f32x4 ar[R_][2];
  float br[R_][4][2];
  auto issue = [&](int c, const int u) {
    const float* ap = a_ptr + 16 * c;
    ar[u][0] = *(const f32x4*)ap;
    ar[u][1] = *(const f32x4*)(ap + a_i);
    const float* bp = b_ptr + (size_t)16 * c * b_s;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      br[u][s][0] = bp[s * b_s];
      br[u][s][1] = bp[s * b_s + 16];
    }
  };

  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int u = 0; u < R_; ++u)
    if (u < nch) issue(u, u);
  for (int c = 0; c < nch; c += R_) {
#pragma unroll
    for (int u = 0; u < R_; ++u) {
      if (c + u < nch) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(ar[u][i][s], br[u][s][j], acc[i][j], 0, 0, 0);
        if (c + u + R_ < nch) issue(c + u + R_, u);
      }
    }
  }

  // ---- partial tiles meet in LDS; wave q finishes the 16x16 quarters
  // t = q, q + S, ... < 4 of the tile
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) red[q][i][j][lane] = acc[i][j];
  __syncthreads();
  // MFMA 16x16 result layout: lane (l16, g) holds rows 4 g .. 4 g + 3 of column l16
  for (int t = q; t < 4; t += S) {
    const int i = t >> 1, j = t & 1;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < S; ++p) v += red[p][i][j][lane];
    const int col = n0 + 16 * j + l16;
    const float bv = args.bias ? args.bias[col] : 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float x = v[r] + bv;
      if (args.relu && x < args.relu_threshold) x = args.relu_threshold;
      args.C[(size_t)(m0 + 16 * i + 4 * g + r) * args.ldc + col] = x;
    }
  }
}

}  // namespace xtc_hip
