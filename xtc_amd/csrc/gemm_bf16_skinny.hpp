// SPDX-License-Identifier: BSD-3-Clause
// bf16 GEMM for skinny A (M <= 16 rows) on gfx950: C[M,N] (fp32) =
// epilogue( A[M,K] (bf16) @ B[K,N] (bf16) ), both row-major.
//
// The cost is streaming B (K x N bf16) once from HBM; the arithmetic is a
// rounding error.  So the kernel is built around the B stream:
//   * a workgroup owns BN = 128 columns and a KC-deep chunk of K (split-K);
//     the grid (N/128 x K/KC) gives each CU a few independent 256-byte-wide
//     B row streams;
//   * B flows through STAGES LDS stages of 64 k-rows x 256 B by LDS DMA
//     (global_load_lds_dwordx4), STAGES-1 slabs ahead of the reads, one
//     vmcnt wait and one barrier per slab;
//   * A (16 x 64 per slab, 2 KB, an L2 hit after the first workgroup of a
//     split) is loaded by every wave straight into the MFMA fragment
//     registers together with the B slab: no LDS slice, no A reads from LDS;
//   * 4 waves each own 32 columns; per 32-deep k-step a wave reads two B
//     fragments (ds_read_b64_tr_b16) and issues two
//     v_mfma_f32_16x16x32_bf16 (B fragment first, so a lane holds 4
//     consecutive columns of one row);
//   * split-K partials go to a workspace [K/KC][16][N] (agent-scope stores);
//     the workgroup that stores the last partial of a column block sums them
//     in split order and applies bias / relu (splitk.hpp), so the result is
//     deterministic and the GEMM stays one launch.
// A rows >= M are loaded from row M-1 (any valid row) and never stored.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "splitk.hpp"

namespace xtc_hip {

struct SkinnyArgs {
  const __bf16* A;
  const __bf16* B;
  float* W;  // partials [splits][16][ldw], or C itself when splits == 1
  float* C;  // [M][ldc]
  const float* bias;
  unsigned* counters;  // [nblocks] arrival counters, zero between launches
  int M, N, K;
  int lda, ldb, ldw, ldc;
  int nblocks;  // N / 128
  int relu;
  float relu_threshold;
};

namespace skinny {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int BN = 128, BK = 64, WAVES = 4;
constexpr int B_STAGE = BK * BN * 2;  // 16 KB: 64 k-rows of 256 B

// 32-byte chunk swizzle of a 256-byte B row: the rows 8g + {0..3} and
// 8g + 8 + {0..3} read by one half-wave land on 8 distinct chunks.
__device__ __forceinline__ int swz_b(int k) { return (k & 3) | ((k >> 1) & 4); }

constexpr int waitcnt_vm(int n) { return (n & 15) | (7 << 4) | (15 << 8) | (((n >> 4) & 3) << 14); }

}  // namespace skinny

template <int KC, int STAGES>
__global__ void __attribute__((amdgpu_flat_work_group_size(256, 256))) gemm_bf16_skinny(SkinnyArgs args) {
  using namespace skinny;
  constexpr int B_DMA_PER_WAVE = B_STAGE / 1024 / WAVES;  // 4
  constexpr int A_LOADS = BK / 32;                        // 16-byte A loads per lane and slab
  constexpr int PER_SLAB = A_LOADS + B_DMA_PER_WAVE;      // vector-memory ops per wave and slab
  constexpr int NK = KC / BK;
  static_assert(KC % BK == 0, "split depth");
  static_assert(STAGES >= 2 && STAGES <= 4 && NK >= STAGES, "stages");
  static_assert((STAGES - 2) * PER_SLAB < 64, "vmcnt range");

  __shared__ __attribute__((aligned(1024))) unsigned char st0[B_STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char st1[B_STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char st2[STAGES > 2 ? B_STAGE : 16];
  __shared__ __attribute__((aligned(1024))) unsigned char st3[STAGES > 3 ? B_STAGE : 16];
  unsigned char* const stages[4] = {st0, st1, st2, st3};

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nb = blockIdx.x % args.nblocks;
  const int split = blockIdx.x / args.nblocks;
  const int n0 = nb * BN;
  const int k0 = split * KC;
  const int l16 = lane & 15;
  const int g = lane >> 4;

  // ---- B slabs: instruction i of wave w fills k-rows 4(4w+i) .. +3 of a
  // stage; lane l -> row +l/16, 16-byte slot l%16, holding global 32-byte
  // chunk (slot/2) ^ swz_b(row), half slot%2.
  int b_off[B_DMA_PER_WAVE];
#pragma unroll
  for (int i = 0; i < B_DMA_PER_WAVE; ++i) {
    const int row = 4 * (wave * B_DMA_PER_WAVE + i) + (lane >> 4);
    const int slot = lane & 15;
    b_off[i] = row * args.ldb + ((slot >> 1) ^ swz_b(row)) * 16 + (slot & 1) * 8;
  }
  const __bf16* b_base = args.B + (size_t)k0 * args.ldb + n0;
  const size_t b_step = (size_t)BK * args.ldb;
  // ---- A fragments straight into registers: lane (l16, g) of every wave
  // holds A[l16][k .. k+7] for k = 32 ks + 8 g of each slab.
  const int a_row = l16 < args.M ? l16 : args.M - 1;
  const __bf16* a_base = args.A + (size_t)a_row * args.lda + k0 + 8 * g;
  u32x4 ar[STAGES][A_LOADS];
  // A loads first, then the B DMAs: the compiler counts both (the builtin
  // DMA is a vector-memory op it knows), so its own waits for ar[] are exact.
  auto issue_slab = [&](int kt, const int si) {
#pragma unroll
    for (int h = 0; h < A_LOADS; ++h) ar[si][h] = *(const u32x4*)(a_base + kt * BK + 32 * h);
    const __bf16* bb = b_base + (size_t)kt * b_step;
    unsigned char* st = stages[si];
#pragma unroll
    for (int i = 0; i < B_DMA_PER_WAVE; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(bb + b_off[i]),
                                       (lds_void*)(st + (wave * B_DMA_PER_WAVE + i) * 1024), 16, 0, 0);
  };

  // ---- fragment coordinates
  const int b_krow0 = 8 * g + (l16 >> 2);
  const int b_f = swz_b(b_krow0);
  const int b_c0 = wave * 2;  // first 32-byte chunk (16 columns) of the wave

  f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s) issue_slab(s, s);

  auto step = [&](int kt, const int s) {
    // this wave's ops of slab kt are done once at most those of the slabs
    // issued after it are outstanding; the barrier then covers every wave's
    // DMAs into stage s
    if (kt + STAGES - 2 < NK)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm((STAGES - 2) * PER_SLAB));
    else
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __syncthreads();
    if (kt + STAGES - 1 < NK) issue_slab(kt + STAGES - 1, (s + STAGES - 1) % STAGES);
    const unsigned char* sb = stages[s];
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      const bf16x8 af = __builtin_bit_cast(bf16x8, ar[s][ks]);
#pragma unroll
      for (int jt = 0; jt < 2; ++jt) {
        const int c32 = (b_c0 + jt) ^ b_f;
        const int off0 = (ks * 32 + b_krow0) * 256 + c32 * 32 + 8 * (l16 & 3);
        i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(sb + off0));
        i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(sb + off0 + 4 * 256));
        const bf16x8 bf = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        acc[jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf, af, acc[jt], 0, 0, 0);
      }
    }
  };
  for (int kt = 0; kt < NK; kt += STAGES) {
#pragma unroll
    for (int s = 0; s < STAGES; ++s)
      if (kt + s < NK) step(kt + s, s);
  }

  // ---- store: lane holds row l16, columns n0 + 32 wave + 16 jt + 4g .. +3
  const int splits = gridDim.x / args.nblocks;
  const bool direct = splits == 1;  // W is C
  if (l16 < args.M) {
    float* row = args.W + ((direct ? 0 : (size_t)split * 16) + l16) * args.ldw;
#pragma unroll
    for (int jt = 0; jt < 2; ++jt) {
      const int n = n0 + wave * 32 + jt * 16 + 4 * g;
      f32x4 v = acc[jt];
      if (direct) {
        if (args.bias) v += *(const f32x4*)(args.bias + n);
        if (args.relu) {
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = v[r] < args.relu_threshold ? args.relu_threshold : v[r];
        }
      }
      if (direct)
        *(f32x4*)(row + n) = v;
      else
        splitk_store4(row + n, v);
    }
  }
  if (direct || !splitk_arrive(args.counters + nb, splits)) return;

  // ---- last workgroup of the column block: C[m][n0 + 4c .. +3] =
  // epilogue( sum_s W[s][m][...] ), 16 x 32 float4 over 256 threads
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int idx = tid + 256 * q;
    const int m = idx >> 5;
    const int n = n0 + 4 * (idx & 31);
    if (m < args.M) {
      f32x4 v = splitk_sum4(args.W + (size_t)m * args.ldw + n, (size_t)16 * args.ldw, splits);
      if (args.bias) v += *(const f32x4*)(args.bias + n);
      if (args.relu) {
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = v[r] < args.relu_threshold ? args.relu_threshold : v[r];
      }
      *(f32x4*)(args.C + (size_t)m * args.ldc + n) = v;
    }
  }
  splitk_release(args.counters + nb);
}

}  // namespace xtc_hip
