// SPDX-License-Identifier: BSD-3-Clause
// fp32 GEMM for aligned shapes on gfx950, LDS-DMA pipeline, one workgroup
// of 8 waves per CU:
//   C[M,N] = epilogue( A[M,K] @ B[K,N] ), fp32 row-major, optional split-K
// with M % BM == 0, N % BN == 0, each split's K range a multiple of BK (16 or 32),
// lda and ldb multiples of 4 and 16-byte aligned operands.
//
// v_mfma_f32_16x16x4_f32 issues at full rate with one or two waves per SIMD
// from one workgroup, and drops to about 65 % with four (measured on MI355X
// with register-only loops).  The register-staged generic kernel (gemm.hpp)
// needs two workgroups per CU to hide its global-load latency.  This kernel
// hides it in one workgroup instead:
//   * 8 waves (WGM x WGN), one workgroup per CU (the stages fill the LDS):
//     two waves per SIMD;
//   * global -> LDS by LDS DMA (global_load_lds_dwordx4, issued from asm),
//     STAGES stages of one BK-deep slab, D = STAGES - 1 slabs ahead of the
//     MFMAs;
//   * per slab, each wave issues the DMA of slab t+D, reads its fragments of
//     slab t (ds_read_b128 for A, ds_read_b32 for B), issues its MFMAs,
//     waits for its own DMA of slab t+1 (s_waitcnt vmcnt) and meets the other
//     waves at one barrier: slab t+1 is then visible, and the stage of slab
//     t, read before the barrier, is free for the DMA of slab t+STAGES.
// LDS layouts (16-byte chunks, XOR-swizzled so that a wave's fragment reads
// hit distinct banks):
//   * A: BM rows of BK floats; chunk c of row r holds global chunk
//     c ^ swz_a(r).  Lane (l16, g) reads A[r][16 kc + 4 g .. +3] with one
//     ds_read_b128: the A values of 4 MFMAs (s = 0..3).
//   * B: BK rows of BN floats; chunk c of row k holds global chunk
//     c ^ (4 ((k >> 2) & 3)).  Lane (l16, g) reads B[16 kc + 4 g + s][n] with
//     ds_read_b32: the four lane groups read rows 4 apart, which the swizzle
//     moves 16 floats (16 banks) apart.
// The MFMA k index of lane group g at step s is physical k = 16 kc + 4 g + s
// for both operands, as in gemm.hpp, and the per-accumulator MFMA sequence
// is the generic kernel's; B is the first operand, so a lane ends up holding
// C[m][n .. n+3] and stores float4s.  Split-K uses the protocol of
// splitk.hpp (partials, arrival counter, the last workgroup sums in split
// order).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemm.hpp"
#include "lds_dma.hpp"
#include "splitk.hpp"

namespace xtc_hip {

namespace f32lds {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) f32x4 lds_f32x4;
typedef __attribute__((address_space(3))) float lds_f32;

constexpr int waitcnt_vm(int n) { return (n & 15) | (7 << 4) | (15 << 8) | (((n >> 4) & 3) << 14); }

// 16-byte chunk swizzle of an A row of BK floats
template <int BK>
__device__ __forceinline__ int swz_a(int r) {
  return BK == 16 ? ((r >> 2) & 3) : ((r >> 1) & 7);
}
// 16-byte chunk swizzle of B row k
__device__ __forceinline__ int swz_b(int k) { return ((k >> 2) & 3) << 2; }

// Workgroup barrier without a memory fence: the waits around it are
// explicit.  The empty asm statements keep memory accesses from moving
// across it, the scheduling barriers keep every instruction on its side.
__device__ __forceinline__ void slab_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
}

}  // namespace f32lds

template <int BM, int BN, int BK, int WGM, int WGN, int STAGES>
__global__ void __attribute__((amdgpu_flat_work_group_size(512, 512))) gemm_f32_lds(GemmArgs args) {
  using namespace f32lds;
  constexpr int TM = BM / WGM / 16, TN = BN / WGN / 16;  // 16x16 tiles per wave
  constexpr int KC = BK / 16;                            // 16-deep k chunks per slab
  constexpr int A_STAGE = BM * BK * 4;
  constexpr int B_STAGE = BK * BN * 4;
  constexpr int STAGE = A_STAGE + B_STAGE;
  constexpr int A_KB = A_STAGE / 1024 / 8;  // DMA instructions per wave per slab
  constexpr int B_KB = B_STAGE / 1024 / 8;
  constexpr int DMA_PER_SLAB = A_KB + B_KB;
  constexpr int A_ROWS_PER_KB = 1024 / (BK * 4);
  constexpr int A_CHUNKS = BK / 4;
  constexpr int B_ROWS_PER_KB = 1024 / (BN * 4);
  constexpr int B_CHUNKS = BN / 4;
  constexpr int D = STAGES - 1;
  static_assert(WGM * WGN == 8 && TM >= 1 && TN >= 1 && TM * 16 * WGM == BM && TN * 16 * WGN == BN, "8 waves");
  static_assert(BK == 16 || BK == 32, "BK");
  static_assert(BN * 4 <= 1024 && 1024 % (BN * 4) == 0, "a DMA kilobyte holds whole B rows");
  static_assert(A_KB * 8 * 1024 == A_STAGE && B_KB * 8 * 1024 == B_STAGE, "stage must split over 8 waves");
  static_assert(STAGES >= 2 && STAGES <= 6 && STAGES * STAGE <= 160 * 1024, "LDS");
  static_assert(D * DMA_PER_SLAB < 64, "vmcnt range");

  __shared__ __attribute__((aligned(1024))) unsigned char st0[STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char st1[STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char st2[STAGES > 2 ? STAGE : 16];
  __shared__ __attribute__((aligned(1024))) unsigned char st3[STAGES > 3 ? STAGE : 16];
  __shared__ __attribute__((aligned(1024))) unsigned char st4[STAGES > 4 ? STAGE : 16];
  __shared__ __attribute__((aligned(1024))) unsigned char st5[STAGES > 5 ? STAGE : 16];
  auto stage = [&](int s) -> unsigned char* {
    return s == 0 ? st0 : s == 1 ? st1 : s == 2 ? st2 : s == 3 ? st3 : s == 4 ? st4 : st5;
  };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN;
  const int wn = wave % WGN;

  int tile_m, tile_n;
  tile_coords(args, tile_m, tile_n);
  const int m0 = tile_m * BM;
  const int n0 = tile_n * BN;
  const int split = blockIdx.z;
  const int k_begin = split * args.k_per_split;
  const int nk = min(args.K - k_begin, args.k_per_split) / BK;

  // ---- LDS DMA sources (16 bytes per lane, 1 KB per instruction)
  int a_off[A_KB];
  int b_off[B_KB];
#pragma unroll
  for (int i = 0; i < A_KB; ++i) {
    const int kb = wave * A_KB + i;
    const int r = kb * A_ROWS_PER_KB + lane / A_CHUNKS;
    a_off[i] = r * args.lda + ((lane % A_CHUNKS) ^ swz_a<BK>(r)) * 4;
  }
#pragma unroll
  for (int i = 0; i < B_KB; ++i) {
    const int kb = wave * B_KB + i;
    const int k = kb * B_ROWS_PER_KB + lane / B_CHUNKS;
    b_off[i] = k * args.ldb + ((lane % B_CHUNKS) ^ swz_b(k)) * 4;
  }
  const float* a_base = (const float*)args.A + (size_t)m0 * args.lda + k_begin;
  const float* b_base = (const float*)args.B + (size_t)k_begin * args.ldb + n0;
  const size_t b_step = (size_t)BK * args.ldb;

  auto issue_slab = [&](int kt, unsigned char* st) {
    const float* ab = a_base + (size_t)kt * BK;
    const float* bb = b_base + (size_t)kt * b_step;
#pragma unroll
    for (int i = 0; i < A_KB; ++i) lds_dma16((const void*)(ab + a_off[i]), st + (wave * A_KB + i) * 1024);
#pragma unroll
    for (int i = 0; i < B_KB; ++i) lds_dma16((const void*)(bb + b_off[i]), st + A_STAGE + (wave * B_KB + i) * 1024);
  };

  // ---- fragment coordinates
  const int l16 = lane & 15;
  const int g = lane >> 4;
  const int a_row0 = wm * (16 * TM) + l16;  // + 16 i
  const int a_sw = swz_a<BK>(a_row0);  // unchanged by + 16 i
  const int b_col0 = wn * (16 * TN) + l16;  // + 16 j

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int s = 0; s < D; ++s)
    if (s < nk) issue_slab(s, stage(s));
  // slab 0 landed (up to D-1 later slabs still in flight), then visible
  if (nk >= D)
    __builtin_amdgcn_s_waitcnt(waitcnt_vm((D - 1) * DMA_PER_SLAB));
  else
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  slab_barrier();

  auto step = [&](int t, const int s) {
    if (t + D < nk) issue_slab(t + D, stage((s + D) % STAGES));
    const unsigned char* sa = stage(s);
    const unsigned char* sb = sa + A_STAGE;
    // the slab's fragments, then its MFMAs
    f32x4 af[KC][TM];
    float bf[KC][4][TN];
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[kc][i] = *(const lds_f32x4*)(sa + (a_row0 + 16 * i) * (BK * 4) + 16 * ((kc * 4 + g) ^ a_sw));
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int k = kc * 16 + 4 * g + q;
        const int sw = swz_b(k);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int col = b_col0 + 16 * j;
          bf[kc][q][j] = *(const lds_f32*)(sb + k * (BN * 4) + 16 * ((col >> 2) ^ sw) + 4 * (col & 3));
        }
      }
    }
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(bf[kc][q][j], af[kc][i][q], acc[i][j], 0, 0, 0);
    // this wave's DMA of slab t+1 has landed (slabs through min(t+D, nk-1) issued)
    if (t + D < nk)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm((D - 1) * DMA_PER_SLAB));
    else
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    if (t + 1 < nk) slab_barrier();
  };
  // slab t lives in stage t % STAGES; the unrolled body fixes it at compile time
  for (int t = 0; t < nk; t += STAGES) {
#pragma unroll
    for (int s = 0; s < STAGES; ++s)
      if (t + s < nk) step(t + s, s);
  }

  // ---- epilogue: lane holds C[m][n .. n+3], m = m0 + 16 TM wm + 16 i + l16,
  // n = n0 + 16 TN wn + 16 j + 4 g
  const int ncol = n0 + wn * (16 * TN) + 4 * g;
  if (args.partial == nullptr) {
    f32x4 bv[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j)
      bv[j] = args.bias ? *(const f32x4*)(args.bias + ncol + 16 * j) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      float* row = args.C + (size_t)(m0 + wm * (16 * TM) + 16 * i + l16) * args.ldc;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        f32x4 v = acc[i][j] + bv[j];
        if (args.relu) {
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = v[r] < args.relu_threshold ? args.relu_threshold : v[r];
        }
        *(f32x4*)(row + ncol + 16 * j) = v;
      }
    }
    return;
  }
  float* plane = args.partial + (size_t)split * args.M * args.N;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    float* row = plane + (size_t)(m0 + wm * (16 * TM) + 16 * i + l16) * args.N;
#pragma unroll
    for (int j = 0; j < TN; ++j) splitk_store4(row + ncol + 16 * j, acc[i][j]);
  }
  if (splitk_arrive(args.counters + tile_m * args.tiles_n + tile_n, (int)gridDim.z)) {
    splitk_finish_tile<BM, BN, 512>(args.partial, args.C, args.bias, args.M, args.N, args.ldc, (int)gridDim.z,
                                    args.relu, args.relu_threshold, m0, n0);
    splitk_release(args.counters + tile_m * args.tiles_n + tile_n);
  }
}

}  // namespace xtc_hip
