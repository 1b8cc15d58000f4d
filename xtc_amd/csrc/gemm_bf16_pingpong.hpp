// SPDX-License-Identifier: BSD-3-Clause
// bf16 GEMM for aligned large shapes on gfx950, "ping-pong" schedule:
//   C[M,N] (fp32) = epilogue( A[M,K] (bf16, row-major) @ B[K,N] (bf16) )
// with M % 256 == 0, N % 256 == 0, K % 32 == 0 and 16-byte aligned rows; B
// row-major (BT = false) or stored transposed (BT = true), as in
// gemm_bf16_lds.hpp, whose LDS layouts, swizzles, fragment reads, MFMA
// tiling, tile raster and K-stagger this kernel shares.
//
// Why a second schedule.  In the 8-wave kernel of gemm_bf16_lds.hpp all
// waves run the same program: after each barrier every wave issues its DMA
// and fragment reads at once and then its MFMAs, so on every SIMD both waves
// compete for LDS in one phase and leave the matrix core idle, then both
// queue MFMAs in the next (MFMA busy measured at 59 %).  Here the 8 waves
// form two groups of 4 (waves 0-3 and 4-7: one of each on every SIMD) that
// run half a step apart:
//   * a step is one 32-deep k-slab: a memory phase (issue the DMA of slab
//     t+D, read the wave's 8 A and 4 B fragments of slab t from LDS, wait for
//     them) and a compute phase (the wave's 32 v_mfma_f32_16x16x32_bf16);
//   * group 1 passes one extra barrier at the start, so every barrier
//     separates "group 0 computes, group 1 reads" from "group 0 reads, group 1
//     computes": each SIMD's matrix core is fed by one wave while the other
//     wave of the SIMD feeds LDS;
//   * both groups pass the same number of barriers: 1 + 2 per slab, group 1
//     skipping the one after its last compute phase that group 0 does not
//     have to wait for (it stores C meanwhile).
// LDS holds STAGES stages of one slab (A 256 x 64 B, B 32 x 512 B or B^T
// 256 x 64 B: 32 KB), and the DMA runs D = STAGES - 1 slabs ahead.
//   * Slab t must have landed before group 0 reads it: every wave waits for
//     its own DMA of slab t+1 (s_waitcnt vmcnt) right before the barrier that
//     opens group 0's memory phase t+1 (group 0 after its compute phase t,
//     group 1 after its memory phase t).  The DMA is issued from asm (no
//     compiler wait-count tracking), so these waits are the only ones.
//   * The DMA of slab t+D goes into the stage of slab t-1, which both groups
//     finished reading (lgkmcnt(0) at the end of every memory phase) before
//     the barrier that precedes the DMA.
// Fragment registers are single-buffered (one slab's 12 fragments): a wave
// reads them only in its memory phase and uses them only in its compute
// phase.  Accumulation order per output element is the K walk, as in
// gemm_bf16_lds.hpp: results are bit-identical to it on exactly summable
// inputs.
//
// Split-K: blockIdx.z picks a range of k_per_split (whole slabs, equal for
// every split) and the walk above runs over it.  With more than one split
// the epilogue stores the fp32 accumulators into the split's partial plane,
// and the last workgroup to arrive at the tile's counter sums the planes in
// split order into C with bias and relu (splitk.hpp), then resets the
// counter for the next launch.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemm_bf16_lds.hpp"
#include "lds_dma.hpp"
#include "splitk.hpp"

namespace xtc_hip {

namespace pingpong {

// s_waitcnt immediate (gfx9 encoding) that waits for lgkmcnt == 0 only.
constexpr int waitcnt_lgkm0() { return 15 | (7 << 4) | (0 << 8) | (3 << 14); }

// A workgroup barrier with no memory fence: the waits around it are
// explicit.  The empty asm statements keep memory accesses from moving
// across it, the scheduling barriers keep every instruction on its side.
__device__ __forceinline__ void phase_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
}

}  // namespace pingpong

template <bool BT, int STAGES>
__global__ void __attribute__((amdgpu_flat_work_group_size(512, 512))) gemm_bf16_pingpong(BigGemmArgs args) {
  using namespace big;
  using namespace pingpong;
  constexpr int BK = 32, WGN = 4, TM = 8, TN = 4, WAVES = 8;
  constexpr int A_STAGE = BM * BK * 2;
  constexpr int B_STAGE = BK * BN * 2;
  constexpr int STAGE = A_STAGE + B_STAGE;
  constexpr int KB_PER_WAVE = (A_STAGE / 1024) / WAVES;  // DMA kilobytes per operand per wave
  constexpr int DMA_PER_SLAB = 2 * KB_PER_WAVE;           // DMA instructions per wave per slab
  constexpr int A_ROWS_PER_KB = 1024 / (2 * BK);
  constexpr int A_CHUNKS = (2 * BK) / 16;
  constexpr int D = STAGES - 1;
  static_assert(STAGES >= 3 && STAGES <= 5 && STAGES * STAGE <= 160 * 1024, "LDS");
  static_assert(KB_PER_WAVE * WAVES * 1024 == A_STAGE, "stage must split evenly over waves");
  static_assert(D * DMA_PER_SLAB < 64, "vmcnt range");

  __shared__ __attribute__((aligned(1024))) unsigned char st0[STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char st1[STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char st2[STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char st3[STAGES > 3 ? STAGE : 16];
  __shared__ __attribute__((aligned(1024))) unsigned char st4[STAGES > 4 ? STAGE : 16];
  auto stage = [&](int s) -> unsigned char* {
    return s == 0 ? st0 : s == 1 ? st1 : s == 2 ? st2 : s == 3 ? st3 : st4;
  };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave-uniform by construction; readfirstlane lets the compiler see it, so
  // the group-dependent barriers below sit behind scalar branches
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN;
  const int wn = wave % WGN;
  const int group = wm;

  int tile_m, tile_n;
  tile_of_block(args, tile_m, tile_n);
  const int m0 = tile_m * BM;
  const int n0 = tile_n * BN;

  // ---- LDS DMA sources, as in gemm_bf16_lds.hpp with BK = 32
  int a_off[KB_PER_WAVE];
  int b_off[KB_PER_WAVE];
#pragma unroll
  for (int i = 0; i < KB_PER_WAVE; ++i) {
    const int kb = wave * KB_PER_WAVE + i;
    const int arow = kb * A_ROWS_PER_KB + lane / A_CHUNKS;
    a_off[i] = arow * args.lda + ((lane % A_CHUNKS) ^ swz_a<BK>(arow)) * 8;
    if constexpr (BT) {
      b_off[i] = arow * args.ldb + ((lane % A_CHUNKS) ^ swz_a<BK>(arow)) * 8;
    } else {
      const int bk = kb * 2 + (lane >> 5);  // 2 k-rows of 512 B per KB
      const int slot = lane & 31;
      b_off[i] = bk * args.ldb + ((slot >> 1) ^ swz_b(bk)) * 16 + (slot & 1) * 8;
    }
  }
  const int split = blockIdx.z;
  const int k_begin = split * args.k_per_split;
  const __bf16* a_base = args.A + (size_t)m0 * args.lda + k_begin;
  const __bf16* b_base = BT ? args.B + (size_t)n0 * args.ldb + k_begin : args.B + (size_t)k_begin * args.ldb + n0;
  const size_t b_step = BT ? (size_t)BK : (size_t)BK * args.ldb;
  const int nk = min(args.K - k_begin, args.k_per_split) / BK;
  // K-stagger: tile (tm, tn) starts its K walk at slab (tm + 2 tn) mod 16
  int kofs = (tile_m + 2 * tile_n) & 15;
  kofs = nk > 0 ? kofs % nk : 0;

  auto issue_slab = [&](int kt, unsigned char* st) {
    int kr = kt + kofs;
    kr = kr >= nk ? kr - nk : kr;
    const __bf16* ab = a_base + (size_t)kr * BK;
    const __bf16* bb = b_base + (size_t)kr * b_step;
#pragma unroll
    for (int i = 0; i < KB_PER_WAVE; ++i) lds_dma16((const void*)(ab + a_off[i]), st + (wave * KB_PER_WAVE + i) * 1024);
#pragma unroll
    for (int i = 0; i < KB_PER_WAVE; ++i)
      lds_dma16((const void*)(bb + b_off[i]), st + A_STAGE + (wave * KB_PER_WAVE + i) * 1024);
  };

  // ---- per-lane fragment read coordinates
  const int l16 = lane & 15;
  const int g = lane >> 4;
  const int a_row0 = wm * (16 * TM) + l16;
  const int a_h = swz_a<BK>(a_row0);
  const int b_krow0 = BT ? wn * (16 * TN) + l16 : 8 * g + (l16 >> 2);
  const int b_f = BT ? swz_a<BK>(b_krow0) : swz_b(b_krow0);
  const int b_c0 = wn * TN;

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
  phase_barrier();
  if (group == 1) phase_barrier();

  // this wave's DMA of slab t+1 has landed (slabs through min(t+D, nk-1) issued)
  auto wait_next = [&](int t) {
    if (t + D < nk)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm((D - 1) * DMA_PER_SLAB));
    else
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  };

  Frags<TM, TN> f;
  auto step = [&](int t, const int s) {
    // ---- memory phase
    if (t + D < nk) issue_slab(t + D, stage((s + D) % STAGES));
    const unsigned char* sa = stage(s);
    read_frags<BK, BT>(f, sa, sa + A_STAGE, 0, a_row0, a_h, g, b_krow0, b_f, b_c0, l16);
    __builtin_amdgcn_s_waitcnt(waitcnt_lgkm0());
    if (group == 1) wait_next(t);
    phase_barrier();
    // ---- compute phase
    mma(acc, f);
    if (group == 0) wait_next(t);
    if (group == 0 || t + 1 < nk) phase_barrier();
  };
  // slab t lives in stage t % STAGES; the unrolled body fixes it at compile time
  for (int t = 0; t < nk; t += STAGES) {
#pragma unroll
    for (int s = 0; s < STAGES; ++s)
      if (t + s < nk) step(t + s, s);
  }

  // ---- epilogue: lane holds C[m][n .. n+3] for each (it, jt); rows in order
  const int mrow = m0 + wm * (16 * TM) + l16;
  const int ncol = n0 + wn * (16 * TN) + 4 * g;
  if (gridDim.z > 1) {
    float* plane = args.partial + (size_t)split * args.M * args.N;
#pragma unroll
    for (int it = 0; it < TM; ++it) {
#pragma unroll
      for (int jt = 0; jt < TN; ++jt) splitk_store4(plane + (size_t)(mrow + it * 16) * args.N + ncol + jt * 16, acc[it][jt]);
    }
    // the arrival flag takes the first word of stage 0: every wave's LDS
    // reads and DMAs are complete before the barrier that opens the arrival
    unsigned* counter = args.counters + tile_m * args.tiles_n + tile_n;
    if (splitk_arrive_in(counter, (int)gridDim.z, reinterpret_cast<unsigned*>(st0))) {
      splitk_finish_tile<BM, BN, 512>(args.partial, args.C, args.bias, args.M, args.N, args.ldc, (int)gridDim.z,
                                      args.relu, args.relu_threshold, m0, n0);
      splitk_release(counter);
    }
    return;
  }
  f32x4 bv[TN];
#pragma unroll
  for (int jt = 0; jt < TN; ++jt)
    bv[jt] = args.bias ? *(const f32x4*)(args.bias + ncol + jt * 16) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int it = 0; it < TM; ++it) {
#pragma unroll
    for (int jt = 0; jt < TN; ++jt) {
      f32x4 v = acc[it][jt] + bv[jt];
      if (args.relu) {
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = v[r] < args.relu_threshold ? args.relu_threshold : v[r];
      }
      *(f32x4*)(args.C + (size_t)(mrow + it * 16) * args.ldc + ncol + jt * 16) = v;
    }
  }
}

}  // namespace xtc_hip
