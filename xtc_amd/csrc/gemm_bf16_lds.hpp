// SPDX-License-Identifier: BSD-3-Clause
// bf16 GEMM for aligned large shapes on gfx950 (CDNA4):
//   C[M,N] (fp32) = epilogue( A[M,K] (bf16, row-major) @ B[K,N] (bf16, row-major) )
// with M % 256 == 0, N % 256 == 0, K % 64 == 0 and 16-byte aligned rows.
//
// Design (one 256x256 output tile per workgroup, 4 waves, one wave per SIMD):
//   * K is walked in 64-deep slabs through two LDS stages of 64 KB each.
//     Global -> LDS moves use the gfx950 LDS DMA (global_load_lds_dwordx4):
//     no VGPR staging, no ds_write; slab k+1 streams in while slab k is
//     multiplied; one s_waitcnt vmcnt(0) + barrier per slab.
//   * A stays row-major in LDS (256 rows x 128 B).  Fragments are read with
//     ds_read_b128; the 16-byte chunk of row r is XOR-swizzled by
//     h(r) = (r & 7) ^ ((r >> 3) & 1), which makes the 16 rows a fragment read
//     touches hit distinct banks for 32- and 64-bank LDS alike.
//   * B stays row-major in LDS (64 k-rows x 512 B) and is read transposed by
//     ds_read_b64_tr_b16: within a 16-lane group, output lane i element q is
//     element (i % 4) of the 8 bytes addressed by lane 4q + i/4, so lane j
//     addresses B[k0 + j/4][n0 + 4(j%4) .. +3] to receive B[k0 .. k0+3][n0+j].
//     Two such reads give the 8 k-values of an MFMA operand.  The 32-byte chunk
//     of k-row k is XOR-swizzled by (k & 3) | ((k >> 1) & 4) for the same
//     bank-conflict reason.
//   * Each wave owns a 128x128 sub-tile: 8x8 v_mfma_f32_16x16x32_bf16 tiles,
//     256 fp32 accumulators per lane.  The MFMA operands are swapped
//     (B-fragment first) so each lane ends up holding 4 consecutive columns of
//     one C row: the epilogue (bias, relu) stores float4s.
//   * Workgroups are remapped so each XCD owns a contiguous range of tiles,
//     rastered in groups of `group_m` tile rows for L2 reuse.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace xtc_hip {

struct BigGemmArgs {
  const __bf16* A;
  const __bf16* B;
  float* C;
  const float* bias;  // [N] or null
  int M, N, K;
  int lda, ldb, ldc;  // elements
  int relu;
  float relu_threshold;
  int tiles_m, tiles_n;
  int group_m;
  int xcd_remap;
};

namespace big {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int NT = 256;                       // 4 waves
constexpr int A_STAGE = BM * BK * 2;          // 32 KB
constexpr int B_STAGE = BK * BN * 2;          // 32 KB
constexpr int STAGE = A_STAGE + B_STAGE;      // 64 KB

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;

__device__ __forceinline__ int swz_a(int row) { return (row & 7) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int swz_b(int k) { return (k & 3) | ((k >> 1) & 4); }

__device__ __forceinline__ void tile_of_block(const BigGemmArgs& a, int& tm, int& tn) {
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

}  // namespace big

namespace big {

// Fragments of one 32-deep k-step for a wave's (16*TM) x (16*TN) sub-tile.
template <int TM, int TN>
struct Frags {
  bf16x8 a[TM];
  bf16x8 b[TN];
};

// Reads k-step `ks` of a stage (A at `sa`, B at `sa + A_STAGE`).
//   A fragment `it`: lane (l16, g) gets A[row0 + it*16 + l16][ks*32 + 8g .. +7]
//   B fragment `jt`: lane (l16, g) gets B[ks*32 + 8g .. +7][col0 + jt*16 + l16]
template <int TM, int TN>
__device__ __forceinline__ void read_frags(Frags<TM, TN>& f, const unsigned char* sa, int ks, int a_row0, int a_h,
                                           int g, int b_krow0, int b_f, int b_c0, int l16) {
  const unsigned char* sb = sa + A_STAGE;
#pragma unroll
  for (int it = 0; it < TM; ++it) {
    const int off = (a_row0 + it * 16) * 128 + 16 * ((ks * 4 + g) ^ a_h);
    f.a[it] = __builtin_bit_cast(bf16x8, *(const lds_u32x4*)(sa + off));
  }
#pragma unroll
  for (int jt = 0; jt < TN; ++jt) {
    const int c32 = (b_c0 + jt) ^ b_f;
    const int off0 = (ks * 32 + b_krow0) * 512 + c32 * 32 + 8 * (l16 & 3);
    i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(sb + off0));
    i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(sb + off0 + 4 * 512));
    f.b[jt] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  }
}

template <int TM, int TN>
__device__ __forceinline__ void mma(f32x4 (&acc)[TM][TN], const Frags<TM, TN>& f) {
#pragma unroll
  for (int it = 0; it < TM; ++it)
#pragma unroll
    for (int jt = 0; jt < TN; ++jt)
      acc[it][jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.b[jt], f.a[it], acc[it][jt], 0, 0, 0);
}

}  // namespace big

// WGM x WGN waves; each wave owns a (256/WGM) x (256/WGN) sub-tile.
template <int WGM, int WGN>
__global__ void __attribute__((amdgpu_flat_work_group_size(WGM * WGN * 64, WGM * WGN * 64)))
gemm_bf16_256x256x64(BigGemmArgs args) {
  using namespace big;
  constexpr int WAVES = WGM * WGN;
  constexpr int TM = BM / WGM / 16;
  constexpr int TN = BN / WGN / 16;
  constexpr int KB_PER_WAVE = (A_STAGE / 1024) / WAVES;  // DMA kilobytes per operand per wave
  static_assert(KB_PER_WAVE * WAVES * 1024 == A_STAGE, "stage must split evenly over waves");
  // Two distinct LDS objects, one per stage, so the compiler can tell the
  // DMA into one stage from the fragment reads of the other.
  __shared__ __attribute__((aligned(1024))) unsigned char stage0[STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char stage1[STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WGN;
  const int wn = wave % WGN;

  int tile_m, tile_n;
  tile_of_block(args, tile_m, tile_n);
  const int m0 = tile_m * BM;
  const int n0 = tile_n * BN;

  // ---- LDS DMA sources: wave `wave` fills KB_PER_WAVE kilobytes of each
  // operand's stage, one instruction per kilobyte (lane l -> 16-byte slot l).
  int a_off[KB_PER_WAVE];
  int b_off[KB_PER_WAVE];
#pragma unroll
  for (int i = 0; i < KB_PER_WAVE; ++i) {
    const int kb = wave * KB_PER_WAVE + i;
    const int arow = kb * 8 + (lane >> 3);  // A: 8 rows of 128 B per KB
    a_off[i] = arow * args.lda + ((lane & 7) ^ swz_a(arow)) * 8;
    const int bk = kb * 2 + (lane >> 5);  // B: 2 k-rows of 512 B per KB
    const int slot = lane & 31;
    b_off[i] = bk * args.ldb + ((slot >> 1) ^ swz_b(bk)) * 16 + (slot & 1) * 8;
  }
  const __bf16* a_base = args.A + (size_t)m0 * args.lda;
  const __bf16* b_base = args.B + n0;
  const size_t b_step = (size_t)BK * args.ldb;

  auto issue_slab = [&](int kt, unsigned char* st) {
    const __bf16* ab = a_base + (size_t)kt * BK;
    const __bf16* bb = b_base + (size_t)kt * b_step;
#pragma unroll
    for (int i = 0; i < KB_PER_WAVE; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(ab + a_off[i]),
                                       (lds_void*)(st + (wave * KB_PER_WAVE + i) * 1024), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < KB_PER_WAVE; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(bb + b_off[i]),
                                       (lds_void*)(st + A_STAGE + (wave * KB_PER_WAVE + i) * 1024), 16, 0, 0);
  };

  // ---- per-lane fragment read coordinates
  const int l16 = lane & 15;
  const int g = lane >> 4;
  const int a_row0 = wm * (16 * TM) + l16;
  const int a_h = swz_a(a_row0);        // depends on l16 only
  const int b_krow0 = 8 * g + (l16 >> 2);
  const int b_f = swz_b(b_krow0);       // unchanged by ks*32 and the +4 half
  const int b_c0 = wn * TN;             // first 32-byte chunk of the wave's columns

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = args.K / BK;
  auto slab = [&](int kt, unsigned char* cur, unsigned char* nxt) {
    if (kt + 1 < nk) issue_slab(kt + 1, nxt);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      Frags<TM, TN> f;
      read_frags(f, cur, ks, a_row0, a_h, g, b_krow0, b_f, b_c0, l16);
      mma(acc, f);
    }
    __builtin_amdgcn_s_waitcnt(0);  // DMA of slab kt+1 landed
    __syncthreads();                // every wave is done with `cur`
  };

  issue_slab(0, stage0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int kt = 0; kt < nk; kt += 2) {
    slab(kt, stage0, stage1);
    if (kt + 1 < nk) slab(kt + 1, stage1, stage0);
  }

  // ---- epilogue: lane holds C[m][n .. n+3] for each (it, jt)
  const int mrow = m0 + wm * (16 * TM) + l16;
  const int ncol = n0 + wn * (16 * TN) + 4 * g;
#pragma unroll
  for (int jt = 0; jt < TN; ++jt) {
    const int n = ncol + jt * 16;
    f32x4 bv = {0.f, 0.f, 0.f, 0.f};
    if (args.bias) bv = *(const f32x4*)(args.bias + n);
#pragma unroll
    for (int it = 0; it < TM; ++it) {
      f32x4 v = acc[it][jt] + bv;
      if (args.relu) {
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = v[r] < args.relu_threshold ? args.relu_threshold : v[r];
      }
      *(f32x4*)(args.C + (size_t)(mrow + it * 16) * args.ldc + n) = v;
    }
  }
}

}  // namespace xtc_hip
