// SPDX-License-Identifier: BSD-3-Clause
// bf16 GEMM for aligned large shapes on gfx950 (CDNA4):
//   C[M,N] (fp32) = epilogue( A[M,K] (bf16, row-major) @ B[K,N] (bf16) )
// with M % 256 == 0, N % 256 == 0, K % BK == 0 and 16-byte aligned rows.
// B is row-major [K][ldb] (BT = false) or stored transposed, [N][ldb] with
// k contiguous (BT = true: the tensor layout [1, 0]).
//
// Design (one 256x256 output tile per workgroup, WGM x WGN waves):
//   * K is walked in BK-deep slabs through STAGES LDS stages (distinct LDS
//     objects, so the compiler can tell the DMA into one stage from the reads
//     of another).  Global -> LDS moves use the gfx950 LDS DMA
//     (global_load_lds_dwordx4): no VGPR staging, no ds_write.  The DMA runs
//     STAGES-1 slabs ahead of the MFMAs; per slab one s_waitcnt vmcnt(N) for
//     exactly the slab about to be read, then one barrier.  Measured on
//     MI355X at 8192^3 (zero inputs, each part alone, the others removed):
//     MFMA 490 us, DMA 481 us even when every panel read hits L2, LDS
//     fragment reads 310 us; all together 735 us.  Serving every panel from
//     L2 saves only 4 %; BK = 32 with 3-5 stages, or a ring of five 32-deep
//     stages with one barrier per 64 k, was 4-10 % slower than BK = 64 with
//     2 stages.  The slab's LDS reads and MFMAs are ordered by hand (slab64).
//   * A stays row-major in LDS (256 rows x 2*BK bytes), read with
//     ds_read_b128.  The 16-byte chunk of row r is XOR-swizzled by r & 7 for
//     128-byte rows (BK=64) and by (r >> 1) & 3 for 64-byte rows (BK=32): the
//     best patterns measured for this access on MI355X (174 and 218 B/clk/CU;
//     contiguous b128 reads give 191).
//   * BT: B's stage has A's shape (256 n-rows x 2*BK bytes), is filled,
//     swizzled and read exactly like A (ds_read_b128), and B fragment jt of
//     a lane is the A-style fragment of n-row col0 + jt*16 + l16.
//   * !BT: B stays row-major in LDS (BK k-rows x 512 B) and is read transposed by
//     ds_read_b64_tr_b16: within a 16-lane group, output lane i element q is
//     element (i % 4) of the 8 bytes addressed by lane 4q + i/4, so lane j
//     addresses B[k0 + j/4][n0 + 4(j%4) .. +3] to receive B[k0 .. k0+3][n0+j].
//     Two such reads give the 8 k-values of an MFMA operand.  The 32-byte chunk
//     of k-row k is XOR-swizzled by (k & 3) | ((k >> 1) & 4): 101 B/clk/CU
//     measured (32 unswizzled, 94 with k & 3 alone).
//   * Each wave owns a (256/WGM) x (256/WGN) sub-tile of
//     v_mfma_f32_16x16x32_bf16 tiles.  The MFMA operands are swapped
//     (B-fragment first) so each lane ends up holding 4 consecutive columns of
//     one C row: the epilogue (bias, relu) stores float4s, row by row.
//   * Workgroups are remapped so each XCD owns a contiguous range of tiles,
//     rastered in groups of `group_m` tile rows for L2 reuse, and each tile
//     starts its K walk at a tile-dependent slab (see kofs) so tiles sharing a
//     panel are not in lockstep.  The rotation changes only the order of the
//     fp32 accumulation.
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
  // split-K (gemm_bf16_pingpong only): split blockIdx.z covers K range
  // [z * k_per_split, (z + 1) * k_per_split); with more than one split the
  // workgroups store fp32 partial sums in partial[splits][M][N] and the last
  // to arrive at its tile's counter sums them into C (splitk.hpp)
  int k_per_split;
  float* partial;
  unsigned* counters;
};

namespace big {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 256, BN = 256;

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;

template <int BK>
__device__ __forceinline__ int swz_a(int row) {
  return BK == 64 ? (row & 7) : ((row >> 1) & 3);
}
__device__ __forceinline__ int swz_b(int k) { return (k & 3) | ((k >> 1) & 4); }

// s_waitcnt immediate (gfx9 encoding) that waits for vmcnt <= n only.
constexpr int waitcnt_vm(int n) { return (n & 15) | (7 << 4) | (15 << 8) | (((n >> 4) & 3) << 14); }

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

// Fragments of one 32-deep k-step for a wave's (16*TM) x (16*TN) sub-tile.
template <int TM, int TN>
struct Frags {
  bf16x8 a[TM];
  bf16x8 b[TN];
};

// Reads k-step `ks` of a stage (A at `sa`, B at `sb`).
//   A fragment `it`: lane (l16, g) gets A[row0 + it*16 + l16][ks*32 + 8g .. +7]
//   B fragment `jt`: lane (l16, g) gets B[ks*32 + 8g .. +7][col0 + jt*16 + l16]
// With BT the B coordinates are those of an A-style operand: b_krow0 is the
// lane's first n-row (wn*16*TN + l16) and b_f its chunk swizzle; b_c0 unused.
template <int BK, bool BT, int TM, int TN>
__device__ __forceinline__ void read_frags(Frags<TM, TN>& f, const unsigned char* sa, const unsigned char* sb, int ks,
                                           int a_row0, int a_h, int g, int b_krow0, int b_f, int b_c0, int l16) {
#pragma unroll
  for (int it = 0; it < TM; ++it) {
    const int off = (a_row0 + it * 16) * (2 * BK) + 16 * ((ks * 4 + g) ^ a_h);
    f.a[it] = __builtin_bit_cast(bf16x8, *(const lds_u32x4*)(sa + off));
  }
#pragma unroll
  for (int jt = 0; jt < TN; ++jt) {
    if constexpr (BT) {
      const int off = (b_krow0 + jt * 16) * (2 * BK) + 16 * ((ks * 4 + g) ^ b_f);
      f.b[jt] = __builtin_bit_cast(bf16x8, *(const lds_u32x4*)(sb + off));
    } else {
      const int c32 = (b_c0 + jt) ^ b_f;
      const int off0 = (ks * 32 + b_krow0) * 512 + c32 * 32 + 8 * (l16 & 3);
      i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(sb + off0));
      i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(sb + off0 + 4 * 512));
      f.b[jt] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
  }
}

// One A fragment (one ds_read_b128) / one B fragment (two ds_read_b64_tr_b16,
// or one ds_read_b128 with BT)
// of k-step ks, with the same addressing as read_frags.
template <int BK, int TM, int TN>
__device__ __forceinline__ void read_a1(Frags<TM, TN>& f, const unsigned char* sa, int ks, int it, int a_row0, int a_h,
                                        int g) {
  const int off = (a_row0 + it * 16) * (2 * BK) + 16 * ((ks * 4 + g) ^ a_h);
  f.a[it] = __builtin_bit_cast(bf16x8, *(const lds_u32x4*)(sa + off));
}
template <int BK, bool BT, int TM, int TN>
__device__ __forceinline__ void read_b1(Frags<TM, TN>& f, const unsigned char* sb, int ks, int jt, int b_krow0, int b_f,
                                        int b_c0, int l16, int g) {
  if constexpr (BT) {
    const int off = (b_krow0 + jt * 16) * (2 * BK) + 16 * ((ks * 4 + g) ^ b_f);
    f.b[jt] = __builtin_bit_cast(bf16x8, *(const lds_u32x4*)(sb + off));
  } else {
    const int c32 = (b_c0 + jt) ^ b_f;
    const int off0 = (ks * 32 + b_krow0) * 512 + c32 * 32 + 8 * (l16 & 3);
    i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(sb + off0));
    i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(sb + off0 + 4 * 512));
    f.b[jt] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  }
}

// The two k-steps of a 64-deep slab in a fixed order (sched_barrier fences
// keep it): the A fragments and the first LA B fragments of k-step 0; then,
// per output column jt, the B fragment jt+LA of k-step 0 and a share of
// k-step 1's fragments followed by the column's TM MFMAs; then all MFMAs of
// k-step 1, whose operands were read during k-step 0.  Every accumulator
// sees k-step 0 before k-step 1, as in the plain loop, so results are
// bit-identical to it.  Left to itself the scheduler issues all 40 reads
// first and waits for every one of them before the first MFMA (an LDS DMA
// in flight makes the compiler's LDS waits all-or-nothing).
template <int BK, bool BT, int TM, int TN>
__device__ __forceinline__ void slab64(f32x4 (&acc)[TM][TN], const unsigned char* sa, const unsigned char* sb,
                                       int a_row0, int a_h, int g, int b_krow0, int b_f, int b_c0, int l16) {
  constexpr int LA = 2;
  constexpr int NF1 = TM + TN;  // k-step 1 fragments
  Frags<TM, TN> f0, f1;
#pragma unroll
  for (int it = 0; it < TM; ++it) read_a1<BK>(f0, sa, 0, it, a_row0, a_h, g);
#pragma unroll
  for (int jt = 0; jt < LA && jt < TN; ++jt) read_b1<BK, BT>(f0, sb, 0, jt, b_krow0, b_f, b_c0, l16, g);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int jt = 0; jt < TN; ++jt) {
    if (jt + LA < TN) read_b1<BK, BT>(f0, sb, 0, jt + LA, b_krow0, b_f, b_c0, l16, g);
#pragma unroll
    for (int q = jt * NF1 / TN; q < (jt + 1) * NF1 / TN; ++q) {
      if (q < TM) read_a1<BK>(f1, sa, 1, q, a_row0, a_h, g);
      else read_b1<BK, BT>(f1, sb, 1, q - TM, b_krow0, b_f, b_c0, l16, g);
    }
#pragma unroll
    for (int it = 0; it < TM; ++it)
      acc[it][jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f0.b[jt], f0.a[it], acc[it][jt], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int jt = 0; jt < TN; ++jt)
#pragma unroll
    for (int it = 0; it < TM; ++it)
      acc[it][jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f1.b[jt], f1.a[it], acc[it][jt], 0, 0, 0);
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
template <int WGM, int WGN, int BK, int STAGES, bool BT = false>
__global__ void __attribute__((amdgpu_flat_work_group_size(WGM * WGN * 64, WGM * WGN * 64)))
gemm_bf16_256x256(BigGemmArgs args) {
  using namespace big;
  constexpr int WAVES = WGM * WGN;
  constexpr int TM = BM / WGM / 16;
  constexpr int TN = BN / WGN / 16;
  constexpr int A_STAGE = BM * BK * 2;
  constexpr int B_STAGE = BK * BN * 2;
  constexpr int STAGE = A_STAGE + B_STAGE;
  constexpr int KB_PER_WAVE = (A_STAGE / 1024) / WAVES;  // DMA kilobytes per operand per wave
  constexpr int DMA_PER_SLAB = 2 * KB_PER_WAVE;           // DMA instructions per wave per slab
  constexpr int A_ROWS_PER_KB = 1024 / (2 * BK);
  constexpr int A_CHUNKS = (2 * BK) / 16;
  static_assert(BK == 32 || BK == 64, "BK");
  static_assert(STAGES >= 2 && STAGES <= 5 && STAGES * STAGE <= 160 * 1024, "LDS");
  static_assert(KB_PER_WAVE * WAVES * 1024 == A_STAGE, "stage must split evenly over waves");
  static_assert((STAGES - 2) * DMA_PER_SLAB < 64, "vmcnt range");

  __shared__ __attribute__((aligned(1024))) unsigned char st0[STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char st1[STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char st2[STAGES > 2 ? STAGE : 16];
  __shared__ __attribute__((aligned(1024))) unsigned char st3[STAGES > 3 ? STAGE : 16];
  __shared__ __attribute__((aligned(1024))) unsigned char st4[STAGES > 4 ? STAGE : 16];
  unsigned char* const stages[5] = {st0, st1, st2, st3, st4};

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
    const int arow = kb * A_ROWS_PER_KB + lane / A_CHUNKS;
    a_off[i] = arow * args.lda + ((lane % A_CHUNKS) ^ swz_a<BK>(arow)) * 8;
    if constexpr (BT) {  // B^T rows like A rows
      b_off[i] = arow * args.ldb + ((lane % A_CHUNKS) ^ swz_a<BK>(arow)) * 8;
    } else {
      const int bk = kb * 2 + (lane >> 5);  // B: 2 k-rows of 512 B per KB
      const int slot = lane & 31;
      b_off[i] = bk * args.ldb + ((slot >> 1) ^ swz_b(bk)) * 16 + (slot & 1) * 8;
    }
  }
  const __bf16* a_base = args.A + (size_t)m0 * args.lda;
  const __bf16* b_base = BT ? args.B + (size_t)n0 * args.ldb : args.B + n0;
  const size_t b_step = BT ? (size_t)BK : (size_t)BK * args.ldb;
  const int nk = args.K / BK;
  // K-stagger: tile (tm, tn) walks K starting at slab (tm + 2 tn) mod 16, so
  // the tiles sharing an A panel (same tm) or a B panel (same tn) do not
  // request the same lines at the same time: one leads and takes the L2
  // miss, the others trail and hit.  In lockstep, nearly every L2 access
  // waited on a miss in flight (measured: 830 -> 787 us at 8192^3).
  int kofs = (tile_m + 2 * tile_n) & 15;
  kofs = nk > 0 ? kofs % nk : 0;

  auto issue_slab = [&](int kt, unsigned char* st) {
    int kr = kt + kofs;
    kr = kr >= nk ? kr - nk : kr;
    const __bf16* ab = a_base + (size_t)kr * BK;
    const __bf16* bb = b_base + (size_t)kr * b_step;
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
  const int a_h = swz_a<BK>(a_row0);    // depends on l16 only
  // !BT: first k-row of the lane's transposed reads and its chunk swizzle
  // (unchanged by ks*32 and the +4 half).  BT: first n-row and its swizzle.
  const int b_krow0 = BT ? wn * (16 * TN) + l16 : 8 * g + (l16 >> 2);
  const int b_f = BT ? swz_a<BK>(b_krow0) : swz_b(b_krow0);
  const int b_c0 = wn * TN;             // !BT: first 32-byte chunk of the wave's columns

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < nk) issue_slab(s, stages[s]);

  // slab kt lives in stage kt % STAGES; the unrolled body fixes it at compile time
  auto step = [&](int kt, const int s) {
    if (kt + STAGES - 2 < nk)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm((STAGES - 2) * DMA_PER_SLAB));  // slab kt landed
    else
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __syncthreads();  // slab kt visible to all waves; stage of slab kt-1 free
    if (kt + STAGES - 1 < nk) issue_slab(kt + STAGES - 1, stages[(s + STAGES - 1) % STAGES]);
    const unsigned char* sa = stages[s];
    if constexpr (BK == 64) {
      slab64<BK, BT>(acc, sa, sa + A_STAGE, a_row0, a_h, g, b_krow0, b_f, b_c0, l16);
    } else {
#pragma unroll
      for (int ks = 0; ks < BK / 32; ++ks) {
        Frags<TM, TN> f;
        read_frags<BK, BT>(f, sa, sa + A_STAGE, ks, a_row0, a_h, g, b_krow0, b_f, b_c0, l16);
        mma(acc, f);
      }
    }
  };
  for (int kt = 0; kt < nk; kt += STAGES) {
#pragma unroll
    for (int s = 0; s < STAGES; ++s)
      if (kt + s < nk) step(kt + s, s);
  }

  // ---- epilogue: lane holds C[m][n .. n+3] for each (it, jt); rows in order
  const int mrow = m0 + wm * (16 * TM) + l16;
  const int ncol = n0 + wn * (16 * TN) + 4 * g;
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
