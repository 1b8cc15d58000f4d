// SPDX-License-Identifier: BSD-3-Clause
// MFMA GEMM / implicit-GEMM conv2d kernel family for gfx950 (CDNA4).
//
// One template covers every matmul-like node of an XTC graph:
//   C[M,N] = epilogue( sum_k A[M,K] * B[K,N] )
// with
//   * T = float  : v_mfma_f32_16x16x4_f32   (fp32 in, fp32 accumulate)
//   * T = bf16   : v_mfma_f32_16x16x32_bf16 (bf16 in, fp32 accumulate)
//   * CONV=true  : A is not a matrix but the implicit im2col view of an NHWC
//                  input; the pad node feeding the conv is folded into the
//                  A loader (out-of-bounds taps read `pad_value`).
// The reference semantics are linalg.fill(0)+linalg.matmul
// (src/xtc/backends/mlir/MlirOps.py:189-270) and the NHWC x RSCF conv
// (src/xtc/graphs/xtc/operators.py:252-347, MlirOps.py:349-404): beta = 0,
// C is fully overwritten.
//
// Structure (per workgroup = one BM x BN output tile):
//   * WGM x WGN waves, each owning a (BM/WGM) x (BN/WGN) wave tile built from
//     16x16 MFMA tiles, accumulators in registers (AGPR/VGPR).
//   * K is walked in BK slabs through two LDS buffers.  Global loads for slab
//     k+1 are issued into registers before the MFMAs of slab k and written to
//     the other LDS buffer afterwards: one barrier per slab.
//   * fp32: A stored row-major [BM][BK+4], B row-major [BK][BN+4].  The k
//     order inside a 16-wide chunk is permuted so that each lane reads A as
//     one 16-byte vector (lane group g handles k = 4g+s on MFMA step s).
//   * bf16: A stored row-major [BM][BK+8]; B is transposed on its way into LDS
//     (8x8 register transpose with v_perm) to Bt[BN][BK+8], so both operands
//     are read as one 16-byte vector per lane per MFMA.
//   * Padded rows make the fragment reads and tile writes bank-conflict free.
//   * Grid: 1-D over tiles, remapped so each XCD owns a contiguous range of
//     tiles, then grouped (GROUP_M tile rows) for L2 reuse; z = split-K.
//   * Epilogue: optional bias[N] and relu fused; split-K writes fp32 partial
//     sums to a workspace and the workgroup that stores a tile's last partial
//     sums them in split order and applies the epilogue (splitk.hpp).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "splitk.hpp"

namespace xtc_hip {

// register sets of global loads in flight in gemm_kernel (see its K loop):
// one by default; the registry adds ring-3 instances of a few small tiles
constexpr int kGemmRing = 1;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

struct GemmArgs {
  const void* A;      // [M][lda] (matrix) or NHWC input (conv)
  const void* B;      // [K][ldb]
  float* C;           // [M][ldc]
  const float* bias;  // [N] or null
  float* partial;     // split-K workspace [splits][M][N] or null
  unsigned* counters; // split-K arrival counters [tiles_m * tiles_n], zero between launches
  int M, N, K;
  int lda, ldb, ldc;
  int k_per_split;    // multiple of BK
  int relu;           // 1: out = max(out, relu_threshold) (numpy maximum, NaN kept)
  float relu_threshold;
  int tiles_m, tiles_n;
  int group_m;        // raster group height in tiles
  int xcd_remap;      // 1: remap block ids so each XCD gets contiguous tiles
  // implicit-GEMM conv view of A (CONV=true)
  int cH, cW, cC;     // input spatial dims / channels (unpadded)
  int cOH, cOW;       // output spatial dims
  int cS;             // kernel width (R is implied by K)
  int cSH, cSW;       // strides
  int cPH, cPW;       // top / left padding folded into the loader
  float pad_value;
};

template <typename T> struct Vec;  // 16-byte chunk of T
template <> struct Vec<float> { static constexpr int N = 4; };
template <> struct Vec<__bf16> { static constexpr int N = 8; };

__device__ __forceinline__ u32x4 ldg16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

__device__ __forceinline__ u32x4 splat16(float v, float) {
  unsigned u = __float_as_uint(v);
  return u32x4{u, u, u, u};
}
__device__ __forceinline__ u32x4 splat16(float v, __bf16) {
  // round-to-nearest-even fp32 -> bf16, replicated in both halves
  unsigned u = __float_as_uint(v);
  unsigned r = ((u >> 16) & 1u) + 0x7fffu;
  unsigned h = (u + r) >> 16;
  unsigned w = h | (h << 16);
  return u32x4{w, w, w, w};
}

// Maps the 1-D block id onto (tile_m, tile_n).
__device__ __forceinline__ void tile_coords(const GemmArgs& a, int& tm, int& tn) {
  int nb = a.tiles_m * a.tiles_n;
  int bid = blockIdx.x;
  if (a.xcd_remap && (nb & 7) == 0) {
    // Workgroups are dispatched round-robin over the 8 XCDs: give XCD x the
    // contiguous id range [x*nb/8, (x+1)*nb/8) so its L2 sees neighbours.
    bid = (bid & 7) * (nb >> 3) + (bid >> 3);
  }
  int gm = a.group_m;
  int per_group = gm * a.tiles_n;
  int group = bid / per_group;
  int first_m = group * gm;
  int gsize = min(a.tiles_m - first_m, gm);
  int in_group = bid - group * per_group;
  tm = first_m + in_group % gsize;
  tn = in_group / gsize;
}

template <typename T, int BM, int BN, int BK, int WGM, int WGN, bool CONV>
struct GemmTile {
  static constexpr int NT = WGM * WGN * 64;
  static constexpr int VEC = Vec<T>::N;
  static constexpr bool F32 = sizeof(T) == 4;
  static constexpr int WTM = BM / WGM;
  static constexpr int WTN = BN / WGN;
  static constexpr int TM = WTM / 16;
  static constexpr int TN = WTN / 16;
  static constexpr int APAD = VEC;  // one 16-byte chunk of padding per row
  static constexpr int AST = BK + APAD;             // A row stride (elements)
  static constexpr int BST = F32 ? (BN + 4) : (BK + 8);  // B row stride
  static constexpr int A_ELEMS = BM * AST;
  static constexpr int B_ELEMS = F32 ? BK * BST : BN * BST;
  static constexpr int STAGE_ELEMS = A_ELEMS + B_ELEMS;
  // A tile: BM rows x (BK/VEC) chunks
  static constexpr int A_CHUNKS_ROW = BK / VEC;
  static constexpr int A_CHUNKS = BM * A_CHUNKS_ROW;
  static constexpr int A_PER_T = (A_CHUNKS + NT - 1) / NT;
  static constexpr bool A_EVEN = A_CHUNKS % NT == 0;
  // B tile (fp32): BK rows x (BN/4) chunks ; (bf16): (BK/8) x (BN/8) 8x8 blocks
  static constexpr int B_CHUNKS_ROW = BN / VEC;
  static constexpr int B_UNITS = F32 ? BK * B_CHUNKS_ROW : (BK / 8) * (BN / 8);
  static constexpr int B_PER_T = (B_UNITS + NT - 1) / NT;
  static constexpr bool B_EVEN = B_UNITS % NT == 0;
  static constexpr int B_REGS = F32 ? B_PER_T : B_PER_T * 8;

  static_assert(BM % (16 * WGM) == 0 && BN % (16 * WGN) == 0, "wave tile");
  static_assert(BK % (F32 ? 16 : 32) == 0, "BK must cover whole MFMA k-steps");
  static_assert(A_CHUNKS % NT == 0 || A_CHUNKS < NT, "A tile must split evenly over threads");
  static_assert(B_UNITS % NT == 0 || B_UNITS < NT, "B tile must split evenly over threads");
};

template <typename T, int BM, int BN, int BK, int WGM, int WGN, bool CONV, int RING = kGemmRing>
__global__ void __attribute__((amdgpu_flat_work_group_size(WGM * WGN * 64, WGM * WGN * 64)))
__attribute__((amdgpu_waves_per_eu(1, 4)))
gemm_kernel(GemmArgs args) {
  static_assert(RING >= 1 && RING <= 4, "register ring depth");
  using P = GemmTile<T, BM, BN, BK, WGM, WGN, CONV>;
  constexpr int NT = P::NT;
  constexpr int VEC = P::VEC;
  constexpr bool F32 = P::F32;

  __shared__ __attribute__((aligned(16))) T smem[2 * P::STAGE_ELEMS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WGN;
  const int wn = wave % WGN;
  const int l16 = lane & 15;
  const int g = lane >> 4;

  int tile_m, tile_n;
  tile_coords(args, tile_m, tile_n);
  const int m0 = tile_m * BM;
  const int n0 = tile_n * BN;
  const int split = blockIdx.z;
  const int k_begin = split * args.k_per_split;
  const int k_end = min(args.K, k_begin + args.k_per_split);
  const int nk = (k_end - k_begin + BK - 1) / BK;

  const T* __restrict__ Ag = reinterpret_cast<const T*>(args.A);
  const T* __restrict__ Bg = reinterpret_cast<const T*>(args.B);
  const u32x4 padv = splat16(args.pad_value, T());

  // ---- per-thread A chunk coordinates (fixed over the K loop) ----
  int a_row[P::A_PER_T];
  int a_col[P::A_PER_T];
  // conv: per row base offsets / window origin
  int a_base[P::A_PER_T];
  int a_ih0[P::A_PER_T];
  int a_iw0[P::A_PER_T];
  bool a_rowok[P::A_PER_T];
#pragma unroll
  for (int i = 0; i < P::A_PER_T; ++i) {
    int c = tid + i * NT;
    const bool mine = P::A_EVEN || c < P::A_CHUNKS;
    if (!mine) c = 0;
    a_row[i] = c / P::A_CHUNKS_ROW;
    a_col[i] = (c % P::A_CHUNKS_ROW) * VEC;
    int m = m0 + a_row[i];
    a_rowok[i] = mine && m < args.M;
    if constexpr (CONV) {
      int mm = a_rowok[i] ? m : 0;
      int ow = mm % args.cOW;
      int t = mm / args.cOW;
      int oh = t % args.cOH;
      int b = t / args.cOH;
      a_ih0[i] = oh * args.cSH - args.cPH;
      a_iw0[i] = ow * args.cSW - args.cPW;
      a_base[i] = b * args.cH;
    } else {
      a_base[i] = m * args.lda;
      a_ih0[i] = 0;
      a_iw0[i] = 0;
    }
  }

  // RING register sets of global loads: slab t lives in set t % RING, and
  // RING slabs are in flight while one is computed from LDS
  u32x4 areg[RING][P::A_PER_T];
  u32x4 breg[RING][P::B_REGS];

  // conv: when the channel count is a multiple of BK, a slab [kt, kt+BK)
  // lies in one filter tap (r, s); its coordinates are computed once per
  // slab from the uniform kt instead of per 16-byte chunk.
  const bool tap_slabs = CONV && args.cC % BK == 0;
  auto load_a = [&](int kt, int slot) {
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
    for (int i = 0; i < P::A_PER_T; ++i) {
      int k = kt + a_col[i];
      bool ok = a_rowok[i] && k < k_end;
      if constexpr (CONV) {
        // k -> (r, s, c) in the RSCF weight order
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
        int ih = a_ih0[i] + r;
        int iw = a_iw0[i] + s;
        bool inb = ok && ih >= 0 && ih < args.cH && iw >= 0 && iw < args.cW;
        if (inb) {
          areg[slot][i] = ldg16(Ag + ((size_t)((a_base[i] + ih) * args.cW + iw) * args.cC + c));
        } else {
          areg[slot][i] = ok ? padv : u32x4{0, 0, 0, 0};
        }
      } else {
        areg[slot][i] = ok ? ldg16(Ag + (size_t)a_base[i] + k) : u32x4{0, 0, 0, 0};
      }
    }
  };

  auto load_b = [&](int kt, int slot) {
    if constexpr (F32) {
#pragma unroll
      for (int i = 0; i < P::B_PER_T; ++i) {
        int c = tid + i * NT;
        const bool mine = P::B_EVEN || c < P::B_UNITS;
        int kr = c / P::B_CHUNKS_ROW;
        int nc = (c % P::B_CHUNKS_ROW) * VEC;
        int k = kt + kr;
        int n = n0 + nc;
        bool ok = mine && k < k_end && n < args.N;
        breg[slot][i] = ok ? ldg16(Bg + (size_t)k * args.ldb + n) : u32x4{0, 0, 0, 0};
      }
    } else {
      // 8x8 blocks: thread -> (k block kc, n block nb), kc fastest
#pragma unroll
      for (int i = 0; i < P::B_PER_T; ++i) {
        int u = tid + i * NT;
        const bool mine = P::B_EVEN || u < P::B_UNITS;
        int kc = u % (BK / 8);
        int nb = u / (BK / 8);
        int n = n0 + nb * 8;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          int k = kt + kc * 8 + e;
          bool ok = mine && k < k_end && n < args.N;
          breg[slot][i * 8 + e] = ok ? ldg16(Bg + (size_t)k * args.ldb + n) : u32x4{0, 0, 0, 0};
        }
      }
    }
  };

  auto store_tiles = [&](T* st, int slot) {
    T* As = st;
    T* Bs = st + P::A_ELEMS;
#pragma unroll
    for (int i = 0; i < P::A_PER_T; ++i) {
      if (P::A_EVEN || tid + i * NT < P::A_CHUNKS)
        *reinterpret_cast<u32x4*>(As + a_row[i] * P::AST + a_col[i]) = areg[slot][i];
    }
    if constexpr (F32) {
#pragma unroll
      for (int i = 0; i < P::B_PER_T; ++i) {
        int c = tid + i * NT;
        if (!(P::B_EVEN || c < P::B_UNITS)) continue;
        int kr = c / P::B_CHUNKS_ROW;
        int nc = (c % P::B_CHUNKS_ROW) * VEC;
        *reinterpret_cast<u32x4*>(Bs + kr * P::BST + nc) = breg[slot][i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < P::B_PER_T; ++i) {
        int u = tid + i * NT;
        if (!(P::B_EVEN || u < P::B_UNITS)) continue;
        int kc = u % (BK / 8);
        int nb = u / (BK / 8);
        const u32x4* r = &breg[slot][i * 8];
        // transpose: column n of the 8x8 block becomes 8 consecutive k values
#pragma unroll
        for (int n = 0; n < 8; ++n) {
          const unsigned sel = (n & 1) ? 0x07060302u : 0x05040100u;
          u32x4 o;
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            o[p] = __builtin_amdgcn_perm(r[2 * p + 1][n >> 1], r[2 * p][n >> 1], sel);
          }
          *reinterpret_cast<u32x4*>(Bs + (nb * 8 + n) * P::BST + kc * 8) = o;
        }
      }
    }
  };

  f32x4 acc[P::TM][P::TN];
#pragma unroll
  for (int i = 0; i < P::TM; ++i)
#pragma unroll
    for (int j = 0; j < P::TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int wrow = wm * P::WTM;  // wave tile origin inside the block tile
  const int wcol = wn * P::WTN;

  auto compute = [&](const T* st) {
    const T* As = st;
    const T* Bs = st + P::A_ELEMS;
    if constexpr (F32) {
#pragma unroll
      for (int kc = 0; kc < BK / 16; ++kc) {
        f32x4 af[P::TM];
#pragma unroll
        for (int i = 0; i < P::TM; ++i) {
          af[i] = *reinterpret_cast<const f32x4*>(
              reinterpret_cast<const float*>(As) + (wrow + i * 16 + l16) * P::AST + kc * 16 + 4 * g);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          float bf[P::TN];
#pragma unroll
          for (int j = 0; j < P::TN; ++j) {
            bf[j] = reinterpret_cast<const float*>(Bs)[(kc * 16 + 4 * g + s) * P::BST + wcol + j * 16 + l16];
          }
#pragma unroll
          for (int i = 0; i < P::TM; ++i)
#pragma unroll
            for (int j = 0; j < P::TN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][s], bf[j], acc[i][j], 0, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < BK / 32; ++ks) {
        bf16x8 af[P::TM];
        bf16x8 bfr[P::TN];
#pragma unroll
        for (int i = 0; i < P::TM; ++i)
          af[i] = *reinterpret_cast<const bf16x8*>(As + (wrow + i * 16 + l16) * P::AST + ks * 32 + 8 * g);
#pragma unroll
        for (int j = 0; j < P::TN; ++j)
          bfr[j] = *reinterpret_cast<const bf16x8*>(Bs + (wcol + j * 16 + l16) * P::BST + ks * 32 + 8 * g);
#pragma unroll
        for (int i = 0; i < P::TM; ++i)
#pragma unroll
          for (int j = 0; j < P::TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
      }
    }
  };

  // Slabs go global -> registers (set t % RING) -> LDS (buffer t & 1) ->
  // MFMA.  Step t issues the loads of slab t + RING into the set slab t
  // left (stored to LDS in step t - 1), computes slab t, then stores slab
  // t + 1, whose loads were issued RING - 1 steps earlier: the in-order
  // vmcnt wait before that store leaves the younger sets in flight.  One
  // barrier per step.  The steps are unrolled by RING so every set index is
  // a constant.
  if (nk > 0) {
    load_a(k_begin, 0);
    load_b(k_begin, 0);
    store_tiles(smem, 0);
#pragma unroll
    for (int r = 1; r < RING; ++r) {
      if (r < nk) {
        load_a(k_begin + r * BK, r);
        load_b(k_begin + r * BK, r);
      }
    }
    __syncthreads();
    for (int it0 = 0; it0 < nk; it0 += RING) {
#pragma unroll
      for (int u = 0; u < RING; ++u) {
        const int it = it0 + u;
        if (it < nk) {
          T* cur = smem + (it & 1) * P::STAGE_ELEMS;
          T* nxt = smem + ((it & 1) ^ 1) * P::STAGE_ELEMS;
          if (it + RING < nk) {
            load_a(k_begin + (it + RING) * BK, u);
            load_b(k_begin + (it + RING) * BK, u);
          }
          compute(cur);
          if (it + 1 < nk) store_tiles(nxt, (u + 1) % RING);
          __syncthreads();
        }
      }
    }
  }

  // ---- epilogue ----
  // MFMA 16x16 result layout: lane holds rows 4*g..4*g+3 of column l16.
  const bool to_partial = args.partial != nullptr;
  float* out = to_partial ? args.partial + (size_t)split * args.M * args.N : args.C;
  const int ldo = to_partial ? args.N : args.ldc;
#pragma unroll
  for (int j = 0; j < P::TN; ++j) {
    int col = n0 + wcol + j * 16 + l16;
    if (col >= args.N) continue;
    float bv = (!to_partial && args.bias) ? args.bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < P::TM; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        int row = m0 + wrow + i * 16 + 4 * g + r;
        if (row < args.M) {
          float v = acc[i][j][r];
          if (!to_partial) {
            v += bv;
            if (args.relu && v < args.relu_threshold) v = args.relu_threshold;
          }
          if (to_partial)
            splitk_store(out + (size_t)row * ldo + col, v);
          else
            out[(size_t)row * ldo + col] = v;
        }
      }
    }
  }
  if (to_partial && splitk_arrive(args.counters + tile_m * args.tiles_n + tile_n, (int)gridDim.z)) {
    splitk_finish_tile<BM, BN, NT>(args.partial, args.C, args.bias, args.M, args.N, args.ldc, (int)gridDim.z,
                                   args.relu, args.relu_threshold, m0, n0);
    splitk_release(args.counters + tile_m * args.tiles_n + tile_n);
  }
}

}  // namespace xtc_hip
