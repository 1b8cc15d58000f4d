// SPDX-License-Identifier: BSD-3-Clause
// Direct NHWC x RSCF conv2d (fp32) on gfx950 for channel counts that are
// multiples of 64:
//   O[b,oh,ow,f] = epilogue( sum_{r,s,c} Ipad[b, oh*sh+r, ow*sw+s, c] * W[r,s,c,f] )
// with the pad of a pad2d producer folded in (out-of-image taps read
// pad_value), as XTCOperConv2D after XTCOperPad2D (operators.py:252-347,
// 350-591).
//
// Why not the implicit-GEMM loader: for shapes like 8x56x56x64 * 3x3x64x64
// (GEMM M=25088, N=64, K=576) each tile walks only K=576 and re-reads every
// input pixel once per filter tap from L2; the global-load latency is then
// exposed on every slab.  Here a workgroup owns a TH x TW block of output
// pixels x 64 filters of one image (8x8 with 2x2 waves; 8x14 with 1x4
// waves: 224 equal blocks for 8x56x56 outputs; or 7x14 with 1x4 waves, 256
// blocks, one on every CU, its last 2 pixels on 4x4x1 MFMAs as described at
// conv_direct_f32_3x3s1):
//   * the input halo ((TH-1)*sh+R) x ((TW-1)*sw+S) pixels x 64 channels is
//     loaded once into LDS (pad_value outside the image), pixel stride 68
//     floats so the 16 pixels read by a lane group fall on distinct banks;
//   * the weights take one of two paths (template parameter WRING):
//     - WRING = 0: they stream one tap (r, s) [64 c][64 f] = 16 KB at a time
//       through 3 LDS stages by LDS DMA (issued from asm, lds_dma.hpp, so
//       the compiler's waits on the LDS operand reads stay exact), two taps
//       ahead, behind a barrier per tap; the 16-byte chunks of weight row c
//       are XOR-swizzled by 4*((c>>2)&3) so the scalar B reads of the four
//       lane groups hit disjoint banks;
//     - WRING > 0: each lane loads its own B fragments of a tap (16 FT
//       floats: its filter column, the 16 channels its MFMA k-slots take)
//       straight from global memory into a ring of WRING taps of registers,
//       WRING taps ahead of the MFMAs.  No weight LDS, no DMA and no
//       barrier inside the K walk; the only barrier publishes the halo.
//       With one wave per SIMD (8x14 blocks: FT = 1) it is 6 % faster than
//       the LDS stages; with FT = 2 (8x8 blocks) 5 % slower, the twice as
//       many 4-byte loads per tap outweighing the saved barriers;
//   * 4 waves (WM x WN), each TH*TW/WM pixels x 64/WN filters of
//     v_mfma_f32_16x16x4_f32; the filter fragment is the first operand, so a
//     lane ends up with 4 consecutive filters of one pixel and stores a float4;
//   * more than 64 channels: the halo is reloaded per 64-channel chunk.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lds_dma.hpp"

namespace xtc_hip {

struct DirectConvArgs {
  const float* I;  // [NB][H][W][C], unpadded
  const float* Wt;  // [R][S][C][F]
  float* O;        // [NB][OH][OW][F]
  const float* bias;
  int NB, H, W, C, F, R, S;
  int sh, sw;
  int pt, pl;      // top / left padding
  int OH, OW;
  float pad_value;
  int relu;
  float relu_threshold;
  int tiles_h, tiles_w;  // ceil(OH/TH), ceil(OW/TW)
};

namespace dconv {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int CB = 64;            // channels per chunk
constexpr int FB = 64;            // filters per workgroup
constexpr int CP = CB + 4;        // halo pixel stride (floats)
constexpr int W_STAGE = CB * FB * 4;  // 16 KB
constexpr int STAGES = 3;
constexpr int NW = 4;             // waves per workgroup
constexpr int NT = NW * 64;
constexpr int DMA_PER_WAVE = W_STAGE / 1024 / NW;  // 4
// halo capacity in pixels for a halo buffer of `bytes`
constexpr int halo_pix(int bytes) { return bytes / (CP * 4); }

__device__ __forceinline__ int swz(int c) { return 4 * ((c >> 2) & 3); }
constexpr int waitcnt_vm(int n) { return (n & 15) | (7 << 4) | (15 << 8) | (((n >> 4) & 3) << 14); }

}  // namespace dconv

// TH x TW output pixels per workgroup, WM x WN waves, HALO_BYTES of LDS for
// the input halo of one 64-channel chunk, weights through LDS stages
// (WRING = 0) or a register ring of WRING taps.
// The remainder pixels' epilogue (1 x 4-wave blocks whose pixel count is not
// a multiple of 16): lane (l16, g) register i holds pixel 16 PT + i of the
// block, filter f, summed over the channels of phase g; the four phases are
// added across lanes and the lanes of phase 0 store.
template <int PT, int REM, int TW>
__device__ __forceinline__ void store_remainder(const DirectConvArgs& a, dconv::f32x4 accr, int img, int oh0,
                                                int ow0, int f, int g) {
#pragma unroll
  for (int i = 0; i < REM; ++i) {
    accr[i] += __shfl_xor(accr[i], 16);
    accr[i] += __shfl_xor(accr[i], 32);
  }
  if (g != 0) return;
  const float bf = a.bias ? a.bias[f] : 0.f;
#pragma unroll
  for (int i = 0; i < REM; ++i) {
    const int p = 16 * PT + i;
    const int oh = oh0 + p / TW, ow = ow0 + p % TW;
    if (oh >= a.OH || ow >= a.OW) continue;
    float v = accr[i] + bf;
    if (a.relu) v = v < a.relu_threshold ? a.relu_threshold : v;
    a.O[(((size_t)img * a.OH + oh) * a.OW + ow) * a.F + f] = v;
  }
}

template <int TH, int TW, int WM, int WN, int HALO_BYTES, int WRING>
__global__ void __attribute__((amdgpu_flat_work_group_size(256, 256))) conv_direct_f32(DirectConvArgs a) {
  using namespace dconv;
  constexpr int HALO_MAX_PIX = halo_pix(HALO_BYTES);
  constexpr int PT = TH * TW / 16 / WM;  // whole 16-pixel tiles per wave
  constexpr int REM = TH * TW - 16 * PT * WM;  // pixels after them (one wave row only)
  constexpr int FT = FB / WN / 16;       // 16-filter tiles per wave
  constexpr bool REG = WRING > 0;
  constexpr int RING = REG ? WRING : STAGES;  // slabs in flight + 1 (LDS) or in registers
  constexpr int WBYTES = REG ? 16 : W_STAGE;
  static_assert(WM * WN == NW && FB % (16 * WN) == 0, "tiling");
  static_assert(REM == 0 || (WM == 1 && FT == 1 && REM <= 4), "remainder pixels: 1 x 4 waves, at most 4");
  static_assert(WRING >= 0 && WRING <= 4, "register ring");
  __shared__ __attribute__((aligned(1024))) float halo[HALO_MAX_PIX * CP];
  __shared__ __attribute__((aligned(1024))) unsigned char w0[WBYTES];
  __shared__ __attribute__((aligned(1024))) unsigned char w1[WBYTES];
  __shared__ __attribute__((aligned(1024))) unsigned char w2[WBYTES];
  unsigned char* const wst[3] = {w0, w1, w2};

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN;  // pixels 16 PT wm .. +16 PT - 1
  const int wn = wave % WN;  // filters 16 FT wn .. +16 FT - 1
  const int l16 = lane & 15;
  const int g = lane >> 4;

  // block -> (image, tile row, tile column, filter block); filters fastest
  const int fblocks = a.F / FB;
  int bid = blockIdx.x;
  const int fb = bid % fblocks;
  bid /= fblocks;
  const int tw = bid % a.tiles_w;
  bid /= a.tiles_w;
  const int th = bid % a.tiles_h;
  const int img = bid / a.tiles_h;
  const int oh0 = th * TH, ow0 = tw * TW;
  const int HH = (TH - 1) * a.sh + a.R;
  const int HW = (TW - 1) * a.sw + a.S;
  const int ih0 = oh0 * a.sh - a.pt;
  const int iw0 = ow0 * a.sw - a.pl;
  const int taps = a.R * a.S;
  const int chunks = a.C / CB;
  const int nslab = chunks * taps;  // weight slabs, chunk-major

  // weight slab t = (chunk, tap): rows c of W[r][s][chunk*64 + c][fb*64 ..]
  int w_row[DMA_PER_WAVE], w_col[DMA_PER_WAVE];
#pragma unroll
  for (int i = 0; i < DMA_PER_WAVE; ++i) {
    const int c = 4 * (wave * DMA_PER_WAVE + i) + (lane >> 4);
    w_row[i] = c;
    w_col[i] = fb * FB + ((lane & 15) ^ swz(c)) * 4;
  }
  auto issue_slab = [&](int t, unsigned char* st) {
    const int chunk = t / taps;
    const int tap = t - chunk * taps;
    const float* base = a.Wt + ((size_t)tap * a.C + chunk * CB) * a.F;
#pragma unroll
    for (int i = 0; i < DMA_PER_WAVE; ++i)
      lds_dma16((const void*)(base + (size_t)w_row[i] * a.F + w_col[i]), st + (wave * DMA_PER_WAVE + i) * 1024);
  };
  // register ring: lane (l16, g) holds
  // W[r][s][chunk*64 + 16 kc + 4 g + st][fb*64 + wn*16*FT + 16 jt + l16]
  float wr[REG ? RING : 1][CB / 16][4][FT];
  const float* const wlane = a.Wt + (size_t)(4 * g) * a.F + fb * FB + wn * 16 * FT + l16;
  auto load_slab = [&](int t, const int u) {
    const int chunk = t / taps;
    const int tap = t - chunk * taps;
    const float* base = wlane + ((size_t)tap * a.C + chunk * CB) * a.F;
#pragma unroll
    for (int kc = 0; kc < CB / 16; ++kc)
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int jt = 0; jt < FT; ++jt) wr[u][kc][st][jt] = base[(size_t)(kc * 16 + st) * a.F + jt * 16];
  };

  // All of a thread's halo loads are issued before its first LDS write (at
  // most HALO_MAX_PIX * 16 / 256 chunks: 8 for 8x8 tiles, 12 for 8x14), so
  // the load latency is paid once rather than once per chunk.
  auto load_halo = [&](int chunk) {
    constexpr int MAXQ = (HALO_MAX_PIX * (CB / 4) + NT - 1) / NT;
    const int n16 = HH * HW * (CB / 4);  // 16-byte chunks
    f32x4 v[MAXQ];
#pragma unroll
    for (int j = 0; j < MAXQ; ++j) {
      const int q = tid + j * NT;
      const int pix = q >> 4;
      const int cc = (q & 15) * 4;
      const int hy = pix / HW, hx = pix - (pix / HW) * HW;
      const int ih = ih0 + hy, iw = iw0 + hx;
      v[j] = f32x4{a.pad_value, a.pad_value, a.pad_value, a.pad_value};
      if (q < n16 && ih >= 0 && ih < a.H && iw >= 0 && iw < a.W)
        v[j] = *(const f32x4*)(a.I + (((size_t)img * a.H + ih) * a.W + iw) * a.C + chunk * CB + cc);
    }
#pragma unroll
    for (int j = 0; j < MAXQ; ++j) {
      const int q = tid + j * NT;
      if (q < n16) *(f32x4*)(halo + (q >> 4) * CP + (q & 15) * 4) = v[j];
    }
  };

  // output pixels of this lane's PT 16-pixel tiles
  int php[PT], pwp[PT];
#pragma unroll
  for (int it = 0; it < PT; ++it) {
    const int p = wm * 16 * PT + it * 16 + l16;
    php[it] = p / TW;
    pwp[it] = p % TW;
  }

  // remainder pixel of this lane's 4x4x1 rows (see conv_direct_f32_3x3s1)
  int rph = 0, rpw = 0;
  if constexpr (REM > 0) {
    const int p = 16 * PT + min(l16 & 3, REM - 1);
    rph = p / TW;
    rpw = p % TW;
  }

  f32x4 acc[PT][FT];
#pragma unroll
  for (int i = 0; i < PT; ++i)
#pragma unroll
    for (int j = 0; j < FT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 accr = f32x4{0.f, 0.f, 0.f, 0.f};

  if constexpr (REG) {
#pragma unroll
    for (int t = 0; t < RING; ++t)
      if (t < nslab) load_slab(t, t);
  } else {
#pragma unroll
    for (int t = 0; t < STAGES - 1; ++t)
      if (t < nslab) issue_slab(t, wst[t]);
  }

  auto step = [&](int t, const int s) {
    const int chunk = t / taps;
    const int tap = t - chunk * taps;
    if (tap == 0) {
      if (chunk > 0) __syncthreads();  // every wave is done with the previous chunk's halo
      load_halo(chunk);
    }
    if constexpr (REG) {
      if (tap == 0) __syncthreads();  // halo visible
    } else {
      if (t + STAGES - 2 < nslab)
        __builtin_amdgcn_s_waitcnt(waitcnt_vm((STAGES - 2) * DMA_PER_WAVE));
      else
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
      __syncthreads();  // slab t (and the halo) visible; stage of slab t-1 free
      if (t + STAGES - 1 < nslab) issue_slab(t + STAGES - 1, wst[(s + STAGES - 1) % STAGES]);
    }
    const float* ws = (const float*)wst[REG ? 0 : s];
    const int r = tap / a.S;
    const int sx = tap - r * a.S;
    int aoff[PT];
#pragma unroll
    for (int it = 0; it < PT; ++it) aoff[it] = ((php[it] * a.sh + r) * HW + pwp[it] * a.sw + sx) * CP + 4 * g;
    const int roff = ((rph * a.sh + r) * HW + rpw * a.sw + sx) * CP + 4 * g;
#pragma unroll
    for (int kc = 0; kc < CB / 16; ++kc) {
      f32x4 av[PT];
#pragma unroll
      for (int it = 0; it < PT; ++it) av[it] = *(const f32x4*)(halo + aoff[it] + kc * 16);
      f32x4 ar;
      if constexpr (REM > 0) ar = *(const f32x4*)(halo + roff + kc * 16);
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int c = kc * 16 + 4 * g + st;
#pragma unroll
        for (int jt = 0; jt < FT; ++jt) {
          const int f = wn * 16 * FT + jt * 16 + l16;
          const float bv = REG ? wr[REG ? s : 0][kc][st][jt] : ws[c * FB + ((f >> 2) ^ swz(c)) * 4 + (f & 3)];
#pragma unroll
          for (int it = 0; it < PT; ++it)
            acc[it][jt] = __builtin_amdgcn_mfma_f32_16x16x4f32(bv, av[it][st], acc[it][jt], 0, 0, 0);
          if constexpr (REM > 0) accr = __builtin_amdgcn_mfma_f32_4x4x1f32(ar[st], bv, accr, 0, 0, 0);
        }
      }
    }
    if constexpr (REG) {
      if (t + RING < nslab) load_slab(t + RING, s);
    }
  };
  for (int t = 0; t < nslab; t += RING) {
#pragma unroll
    for (int s = 0; s < RING; ++s)
      if (t + s < nslab) step(t + s, s);
  }

  // lane holds filters f0 .. f0+3 of pixel (php, pwp) for each (it, jt)
#pragma unroll
  for (int it = 0; it < PT; ++it) {
    const int oh = oh0 + php[it], ow = ow0 + pwp[it];
    if (oh >= a.OH || ow >= a.OW) continue;
    float* out = a.O + (((size_t)img * a.OH + oh) * a.OW + ow) * a.F + fb * FB;
#pragma unroll
    for (int jt = 0; jt < FT; ++jt) {
      const int f = wn * 16 * FT + jt * 16 + 4 * g;
      f32x4 v = acc[it][jt];
      if (a.bias) v += *(const f32x4*)(a.bias + fb * FB + f);
      if (a.relu) {
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = v[q] < a.relu_threshold ? a.relu_threshold : v[q];
      }
      *(f32x4*)(out + f) = v;
    }
  }
  if constexpr (REM > 0) store_remainder<PT, REM, TW>(a, accr, img, oh0, ow0, fb * FB + wn * 16 + l16, g);
}

// The register-ring path above for a 3x3 window at stride 1, with the window,
// the strides and the halo's width fixed at compile time (1 x 4 waves, 64
// filters per workgroup, FT = 1).  Same blocks, fragments, weight ring and
// accumulation order as conv_direct_f32<TH, TW, 1, 4, *, WRING>, so results
// are bit-identical to it; what changes is the instruction stream between the
// MFMAs.  In the general kernel every step recomputes the lane's halo offsets
// from runtime strides and window sizes (integer multiplies, a division by S)
// and each weight load its 64-bit address, and those VALU instructions share
// the wave's issue with its MFMAs: measured on the C4 shape (8x56x56x64, 3x3,
// 224 blocks), the MFMAs alone of the general kernel take 21.3 us against
// 15.3 us for a register-only loop of the same MFMA count, and 18.5 us once
// the per-step offset arithmetic is removed.  Here the taps are unrolled, so
// each fragment read is one ds_read_b128 at an immediate offset from one of 7
// per-lane base registers, and each weight load adds a constant row offset to
// a per-lane pointer.  C4: 23.1 -> 20.6 us, bit-identical on integer and
// random inputs.
//
// A block whose pixel count is not a multiple of 16 (TH x TW = 16 PT + REM,
// REM <= 4) runs its PT whole tiles as above and its last REM pixels on
// v_mfma_f32_4x4x1_16b_f32, whose 16 independent 4x4 blocks take the same
// operands the ring and the halo already hold: block b = 4 g + fg of lane
// (l16, g) multiplies pixel i (rows, i = l16 & 3, clamped to REM - 1) by
// filters 16 wn + 4 fg .. + 3 (columns) over the channels 16 kc + 4 g + st,
// so each (tap, k-chunk) adds one ds_read_b128 and 4 of these MFMAs (a quarter
// of a 16x16x4's cycles) instead of a 16-pixel tile, and the four channel
// phases g are summed across lanes at the end.  7 x 14 blocks (6 tiles + 2
// pixels) cover 8x56x56 outputs in 256 blocks, one per CU, with 6.25 tiles
// of MFMA cycles per SIMD instead of the 7 of 8 x 14 blocks on 224 CUs.  The
// remainder pixels sum their channels in another order than the tiles, so
// they are exact on exactly summable inputs and within fp32 rounding
// otherwise.
template <int TH, int TW, int WRING>
__global__ void __attribute__((amdgpu_flat_work_group_size(256, 256))) conv_direct_f32_3x3s1(DirectConvArgs a) {
  using namespace dconv;
  constexpr int R = 3, S = 3, TAPS = R * S;
  constexpr int HH = TH + R - 1, HW = TW + S - 1;  // halo of one block at stride 1
  constexpr int NPIX = HH * HW;
  constexpr int PT = TH * TW / 16;  // whole 16-pixel tiles per wave
  constexpr int REM = TH * TW - 16 * PT;  // pixels after them, on 4x4x1 MFMAs
  constexpr int RING = WRING;
  static_assert(REM <= 4, "at most 4 pixels after the whole tiles");
  static_assert(RING >= 1 && TAPS % RING == 0, "the ring slot of tap t of any chunk is t % RING");
  __shared__ __attribute__((aligned(1024))) float halo[NPIX * CP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wn = __builtin_amdgcn_readfirstlane(tid >> 6);  // filters 16 wn .. 16 wn + 15
  const int l16 = lane & 15;
  const int g = lane >> 4;

  // block -> (image, tile row, tile column, filter block); filters fastest
  const int fblocks = a.F / FB;
  int bid = blockIdx.x;
  const int fb = bid % fblocks;
  bid /= fblocks;
  const int tw = bid % a.tiles_w;
  bid /= a.tiles_w;
  const int th = bid % a.tiles_h;
  const int img = bid / a.tiles_h;
  const int oh0 = th * TH, ow0 = tw * TW;
  const int ih0 = oh0 - a.pt;
  const int iw0 = ow0 - a.pl;
  const int chunks = a.C / CB;
  const int nslab = chunks * TAPS;  // weight slabs, chunk-major
  const int F = a.F;

  // register ring: lane (l16, g) holds W[tap][chunk*64 + 16 kc + 4 g + st][fb*64 + 16 wn + l16]
  float wr[RING][CB / 16][4];
  const float* const wlane = a.Wt + (size_t)(4 * g) * F + fb * FB + wn * 16 + l16;
  auto load_slab = [&](int t, const int u) {
    const int chunk = t / TAPS;
    const int tap = t - chunk * TAPS;
    const float* base = wlane + ((size_t)tap * a.C + chunk * CB) * F;
#pragma unroll
    for (int kc = 0; kc < CB / 16; ++kc)
#pragma unroll
      for (int st = 0; st < 4; ++st) wr[u][kc][st] = base[(size_t)(kc * 16 + st) * F];
  };
  // the halo of one 64-channel chunk, every global load issued before the
  // first LDS write (pad_value outside the image)
  auto load_halo = [&](int chunk) {
    constexpr int N16 = NPIX * (CB / 4);  // 16-byte pieces
    constexpr int MAXQ = (N16 + NT - 1) / NT;
    f32x4 v[MAXQ];
#pragma unroll
    for (int j = 0; j < MAXQ; ++j) {
      const int q = tid + j * NT;
      const int pix = q >> 4;
      const int ih = ih0 + pix / HW, iw = iw0 + pix % HW;
      v[j] = f32x4{a.pad_value, a.pad_value, a.pad_value, a.pad_value};
      if (q < N16 && ih >= 0 && ih < a.H && iw >= 0 && iw < a.W)
        v[j] = *(const f32x4*)(a.I + (((size_t)img * a.H + ih) * a.W + iw) * a.C + chunk * CB + (q & 15) * 4);
    }
#pragma unroll
    for (int j = 0; j < MAXQ; ++j) {
      const int q = tid + j * NT;
      if (q < N16) *(f32x4*)(halo + (q >> 4) * CP + (q & 15) * 4) = v[j];
    }
  };
  // LDS offset (floats) of the lane's pixel of tile it at tap (0, 0), channel 4 g
  int abase[PT];
#pragma unroll
  for (int it = 0; it < PT; ++it) {
    const int p = it * 16 + l16;
    abase[it] = ((p / TW) * HW + p % TW) * CP + 4 * g;
  }

  // remainder: the lane's pixel 16 PT + min(l16 & 3, REM - 1) at tap (0, 0), channel 4 g
  int rbase = 0;
  if constexpr (REM > 0) {
    const int p = 16 * PT + min(l16 & 3, REM - 1);
    rbase = ((p / TW) * HW + p % TW) * CP + 4 * g;
  }

  f32x4 acc[PT];
#pragma unroll
  for (int i = 0; i < PT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 accr = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < RING; ++t)
    if (t < nslab) load_slab(t, t);

  for (int chunk = 0; chunk < chunks; ++chunk) {
    if (chunk > 0) __syncthreads();  // every wave is done with the previous chunk's halo
    load_halo(chunk);
    __syncthreads();  // halo visible
    const int t0 = chunk * TAPS;
#pragma unroll
    for (int tap = 0; tap < TAPS; ++tap) {
      const int u = tap % RING;
      const int toff = ((tap / S) * HW + tap % S) * CP;  // compile-time
#pragma unroll
      for (int kc = 0; kc < CB / 16; ++kc) {
        f32x4 av[PT];
#pragma unroll
        for (int it = 0; it < PT; ++it) av[it] = *(const f32x4*)(halo + abase[it] + toff + kc * 16);
        f32x4 ar;
        if constexpr (REM > 0) ar = *(const f32x4*)(halo + rbase + toff + kc * 16);
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const float bv = wr[u][kc][st];
#pragma unroll
          for (int it = 0; it < PT; ++it) acc[it] = __builtin_amdgcn_mfma_f32_16x16x4f32(bv, av[it][st], acc[it], 0, 0, 0);
          if constexpr (REM > 0) accr = __builtin_amdgcn_mfma_f32_4x4x1f32(ar[st], bv, accr, 0, 0, 0);
        }
      }
      if (t0 + tap + RING < nslab) load_slab(t0 + tap + RING, u);
    }
  }

  // lane holds filters 16 wn + 4 g .. + 3 of pixel it*16 + l16
#pragma unroll
  for (int it = 0; it < PT; ++it) {
    const int p = it * 16 + l16;
    const int oh = oh0 + p / TW, ow = ow0 + p % TW;
    if (oh >= a.OH || ow >= a.OW) continue;
    const int f = wn * 16 + 4 * g;
    f32x4 v = acc[it];
    if (a.bias) v += *(const f32x4*)(a.bias + fb * FB + f);
    if (a.relu) {
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = v[q] < a.relu_threshold ? a.relu_threshold : v[q];
    }
    *(f32x4*)(a.O + (((size_t)img * a.OH + oh) * a.OW + ow) * F + fb * FB + f) = v;
  }

  if constexpr (REM > 0) store_remainder<PT, REM, TW>(a, accr, img, oh0, ow0, fb * FB + wn * 16 + l16, g);
}

}  // namespace xtc_hip
