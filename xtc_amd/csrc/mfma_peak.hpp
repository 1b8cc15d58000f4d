// SPDX-License-Identifier: BSD-3-Clause
// Register-resident MFMA throughput kernels: the measured peak behind
// xtc_hip_evaluate_flops, the device counterpart of the reference's
// evaluate_flops microbenchmark (src/xtc/csrcs/runtimes/host/evaluate_flops.c:
// 431-494, which times independent FMA chains in registers).
//
// Each wave loads its operand fragments once, then issues `iters` rounds of
// independent MFMAs into 32 (bf16) or 16 (fp32, fp64) accumulators: no memory
// traffic and no dependency stall inside a round, so the time is the matrix
// cores' issue rate at the operands' switching activity.  One workgroup of 4
// waves per SIMD quad (one wave per SIMD), two workgroups per CU.  The
// accumulators are reduced into `out` so that no MFMA is dead code.
#pragma once
#include <hip/hip_runtime.h>

namespace xtc_hip {
namespace peak {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
// bf16: a round is 8 A x 4 B fragments = 32 MFMAs of 16x16x32, 2^19 FLOP per wave
constexpr int kBf16Frags = 12;          // 16-byte operand fragments per lane
constexpr double kBf16FmaPerRound = 32.0 * 16 * 16 * 32;
// fp32: a round is 4 k-steps of 4 A x 4 B = 64 MFMAs of 16x16x4, 2^17 FLOP per wave
constexpr int kF32Frags = 32;           // 4-byte operands per lane
constexpr double kF32FmaPerRound = 64.0 * 16 * 16 * 4;

__global__ void __launch_bounds__(kThreads) mfma_peak_bf16(const u32x4* __restrict__ in, float* __restrict__ out,
                                                          int iters) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  bf16x8 a[8], b[4];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = __builtin_bit_cast(bf16x8, in[(wave * kBf16Frags + i) * 64 + lane]);
#pragma unroll
  for (int i = 0; i < 4; ++i) b[i] = __builtin_bit_cast(bf16x8, in[(wave * kBf16Frags + 8 + i) * 64 + lane]);
  f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int t = 0; t < iters; ++t) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b[j], a[i], acc[i][j], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) s += acc[i][j][0] + acc[i][j][3];
  out[blockIdx.x * kThreads + threadIdx.x] = s;
}

__global__ void __launch_bounds__(kThreads) mfma_peak_f32(const float* __restrict__ in, float* __restrict__ out,
                                                         int iters) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  float a[16], b[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) a[i] = in[(wave * kF32Frags + i) * 64 + lane];
#pragma unroll
  for (int i = 0; i < 16; ++i) b[i] = in[(wave * kF32Frags + 16 + i) * 64 + lane];
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int t = 0; t < iters; ++t) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(b[4 * q + j], a[4 * q + i], acc[i][j], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) s += acc[i][j][0] + acc[i][j][3];
  out[blockIdx.x * kThreads + threadIdx.x] = s;
}

// fp64: a round is 2 k-steps of 4 A x 4 B = 32 MFMAs of 16x16x4 f64
constexpr int kF64Frags = 16;           // 8-byte operands per lane
constexpr double kF64FmaPerRound = 32.0 * 16 * 16 * 4;
typedef double f64x4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(kThreads) mfma_peak_f64(const double* __restrict__ in, float* __restrict__ out,
                                                         int iters) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  double a[8], b[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = in[(wave * kF64Frags + i) * 64 + lane];
#pragma unroll
  for (int i = 0; i < 8; ++i) b[i] = in[(wave * kF64Frags + 8 + i) * 64 + lane];
  f64x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f64x4{0.0, 0.0, 0.0, 0.0};
  for (int t = 0; t < iters; ++t) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(b[4 * q + j], a[4 * q + i], acc[i][j], 0, 0, 0);
  }
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) s += acc[i][j][0] + acc[i][j][3];
  out[blockIdx.x * kThreads + threadIdx.x] = (float)s;
}

}  // namespace peak
}  // namespace xtc_hip
