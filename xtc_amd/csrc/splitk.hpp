// SPDX-License-Identifier: BSD-3-Clause
// Split-K completion inside the GEMM launch: the workgroup that stores the
// last partial tile of an output tile sums all of them, so a split-K GEMM
// is one kernel (no second reduce launch, no launch gap).
//
// Protocol, per output tile with `splits` workgroups along K:
//   1. every workgroup stores its fp32 partial tile to the workspace with the
//      agent-scope cache policy (gfx950: global_store ... sc1, written
//      through to the device coherence point, so the other XCDs' L2s never
//      hold it dirty): 16-byte stores where the tile allows, else the 4-byte
//      agent-scope atomic store, which compiles to the same policy;
//   2. every thread waits for its stores to complete (vmcnt(0)), the
//      workgroup synchronises and one lane increments the tile's arrival
//      counter (agent-scope atomic add);
//   3. the workgroup that sees splits-1 is the last one: it reads the
//      partials back with sc1 loads (16 bytes, or 4-byte agent-scope atomic
//      loads), sums partial[0..splits-1] in split order (the result does not
//      depend on which workgroup arrived last), applies bias / relu, stores C
//      and sets the counter back to 0 for the next launch.
// Every access to the published data carries the agent-scope policy, so no
// L2 write-back (buffer_wbl2) or invalidate (buffer_inv) is needed: a
// release/acquire fence at agent scope would write back and invalidate the
// whole L2 of the XCD in every workgroup, which costs more than the reduce.
// The 16-byte accesses halve the instructions of the 8-byte atomic pairs
// they replaced and make the C5 MLP 4 % faster.
// Counters start at zero (the host clears them with a kernel when it
// allocates them, and before every call of the no-allocation entry point)
// and every launch leaves them at zero.  Two launches that share the
// counters and the workspace must not overlap: the host keeps both per
// launch stream.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace xtc_hip {

namespace splitk {
typedef float f32x4 __attribute__((ext_vector_type(4)));
// s_waitcnt vmcnt(0), expcnt and lgkmcnt left at their maximum (no wait)
constexpr int kWaitVm0 = (7 << 4) | (15 << 8);
}  // namespace splitk

__device__ __forceinline__ void splitk_store(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float splitk_load(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16-byte aligned p: one 16-byte store with the agent-scope cache policy
// (sc1, what an agent-scope atomic store of 8 bytes compiles to), issued from
// asm because no atomic is 16 bytes wide; its completion is waited for in
// splitk_arrive (s_waitcnt vmcnt(0)).  The compiler does not count wait
// states into inline asm, so the asm opens with 24 of them: the most an
// MFMA result needs before a memory instruction reads it (16-pass XDL ops
// need 19).  The trailing s_nop covers the one wait state a VALU write of
// the data registers needs after a store of more than 8 bytes.
__device__ __forceinline__ void splitk_store4(float* p, splitk::f32x4 v) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\tglobal_store_dwordx4 %0, %1, off sc1\n\ts_nop 0" ::"v"(p), "v"(v)
               : "memory");
}

__device__ __forceinline__ splitk::f32x4 splitk_load4(const float* p) {
  uint64_t* q = reinterpret_cast<uint64_t*>(const_cast<float*>(p));
  const uint64_t lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t hi = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return splitk::f32x4{__uint_as_float((unsigned)lo), __uint_as_float((unsigned)(lo >> 32)),
                       __uint_as_float((unsigned)hi), __uint_as_float((unsigned)(hi >> 32))};
}

// Loads of 16 bytes with the agent-scope cache policy (sc1), from asm; each
// asm block waits for its own loads (s_waitcnt vmcnt(0)) before its outputs
// are defined.
#define XTC_SPLITK_LD(i, a) "global_load_dwordx4 %" #i ", %" #a ", off sc1\n\t"
__device__ __forceinline__ void splitk_ld8(splitk::f32x4* t, const float* p, size_t stride) {
  asm volatile(XTC_SPLITK_LD(0, 8) XTC_SPLITK_LD(1, 9) XTC_SPLITK_LD(2, 10) XTC_SPLITK_LD(3, 11)
               XTC_SPLITK_LD(4, 12) XTC_SPLITK_LD(5, 13) XTC_SPLITK_LD(6, 14) XTC_SPLITK_LD(7, 15) "s_waitcnt vmcnt(0)"
               : "=&v"(t[0]), "=&v"(t[1]), "=&v"(t[2]), "=&v"(t[3]), "=&v"(t[4]), "=&v"(t[5]), "=&v"(t[6]),
                 "=&v"(t[7])
               : "v"(p), "v"(p + stride), "v"(p + 2 * stride), "v"(p + 3 * stride), "v"(p + 4 * stride),
                 "v"(p + 5 * stride), "v"(p + 6 * stride), "v"(p + 7 * stride)
               : "memory");
}
__device__ __forceinline__ void splitk_ld4(splitk::f32x4* t, const float* p, size_t stride) {
  asm volatile(XTC_SPLITK_LD(0, 4) XTC_SPLITK_LD(1, 5) XTC_SPLITK_LD(2, 6) XTC_SPLITK_LD(3, 7) "s_waitcnt vmcnt(0)"
               : "=&v"(t[0]), "=&v"(t[1]), "=&v"(t[2]), "=&v"(t[3])
               : "v"(p), "v"(p + stride), "v"(p + 2 * stride), "v"(p + 3 * stride)
               : "memory");
}
__device__ __forceinline__ void splitk_ld2(splitk::f32x4* t, const float* p, size_t stride) {
  asm volatile(XTC_SPLITK_LD(0, 2) XTC_SPLITK_LD(1, 3) "s_waitcnt vmcnt(0)"
               : "=&v"(t[0]), "=&v"(t[1])
               : "v"(p), "v"(p + stride)
               : "memory");
}
__device__ __forceinline__ void splitk_ld1(splitk::f32x4* t, const float* p) {
  asm volatile(XTC_SPLITK_LD(0, 1) "s_waitcnt vmcnt(0)" : "=&v"(t[0]) : "v"(p) : "memory");
}
#undef XTC_SPLITK_LD

// sum_{s < splits} p[s * stride] in split order, starting from +0.0, up to 8
// loads in flight.  Only the splits that exist are loaded: these loads go
// past the L2.
__device__ __forceinline__ splitk::f32x4 splitk_sum4(const float* p, size_t stride, int splits) {
  splitk::f32x4 v = {0.f, 0.f, 0.f, 0.f};
  splitk::f32x4 t[8];
  int s = 0;
  for (; s + 8 <= splits; s += 8) {
    splitk_ld8(t, p + (size_t)s * stride, stride);
#pragma unroll
    for (int j = 0; j < 8; ++j) v += t[j];
  }
  if (s + 4 <= splits) {
    splitk_ld4(t, p + (size_t)s * stride, stride);
#pragma unroll
    for (int j = 0; j < 4; ++j) v += t[j];
    s += 4;
  }
  if (s + 2 <= splits) {
    splitk_ld2(t, p + (size_t)s * stride, stride);
    v += t[0];
    v += t[1];
    s += 2;
  }
  if (s < splits) {
    splitk_ld1(t, p + (size_t)s * stride);
    v += t[0];
  }
  return v;
}

__device__ __forceinline__ float splitk_sum1(const float* p, size_t stride, int splits) {
  constexpr int kBatch = 8;
  float v = 0.f;
  for (int s0 = 0; s0 < splits; s0 += kBatch) {
    float t[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j)
      if (s0 + j < splits) t[j] = splitk_load(p + (size_t)(s0 + j) * stride);
#pragma unroll
    for (int j = 0; j < kBatch; ++j)
      if (s0 + j < splits) v += t[j];
  }
  return v;
}

// Step 2: true in the last-arriving workgroup only.  Called by every thread
// of the workgroup (1-D blocks) after its splitk_store calls.  `flag` is one
// LDS word that no thread touches between the first barrier here and the
// return (a kernel whose LDS is full passes a word of its own, free by then).
__device__ __forceinline__ bool splitk_arrive_in(unsigned* counter, int splits, unsigned* flag) {
  __builtin_amdgcn_s_waitcnt(splitk::kWaitVm0);
  __syncthreads();
  if (threadIdx.x == 0)
    *flag = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(splits - 1)
                ? 1u
                : 0u;
  __syncthreads();
  return *flag != 0;
}

__device__ __forceinline__ bool splitk_arrive(unsigned* counter, int splits) {
  __shared__ unsigned s_last;
  return splitk_arrive_in(counter, splits, &s_last);
}

// Ends the protocol in the last workgroup (after its reads of the partials).
__device__ __forceinline__ void splitk_release(unsigned* counter) {
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The last workgroup's sum over one BM x BN output tile at (m0, n0):
// C[m][n] = epilogue( sum_s partial[s][m][n] ), partial is [splits][M][N].
// Four columns per thread when N, ldc and the pointers allow it; the sums
// are the same element by element either way.
template <int BM, int BN, int NT>
__device__ __forceinline__ void splitk_finish_tile(const float* partial, float* C, const float* bias, int M,
                                                   int N, int ldc, int splits, int relu, float thr, int m0,
                                                   int n0) {
  using splitk::f32x4;
  const size_t plane = (size_t)M * N;
  const int tid = threadIdx.x;
  const bool vec = BN % 4 == 0 && ((N | ldc) & 3) == 0 && (((uintptr_t)C | (uintptr_t)partial) & 15) == 0 &&
                   (bias == nullptr || ((uintptr_t)bias & 15) == 0);
  if (vec) {
    for (int idx = tid; idx < BM * BN / 4; idx += NT) {
      const int m = m0 + idx / (BN / 4);
      const int n = n0 + 4 * (idx % (BN / 4));
      if (m >= M || n >= N) continue;
      f32x4 v = splitk_sum4(partial + (size_t)m * N + n, plane, splits);
      if (bias) v += *(const f32x4*)(bias + n);
      if (relu) {
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = v[r] < thr ? thr : v[r];
      }
      *(f32x4*)(C + (size_t)m * ldc + n) = v;
    }
  } else {
    for (int idx = tid; idx < BM * BN; idx += NT) {
      const int m = m0 + idx / BN;
      const int n = n0 + idx % BN;
      if (m >= M || n >= N) continue;
      float v = splitk_sum1(partial + (size_t)m * N + n, plane, splits);
      if (bias) v += bias[n];
      if (relu && v < thr) v = thr;
      C[(size_t)m * ldc + n] = v;
    }
  }
}

}  // namespace xtc_hip
