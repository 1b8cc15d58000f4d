// SPDX-License-Identifier: BSD-3-Clause
// libxtc_hip runtime: device management, operator dispatch, auxiliary
// HBM-bound kernels and the timing harness behind include/xtc_hip.h.
#include <hip/hip_runtime.h>

#include <dlfcn.h>
#include <linux/perf_event.h>
#include <math.h>
#include <sys/syscall.h>
#include <unistd.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <time.h>

#include <atomic>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "gemm_bf16_lds.hpp"
#include "gemm_bf16_skinny.hpp"
#include "gemm_bf16_pingpong.hpp"
#include "gemm_f32_splitwave.hpp"
#include "gemm_f32_lds.hpp"
#include "gemm_f64.hpp"
#include "conv_direct.hpp"
#include "mfma_peak.hpp"
#include "registry.hpp"
#include "xtc_hip.h"

using namespace xtc_hip;

// Scratch memory of xtc_hip_matmul_noalloc: one copy per device, for the
// whole life of the process.  Host code never uses this name as an address
// (in host code it is only a stand-in for the device symbol): xtc_hip_init
// looks up each device's address of it once (DeviceState::scratch_ptr).
static __device__ __align__(256) unsigned char scratch[XTC_HIP_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_last_error;

int fail(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return 1;
}

#define HIP_TRY(expr)                                                          \
  do {                                                                         \
    hipError_t e_ = (expr);                                                    \
    if (e_ != hipSuccess)                                                      \
      return fail("%s failed: %s", #expr, hipGetErrorString(e_));              \
  } while (0)

constexpr int kMaxDevices = 16;

// Scratch memory of one stream: split-K partial sums and arrival counters
// (zero between launches), and natural copies of transposed operands.  Each
// stream has its own, so launches on different streams never share scratch
// and may overlap; launches on one stream are ordered by the stream.
struct StreamScratch {
  void* workspace = nullptr;
  size_t workspace_bytes = 0;
  unsigned* counters = nullptr;
  size_t counters_len = 0;
  void* staging[2] = {nullptr, nullptr};
  size_t staging_bytes[2] = {0, 0};
};

struct DeviceState {
  bool ready = false;
  int cus = 0;  // compute units
  hipStream_t stream = nullptr;
  void* scratch_ptr = nullptr;  // this device's address of `scratch`
  // completion word of the library stream in coherent host memory, and the
  // last sequence number queued for it (xtc_hip_synchronize)
  unsigned* done_flag = nullptr;
  std::atomic<unsigned> done_seq{0};
  // taking a sequence number and queuing its store happen under this lock,
  // so concurrent callers queue their stores in number order and the word
  // only grows
  std::mutex done_mutex;
  std::unordered_map<hipStream_t, StreamScratch> scratch;  // by launch stream
  std::string arch, name;
};

std::mutex g_mutex;
DeviceState g_dev[kMaxDevices];
int g_current = -1;

DeviceState* current_state() {
  if (g_current < 0) return nullptr;
  DeviceState* d = &g_dev[g_current];
  return d->ready ? d : nullptr;
}

hipStream_t pick_stream(void* s) {
  if (s) return (hipStream_t)s;
  DeviceState* d = current_state();
  return d ? d->stream : nullptr;
}

double now_s() {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

// Scratch of stream `s` on the current device, or null.  The caller holds
// g_mutex.
StreamScratch* stream_scratch(hipStream_t s) {
  DeviceState* d = current_state();
  return d ? &d->scratch[s] : nullptr;
}

// Replaces *buf by a buffer of `bytes` after the launches of stream `s` that
// may still use the old one are done.  False on failure.
bool regrow(void** buf, size_t* have, size_t bytes, hipStream_t s) {
  if (*buf) {
    if (hipStreamSynchronize(s) != hipSuccess) return false;
    hipFree(*buf);
    *buf = nullptr;
    *have = 0;
  }
  if (hipMalloc(buf, bytes) != hipSuccess) return false;
  *have = bytes;
  return true;
}

// Grows the split-K workspace of stream `s`.  Returns null on failure.
void* workspace(size_t bytes, hipStream_t s) {
  std::lock_guard<std::mutex> lk(g_mutex);
  StreamScratch* x = stream_scratch(s);
  if (!x) return nullptr;
  if (x->workspace_bytes < bytes && !regrow(&x->workspace, &x->workspace_bytes, bytes, s)) return nullptr;
  return x->workspace;
}

// Grows staging buffer `slot` (0: A, 1: B) of stream `s`.  Returns null on
// failure.
void* staging(int slot, size_t bytes, hipStream_t s) {
  std::lock_guard<std::mutex> lk(g_mutex);
  StreamScratch* x = stream_scratch(s);
  if (!x) return nullptr;
  if (x->staging_bytes[slot] < bytes && !regrow(&x->staging[slot], &x->staging_bytes[slot], bytes, s))
    return nullptr;
  return x->staging[slot];
}

bool zero_fill(void* p, size_t bytes, hipStream_t s);

// Grows the split-K arrival counters (splitk.hpp) of stream `s` to at least
// n entries.  New counters are cleared here, once, on `s` (by a kernel, not
// a memset node, so the call may be captured in a graph); every split-K
// launch leaves them at zero.  The stream's record is only updated once the
// clear is queued.  Returns null on failure.
unsigned* split_counters(size_t n, hipStream_t s) {
  std::lock_guard<std::mutex> lk(g_mutex);
  StreamScratch* x = stream_scratch(s);
  if (!x) return nullptr;
  if (x->counters_len < n) {
    const size_t len = n < 4096 ? 4096 : n;
    size_t bytes = x->counters_len * sizeof(unsigned);
    void* p = x->counters;
    x->counters = nullptr;  // regrow frees the old array first
    x->counters_len = 0;
    if (!regrow(&p, &bytes, len * sizeof(unsigned), s)) return nullptr;
    if (!zero_fill(p, bytes, s)) {
      hipFree(p);
      return nullptr;
    }
    x->counters = (unsigned*)p;
    x->counters_len = len;
  }
  return x->counters;
}

// Where one call takes its scratch memory from (split-K partial sums and
// arrival counters, natural copies of transposed operands).
//  * Growing mode (`fixed` null, xtc_hip_matmul and xtc_hip_conv2d): the
//    per-stream buffers above, allocated or enlarged on demand.
//  * Fixed mode (xtc_hip_matmul_noalloc): consecutive 256-byte aligned pieces
//    of the device's static `scratch` array, at most `cap` bytes in all;
//    nothing is allocated, and the counters are cleared by a kernel on the
//    call's stream before the launch that uses them.
struct Scratch {
  hipStream_t s;
  char* fixed = nullptr;
  size_t cap = 0;
  size_t used = 0;

  void* take(size_t bytes, const char* what) {
    const size_t off = (used + 255) & ~(size_t)255;
    if (off > cap || bytes > cap - off) {
      fail("xtc_hip_matmul_noalloc: %s need %zu bytes at offset %zu of the %zu-byte scratch", what, bytes, off,
           cap);
      return nullptr;
    }
    used = off + bytes;
    return fixed + off;
  }
  float* partials(size_t bytes) {
    if (fixed) return (float*)take(bytes, "split-K partial sums");
    void* p = workspace(bytes, s);
    if (!p) fail("cannot allocate %zu bytes of split-K workspace", bytes);
    return (float*)p;
  }
  unsigned* counters(size_t n) {
    if (fixed) {
      unsigned* p = (unsigned*)take(n * sizeof(unsigned), "split-K counters");
      if (p && !zero_fill(p, n * sizeof(unsigned), s)) {
        fail("cannot clear %zu split-K counters", n);
        return nullptr;
      }
      return p;
    }
    unsigned* p = split_counters(n, s);
    if (!p) fail("cannot allocate %zu split-K counters", n);
    return p;
  }
  void* stage(int slot, size_t bytes) {
    if (fixed) return take(bytes, "transposed operand copies");
    void* p = staging(slot, bytes, s);
    if (!p) fail("cannot allocate %zu bytes of transpose staging", bytes);
    return p;
  }
};

// ------------------------------------------------------------ aux kernels

__global__ void fill_zero_kernel(uint4* p, uint64_t n16, unsigned char* tail, int ntail) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (; i < n16; i += stride) p[i] = make_uint4(0, 0, 0, 0);
  if (blockIdx.x == 0 && (int)threadIdx.x < ntail) tail[threadIdx.x] = 0;
}

int grid_for(uint64_t n, int block);

// Queues a zero fill of `bytes` at 16-byte aligned p on `s`.
bool zero_fill(void* p, size_t bytes, hipStream_t s) {
  const uint64_t n16 = bytes / 16;
  const int ntail = (int)(bytes % 16);
  hipLaunchKernelGGL(fill_zero_kernel, dim3(grid_for(n16 ? n16 : 1, 256)), dim3(256), 0, s, (uint4*)p, n16,
                     (unsigned char*)p + n16 * 16, ntail);
  return hipGetLastError() == hipSuccess;
}

// Release store of `v` to the host-visible completion word (xtc_hip_synchronize):
// stream order puts it after every earlier launch of the stream.
__global__ void stream_done_kernel(unsigned* flag, unsigned v) {
  if (threadIdx.x == 0) __hip_atomic_store(flag, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

__global__ void relu_kernel(const float* __restrict__ x, float* __restrict__ y, uint64_t n,
                            float thr) {
  uint64_t n4 = n / 4;
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  const float4* x4 = reinterpret_cast<const float4*>(x);
  float4* y4 = reinterpret_cast<float4*>(y);
  for (uint64_t j = i; j < n4; j += stride) {
    float4 v = x4[j];
    v.x = v.x < thr ? thr : v.x;
    v.y = v.y < thr ? thr : v.y;
    v.z = v.z < thr ? thr : v.z;
    v.w = v.w < thr ? thr : v.w;
    y4[j] = v;
  }
  for (uint64_t j = n4 * 4 + i; j < n; j += stride) {
    float v = x[j];
    y[j] = v < thr ? thr : v;
  }
}

struct PadDims {
  int ndim;
  int64_t in_shape[8];
  int64_t out_shape[8];
  int64_t before[8];
};

__global__ void pad_kernel(const float* __restrict__ x, float* __restrict__ y, PadDims d,
                           uint64_t total, float value) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (; i < total; i += stride) {
    uint64_t rem = i;
    int64_t src = 0;
    int64_t src_stride = 1;
    bool inside = true;
    for (int k = d.ndim - 1; k >= 0; --k) {
      int64_t o = (int64_t)(rem % (uint64_t)d.out_shape[k]);
      rem /= (uint64_t)d.out_shape[k];
      int64_t s = o - d.before[k];
      inside = inside && s >= 0 && s < d.in_shape[k];
      src += s * src_stride;
      src_stride *= d.in_shape[k];
    }
    float v = value;
    if (inside) v = x[src];
    y[i] = v;
  }
}

// Constant pad with no padding on the innermost dim: the output is rows of
// that dim, each a copy of one input row or all `value`; 16-byte accesses
// (the row length and both pointers are multiples of 4 floats / 16 bytes).
// The row index is decomposed over the outer dims once per 4 elements.
__global__ void pad_rows_kernel(const float4* __restrict__ x, float4* __restrict__ y, PadDims d, uint64_t total4,
                                float value) {
  const int inner4 = (int)(d.out_shape[d.ndim - 1] / 4);
  const float4 pv = make_float4(value, value, value, value);
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total4; i += stride) {
    uint64_t row = i / (uint64_t)inner4;
    const int col = (int)(i - row * (uint64_t)inner4);
    int64_t src = 0, src_stride = 1;
    bool inside = true;
    for (int k = d.ndim - 2; k >= 0; --k) {
      const int64_t o = (int64_t)(row % (uint64_t)d.out_shape[k]);
      row /= (uint64_t)d.out_shape[k];
      const int64_t sk = o - d.before[k];
      inside = inside && sk >= 0 && sk < d.in_shape[k];
      src += sk * src_stride;
      src_stride *= d.in_shape[k];
    }
    y[i] = inside ? x[src * inner4 + col] : pv;
  }
}

// Crop of a row-major tensor (unpad): out[o] = in[o + before] per dim, for
// elements of T (2, 4 or 8 bytes; bf16 tensors move as their 16-bit words).
// d.in_shape is the padded input, d.out_shape the cropped output.
template <typename T>
__global__ void unpad_kernel(const T* __restrict__ x, T* __restrict__ y, PadDims d, uint64_t total) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    uint64_t rem = i;
    int64_t src = 0, src_stride = 1;
    for (int k = d.ndim - 1; k >= 0; --k) {
      const int64_t o = (int64_t)(rem % (uint64_t)d.out_shape[k]);
      rem /= (uint64_t)d.out_shape[k];
      src += (o + d.before[k]) * src_stride;
      src_stride *= d.in_shape[k];
    }
    y[i] = x[src];
  }
}

// Crop that keeps the innermost dim whole: 16-byte copies of its rows (the
// row length in bytes and both pointers are multiples of 16).
__global__ void unpad_rows_kernel(const uint4* __restrict__ x, uint4* __restrict__ y, PadDims d, uint64_t total16,
                                  int64_t inner16) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total16; i += stride) {
    uint64_t row = i / (uint64_t)inner16;
    const int64_t col = (int64_t)(i - row * (uint64_t)inner16);
    int64_t src = 0, src_stride = 1;
    for (int k = d.ndim - 2; k >= 0; --k) {
      const int64_t o = (int64_t)(row % (uint64_t)d.out_shape[k]);
      row /= (uint64_t)d.out_shape[k];
      src += (o + d.before[k]) * src_stride;
      src_stride *= d.in_shape[k];
    }
    y[i] = x[src * inner16 + col];
  }
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  unsigned u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40u);
  unsigned r = ((u >> 16) & 1u) + 0x7fffu;
  return (uint16_t)((u + r) >> 16);
}

// The casts move 8 elements per thread and step (two 16-byte fp32 accesses,
// one 16-byte bf16 access) when both pointers are 16-byte aligned; the last
// n % 8 elements, or all of them otherwise, one at a time.
__global__ void cast_f32_bf16_kernel(const float* x, uint16_t* y, uint64_t n, int vec) {
  const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  uint64_t done = 0;
  if (vec) {
    const uint64_t n8 = n / 8;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    uint4* y8 = reinterpret_cast<uint4*>(y);
    for (uint64_t i = tid; i < n8; i += stride) {
      const float4 a = x4[2 * i], b = x4[2 * i + 1];
      uint4 o;
      o.x = f32_to_bf16_rne(a.x) | ((unsigned)f32_to_bf16_rne(a.y) << 16);
      o.y = f32_to_bf16_rne(a.z) | ((unsigned)f32_to_bf16_rne(a.w) << 16);
      o.z = f32_to_bf16_rne(b.x) | ((unsigned)f32_to_bf16_rne(b.y) << 16);
      o.w = f32_to_bf16_rne(b.z) | ((unsigned)f32_to_bf16_rne(b.w) << 16);
      y8[i] = o;
    }
    done = n8 * 8;
  }
  for (uint64_t i = done + tid; i < n; i += stride) y[i] = f32_to_bf16_rne(x[i]);
}

__global__ void cast_bf16_f32_kernel(const uint16_t* x, float* y, uint64_t n, int vec) {
  const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  uint64_t done = 0;
  if (vec) {
    const uint64_t n8 = n / 8;
    const uint4* x8 = reinterpret_cast<const uint4*>(x);
    float4* y4 = reinterpret_cast<float4*>(y);
    for (uint64_t i = tid; i < n8; i += stride) {
      const uint4 v = x8[i];
      y4[2 * i] = make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                              __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u));
      y4[2 * i + 1] = make_float4(__uint_as_float(v.z << 16), __uint_as_float(v.z & 0xffff0000u),
                                  __uint_as_float(v.w << 16), __uint_as_float(v.w & 0xffff0000u));
    }
    done = n8 * 8;
  }
  for (uint64_t i = done + tid; i < n; i += stride) y[i] = __uint_as_float(((unsigned)x[i]) << 16);
}

template <typename T>
__device__ __forceinline__ float to_f32(T v);
template <>
__device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f32<uint16_t>(uint16_t v) {
  return __uint_as_float(((unsigned)v) << 16);
}

// Reference-shaped fallback for shapes the MFMA tiles cannot take (row
// strides or K not a multiple of the 16-byte vector): one output per thread.
template <typename T>
__global__ void gemm_naive_kernel(const T* A, const T* B, float* C, const float* bias, int M,
                                  int N, int K, int lda, int ldb, int ldc, int relu, float thr) {
  uint64_t total = (uint64_t)M * N;
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    int m = (int)(i / N);
    int n = (int)(i % N);
    float acc = 0.f;
    for (int k = 0; k < K; ++k)
      acc = fmaf(to_f32(A[(size_t)m * lda + k]), to_f32(B[(size_t)k * ldb + n]), acc);
    if (bias) acc += bias[n];
    if (relu && acc < thr) acc = thr;
    C[(size_t)m * ldc + n] = acc;
  }
}

template <typename T>
__global__ void conv_naive_kernel(const T* I, const T* Wt, float* O, const float* bias, int NB,
                                  int H, int W, int C, int F, int R, int S, int sh, int sw,
                                  int ph, int pw, int OH, int OW, float padv, int relu,
                                  float thr) {
  uint64_t total = (uint64_t)NB * OH * OW * F;
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
  int f = (int)(i % F);
  int m = (int)(i / F);
  int ow = m % OW;
  int t = m / OW;
  int oh = t % OH;
  int b = t / OH;
  float acc = 0.f;
  for (int r = 0; r < R; ++r)
    for (int s = 0; s < S; ++s) {
      int ih = oh * sh + r - ph;
      int iw = ow * sw + s - pw;
      bool inb = ih >= 0 && ih < H && iw >= 0 && iw < W;
      for (int c = 0; c < C; ++c) {
        float iv = inb ? to_f32(I[(((size_t)b * H + ih) * W + iw) * C + c]) : padv;
        acc = fmaf(iv, to_f32(Wt[(((size_t)r * S + s) * C + c) * F + f]), acc);
      }
    }
  if (bias) acc += bias[f];
  if (relu && acc < thr) acc = thr;
  O[(size_t)m * F + f] = acc;
  }
}

// fp64 forms of the two fallbacks: fp64 operands, accumulation and output.
__global__ void gemm_naive_f64_kernel(const double* A, const double* B, double* C, const double* bias, int M, int N,
                                      int K, int lda, int ldb, int ldc, int relu, double thr) {
  const uint64_t total = (uint64_t)M * N;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int m = (int)(i / N), n = (int)(i % N);
    double acc = 0.0;
    for (int k = 0; k < K; ++k) acc = fma(A[(size_t)m * lda + k], B[(size_t)k * ldb + n], acc);
    if (bias) acc += bias[n];
    if (relu && acc < thr) acc = thr;
    C[(size_t)m * ldc + n] = acc;
  }
}

__global__ void conv_naive_f64_kernel(const double* I, const double* Wt, double* O, const double* bias, int NB, int H,
                                      int W, int C, int F, int R, int S, int sh, int sw, int ph, int pw, int OH,
                                      int OW, double padv, int relu, double thr) {
  const uint64_t total = (uint64_t)NB * OH * OW * F;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int f = (int)(i % F);
    const int m = (int)(i / F);
    const int ow = m % OW, t = m / OW;
    const int oh = t % OH, b = t / OH;
    double acc = 0.0;
    for (int r = 0; r < R; ++r)
      for (int s = 0; s < S; ++s) {
        const int ih = oh * sh + r - ph, iw = ow * sw + s - pw;
        const bool inb = ih >= 0 && ih < H && iw >= 0 && iw < W;
        for (int c = 0; c < C; ++c) {
          const double iv = inb ? I[(((size_t)b * H + ih) * W + iw) * C + c] : padv;
          acc = fma(iv, Wt[(((size_t)r * S + s) * C + c) * F + f], acc);
        }
      }
    if (bias) acc += bias[f];
    if (relu && acc < thr) acc = thr;
    O[(size_t)m * F + f] = acc;
  }
}

__global__ void relu_f64_kernel(const double* __restrict__ x, double* __restrict__ y, uint64_t n, double thr) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const double v = x[i];
    y[i] = v < thr ? thr : v;
  }
}

__global__ void pad_f64_kernel(const double* __restrict__ x, double* __restrict__ y, PadDims d, uint64_t total,
                               double value) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    uint64_t rem = i;
    int64_t src = 0, src_stride = 1;
    bool inside = true;
    for (int k = d.ndim - 1; k >= 0; --k) {
      const int64_t o = (int64_t)(rem % (uint64_t)d.out_shape[k]);
      rem /= (uint64_t)d.out_shape[k];
      const int64_t sk = o - d.before[k];
      inside = inside && sk >= 0 && sk < d.in_shape[k];
      src += sk * src_stride;
      src_stride *= d.in_shape[k];
    }
    y[i] = inside ? x[src] : value;
  }
}

// dst[r][c] = src[r][c] for c < C, 0 for C <= c < Cp, over `rows` rows of C
// (src) and Cp (dst) elements: the channel padding that gives a conv input
// (rows = N*H*W pixels) or its RSCF weights (rows = R*S taps, C*F and Cp*F
// elements) 16-byte channel vectors.  HBM-bound copy.
template <typename T>
__global__ void __launch_bounds__(256) pad_channels_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                           uint64_t rows, uint32_t C, uint32_t Cp) {
  const uint64_t total = rows * Cp;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const uint64_t r = i / Cp;
    const uint32_t c = (uint32_t)(i - r * Cp);
    dst[i] = c < C ? src[r * C + c] : T(0);
  }
}

float bf16_round_host(float v) {
  unsigned u;
  memcpy(&u, &v, 4);
  unsigned r = ((u >> 16) & 1u) + 0x7fffu;
  u = ((u + r) >> 16) << 16;
  float o;
  memcpy(&o, &u, 4);
  return o;
}

int grid_for(uint64_t n, int block) {
  uint64_t g = (n + block - 1) / block;
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return (int)g;
}

// Tiles of the direct conv kernel (conv_direct.hpp): BM output pixels as a
// TH x TW block, 64 filters, slabs of 16 channels per MFMA k-group, WGM x WGN
// waves, and the LDS of the input halo.  8x8 (2x2 waves) shares its tile
// with a generic implicit-GEMM instance, which runs the shapes the direct
// kernel does not take; 8x14 (1x4 waves, 224 equal blocks for 8x56x56
// outputs) and 7x14 (1x4 waves, 6 whole 16-pixel tiles and 2 pixels on
// 4x4x1 MFMAs; 256 blocks for 8x56x56, one per CU) exist only here.  8x8
// streams its weights through LDS stages, the 1x4-wave blocks through a
// register ring of 3 taps (the faster path for each in one process).
typedef void (*DirectConvLaunch)(const DirectConvArgs&, dim3, hipStream_t);
template <int TH, int TW, int WM, int WN, int HALO_BYTES, int WRING>
void launch_conv_direct(const DirectConvArgs& a, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((conv_direct_f32<TH, TW, WM, WN, HALO_BYTES, WRING>), grid, dim3(dconv::NT), 0, s, a);
}
template <int TH, int TW, int WRING>
void launch_conv_direct_3x3s1(const DirectConvArgs& a, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((conv_direct_f32_3x3s1<TH, TW, WRING>), grid, dim3(dconv::NT), 0, s, a);
}
struct DirectConvTile {
  xtc_hip_tile tile;
  int th, tw, halo_bytes;
  int wring;  // 0: weights through dconv::STAGES LDS stages, else register ring depth
  DirectConvLaunch launch;
  // the same blocks and ring for a 3x3 window at stride 1, its offsets fixed
  // at compile time (bit-identical to `launch`); null where there is none
  DirectConvLaunch launch_3x3s1;
  int lds_bytes() const { return halo_bytes + (wring ? 0 : dconv::STAGES * dconv::W_STAGE); }
  int depth() const { return wring ? wring : dconv::STAGES; }
};
const DirectConvTile kDirectConv[] = {
    {{64, 64, 16, 2, 2}, 8, 8, 32 * 1024, 0, &launch_conv_direct<8, 8, 2, 2, 32 * 1024, 0>, nullptr},
    {{112, 64, 16, 1, 4}, 8, 14, 48 * 1024, 3, &launch_conv_direct<8, 14, 1, 4, 48 * 1024, 3>,
     &launch_conv_direct_3x3s1<8, 14, 3>},
    {{98, 64, 16, 1, 4}, 7, 14, 48 * 1024, 3, &launch_conv_direct<7, 14, 1, 4, 48 * 1024, 3>,
     &launch_conv_direct_3x3s1<7, 14, 3>},
};

bool same_tile(const xtc_hip_tile& a, const xtc_hip_tile& b) {
  return a.bm == b.bm && a.bn == b.bn && a.bk == b.bk && a.wgm == b.wgm && a.wgn == b.wgn;
}

const DirectConvTile* direct_conv_tile(const xtc_hip_tile& t) {
  for (const DirectConvTile& d : kDirectConv)
    if (same_tile(d.tile, t)) return &d;
  return nullptr;
}

// Registry entries of the tiles only the direct conv kernel implements
// (launch null: no implicit-GEMM instance behind them).
const GemmEntry* direct_only_entries(int* n) {
  static const std::vector<GemmEntry> v = [] {
    std::vector<GemmEntry> out;
    int nreg = 0;
    const GemmEntry* e = gemm_registry(&nreg);
    for (const DirectConvTile& d : kDirectConv) {
      bool generic = false;
      for (int i = 0; i < nreg; ++i)
        generic = generic || (e[i].dtype == XTC_HIP_F32 && e[i].conv == 1 &&
                              same_tile(xtc_hip_tile{e[i].bm, e[i].bn, e[i].bk, e[i].wgm, e[i].wgn}, d.tile));
      if (!generic)
        out.push_back(GemmEntry{XTC_HIP_F32, 1, d.tile.bm, d.tile.bn, d.tile.bk, d.tile.wgm, d.tile.wgn,
                                d.lds_bytes(), dconv::NT, nullptr});
    }
    return out;
  }();
  *n = (int)v.size();
  return v.data();
}

// fp64 tiles (gemm_f64.hpp): 16-deep slabs, WGM x WGN waves of 16x16 fp64
// MFMA tiles, for matmul and the implicit-GEMM conv loader alike.
typedef void (*GemmLaunch64)(const GemmArgs64&, dim3, hipStream_t);
template <int BM, int BN, int WGM, int WGN, bool CONV>
void launch_gemm_f64(const GemmArgs64& a, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((gemm_f64_kernel<BM, BN, WGM, WGN, CONV>), grid, dim3(WGM * WGN * 64), 0, s, a);
}
struct F64Tile {
  int conv;
  xtc_hip_tile tile;
  GemmLaunch64 launch;
  int lds_bytes() const { return 2 * (tile.bm * (16 + 2) + 16 * (tile.bn + 8)) * 8; }
};
#define XTC_F64_TILES(CONV)                                                      \
  {CONV, {32, 32, 16, 1, 1}, &launch_gemm_f64<32, 32, 1, 1, CONV>},              \
      {CONV, {64, 32, 16, 2, 1}, &launch_gemm_f64<64, 32, 2, 1, CONV>},          \
      {CONV, {32, 64, 16, 1, 2}, &launch_gemm_f64<32, 64, 1, 2, CONV>},          \
      {CONV, {64, 64, 16, 2, 2}, &launch_gemm_f64<64, 64, 2, 2, CONV>},          \
      {CONV, {128, 64, 16, 2, 2}, &launch_gemm_f64<128, 64, 2, 2, CONV>},        \
      {CONV, {64, 128, 16, 2, 2}, &launch_gemm_f64<64, 128, 2, 2, CONV>},        \
      {CONV, {128, 128, 16, 2, 2}, &launch_gemm_f64<128, 128, 2, 2, CONV>}
const F64Tile kF64Tiles[] = {XTC_F64_TILES(false), XTC_F64_TILES(true)};
#undef XTC_F64_TILES

const F64Tile* f64_tile(int conv, const xtc_hip_tile& t) {
  for (const F64Tile& f : kF64Tiles)
    if (f.conv == conv && same_tile(f.tile, t)) return &f;
  return nullptr;
}

// Registry entries of the fp64 tiles, for listing and lookup (their launch
// goes through f64_tile: the kernel takes fp64 arguments).
const GemmEntry* f64_entries(int* n) {
  static const std::vector<GemmEntry> v = [] {
    std::vector<GemmEntry> out;
    for (const F64Tile& f : kF64Tiles)
      out.push_back(GemmEntry{XTC_HIP_F64, f.conv, f.tile.bm, f.tile.bn, f.tile.bk, f.tile.wgm, f.tile.wgn,
                              f.lds_bytes(), f.tile.wgm * f.tile.wgn * 64, nullptr, nullptr});
    return out;
  }();
  *n = (int)v.size();
  return v.data();
}

const GemmEntry* find_entry(int dtype, int conv, const xtc_hip_tile& t) {
  int n = 0;
  const GemmEntry* e = gemm_registry(&n);
  for (int i = 0; i < n; ++i) {
    if (e[i].dtype == dtype && e[i].conv == conv && e[i].bm == t.bm && e[i].bn == t.bn &&
        e[i].bk == t.bk && e[i].wgm == t.wgm && e[i].wgn == t.wgn)
      return &e[i];
  }
  const GemmEntry* x = direct_only_entries(&n);
  for (int i = 0; i < n; ++i)
    if (x[i].dtype == dtype && x[i].conv == conv && same_tile(xtc_hip_tile{x[i].bm, x[i].bn, x[i].bk, x[i].wgm, x[i].wgn}, t))
      return &x[i];
  x = f64_entries(&n);
  for (int i = 0; i < n; ++i)
    if (x[i].dtype == dtype && x[i].conv == conv && same_tile(xtc_hip_tile{x[i].bm, x[i].bn, x[i].bk, x[i].wgm, x[i].wgn}, t))
      return &x[i];
  return nullptr;
}

bool has_entry(int dtype, int conv, int bm, int bn, int bk, int wgm, int wgn) {
  xtc_hip_tile t{bm, bn, bk, wgm, wgn};
  return find_entry(dtype, conv, t) != nullptr;
}

// Default tiles.  Chosen by shape class; tuned on MI355X with loop-explore.
void default_tile(int dtype, int conv, int M, int N, int K, xtc_hip_tile* t, int* split_k) {
  *split_k = 1;
  if (dtype == XTC_HIP_F64) {
    // fp64: the largest tile that still gives every CU a workgroup, then
    // split K (ragged splits allowed, at least 4 slabs each) until about
    // 512 workgroups
    const xtc_hip_tile cand[] = {
        {128, 128, 16, 2, 2}, {128, 64, 16, 2, 2}, {64, 64, 16, 2, 2}, {64, 32, 16, 2, 1}, {32, 32, 16, 1, 1}};
    *t = cand[4];
    for (const xtc_hip_tile& c : cand) {
      if (N <= 32 && c.bn > 32) continue;  // N-narrow: no half-empty 64-wide tiles
      if ((int64_t)((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn) >= 256) {
        *t = c;
        break;
      }
    }
    const int64_t tiles = (int64_t)((M + t->bm - 1) / t->bm) * ((N + t->bn - 1) / t->bn);
    int s = 1;
    while (s < 16 && tiles * s * 2 <= 512 && K / (2 * s) >= 64) s *= 2;
    *split_k = s;
    return;
  }
  auto pick = [&](int bm, int bn, int bk, int wgm, int wgn) {
    if (has_entry(dtype, conv, bm, bn, bk, wgm, wgn)) {
      *t = xtc_hip_tile{bm, bn, bk, wgm, wgn};
      return true;
    }
    return false;
  };
  const bool f32 = dtype == XTC_HIP_F32;
  const int bk = f32 ? 32 : 64;
  // Fewer 64x64 tiles than the chip has CUs (256; 512 for a matmul) over a
  // deep K: split K, completed inside the launch, by powers of two up to
  // 1024 workgroups and 32 splits, with at least 4 slabs per split; from
  // 128 tiles on, only over a K of at least 512.  Measured on MI355X over
  // the op-name layers: ResNet18_12 148 -> 24 us, MobilNet_09 314 -> 37 us,
  // MobilNet_02 (196 tiles, K 576) 34 -> 26 us, Llama3_QK 242 -> 89 us,
  // 512^3 fp32 19 -> 13 us; Yolo9000_09 (146 tiles, K 256) lost 7-12 % at
  // split 2 or 4 against its direct conv, and shapes with more tiles gain
  // little or lose (C4's 392 tiles keep the direct conv).
  // Convs and fp32 matmuls also split into unequal parts (the last split
  // shorter) up to 8; a conv's K = R*S*C rarely splits into whole slabs
  // (bf16 AlexNet_02 3x3x192,
  // 27 64-deep slabs: 35.4 us at split 1 -> 15.0 us at split 4; AlexNet_03
  // 36.1 -> 16.2 us at 8; ResNet18_02 15.2 -> 12.8 us at 2; fp32 AlexNet_02
  // 26.7 us at split 4 -> 18.4 us at 8; fp32 Polybench_large, 37.5 slabs
  // of 32: 56.2 -> 42.2 us).  Beyond 8 the unequal splits gain nothing
  // (bf16 MobilNet_07, K 4608: 18.6 us at 8, 19.2 at 16); bf16 matmuls
  // keep whole slabs (Polybench_large: 22.4 us unsplit, 28.7 at split 2).
  // fp32 matmuls split up to 2304 workgroups, 9 per CU, and 16 splits
  // (Gemma27B_QK 256x4608x8192, 288 tiles: 245 us at split 2, 185 us at
  // split 8; 768x768x4096: 67 -> 57 us at split 16; Polybench_large 43 ->
  // 42 us; 256x1024x4096: 30.4 us at split 16, 38.1 us at 32).
  const bool ragged = conv || f32;
  const int64_t cap = f32 && !conv ? 2304 : 1024;
  const int smax = f32 && !conv ? 16 : 32;
  auto fill = [&](int64_t below) {
    const int64_t tiles = (int64_t)((M + t->bm - 1) / t->bm) * ((N + t->bn - 1) / t->bn);
    if (tiles >= below || (tiles >= 128 && K < 512)) return;
    int s = 1;
    while (s < smax && tiles * s * 2 <= cap && K / (2 * s) >= 4 * t->bk &&
           ((K % (2 * s) == 0 && (K / (2 * s)) % t->bk == 0) || (ragged && 2 * s <= 8)))
      s *= 2;
    *split_k = s;
  };
  if (conv && f32 && N % 64 == 0 && K % 64 == 0 && pick(64, 64, 16, 2, 2)) {
    fill(256);
    return;
  }
  // other fp32 convs: 64x64x16 when its fill rule splits K (SqueezeNet_13
  // 3x3x48, 36 tiles: 23.0 us on 64x64x32 -> 12.2 us at split 4;
  // SqueezeNet_08/14 1x1, 12 tiles: 11.4/13.9 -> 9.8/11.1 us), else the
  // 64x64x32 tile below, which wins unsplit (Yolo9000_02: 41.8 us against
  // 48.2 on 64x64x16)
  if (conv && f32 && pick(64, 64, 16, 2, 2)) {
    fill(256);
    if (*split_k > 1) return;
  }
  if (M <= 16) {
    // skinny bf16 with aligned N and K: the B-streaming kernel
    // (gemm_bf16_skinny.hpp) behind tile 16x128x64, 1x4 waves, 1024-deep splits
    if (!f32 && N % 128 == 0 && (K % 1024 == 0 || K % 512 == 0) && pick(16, 128, 64, 1, 4)) {
      *split_k = K % 1024 == 0 ? K / 1024 : K / 512;
      return;
    }
    // skinny: stream B once; split K until the grid fills the chip
    int bn = 128;
    if (pick(16, bn, bk, 1, 4) || pick(16, 64, bk, 1, 4)) {
      int tiles = (N + t->bn - 1) / t->bn;
      int s = 1;
      while (tiles * s < 1024 && K / (s * 2) >= 4 * bk) s *= 2;
      *split_k = s;
      return;
    }
  }
  if (!conv && N <= 64 && pick(64, 32, bk, 2, 2)) {
    // N-narrow: 64x32 tiles leave few workgroups, so split K until about
    // 1024 of them stream A (at M = 8192, N = 16, K = 8192: split 8, 4.4x
    // faster than one 64x64 tile per 64 rows)
    const int64_t tiles = (int64_t)((M + 63) / 64) * ((N + 31) / 32);
    int s = 1;
    while (tiles * s < 1024 && K % (2 * s) == 0 && (K / (2 * s)) % bk == 0 && K / (2 * s) >= 8 * bk) s *= 2;
    *split_k = s;
    return;
  }
  if (!f32 && !conv && M >= 128 && N >= 128) {
    // bf16 matmuls, measured on MI355X over the op-name layers:
    //  * aligned shapes with at least 128 256x256 tiles take the ping-pong
    //    LDS-DMA kernel behind 256x256x32 (Gemma7B_FC 3072x24576x3072:
    //    797 -> 406 us against 128x128x64; Gemma7B_In, K 256: 32.8 -> 19.3 us);
    //  * the rest take 128x128x64 (Polybench_extralarge 2000x2304x2600:
    //    68 us, against 98 us at 64x64x64 and 274 us at 256x256x64), with
    //    fewer than 256 tiles split K up to 512 workgroups, at least 4 slabs
    //    per split (Gemma27B_QKV 256x8192x4608: 85 -> 43 us at split 4),
    //    when that makes at least 256 workgroups; smaller grids keep the
    //    64x64 tiles below (Polybench_large 1000x1104x1200, whose K splits
    //    into no whole slabs: 23 us at 64x64x64, 34 us on 72 128x128 tiles)
    if (M % 256 == 0 && N % 256 == 0 && K % 32 == 0 && (int64_t)(M / 256) * (N / 256) >= 128 &&
        pick(256, 256, 32, 2, 4))
      return;
    const int64_t tiles = (int64_t)((M + 127) / 128) * ((N + 127) / 128);
    int s = 1;
    while (tiles < 256 && s < 32 && tiles * s * 2 <= 512 && K % (2 * s) == 0 && (K / (2 * s)) % 64 == 0 &&
           K / (2 * s) >= 4 * 64)
      s *= 2;
    if (tiles * s >= 256 && pick(128, 128, 64, 2, 2)) {
      *split_k = s;
      return;
    }
  }
  // aligned fp32 shapes with fewer than 256 128x128 tiles (the M = 128-256
  // projections): the LDS-DMA fp32 kernel behind 128x128x32, 2x4 waves,
  // split K by powers of two, at least 1024 deep each, to between 224 and
  // 256 workgroups, one wave over the chip (Gemma27B_QKV 256x8192x4608, 128 tiles: 201 -> 154 us at
  // split 2; Gemma9B_QK 256x3584x8192, 56 tiles: 162 -> 138 us at split 4;
  // Llama3_QKV 86 -> 76 us).  Past 256 workgroups the second wave costs more
  // than the split gains (Gemma27B_QK, 72 tiles: 261 us at split 2, 264 us
  // at split 4), and 192 leave too many CUs idle (Gemma7B_QK, 48 tiles:
  // 128 -> 138 us), so those keep the 64x64 split-K rule below, as do
  // shallow splits (256x1024x4096 at split 16, 256 deep: 36.7 us against
  // 30.1 us on 64x64 tiles at split 8).
  if (f32 && !conv && M % 128 == 0 && N % 128 == 0 && K % 32 == 0) {
    const int64_t tiles = (int64_t)(M / 128) * (N / 128);
    int s = 1;
    while (s < 32 && tiles * s * 2 <= 256 && K % (32 * s * 2) == 0 && K / (s * 2) >= 1024) s *= 2;
    if (tiles < 256 && s > 1 && tiles * s >= 224 && pick(128, 128, 32, 2, 4)) {
      *split_k = s;
      return;
    }
  }
  // large aligned fp32 shapes with at least one 256x128 tile per CU: the
  // LDS-DMA fp32 kernel behind this tile
  if (f32 && !conv && M % 256 == 0 && N % 128 == 0 && K % 32 == 0 && (int64_t)(M / 256) * (N / 128) >= 256 &&
      pick(256, 128, 32, 4, 2))
    return;
  if (M >= 2048 && N >= 2048) {
    if (pick(128, 128, bk, 2, 2)) return;
  }
  if (!f32 && conv && N >= 96 && (int64_t)((M + 127) / 128) * ((N + 127) / 128) >= 256 && pick(128, 128, 64, 2, 2))
    // bf16 convs with at least 256 128x128 tiles over 96 filters or more
    // (measured on MI355X: Yolo9000_23 1x1, 289 x 28272 x 1024: 86.7 -> 78.3
    // us against 64x64x64; SqueezeNet_00 7x7/2 over 96 filters: 39.2 -> 36.2
    // us; narrower convs lose with the half-empty 128-wide tile)
    return;
  if (pick(64, 64, bk, 2, 2)) {
    // fp32 matmuls over a K of 2048 or more split up to 1152 tiles in two
    // (Polybench_extralarge 2000x2304x2600, 1152 tiles: 263 -> 232 us;
    // 256x8192xK Gemma projections, 512 tiles: 8-10 % faster at split 2)
    fill(conv ? 256 : f32 && K >= 2048 ? cap / 2 + 1 : 512);
    // bf16 convs that split K four ways or more and still make at least
    // 256 workgroups of 128x64 tiles: the same split on those tiles
    // (Yolo9000_12 3x3, 1156 x 512 x 2304, split 4, 320 workgroups: 31.3
    // -> 26.4 us; Yolo9000_18, 289 x 1024 x 4608, split 8, 384: 31.5 ->
    // 27.3 us).  Smaller grids lose (MobilNet_05, 112 workgroups: 18.1 ->
    // 24.4 us; Yolo9000_19, 96: 12.4 -> 16.6 us), and so do the mostly
    // empty 128-row tiles under 128 pixels (ResNet18_12: 17.6 -> 20.2 us)
    if (!f32 && conv && M >= 128 && *split_k >= 4 &&
        (int64_t)((M + 127) / 128) * ((N + 63) / 64) * *split_k >= 256)
      pick(128, 64, 64, 2, 2);
    return;
  }
  int n = 0;
  const GemmEntry* e = gemm_registry(&n);
  for (int i = 0; i < n; ++i)
    if (e[i].dtype == dtype && e[i].conv == conv) {
      *t = xtc_hip_tile{e[i].bm, e[i].bn, e[i].bk, e[i].wgm, e[i].wgn};
      return;
    }
  *t = xtc_hip_tile{0, 0, 0, 0, 0};
}

// K per split (a multiple of the slab depth bk) for `split_k` requested
// splits of K.
int split_depth(int K, int split_k, int bk) {
  if (split_k < 1) split_k = 1;
  const int kps = (K + split_k - 1) / split_k;
  return (kps + bk - 1) / bk * bk;
}

// Splits a launch runs for K, split_k and slab depth bk.
int effective_splits(int K, int split_k, int bk) {
  const int kps = split_depth(K, split_k, bk);
  return (K + kps - 1) / kps;
}

// Ring instances of the generic template (three register sets of loads in
// flight, pipeline depth 4) for entry e at `splits` splits: 0 none, 1 one
// exists and depth 2 is the default, 2 one exists and is the default.  Split
// K makes each workgroup's K walk short and its load latency exposed: the
// ring is then 10-20 % faster (ResNet18_09 conv at split 16: 20.1 -> 17.6
// us, 512^3 fp32 at split 4: 12.8 -> 11.0 us); with one split it gains
// nothing or loses up to 6 %.
int generic_ring(const GemmEntry* e, int splits) {
  if (!e || !e->launch_ring) return 0;
  return splits > 1 ? 2 : 1;
}

// `stages` 0 (default), 2 or 4 (the ring instance, when e has one).
int launch_gemm_common(GemmArgs& a, const GemmEntry* e, int split_k, int stages, int group_m, int xcd_remap,
                       Scratch& x) {
  const hipStream_t s = x.s;
  a.tiles_m = (a.M + e->bm - 1) / e->bm;
  a.tiles_n = (a.N + e->bn - 1) / e->bn;
  a.group_m = group_m > 0 ? group_m : 8;
  a.xcd_remap = xcd_remap;
  const int kps = split_depth(a.K, split_k, e->bk);
  const int splits = (a.K + kps - 1) / kps;
  a.k_per_split = kps;
  a.partial = nullptr;
  a.counters = nullptr;
  if (splits > 1) {
    size_t bytes = (size_t)splits * a.M * a.N * sizeof(float);
    a.partial = x.partials(bytes);
    if (!a.partial) return 1;
    a.counters = x.counters((size_t)a.tiles_m * a.tiles_n);
    if (!a.counters) return 1;
  }
  dim3 grid((unsigned)(a.tiles_m * a.tiles_n), 1, (unsigned)splits);
  const bool ring = e->launch_ring && (stages == 4 || (stages == 0 && splits > 1));
  (ring ? e->launch_ring : e->launch)(a, grid, s);
  HIP_TRY(hipGetLastError());
  return 0;
}

// Split-K set-up and grid of an fp64 launch, as launch_gemm_common for the
// fp32 / bf16 template (fp64 partial planes).
int launch_f64_common(GemmArgs64& a, const F64Tile* f, int split_k, int group_m, int xcd_remap, Scratch& x) {
  a.tiles_m = (a.M + f->tile.bm - 1) / f->tile.bm;
  a.tiles_n = (a.N + f->tile.bn - 1) / f->tile.bn;
  a.group_m = group_m > 0 ? group_m : 8;
  a.xcd_remap = xcd_remap;
  const int kps = split_depth(a.K, split_k, f->tile.bk);
  const int splits = (a.K + kps - 1) / kps;
  a.k_per_split = kps;
  a.partial = nullptr;
  a.counters = nullptr;
  if (splits > 1) {
    a.partial = (double*)x.partials((size_t)splits * a.M * a.N * sizeof(double));
    if (!a.partial) return 1;
    a.counters = x.counters((size_t)a.tiles_m * a.tiles_n);
    if (!a.counters) return 1;
  }
  f->launch(a, dim3((unsigned)(a.tiles_m * a.tiles_n), 1, (unsigned)splits), x.s);
  HIP_TRY(hipGetLastError());
  return 0;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// The LDS-DMA bf16 kernels implement the 256x256x64 tiles with 2x4 and 4x2
// waves (gemm_bf16_lds.hpp) and the 256x256x32 tile with 2x4 waves
// (gemm_bf16_pingpong.hpp) when the shape needs no bounds checks, for B
// row-major (bt = false, ldb >= N) or stored transposed (bt = true, ldb >= K).
// The ping-pong kernel also splits K, into equal ranges of whole slabs.
// XTC_HIP_GENERIC_GEMM=1 forces the generic template (for A/B comparisons).
bool lds_dma_gemm_applies(const xtc_hip_matmul_desc& d, const xtc_hip_tile& t, int split_k, int lda,
                          int ldb, int ldc, const void* A, const void* B, const void* C,
                          const void* bias, bool bt) {
  static const bool disabled = [] {
    const char* v = getenv("XTC_HIP_GENERIC_GEMM");
    return v && v[0] == '1';
  }();
  const int splits = split_k < 1 ? 1 : split_k;
  if (disabled || d.dtype != XTC_HIP_BF16 || (splits > 1 && t.bk != 32)) return false;
  if (t.bm != 256 || t.bn != 256) return false;
  // bk 64: gemm_bf16_lds.hpp with 2x4 or 4x2 waves; bk 32: gemm_bf16_pingpong.hpp, 2x4
  if (t.bk == 64) {
    if (!((t.wgm == 2 && t.wgn == 4) || (t.wgm == 4 && t.wgn == 2))) return false;
  } else if (t.bk != 32 || t.wgm != 2 || t.wgn != 4) {
    return false;
  }
  if (d.M % 256 || d.N % 256 || d.K % (t.bk * splits)) return false;
  if (lda % 8 || ldb % 8 || ldc % 4) return false;
  if (!aligned16(A) || !aligned16(B) || !aligned16(C) || (bias && !aligned16(bias))) return false;
  // element offsets of one tile row/column range must fit in 32 bits
  if ((int64_t)256 * lda > INT32_MAX || (int64_t)(bt ? 256 : 64) * ldb > INT32_MAX) return false;
  return true;
}

// The skinny bf16 kernel (gemm_bf16_skinny.hpp) implements tile 16x128x64
// with 1x4 waves for M <= 16 when each split covers 512 or 1024 of K and the
// shape needs no bounds checks.
bool skinny_gemm_applies(const xtc_hip_matmul_desc& d, const xtc_hip_tile& t, int split_k, int lda,
                         int ldb, int ldc, const void* A, const void* B, const void* C,
                         const void* bias) {
  static const bool disabled = [] {
    const char* v = getenv("XTC_HIP_GENERIC_GEMM");
    return v && v[0] == '1';
  }();
  if (disabled || d.dtype != XTC_HIP_BF16) return false;
  if (t.bm != 16 || t.bn != 128 || t.bk != 64 || t.wgm != 1 || t.wgn != 4) return false;
  const int splits = split_k < 1 ? 1 : split_k;
  if (d.M > 16 || d.N % 128 || d.K % splits) return false;
  const int kc = d.K / splits;
  if (kc != 512 && kc != 1024) return false;
  if (lda % 8 || ldb % 8 || ldc % 4) return false;
  if (!aligned16(A) || !aligned16(B) || !aligned16(C) || (bias && !aligned16(bias))) return false;
  if ((int64_t)64 * ldb > INT32_MAX) return false;
  return true;
}

// The LDS-DMA fp32 kernel (gemm_f32_lds.hpp) implements the 128x256x32 (2x4
// waves), 256x128x32 (4x2 waves) and 128x128x32 (2x4 waves) fp32 tiles,
// split-K included, when the
// shape needs no bounds checks: one workgroup of 8 waves per CU.
bool f32_lds_gemm_applies(const xtc_hip_matmul_desc& d, const xtc_hip_tile& t, int split_k, int lda,
                          int ldb, int ldc, const void* A, const void* B, const void* C,
                          const void* bias) {
  static const bool disabled = [] {
    const char* v = getenv("XTC_HIP_GENERIC_GEMM");
    return v && v[0] == '1';
  }();
  if (disabled || d.dtype != XTC_HIP_F32) return false;
  const bool t1 = t.bm == 128 && t.bn == 256 && t.wgm == 2 && t.wgn == 4;
  const bool t2 = t.bm == 256 && t.bn == 128 && t.wgm == 4 && t.wgn == 2;
  const bool t3 = t.bm == 128 && t.bn == 128 && t.wgm == 2 && t.wgn == 4;
  // BK 32 (3 stages) for all three tiles; BK 16 (deeper stages) for the two
  // 256-wide ones
  if (!(t1 || t2 || t3) || !(t.bk == 32 || (t.bk == 16 && !t3))) return false;
  const int splits = split_k < 1 ? 1 : split_k;
  if (d.M % t.bm || d.N % t.bn || d.K % (t.bk * splits)) return false;
  if (lda % 4 || ldb % 4 || ldc % 4) return false;
  if (!aligned16(A) || !aligned16(B) || !aligned16(C) || (bias && !aligned16(bias))) return false;
  // element offsets of one tile's rows must fit in 32 bits
  if ((int64_t)t.bm * lda > INT32_MAX || (int64_t)32 * ldb > INT32_MAX) return false;
  return true;
}

template <int BM, int BN, int BK, int WGM, int WGN, int STAGES>
void launch_f32_lds(const GemmArgs& a, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((gemm_f32_lds<BM, BN, BK, WGM, WGN, STAGES>), grid, dim3(512), 0, s, a);
}

// Compiled pipeline depths (LDS stages) of the LDS-DMA fp32 kernel, per tile;
// the first entry of a tile is its default.  BK 16 stages are 24 KB (up to
// 6 fit), BK 32 stages 48 KB for the 256-wide tiles (up to 3) and 32 KB for
// 128x128 (up to 4: five would leave no room for the split-K flag).  Against 3 stages of BK 32, 4-5 stages of BK 16
// measured 2-4 % faster on one box and 1-1.5 % slower on another.
struct F32LdsVariant {
  int bm, bn, bk, wgm, wgn, stages;
  GemmLaunch launch;
};
const F32LdsVariant kF32Lds[] = {
    {256, 128, 16, 4, 2, 4, &launch_f32_lds<256, 128, 16, 4, 2, 4>},
    {256, 128, 16, 4, 2, 3, &launch_f32_lds<256, 128, 16, 4, 2, 3>},
    {256, 128, 16, 4, 2, 5, &launch_f32_lds<256, 128, 16, 4, 2, 5>},
    {256, 128, 16, 4, 2, 6, &launch_f32_lds<256, 128, 16, 4, 2, 6>},
    {128, 256, 16, 2, 4, 5, &launch_f32_lds<128, 256, 16, 2, 4, 5>},
    {128, 256, 16, 2, 4, 3, &launch_f32_lds<128, 256, 16, 2, 4, 3>},
    {128, 256, 16, 2, 4, 4, &launch_f32_lds<128, 256, 16, 2, 4, 4>},
    {128, 256, 16, 2, 4, 6, &launch_f32_lds<128, 256, 16, 2, 4, 6>},
    {256, 128, 32, 4, 2, 3, &launch_f32_lds<256, 128, 32, 4, 2, 3>},
    {256, 128, 32, 4, 2, 2, &launch_f32_lds<256, 128, 32, 4, 2, 2>},
    {128, 256, 32, 2, 4, 3, &launch_f32_lds<128, 256, 32, 2, 4, 3>},
    {128, 256, 32, 2, 4, 2, &launch_f32_lds<128, 256, 32, 2, 4, 2>},
    {128, 128, 32, 2, 4, 3, &launch_f32_lds<128, 128, 32, 2, 4, 3>},
    {128, 128, 32, 2, 4, 2, &launch_f32_lds<128, 128, 32, 2, 4, 2>},
    {128, 128, 32, 2, 4, 4, &launch_f32_lds<128, 128, 32, 2, 4, 4>},
};

// The variant of tile t with `stages` (0: the tile's default), or null.
const F32LdsVariant* f32_lds_variant(const xtc_hip_tile& t, int stages) {
  for (const F32LdsVariant& v : kF32Lds)
    if (v.bm == t.bm && v.bn == t.bn && v.bk == t.bk && v.wgm == t.wgm && v.wgn == t.wgn &&
        (stages == 0 || v.stages == stages))
      return &v;
  return nullptr;
}

// The split-wave fp32 kernel (gemm_f32_splitwave.hpp) implements the
// one-wave 32x32x16 tile with split-K 2..8 when the shape is aligned: the
// splits of a tile are the waves of one workgroup instead of workgroups of
// the grid (same partial sums, same summation order).
bool splitwave_gemm_applies(const xtc_hip_matmul_desc& d, const xtc_hip_tile& t, int split_k, int lda,
                            const void* A) {
  static const bool disabled = [] {
    const char* v = getenv("XTC_HIP_GENERIC_GEMM");
    return v && v[0] == '1';
  }();
  if (disabled || d.dtype != XTC_HIP_F32) return false;
  if (t.bm != 32 || t.bn != 32 || t.bk != 16 || t.wgm != 1 || t.wgn != 1) return false;
  if (split_k < 2 || split_k > 8) return false;
  if (d.M % 32 || d.N % 32 || d.K % (16 * split_k)) return false;
  if (lda % 4 || !aligned16(A)) return false;
  return true;
}

// Pipeline depths (register ring chunks) of the split-wave kernel, default
// first.
constexpr int kSplitWaveDepths[] = {4, 2, 8};

template <int S>
void launch_splitwave_s(int depth, dim3 grid, const GemmArgs& a, hipStream_t s) {
  if (depth == 2)
    hipLaunchKernelGGL((gemm_f32_splitwave<S, 2>), grid, dim3(S * 64), 0, s, a);
  else if (depth == 4)
    hipLaunchKernelGGL((gemm_f32_splitwave<S, 4>), grid, dim3(S * 64), 0, s, a);
  else
    hipLaunchKernelGGL((gemm_f32_splitwave<S, 8>), grid, dim3(S * 64), 0, s, a);
}

int launch_splitwave_gemm(const xtc_hip_matmul_desc& d, int split_k, int stages, int lda, int ldb, int ldc,
                          const void* A, const void* B, float* C, const float* bias, hipStream_t s) {
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  a.A = A;
  a.B = B;
  a.C = C;
  a.bias = bias;
  a.M = d.M;
  a.N = d.N;
  a.K = d.K;
  a.lda = lda;
  a.ldb = ldb;
  a.ldc = ldc;
  a.relu = d.relu;
  a.relu_threshold = d.relu_threshold;
  a.tiles_m = d.M / 32;
  a.tiles_n = d.N / 32;
  a.group_m = d.group_m > 0 ? d.group_m : 8;
  a.xcd_remap = d.xcd_remap;
  a.k_per_split = d.K / split_k;
  dim3 grid((unsigned)(a.tiles_m * a.tiles_n));
  const int depth = stages > 0 ? stages : kSplitWaveDepths[0];
  switch (split_k) {
    case 2: launch_splitwave_s<2>(depth, grid, a, s); break;
    case 3: launch_splitwave_s<3>(depth, grid, a, s); break;
    case 4: launch_splitwave_s<4>(depth, grid, a, s); break;
    case 5: launch_splitwave_s<5>(depth, grid, a, s); break;
    case 6: launch_splitwave_s<6>(depth, grid, a, s); break;
    case 7: launch_splitwave_s<7>(depth, grid, a, s); break;
    default: launch_splitwave_s<8>(depth, grid, a, s); break;
  }
  HIP_TRY(hipGetLastError());
  return 0;
}

int launch_skinny_gemm(const xtc_hip_matmul_desc& d, int split_k, int stages, int lda, int ldb, int ldc,
                       const void* A, const void* B, float* C, const float* bias, Scratch& x) {
  const hipStream_t s = x.s;
  const int splits = split_k < 1 ? 1 : split_k;
  SkinnyArgs a;
  a.A = (const __bf16*)A;
  a.B = (const __bf16*)B;
  a.bias = bias;
  a.M = d.M;
  a.N = d.N;
  a.K = d.K;
  a.lda = lda;
  a.ldb = ldb;
  a.nblocks = d.N / 128;
  a.relu = d.relu;
  a.relu_threshold = d.relu_threshold;
  a.C = C;
  a.ldc = ldc;
  a.counters = nullptr;
  if (splits == 1) {
    a.W = C;
    a.ldw = ldc;
  } else {
    size_t bytes = (size_t)splits * 16 * d.N * sizeof(float);
    a.W = x.partials(bytes);
    if (!a.W) return 1;
    a.ldw = d.N;
    a.counters = x.counters((size_t)a.nblocks);
    if (!a.counters) return 1;
  }
  dim3 grid((unsigned)(a.nblocks * splits));
  const bool kc1024 = d.K / splits == 1024;
  const int st = stages ? stages : 4;
  if (kc1024 && st == 4)
    hipLaunchKernelGGL((gemm_bf16_skinny<1024, 4>), grid, dim3(256), 0, s, a);
  else if (kc1024 && st == 3)
    hipLaunchKernelGGL((gemm_bf16_skinny<1024, 3>), grid, dim3(256), 0, s, a);
  else if (kc1024 && st == 2)
    hipLaunchKernelGGL((gemm_bf16_skinny<1024, 2>), grid, dim3(256), 0, s, a);
  else if (!kc1024 && st == 4)
    hipLaunchKernelGGL((gemm_bf16_skinny<512, 4>), grid, dim3(256), 0, s, a);
  else if (!kc1024 && st == 3)
    hipLaunchKernelGGL((gemm_bf16_skinny<512, 3>), grid, dim3(256), 0, s, a);
  else if (!kc1024 && st == 2)
    hipLaunchKernelGGL((gemm_bf16_skinny<512, 2>), grid, dim3(256), 0, s, a);
  else
    return fail("skinny bf16 kernel: no %d-stage pipeline", st);
  HIP_TRY(hipGetLastError());
  return 0;
}

// The direct conv kernel (conv_direct.hpp) implements the tiles of
// kDirectConv for fp32 when C and F are multiples of 64 and the input halo
// of one output block fits its LDS buffer.  XTC_HIP_GENERIC_GEMM=1 turns it
// off for the tiles a generic instance also implements.
bool direct_conv_applies(const xtc_hip_conv2d_desc& d, const xtc_hip_tile& t, int split_k, int OH, int OW,
                         const void* I, const void* W, const void* O, const void* bias) {
  static const bool disabled = [] {
    const char* v = getenv("XTC_HIP_GENERIC_GEMM");
    return v && v[0] == '1';
  }();
  const DirectConvTile* dt = direct_conv_tile(t);
  const GemmEntry* e = find_entry(XTC_HIP_F32, 1, t);
  const bool direct_only = e && e->launch == nullptr;
  if (!dt || (disabled && !direct_only) || d.dtype != XTC_HIP_F32 || split_k > 1) return false;
  if (d.C % 64 || d.F % 64) return false;
  const int hh = (dt->th - 1) * d.stride_h + d.R, hw = (dt->tw - 1) * d.stride_w + d.S;
  if (hh * hw > dconv::halo_pix(dt->halo_bytes)) return false;
  if (!aligned16(I) || !aligned16(W) || !aligned16(O) || (bias && !aligned16(bias))) return false;
  if ((int64_t)d.R * d.S * d.C * d.F > INT32_MAX || (int64_t)d.N * OH * OW > INT32_MAX) return false;
  return true;
}

int launch_direct_conv(const xtc_hip_conv2d_desc& d, const xtc_hip_tile& t, int OH, int OW, const void* I,
                       const void* W, float* O, const float* bias, hipStream_t s) {
  const DirectConvTile* dt = direct_conv_tile(t);
  DirectConvArgs a;
  a.I = (const float*)I;
  a.Wt = (const float*)W;
  a.O = O;
  a.bias = bias;
  a.NB = d.N;
  a.H = d.H;
  a.W = d.W;
  a.C = d.C;
  a.F = d.F;
  a.R = d.R;
  a.S = d.S;
  a.sh = d.stride_h;
  a.sw = d.stride_w;
  a.pt = d.pad_top;
  a.pl = d.pad_left;
  a.OH = OH;
  a.OW = OW;
  a.pad_value = d.pad_value;
  a.relu = d.relu;
  a.relu_threshold = d.relu_threshold;
  a.tiles_h = (OH + dt->th - 1) / dt->th;
  a.tiles_w = (OW + dt->tw - 1) / dt->tw;
  const uint64_t blocks = (uint64_t)d.N * a.tiles_h * a.tiles_w * (d.F / dconv::FB);
  if (blocks > 0x7fffffffu) return fail("conv2d grid too large");
  const bool fixed = dt->launch_3x3s1 && d.R == 3 && d.S == 3 && d.stride_h == 1 && d.stride_w == 1;
  (fixed ? dt->launch_3x3s1 : dt->launch)(a, dim3((unsigned)blocks), s);
  HIP_TRY(hipGetLastError());
  return 0;
}

// The tile a conv2d descriptor gets when it leaves `tile` zeroed: the shape
// class default of default_tile, upgraded from the 8x8 direct conv block to
// a 1x4-wave one when the direct kernel takes the shape with it, the window
// is wider than 1x1 (the wider block shares more of the input halo) and its
// blocks fit in one wave over the chip's 256 CUs: 7x14 (6.125 tiles of MFMA
// per wave) where its blocks fit, else 8x14 (7 tiles).  Measured on MI355X:
// C4 (8x56x56, 3x3) 26.8 us on 8x8, 23.0 on 8x14 (224 blocks), 21.9 -> 20.2
// us from 8x14 to 7x14 (256 blocks) on the 3x3 stride-1 kernel; Yolo9000_08
// (68x68, 3x3, 180 blocks) 47.6 -> 41.3 us from 8x8 to 8x14; but
// Yolo9000_04 (340 blocks) 39.8 -> 41.4 us, and the 1x1 convs lose
// (Yolo9000_09 10.6 -> 15.6 us, ResNet18_03 5.0 -> 6.8).
void default_conv_tile(const xtc_hip_conv2d_desc& d, int OH, int OW, xtc_hip_tile* t, int* split_k) {
  default_tile(d.dtype, 1, d.N * OH * OW, d.F, d.R * d.S * d.C, t, split_k);
  if (d.R * d.S == 1 || !same_tile(*t, xtc_hip_tile{64, 64, 16, 2, 2})) return;
  const void* p = (const void*)(uintptr_t)256;
  for (const xtc_hip_tile wide : {xtc_hip_tile{98, 64, 16, 1, 4}, xtc_hip_tile{112, 64, 16, 1, 4}}) {
    const DirectConvTile* dw = direct_conv_tile(wide);
    if (!dw) continue;
    const int64_t blocks =
        (int64_t)d.N * ((OH + dw->th - 1) / dw->th) * ((OW + dw->tw - 1) / dw->tw) * (d.F / dconv::FB);
    if (blocks <= 256 && direct_conv_applies(d, wide, *split_k, OH, OW, p, p, p, nullptr)) {
      *t = wide;
      return;
    }
  }
}

int launch_lds_dma_gemm(const xtc_hip_matmul_desc& d, const xtc_hip_tile& t, int split_k, int stages, int lda,
                        int ldb, int ldc, const void* A, const void* B, float* C, const float* bias, Scratch& x,
                        bool bt) {
  const hipStream_t s = x.s;
  const int splits = split_k < 1 ? 1 : split_k;
  BigGemmArgs a;
  a.A = (const __bf16*)A;
  a.B = (const __bf16*)B;
  a.C = C;
  a.bias = bias;
  a.M = d.M;
  a.N = d.N;
  a.K = d.K;
  a.lda = lda;
  a.ldb = ldb;
  a.ldc = ldc;
  a.relu = d.relu;
  a.relu_threshold = d.relu_threshold;
  a.tiles_m = d.M / 256;
  a.tiles_n = d.N / 256;
  a.group_m = d.group_m > 0 ? d.group_m : 8;  // 8 <= 16 at 8192^3, zero and random data
  a.xcd_remap = d.xcd_remap;
  a.k_per_split = d.K / splits;
  a.partial = nullptr;
  a.counters = nullptr;
  if (splits > 1) {
    a.partial = x.partials((size_t)splits * d.M * d.N * sizeof(float));
    if (!a.partial) return 1;
    a.counters = x.counters((size_t)a.tiles_m * a.tiles_n);
    if (!a.counters) return 1;
  }
  dim3 grid((unsigned)(a.tiles_m * a.tiles_n), 1, (unsigned)splits);
  if (t.bk == 32) {  // 2x4 waves: the ping-pong schedule, 3-5 stages of 32 KB
    const int st = stages ? stages : 4;
    if (bt && st == 4)
      hipLaunchKernelGGL((gemm_bf16_pingpong<true, 4>), grid, dim3(512), 0, s, a);
    else if (!bt && st == 4)
      hipLaunchKernelGGL((gemm_bf16_pingpong<false, 4>), grid, dim3(512), 0, s, a);
    else if (bt && st == 3)
      hipLaunchKernelGGL((gemm_bf16_pingpong<true, 3>), grid, dim3(512), 0, s, a);
    else if (!bt && st == 3)
      hipLaunchKernelGGL((gemm_bf16_pingpong<false, 3>), grid, dim3(512), 0, s, a);
    else if (bt && st == 5)
      hipLaunchKernelGGL((gemm_bf16_pingpong<true, 5>), grid, dim3(512), 0, s, a);
    else if (!bt && st == 5)
      hipLaunchKernelGGL((gemm_bf16_pingpong<false, 5>), grid, dim3(512), 0, s, a);
    else
      return fail("ping-pong bf16 kernel: no %d-stage pipeline", st);
  } else if (stages != 0 && stages != 2) {
    return fail("256x256x64 bf16 kernel: no %d-stage pipeline", stages);
  } else if (t.wgm == 2) {
    if (bt)
      hipLaunchKernelGGL((gemm_bf16_256x256<2, 4, 64, 2, true>), grid, dim3(512), 0, s, a);
    else
      hipLaunchKernelGGL((gemm_bf16_256x256<2, 4, 64, 2, false>), grid, dim3(512), 0, s, a);
  } else {
    if (bt)
      hipLaunchKernelGGL((gemm_bf16_256x256<4, 2, 64, 2, true>), grid, dim3(512), 0, s, a);
    else
      hipLaunchKernelGGL((gemm_bf16_256x256<4, 2, 64, 2, false>), grid, dim3(512), 0, s, a);
  }
  HIP_TRY(hipGetLastError());
  return 0;
}

// dst[c][r] = src[r][c] for r < R, c < Cc; src rows ld_src apart, dst dense
// [Cc][R].  64x64 tiles through LDS (padded row: the column reads hit 64
// distinct banks), coalesced 64-element rows on both sides.  HBM-bound:
// sizeof(T) bytes read + written per element.
template <typename T>
__global__ void __launch_bounds__(256) transpose_kernel(const T* __restrict__ src, T* __restrict__ dst, int R, int Cc,
                                                        int ld_src) {
  __shared__ T tile[64][65];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
  for (int i = ty; i < 64; i += 4) {
    const int r = r0 + i, c = c0 + tx;
    if (r < R && c < Cc) tile[i][tx] = src[(size_t)r * ld_src + c];
  }
  __syncthreads();
#pragma unroll
  for (int i = ty; i < 64; i += 4) {
    const int c = c0 + i, r = r0 + tx;
    if (c < Cc && r < R) dst[(size_t)c * R + r] = tile[tx][i];
  }
}

// The same transpose with 16-byte accesses on both sides, for R, Cc and
// ld_src multiples of the 16-byte vector (4 fp32 or 8 bf16 elements) and
// 16-byte aligned src and dst.  A workgroup of 256 threads moves a TILE x
// TILE block: TILE / VEC threads load each source row as vectors and write
// them into a padded LDS tile element by element; after the barrier each
// thread gathers one vector's worth of a source column (VEC elements of
// consecutive rows) and stores it as one vector of a dst row.  Vectors
// wholly outside the matrix are skipped, so ragged edges need no element
// masks.
template <typename T, int TILE>
__global__ void __launch_bounds__(256) transpose_vec_kernel(const T* __restrict__ src, T* __restrict__ dst, int R,
                                                            int Cc, int ld_src) {
  constexpr int VEC = 16 / (int)sizeof(T);
  constexpr int TPR = TILE / VEC;  // threads per tile row
  constexpr int RPP = 256 / TPR;   // rows per pass
  static_assert(TPR <= 256 && 256 % TPR == 0, "tile");
  __shared__ T tile[TILE][TILE + 1];
  union Vec16 {
    uint4 v;
    T e[VEC];
  };
  const int r0 = blockIdx.y * TILE, c0 = blockIdx.x * TILE;
  const int tv = threadIdx.x % TPR, tr = threadIdx.x / TPR;
#pragma unroll
  for (int p = 0; p < TILE / RPP; ++p) {
    const int i = tr + p * RPP;
    const int r = r0 + i, c = c0 + tv * VEC;
    if (r < R && c < Cc) {
      Vec16 u;
      u.v = *(const uint4*)(src + (size_t)r * ld_src + c);
#pragma unroll
      for (int j = 0; j < VEC; ++j) tile[i][tv * VEC + j] = u.e[j];
    }
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < TILE / RPP; ++p) {
    const int i = tr + p * RPP;
    const int c = c0 + i, r = r0 + tv * VEC;
    if (c < Cc && r < R) {
      Vec16 u;
#pragma unroll
      for (int j = 0; j < VEC; ++j) u.e[j] = tile[tv * VEC + j][i];
      *(uint4*)(dst + (size_t)c * R + r) = u.v;
    }
  }
}

// Block edge of the vector transpose per element size.  At 8192^2, in one
// process: fp32 32 -> 110 us, 128 -> 116 us, 64 -> 123 us; bf16 128 -> 40 us,
// 64 -> 45 us, 256 -> 61 us.
constexpr int kTransposeTileF32 = 32;
constexpr int kTransposeTileBf16 = 128;
constexpr int kTransposeTileF64 = 32;

// Dense [Cc][R] copy of the R x Cc matrix at src (row stride ld_src) in
// staging buffer `slot`; null on failure (g_last_error set).
const void* transposed_copy(int slot, const void* src, int R, int Cc, int ld_src, int elem_bytes, Scratch& x) {
  const hipStream_t s = x.s;
  const size_t bytes = (size_t)R * Cc * elem_bytes;
  void* dst = x.stage(slot, bytes);
  if (!dst) return nullptr;
  const int vec = 16 / elem_bytes;
  const int vtile = elem_bytes == 8 ? kTransposeTileF64 : elem_bytes == 4 ? kTransposeTileF32 : kTransposeTileBf16;
  if (R % vec == 0 && Cc % vec == 0 && ld_src % vec == 0 && aligned16(src) && aligned16(dst) &&
      (R + vtile - 1) / vtile <= 65535) {
    dim3 grid((unsigned)((Cc + vtile - 1) / vtile), (unsigned)((R + vtile - 1) / vtile));
    if (elem_bytes == 8)
      hipLaunchKernelGGL((transpose_vec_kernel<uint64_t, kTransposeTileF64>), grid, dim3(256), 0, s,
                         (const uint64_t*)src, (uint64_t*)dst, R, Cc, ld_src);
    else if (elem_bytes == 4)
      hipLaunchKernelGGL((transpose_vec_kernel<float, kTransposeTileF32>), grid, dim3(256), 0, s, (const float*)src,
                         (float*)dst, R, Cc, ld_src);
    else
      hipLaunchKernelGGL((transpose_vec_kernel<uint16_t, kTransposeTileBf16>), grid, dim3(256), 0, s,
                         (const uint16_t*)src, (uint16_t*)dst, R, Cc, ld_src);
    if (hipGetLastError() != hipSuccess) {
      fail("transpose launch failed");
      return nullptr;
    }
    return dst;
  }
  dim3 grid((unsigned)((Cc + 63) / 64), (unsigned)((R + 63) / 64));
  if (grid.y > 65535u) {
    fail("transpose: %d rows exceed the grid limit", R);
    return nullptr;
  }
  if (elem_bytes == 8)
    hipLaunchKernelGGL(transpose_kernel<uint64_t>, grid, dim3(256), 0, s, (const uint64_t*)src, (uint64_t*)dst, R,
                       Cc, ld_src);
  else if (elem_bytes == 4)
    hipLaunchKernelGGL(transpose_kernel<float>, grid, dim3(256), 0, s, (const float*)src, (float*)dst, R, Cc, ld_src);
  else
    hipLaunchKernelGGL(transpose_kernel<uint16_t>, grid, dim3(256), 0, s, (const uint16_t*)src, (uint16_t*)dst, R,
                       Cc, ld_src);
  if (hipGetLastError() != hipSuccess) {
    fail("transpose launch failed");
    return nullptr;
  }
  return dst;
}

// The kernel family a matmul runs on, chosen from the shape, tile, split,
// strides and operand alignment in the order of matmul_impl.
enum class MatmulPath { LdsDmaBt, Naive, LdsDma, Skinny, SplitWave, F32Lds, F64, Generic };

const char* path_name(MatmulPath p) {
  switch (p) {
    case MatmulPath::LdsDmaBt:
    case MatmulPath::LdsDma:
      return "LDS-DMA bf16";
    case MatmulPath::Naive:
      return "scalar";
    case MatmulPath::Skinny:
      return "skinny bf16";
    case MatmulPath::SplitWave:
      return "split-wave fp32";
    case MatmulPath::F32Lds:
      return "LDS-DMA fp32";
    case MatmulPath::F64:
      return "fp64";
    default:
      return "generic";
  }
}

// Pipeline depths the kernel of path p compiles for tile t: LDS stages of
// the LDS-DMA kernels, the generic template's register-staged double buffer
// (2) and, for the tiles with a ring instance (`ring`, generic_ring), its
// three register sets (4), the split-wave kernel's ring of register chunks,
// 1 for the scalar kernel.  out[0] is the default.  Returns the count.
int path_depths(MatmulPath p, const xtc_hip_tile& t, int ring, int* out, int max) {
  int tmp[16];
  int n = 0;
  switch (p) {
    case MatmulPath::LdsDmaBt:
    case MatmulPath::LdsDma:
      if (t.bk == 32) {
        tmp[n++] = 4;
        tmp[n++] = 3;
        tmp[n++] = 5;
      } else {
        tmp[n++] = 2;
      }
      break;
    case MatmulPath::Skinny:
      tmp[n++] = 4;
      tmp[n++] = 3;
      tmp[n++] = 2;
      break;
    case MatmulPath::SplitWave:
      for (int v : kSplitWaveDepths) tmp[n++] = v;
      break;
    case MatmulPath::F32Lds:
      for (const F32LdsVariant& v : kF32Lds)
        if (v.bm == t.bm && v.bn == t.bn && v.bk == t.bk && v.wgm == t.wgm && v.wgn == t.wgn && n < 16)
          tmp[n++] = v.stages;
      break;
    case MatmulPath::Naive:
      tmp[n++] = 1;
      break;
    case MatmulPath::F64:
      tmp[n++] = 2;  // register-staged double buffer
      break;
    default:
      if (ring == 2) tmp[n++] = 4;
      tmp[n++] = 2;
      if (ring == 1) tmp[n++] = 4;
      break;
  }
  for (int i = 0; i < n && i < max; ++i) out[i] = tmp[i];
  return n;
}

// 0 if `stages` (0 = default) is a depth of path p for tile t, else fails.
int check_depth(MatmulPath p, const xtc_hip_tile& t, int ring, int stages) {
  if (stages == 0) return 0;
  int depths[16];
  const int n = path_depths(p, t, ring, depths, 16);
  char list[96] = "";
  for (int i = 0; i < n; ++i) {
    if (depths[i] == stages) return 0;
    const size_t used = strlen(list);
    snprintf(list + used, sizeof(list) - used, i ? ", %d" : "%d", depths[i]);
  }
  return fail("the %s kernel for tile %dx%dx%d waves %dx%d has pipeline depths {%s}, not %d", path_name(p), t.bm,
              t.bn, t.bk, t.wgm, t.wgn, list, stages);
}

// Strides, tile and split of descriptor d after defaults.  Returns 0, or
// fails.
int resolve_matmul(const xtc_hip_matmul_desc& d, int* lda, int* ldb, int* ldc, xtc_hip_tile* t, int* split_k) {
  if (d.dtype != XTC_HIP_F32 && d.dtype != XTC_HIP_BF16 && d.dtype != XTC_HIP_F64) return fail("bad dtype %d", d.dtype);
  if (d.M <= 0 || d.N <= 0 || d.K <= 0) return fail("bad shape %dx%dx%d", d.M, d.N, d.K);
  if (d.stages < 0) return fail("bad pipeline depth %d", d.stages);
  const bool ta = d.trans_a != 0, tb = d.trans_b != 0;
  *lda = d.lda ? d.lda : (ta ? d.M : d.K);
  *ldb = d.ldb ? d.ldb : (tb ? d.K : d.N);
  *ldc = d.ldc ? d.ldc : d.N;
  if (*lda < (ta ? d.M : d.K) || *ldb < (tb ? d.K : d.N) || *ldc < d.N)
    return fail("leading dimension smaller than shape");
  *t = d.tile;
  *split_k = d.split_k;
  if (t->bm == 0) {
    int sk = 1;
    default_tile(d.dtype, 0, d.M, d.N, d.K, t, &sk);
    if (*split_k <= 0) *split_k = sk;
  }
  return 0;
}

// The path of a matmul whose operands, after any transposed copy, are A/B
// with strides lda/ldb (the B^T-direct case is decided before the copies).
int natural_path(const xtc_hip_matmul_desc& d, const xtc_hip_tile& t, int split_k, int lda, int ldb, int ldc,
                 const void* A, const void* B, const void* C, const void* bias, MatmulPath* path) {
  const int vec = d.dtype == XTC_HIP_F32 ? 4 : d.dtype == XTC_HIP_F64 ? 2 : 8;
  const bool vec_ok = lda % vec == 0 && ldb % vec == 0 && d.K % vec == 0 && d.N % vec == 0 && aligned16(A) &&
                      aligned16(B);
  if (!vec_ok) {
    *path = MatmulPath::Naive;
    return 0;
  }
  if (d.dtype == XTC_HIP_F64) {
    if (!f64_tile(0, t))
      return fail("no fp64 matmul kernel instance for tile %dx%dx%d waves %dx%d", t.bm, t.bn, t.bk, t.wgm, t.wgn);
    *path = MatmulPath::F64;
    return 0;
  }
  if (!find_entry(d.dtype, 0, t))
    return fail("no matmul kernel instance for dtype %d tile %dx%dx%d waves %dx%d", d.dtype, t.bm, t.bn, t.bk, t.wgm,
                t.wgn);
  if (lds_dma_gemm_applies(d, t, split_k, lda, ldb, ldc, A, B, C, (const float*)bias, false))
    *path = MatmulPath::LdsDma;
  else if (skinny_gemm_applies(d, t, split_k, lda, ldb, ldc, A, B, C, (const float*)bias))
    *path = MatmulPath::Skinny;
  else if (splitwave_gemm_applies(d, t, split_k, lda, A))
    *path = MatmulPath::SplitWave;
  else if (f32_lds_gemm_applies(d, t, split_k, lda, ldb, ldc, A, B, C, (const float*)bias))
    *path = MatmulPath::F32Lds;
  else
    *path = MatmulPath::Generic;
  return 0;
}

// xtc_hip_matmul with its scratch taken from `x` (whose stream is the
// descriptor's).
// The fp64 GEMM of descriptor d on A/B with strides lda/ldb (after any
// transposed copy): the fp64 MFMA kernel, split-K partials in fp64.
int launch_f64_gemm(const xtc_hip_matmul_desc& d, const xtc_hip_tile& t, int split_k, int lda, int ldb, int ldc,
                    const void* A, const void* B, void* C, const void* bias, Scratch& x) {
  const F64Tile* f = f64_tile(0, t);
  GemmArgs64 a;
  memset(&a, 0, sizeof(a));
  a.A = (const double*)A;
  a.B = (const double*)B;
  a.C = (double*)C;
  a.bias = (const double*)bias;
  a.M = d.M;
  a.N = d.N;
  a.K = d.K;
  a.lda = lda;
  a.ldb = ldb;
  a.ldc = ldc;
  a.relu = d.relu;
  a.relu_threshold = d.relu_threshold_f64;
  return launch_f64_common(a, f, split_k, d.group_m, d.xcd_remap, x);
}

int matmul_impl(const xtc_hip_matmul_desc& d, const void* A, const void* B, void* Cv, const void* biasv,
                Scratch& x) {
  float* C = (float*)Cv;
  const float* bias = (const float*)biasv;
  if (!A || !B || !C) return fail("null operand");
  int lda, ldb, ldc, split_k;
  xtc_hip_tile t;
  if (resolve_matmul(d, &lda, &ldb, &ldc, &t, &split_k)) return 1;
  const bool ta = d.trans_a != 0, tb = d.trans_b != 0;
  const hipStream_t s = x.s;
  // B stored transposed feeds the LDS-DMA kernel directly (B^T tiles are
  // read like A tiles); every other transposed operand gets a natural copy
  // in a staging buffer first (one HBM-bound transpose).
  if (tb && !ta && lds_dma_gemm_applies(d, t, split_k, lda, ldb, ldc, A, B, C, bias, true)) {
    if (check_depth(MatmulPath::LdsDmaBt, t, 0, d.stages)) return 1;
    return launch_lds_dma_gemm(d, t, split_k, d.stages, lda, ldb, ldc, A, B, C, bias, x, true);
  }
  const int esz = d.dtype == XTC_HIP_F64 ? 8 : d.dtype == XTC_HIP_F32 ? 4 : 2;
  if (ta) {
    A = transposed_copy(0, A, d.K, d.M, lda, esz, x);
    if (!A) return 1;
    lda = d.K;
  }
  if (tb) {
    B = transposed_copy(1, B, d.N, d.K, ldb, esz, x);
    if (!B) return 1;
    ldb = d.N;
  }
  MatmulPath path;
  if (natural_path(d, t, split_k, lda, ldb, ldc, A, B, C, bias, &path)) return 1;
  const int ring =
      path == MatmulPath::Generic ? generic_ring(find_entry(d.dtype, 0, t), effective_splits(d.K, split_k, t.bk)) : 0;
  if (check_depth(path, t, ring, d.stages)) return 1;
  if (path == MatmulPath::Naive) {
    dim3 grid(grid_for((uint64_t)d.M * d.N, 128));
    if (d.dtype == XTC_HIP_F64)
      hipLaunchKernelGGL(gemm_naive_f64_kernel, grid, dim3(128), 0, s, (const double*)A, (const double*)B,
                         (double*)Cv, (const double*)biasv, d.M, d.N, d.K, lda, ldb, ldc, d.relu,
                         d.relu_threshold_f64);
    else if (d.dtype == XTC_HIP_F32)
      hipLaunchKernelGGL(gemm_naive_kernel<float>, grid, dim3(128), 0, s, (const float*)A,
                         (const float*)B, C, bias, d.M, d.N, d.K, lda, ldb, ldc, d.relu,
                         d.relu_threshold);
    else
      hipLaunchKernelGGL(gemm_naive_kernel<uint16_t>, grid, dim3(128), 0, s,
                         (const uint16_t*)A, (const uint16_t*)B, C, bias, d.M, d.N, d.K, lda,
                         ldb, ldc, d.relu, d.relu_threshold);
    HIP_TRY(hipGetLastError());
    return 0;
  }
  if (path == MatmulPath::F64) return launch_f64_gemm(d, t, split_k, lda, ldb, ldc, A, B, Cv, biasv, x);
  if (path == MatmulPath::LdsDma)
    return launch_lds_dma_gemm(d, t, split_k, d.stages, lda, ldb, ldc, A, B, C, bias, x, false);
  if (path == MatmulPath::Skinny) return launch_skinny_gemm(d, split_k, d.stages, lda, ldb, ldc, A, B, C, bias, x);
  if (path == MatmulPath::SplitWave)
    return launch_splitwave_gemm(d, split_k, d.stages, lda, ldb, ldc, A, B, C, bias, s);
  const GemmEntry* e = find_entry(d.dtype, 0, t);
  GemmEntry lds_entry;
  if (path == MatmulPath::F32Lds) {
    // same tiles, split-K set-up and grid as the generic instance; only the
    // kernel differs
    lds_entry = *e;
    lds_entry.launch = f32_lds_variant(t, d.stages)->launch;
    lds_entry.launch_ring = nullptr;
    e = &lds_entry;
  }
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  a.A = A;
  a.B = B;
  a.C = C;
  a.bias = bias;
  a.M = d.M;
  a.N = d.N;
  a.K = d.K;
  a.lda = lda;
  a.ldb = ldb;
  a.ldc = ldc;
  a.relu = d.relu;
  a.relu_threshold = d.relu_threshold;
  return launch_gemm_common(a, e, split_k, path == MatmulPath::Generic ? d.stages : 0, d.group_m, d.xcd_remap, x);
}

}  // namespace

extern "C" {

const char* xtc_hip_last_error(void) { return g_last_error.c_str(); }

int xtc_hip_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

int xtc_hip_init(int device) {
  if (device < 0 || device >= kMaxDevices) return fail("invalid device %d", device);
  int n = xtc_hip_device_count();
  if (device >= n) return fail("device %d not present (%d visible)", device, n);
  std::lock_guard<std::mutex> lk(g_mutex);
  HIP_TRY(hipSetDevice(device));
  DeviceState& d = g_dev[device];
  if (!d.ready) {
    HIP_TRY(hipStreamCreateWithFlags(&d.stream, hipStreamNonBlocking));
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, device));
    HIP_TRY(hipGetSymbolAddress(&d.scratch_ptr, HIP_SYMBOL(scratch)));
    HIP_TRY(hipHostMalloc((void**)&d.done_flag, 256, hipHostMallocCoherent));
    *d.done_flag = 0;
    d.arch = prop.gcnArchName;
    d.name = prop.name;
    d.cus = prop.multiProcessorCount;
    d.ready = true;
  }
  g_current = device;
  return 0;
}

static int copy_str(const std::string& s, char* buf, int len) {
  if (!buf || len <= 0) return fail("null buffer");
  snprintf(buf, (size_t)len, "%s", s.c_str());
  return 0;
}

int xtc_hip_device_arch(char* buf, int len) {
  DeviceState* d = current_state();
  if (!d) return fail("xtc_hip_init not called");
  return copy_str(d->arch, buf, len);
}

int xtc_hip_device_name(char* buf, int len) {
  DeviceState* d = current_state();
  if (!d) return fail("xtc_hip_init not called");
  return copy_str(d->name, buf, len);
}

void* xtc_hip_stream(void) {
  DeviceState* d = current_state();
  return d ? (void*)d->stream : nullptr;
}

int xtc_hip_synchronize(void) {
  DeviceState* d = current_state();
  if (!d) return fail("xtc_hip_init not called");
  // A one-thread kernel queued behind the work stores the call's sequence
  // number to coherent host memory, and the host spins on that word: the
  // round trip is about 6 us where a stream synchronisation takes 11 us (the
  // runtime's completion signal), which decides the time of short
  // synchronous payloads.  The spin asks the stream itself every 50 us, so
  // it also ends on completion without the store and on an error.
  unsigned seq;
  hipError_t launched;
  {
    std::lock_guard<std::mutex> lock(d->done_mutex);
    seq = d->done_seq.fetch_add(1u) + 1u;
    hipLaunchKernelGGL(stream_done_kernel, dim3(1), dim3(64), 0, d->stream, d->done_flag, seq);
    launched = hipGetLastError();
  }
  if (launched != hipSuccess) {
    HIP_TRY(hipStreamSynchronize(d->stream));
    return 0;
  }
  double next_query = now_s() + 50e-6;
  while ((int)(__atomic_load_n(d->done_flag, __ATOMIC_ACQUIRE) - seq) < 0) {
    __builtin_ia32_pause();
    if (now_s() >= next_query) {
      const hipError_t e = hipStreamQuery(d->stream);
      if (e == hipSuccess) break;
      if (e != hipErrorNotReady) return fail("xtc_hip_synchronize: %s", hipGetErrorString(e));
      next_query = now_s() + 50e-6;
    }
  }
  return 0;
}

void* xtc_hip_stream_create(void) {
  if (!current_state()) {
    fail("xtc_hip_init not called");
    return nullptr;
  }
  hipStream_t s = nullptr;
  if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) {
    fail("hipStreamCreateWithFlags failed");
    return nullptr;
  }
  return (void*)s;
}

int xtc_hip_stream_synchronize(void* stream) {
  if (!current_state()) return fail("xtc_hip_init not called");
  HIP_TRY(hipStreamSynchronize(pick_stream(stream)));
  return 0;
}

int xtc_hip_stream_destroy(void* stream) {
  DeviceState* d = current_state();
  if (!d) return fail("xtc_hip_init not called");
  hipStream_t s = (hipStream_t)stream;
  if (!s || s == d->stream) return fail("the library stream cannot be destroyed");
  if (xtc_hip_stream_release(stream)) return 1;
  HIP_TRY(hipStreamDestroy(s));
  return 0;
}

int xtc_hip_stream_release(void* stream) {
  DeviceState* d = current_state();
  if (!d) return fail("xtc_hip_init not called");
  hipStream_t s = pick_stream(stream);
  HIP_TRY(hipStreamSynchronize(s));
  std::lock_guard<std::mutex> lk(g_mutex);
  auto it = d->scratch.find(s);
  if (it != d->scratch.end()) {
    StreamScratch& x = it->second;
    if (x.workspace) hipFree(x.workspace);
    if (x.counters) hipFree(x.counters);
    for (void* p : x.staging)
      if (p) hipFree(p);
    d->scratch.erase(it);
  }
  return 0;
}

void* xtc_hip_malloc(uint64_t bytes) {
  if (!current_state()) {
    fail("xtc_hip_init not called");
    return nullptr;
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
  if (e != hipSuccess) {
    fail("hipMalloc(%llu) failed: %s", (unsigned long long)bytes, hipGetErrorString(e));
    return nullptr;
  }
  return p;
}

int xtc_hip_free(void* ptr) {
  if (!ptr) return 0;
  DeviceState* d = current_state();
  if (d) HIP_TRY(hipStreamSynchronize(d->stream));
  HIP_TRY(hipFree(ptr));
  return 0;
}

static int copy_sync(void* dst, const void* src, uint64_t bytes, hipMemcpyKind kind) {
  DeviceState* d = current_state();
  if (!d) return fail("xtc_hip_init not called");
  if (bytes == 0) return 0;
  HIP_TRY(hipMemcpyAsync(dst, src, bytes, kind, d->stream));
  HIP_TRY(hipStreamSynchronize(d->stream));
  return 0;
}

int xtc_hip_memcpy_h2d(void* dst, const void* src, uint64_t bytes) {
  return copy_sync(dst, src, bytes, hipMemcpyHostToDevice);
}
int xtc_hip_memcpy_d2h(void* dst, const void* src, uint64_t bytes) {
  return copy_sync(dst, src, bytes, hipMemcpyDeviceToHost);
}
int xtc_hip_memcpy_d2d(void* dst, const void* src, uint64_t bytes) {
  return copy_sync(dst, src, bytes, hipMemcpyDeviceToDevice);
}

int xtc_hip_memset_zero(void* ptr, uint64_t bytes) {
  DeviceState* d = current_state();
  if (!d) return fail("xtc_hip_init not called");
  if (bytes == 0) return 0;
  if (!aligned16(ptr)) return fail("memset_zero: pointer not 16-byte aligned");
  uint64_t n16 = bytes / 16;
  int ntail = (int)(bytes % 16);
  hipLaunchKernelGGL(fill_zero_kernel, dim3(grid_for(n16 ? n16 : 1, 256)), dim3(256), 0,
                     d->stream, (uint4*)ptr, n16, (unsigned char*)ptr + n16 * 16, ntail);
  HIP_TRY(hipGetLastError());
  HIP_TRY(hipStreamSynchronize(d->stream));
  return 0;
}

void* xtc_hip_event_create(void) {
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) {
    fail("hipEventCreate failed");
    return nullptr;
  }
  return (void*)e;
}

int xtc_hip_event_record(void* event, void* stream) {
  HIP_TRY(hipEventRecord((hipEvent_t)event, pick_stream(stream)));
  return 0;
}

int xtc_hip_event_elapsed_ms(void* start, void* stop, float* ms) {
  HIP_TRY(hipEventSynchronize((hipEvent_t)stop));
  HIP_TRY(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
  return 0;
}

int xtc_hip_event_destroy(void* event) {
  HIP_TRY(hipEventDestroy((hipEvent_t)event));
  return 0;
}

int xtc_hip_matmul_desc_size(void) { return (int)sizeof(xtc_hip_matmul_desc); }
int xtc_hip_conv2d_desc_size(void) { return (int)sizeof(xtc_hip_conv2d_desc); }

int xtc_hip_gemm_instance_count(void) {
  int n = 0, m = 0, q = 0;
  gemm_registry(&n);
  direct_only_entries(&m);
  f64_entries(&q);
  return n + m + q;
}

int xtc_hip_gemm_instance_get(int index, xtc_hip_gemm_instance* out) {
  int n = 0, m = 0, q = 0;
  const GemmEntry* e = gemm_registry(&n);
  const GemmEntry* x = direct_only_entries(&m);
  const GemmEntry* y = f64_entries(&q);
  if (index < 0 || index >= n + m + q || !out) return fail("instance index %d out of range", index);
  if (index >= n + m) {
    e = y;
    index -= n + m;
  } else if (index >= n) {
    e = x;
    index -= n;
  }
  out->dtype = e[index].dtype;
  out->conv = e[index].conv;
  out->tile = xtc_hip_tile{e[index].bm, e[index].bn, e[index].bk, e[index].wgm, e[index].wgn};
  out->lds_bytes = e[index].lds_bytes;
  out->threads = e[index].threads;
  return 0;
}

int xtc_hip_default_tile(int dtype, int conv, int M, int N, int K, xtc_hip_tile* out,
                         int* split_k) {
  if (!out || !split_k) return fail("null output");
  default_tile(dtype, conv, M, N, K, out, split_k);
  if (out->bm == 0) return fail("no kernel instance for dtype %d conv %d", dtype, conv);
  return 0;
}

int xtc_hip_conv2d_default_tile(const xtc_hip_conv2d_desc* desc, xtc_hip_tile* out, int* split_k) {
  if (!desc || !out || !split_k) return fail("null argument");
  const xtc_hip_conv2d_desc& d = *desc;
  const int HP = d.H + d.pad_top + d.pad_bottom;
  const int WP = d.W + d.pad_left + d.pad_right;
  if (d.stride_h <= 0 || d.stride_w <= 0 || HP < d.R || WP < d.S) return fail("bad conv2d descriptor");
  default_conv_tile(d, (HP - d.R) / d.stride_h + 1, (WP - d.S) / d.stride_w + 1, out, split_k);
  if (out->bm == 0) return fail("no conv2d kernel instance for dtype %d", d.dtype);
  return 0;
}

int xtc_hip_matmul_pipeline_depths(const xtc_hip_matmul_desc* desc, int* depths, int max_depths) {
  if (!desc || !depths || max_depths < 1) return -fail("null argument");
  const xtc_hip_matmul_desc& d = *desc;
  int lda, ldb, ldc, split_k;
  xtc_hip_tile t;
  if (resolve_matmul(d, &lda, &ldb, &ldc, &t, &split_k)) return -1;
  // operands as the allocators hand them out: 256-byte aligned
  const void* p = (const void*)(uintptr_t)256;
  MatmulPath path;
  if (d.trans_b && !d.trans_a && lds_dma_gemm_applies(d, t, split_k, lda, ldb, ldc, p, p, p, nullptr, true)) {
    path = MatmulPath::LdsDmaBt;
  } else {
    if (d.trans_a) lda = d.K;
    if (d.trans_b) ldb = d.N;
    if (natural_path(d, t, split_k, lda, ldb, ldc, p, p, p, nullptr, &path)) return -1;
  }
  const int ring =
      path == MatmulPath::Generic ? generic_ring(find_entry(d.dtype, 0, t), effective_splits(d.K, split_k, t.bk)) : 0;
  return path_depths(path, t, ring, depths, max_depths);
}

int xtc_hip_conv2d_pipeline_depths(const xtc_hip_conv2d_desc* desc, int* depths, int max_depths) {
  if (!desc || !depths || max_depths < 1) return -fail("null argument");
  xtc_hip_conv2d_desc d = *desc;
  const int HP = d.H + d.pad_top + d.pad_bottom;
  const int WP = d.W + d.pad_left + d.pad_right;
  if (d.stride_h <= 0 || d.stride_w <= 0 || HP < d.R || WP < d.S) return -fail("bad conv2d descriptor");
  const int OH = (HP - d.R) / d.stride_h + 1;
  const int OW = (WP - d.S) / d.stride_w + 1;
  const int vec = d.dtype == XTC_HIP_F32 ? 4 : d.dtype == XTC_HIP_F64 ? 2 : 8;
  const bool padded = d.pad_top || d.pad_bottom || d.pad_left || d.pad_right;
  const double pad_value = d.dtype == XTC_HIP_F64 ? d.pad_value_f64 : (double)d.pad_value;
  if (d.C % vec && d.F % vec == 0 && (!padded || isfinite(pad_value))) {
    // xtc_hip_conv2d stages such a conv with zero channels up to the next
    // whole vector and runs the MFMA conv on the copies: describe that kernel
    d.C = (d.C + vec - 1) / vec * vec;
  }
  if (d.C % vec || d.F % vec) {
    depths[0] = 1;  // scalar kernel
    return 1;
  }
  xtc_hip_tile t = d.tile;
  int split_k = d.split_k;
  if (t.bm == 0) {
    int sk = 1;
    default_conv_tile(d, OH, OW, &t, &sk);
    if (split_k <= 0) split_k = sk;
  }
  const GemmEntry* e = find_entry(d.dtype, 1, t);
  if (!e)
    return -fail("no conv2d kernel instance for dtype %d tile %dx%dx%d waves %dx%d", d.dtype, t.bm, t.bn, t.bk,
                 t.wgm, t.wgn);
  const void* p = (const void*)(uintptr_t)256;
  if (d.dtype == XTC_HIP_F64) {
    depths[0] = 2;  // the fp64 kernel's register-staged double buffer
    return 1;
  }
  // the direct kernel keeps its weight taps in LDS stages or a register
  // ring; the implicit-GEMM loader double-buffers through registers, with
  // three register sets in flight on the tiles that have a ring instance
  // when K is split
  if (direct_conv_applies(d, t, split_k, OH, OW, p, p, p, nullptr))
    depths[0] = direct_conv_tile(t)->depth();
  else if (e->launch)
    depths[0] = generic_ring(e, effective_splits(d.R * d.S * d.C, split_k > 0 ? split_k : 1, t.bk)) == 2 ? 4 : 2;
  else
    return -fail("conv2d tile %dx%dx%d waves %dx%d exists only in the direct conv kernel, which does not take "
                 "this shape",
                 t.bm, t.bn, t.bk, t.wgm, t.wgn);
  return 1;
}

int xtc_hip_matmul(const xtc_hip_matmul_desc* desc, const void* A, const void* B, void* C,
                   const void* bias) {
  if (!desc) return fail("null descriptor");
  if (!current_state()) return fail("xtc_hip_init not called");
  Scratch x{pick_stream(desc->stream)};
  return matmul_impl(*desc, A, B, C, bias, x);
}

int xtc_hip_matmul_noalloc(const xtc_hip_matmul_desc* desc, const void* A, const void* B, void* C,
                           const void* bias) {
  if (!desc) return fail("null descriptor");
  DeviceState* dev = current_state();
  if (!dev) return fail("xtc_hip_init not called");
  if (!dev->scratch_ptr) return fail("xtc_hip_matmul_noalloc: no scratch address for this device");
  Scratch x{pick_stream(desc->stream)};
  x.fixed = (char*)dev->scratch_ptr;
  x.cap = XTC_HIP_NOALLOC_SCRATCH_BYTES;
  return matmul_impl(*desc, A, B, C, bias, x);
}

int xtc_hip_conv2d(const xtc_hip_conv2d_desc* desc, const void* input, const void* weight,
                   void* outv, const void* biasv) {
  if (!desc) return fail("null descriptor");
  if (!current_state()) return fail("xtc_hip_init not called");
  if (!input || !weight || !outv) return fail("null operand");
  float* out = (float*)outv;
  const float* bias = (const float*)biasv;
  const xtc_hip_conv2d_desc& d = *desc;
  if (d.dtype != XTC_HIP_F32 && d.dtype != XTC_HIP_BF16 && d.dtype != XTC_HIP_F64) return fail("bad dtype %d", d.dtype);
  const bool f64 = d.dtype == XTC_HIP_F64;
  if (d.N <= 0 || d.H <= 0 || d.W <= 0 || d.C <= 0 || d.F <= 0 || d.R <= 0 || d.S <= 0 ||
      d.stride_h <= 0 || d.stride_w <= 0 || d.pad_top < 0 || d.pad_bottom < 0 ||
      d.pad_left < 0 || d.pad_right < 0)
    return fail("bad conv2d descriptor");
  const int HP = d.H + d.pad_top + d.pad_bottom;
  const int WP = d.W + d.pad_left + d.pad_right;
  if (HP < d.R || WP < d.S) return fail("conv2d window larger than padded input");
  const int OH = (HP - d.R) / d.stride_h + 1;
  const int OW = (WP - d.S) / d.stride_w + 1;
  hipStream_t s = pick_stream(d.stream);
  const int vec = d.dtype == XTC_HIP_F32 ? 4 : f64 ? 2 : 8;
  const int M = d.N * OH * OW;
  const int K = d.R * d.S * d.C;
  const bool vec_ok = d.C % vec == 0 && d.F % vec == 0 && aligned16(input) && aligned16(weight);
  const bool padded = d.pad_top || d.pad_bottom || d.pad_left || d.pad_right;
  if (!vec_ok && d.F % vec == 0 && (!padded || isfinite(f64 ? d.pad_value_f64 : (double)d.pad_value))) {
    // Channels that are not whole 16-byte vectors (C = 3 image inputs): the
    // input and the weights are copied with zero channels up to Cp, a
    // multiple of the vector, and the MFMA conv runs on the copies.  A zero
    // channel adds exact zeros (input 0 or a finite pad value, times a zero
    // weight), so the result is the conv over the C real channels.
    const int Cp = (d.C + vec - 1) / vec * vec;
    const size_t esz = f64 ? 8 : d.dtype == XTC_HIP_F32 ? 4 : 2;
    const uint64_t pixels = (uint64_t)d.N * d.H * d.W, taps = (uint64_t)d.R * d.S;
    if ((uint64_t)Cp * d.F > 0xffffffffu) return fail("conv2d: %d x %d channels too many to stage", Cp, d.F);
    Scratch x{s};
    void* in_c = x.stage(0, pixels * Cp * esz);
    void* w_c = in_c ? x.stage(1, taps * Cp * d.F * esz) : nullptr;
    if (!in_c || !w_c) return 1;
    if (f64) {  // zero bits are +0.0: the 8-byte copy needs no fp type
      hipLaunchKernelGGL(pad_channels_kernel<uint64_t>, dim3(grid_for(pixels * Cp, 256)), dim3(256), 0, s,
                         (const uint64_t*)input, (uint64_t*)in_c, pixels, (uint32_t)d.C, (uint32_t)Cp);
      hipLaunchKernelGGL(pad_channels_kernel<uint64_t>, dim3(grid_for(taps * Cp * d.F, 256)), dim3(256), 0, s,
                         (const uint64_t*)weight, (uint64_t*)w_c, taps, (uint32_t)(d.C * d.F),
                         (uint32_t)(Cp * d.F));
    } else if (d.dtype == XTC_HIP_F32) {
      hipLaunchKernelGGL(pad_channels_kernel<float>, dim3(grid_for(pixels * Cp, 256)), dim3(256), 0, s,
                         (const float*)input, (float*)in_c, pixels, (uint32_t)d.C, (uint32_t)Cp);
      hipLaunchKernelGGL(pad_channels_kernel<float>, dim3(grid_for(taps * Cp * d.F, 256)), dim3(256), 0, s,
                         (const float*)weight, (float*)w_c, taps, (uint32_t)(d.C * d.F), (uint32_t)(Cp * d.F));
    } else {
      hipLaunchKernelGGL(pad_channels_kernel<uint16_t>, dim3(grid_for(pixels * Cp, 256)), dim3(256), 0, s,
                         (const uint16_t*)input, (uint16_t*)in_c, pixels, (uint32_t)d.C, (uint32_t)Cp);
      hipLaunchKernelGGL(pad_channels_kernel<uint16_t>, dim3(grid_for(taps * Cp * d.F, 256)), dim3(256), 0, s,
                         (const uint16_t*)weight, (uint16_t*)w_c, taps, (uint32_t)(d.C * d.F),
                         (uint32_t)(Cp * d.F));
    }
    HIP_TRY(hipGetLastError());
    xtc_hip_conv2d_desc dc = d;
    dc.C = Cp;
    return xtc_hip_conv2d(&dc, in_c, w_c, outv, biasv);
  }
  if (!vec_ok) {
    dim3 grid(grid_for((uint64_t)M * d.F, 128));
    if (f64)
      hipLaunchKernelGGL(conv_naive_f64_kernel, grid, dim3(128), 0, s, (const double*)input, (const double*)weight,
                         (double*)outv, (const double*)biasv, d.N, d.H, d.W, d.C, d.F, d.R, d.S, d.stride_h,
                         d.stride_w, d.pad_top, d.pad_left, OH, OW, d.pad_value_f64, d.relu, d.relu_threshold_f64);
    else if (d.dtype == XTC_HIP_F32)
      hipLaunchKernelGGL(conv_naive_kernel<float>, grid, dim3(128), 0, s, (const float*)input,
                         (const float*)weight, out, bias, d.N, d.H, d.W, d.C, d.F, d.R, d.S,
                         d.stride_h, d.stride_w, d.pad_top, d.pad_left, OH, OW, d.pad_value,
                         d.relu, d.relu_threshold);
    else
      hipLaunchKernelGGL(conv_naive_kernel<uint16_t>, grid, dim3(128), 0, s,
                         (const uint16_t*)input, (const uint16_t*)weight, out, bias, d.N, d.H,
                         d.W, d.C, d.F, d.R, d.S, d.stride_h, d.stride_w, d.pad_top, d.pad_left,
                         OH, OW, bf16_round_host(d.pad_value), d.relu, d.relu_threshold);
    HIP_TRY(hipGetLastError());
    return 0;
  }
  xtc_hip_tile t = d.tile;
  int split_k = d.split_k;
  if (t.bm == 0) {
    int sk = 1;
    default_conv_tile(d, OH, OW, &t, &sk);
    if (split_k <= 0) split_k = sk;
  }
  const GemmEntry* e = find_entry(d.dtype, 1, t);
  if (!e)
    return fail("no conv2d kernel instance for dtype %d tile %dx%dx%d waves %dx%d", d.dtype,
                t.bm, t.bn, t.bk, t.wgm, t.wgn);
  if (f64) {
    GemmArgs64 a;
    memset(&a, 0, sizeof(a));
    a.A = (const double*)input;
    a.B = (const double*)weight;
    a.C = (double*)outv;
    a.bias = (const double*)biasv;
    a.M = M;
    a.N = d.F;
    a.K = K;
    a.lda = K;
    a.ldb = d.F;
    a.ldc = d.F;
    a.relu = d.relu;
    a.relu_threshold = d.relu_threshold_f64;
    a.cH = d.H;
    a.cW = d.W;
    a.cC = d.C;
    a.cOH = OH;
    a.cOW = OW;
    a.cS = d.S;
    a.cSH = d.stride_h;
    a.cSW = d.stride_w;
    a.cPH = d.pad_top;
    a.cPW = d.pad_left;
    a.pad_value = d.pad_value_f64;
    Scratch x{s};
    return launch_f64_common(a, f64_tile(1, t), split_k, d.group_m, d.xcd_remap, x);
  }
  if (direct_conv_applies(d, t, split_k, OH, OW, input, weight, out, bias))
    return launch_direct_conv(d, t, OH, OW, input, weight, out, bias, s);
  if (!e->launch)
    return fail("conv2d tile %dx%dx%d waves %dx%d exists only in the direct conv kernel, which needs fp32, no "
                "split-K, C and F multiples of 64, 16-byte aligned operands and an input halo that fits its "
                "LDS buffer",
                t.bm, t.bn, t.bk, t.wgm, t.wgn);
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  a.A = input;
  a.B = weight;
  a.C = out;
  a.bias = bias;
  a.M = M;
  a.N = d.F;
  a.K = K;
  a.lda = K;
  a.ldb = d.F;
  a.ldc = d.F;
  a.relu = d.relu;
  a.relu_threshold = d.relu_threshold;
  a.cH = d.H;
  a.cW = d.W;
  a.cC = d.C;
  a.cOH = OH;
  a.cOW = OW;
  a.cS = d.S;
  a.cSH = d.stride_h;
  a.cSW = d.stride_w;
  a.cPH = d.pad_top;
  a.cPW = d.pad_left;
  a.pad_value = d.pad_value;
  Scratch x{s};
  return launch_gemm_common(a, e, split_k, 0, d.group_m, d.xcd_remap, x);
}

int xtc_hip_relu(const float* x, float* y, uint64_t n, float threshold, void* stream) {
  if (!current_state()) return fail("xtc_hip_init not called");
  if (n == 0) return 0;
  if (!x || !y) return fail("null operand");
  if (!aligned16(x) || !aligned16(y)) return fail("relu: operands must be 16-byte aligned");
  hipLaunchKernelGGL(relu_kernel, dim3(grid_for((n + 3) / 4, 256)), dim3(256), 0,
                     pick_stream(stream), x, y, n, threshold);
  HIP_TRY(hipGetLastError());
  return 0;
}

int xtc_hip_pad(const float* x, float* y, int ndim, const int64_t* shape, const int64_t* before,
                const int64_t* after, float value, void* stream) {
  if (!current_state()) return fail("xtc_hip_init not called");
  if (ndim < 1 || ndim > 8) return fail("pad: rank %d unsupported", ndim);
  if (!x || !y || !shape || !before || !after) return fail("null operand");
  PadDims d;
  memset(&d, 0, sizeof(d));
  d.ndim = ndim;
  uint64_t total = 1;
  for (int k = 0; k < ndim; ++k) {
    if (shape[k] < 0 || before[k] < 0 || after[k] < 0) return fail("pad: negative extent");
    d.in_shape[k] = shape[k];
    d.before[k] = before[k];
    d.out_shape[k] = shape[k] + before[k] + after[k];
    total *= (uint64_t)d.out_shape[k];
  }
  if (total == 0) return 0;
  const int last = ndim - 1;
  if (before[last] == 0 && after[last] == 0 && shape[last] % 4 == 0 && aligned16(x) && aligned16(y)) {
    hipLaunchKernelGGL(pad_rows_kernel, dim3(grid_for(total / 4, 256)), dim3(256), 0, pick_stream(stream),
                       (const float4*)x, (float4*)y, d, total / 4, value);
    HIP_TRY(hipGetLastError());
    return 0;
  }
  hipLaunchKernelGGL(pad_kernel, dim3(grid_for(total, 256)), dim3(256), 0, pick_stream(stream),
                     x, y, d, total, value);
  HIP_TRY(hipGetLastError());
  return 0;
}

int xtc_hip_relu_f64(const double* x, double* y, uint64_t n, double threshold, void* stream) {
  if (!current_state()) return fail("xtc_hip_init not called");
  if (n == 0) return 0;
  if (!x || !y) return fail("null operand");
  hipLaunchKernelGGL(relu_f64_kernel, dim3(grid_for(n, 256)), dim3(256), 0, pick_stream(stream), x, y, n, threshold);
  HIP_TRY(hipGetLastError());
  return 0;
}

int xtc_hip_pad_f64(const double* x, double* y, int ndim, const int64_t* shape, const int64_t* before,
                    const int64_t* after, double value, void* stream) {
  if (!current_state()) return fail("xtc_hip_init not called");
  if (ndim < 1 || ndim > 8) return fail("pad: rank %d unsupported", ndim);
  if (!x || !y || !shape || !before || !after) return fail("null operand");
  PadDims d;
  memset(&d, 0, sizeof(d));
  d.ndim = ndim;
  uint64_t total = 1;
  for (int k = 0; k < ndim; ++k) {
    if (shape[k] < 0 || before[k] < 0 || after[k] < 0) return fail("pad: negative extent");
    d.in_shape[k] = shape[k];
    d.before[k] = before[k];
    d.out_shape[k] = shape[k] + before[k] + after[k];
    total *= (uint64_t)d.out_shape[k];
  }
  if (total == 0) return 0;
  hipLaunchKernelGGL(pad_f64_kernel, dim3(grid_for(total, 256)), dim3(256), 0, pick_stream(stream), x, y, d, total,
                     value);
  HIP_TRY(hipGetLastError());
  return 0;
}

int xtc_hip_unpad(const void* x, void* y, int elem_bytes, int ndim, const int64_t* shape, const int64_t* before,
                  const int64_t* after, void* stream) {
  if (!current_state()) return fail("xtc_hip_init not called");
  if (ndim < 1 || ndim > 8) return fail("unpad: rank %d unsupported", ndim);
  if (elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8) return fail("unpad: element size %d unsupported", elem_bytes);
  if (!x || !y || !shape || !before || !after) return fail("null operand");
  PadDims d;
  memset(&d, 0, sizeof(d));
  d.ndim = ndim;
  uint64_t total = 1;
  for (int k = 0; k < ndim; ++k) {
    if (shape[k] < 0 || before[k] < 0 || after[k] < 0) return fail("unpad: negative extent");
    if (before[k] + after[k] > shape[k])
      return fail("unpad: crop %lld + %lld exceeds dim %d of size %lld", (long long)before[k], (long long)after[k], k,
                  (long long)shape[k]);
    d.in_shape[k] = shape[k];
    d.before[k] = before[k];
    d.out_shape[k] = shape[k] - before[k] - after[k];
    total *= (uint64_t)d.out_shape[k];
  }
  if (total == 0) return 0;
  const int last = ndim - 1;
  const int64_t row_bytes = shape[last] * elem_bytes;
  if (before[last] == 0 && after[last] == 0 && row_bytes % 16 == 0 && aligned16(x) && aligned16(y)) {
    const uint64_t total16 = total * (uint64_t)elem_bytes / 16;
    hipLaunchKernelGGL(unpad_rows_kernel, dim3(grid_for(total16, 256)), dim3(256), 0, pick_stream(stream),
                       (const uint4*)x, (uint4*)y, d, total16, row_bytes / 16);
  } else if (elem_bytes == 2) {
    hipLaunchKernelGGL(unpad_kernel<uint16_t>, dim3(grid_for(total, 256)), dim3(256), 0, pick_stream(stream),
                       (const uint16_t*)x, (uint16_t*)y, d, total);
  } else if (elem_bytes == 4) {
    hipLaunchKernelGGL(unpad_kernel<uint32_t>, dim3(grid_for(total, 256)), dim3(256), 0, pick_stream(stream),
                       (const uint32_t*)x, (uint32_t*)y, d, total);
  } else {
    hipLaunchKernelGGL(unpad_kernel<uint64_t>, dim3(grid_for(total, 256)), dim3(256), 0, pick_stream(stream),
                       (const uint64_t*)x, (uint64_t*)y, d, total);
  }
  HIP_TRY(hipGetLastError());
  return 0;
}

int xtc_hip_cast_f32_to_bf16(const float* x, uint16_t* y, uint64_t n, void* stream) {
  if (!current_state()) return fail("xtc_hip_init not called");
  if (n == 0) return 0;
  const int vec = aligned16(x) && aligned16(y);
  hipLaunchKernelGGL(cast_f32_bf16_kernel, dim3(grid_for(vec ? (n + 7) / 8 : n, 256)), dim3(256), 0,
                     pick_stream(stream), x, y, n, vec);
  HIP_TRY(hipGetLastError());
  return 0;
}

int xtc_hip_cast_bf16_to_f32(const uint16_t* x, float* y, uint64_t n, void* stream) {
  if (!current_state()) return fail("xtc_hip_init not called");
  if (n == 0) return 0;
  const int vec = aligned16(x) && aligned16(y);
  hipLaunchKernelGGL(cast_bf16_f32_kernel, dim3(grid_for(vec ? (n + 7) / 8 : n, 256)), dim3(256), 0,
                     pick_stream(stream), x, y, n, vec);
  HIP_TRY(hipGetLastError());
  return 0;
}

// ------------------------------------------------------------ timing harness

typedef void (*fn0)(void);
typedef void (*fn8)(void*, void*, void*, void*, void*, void*, void*, void*);

static inline void call_payload(void (*func)(void), void** args, int nargs) {
  void* a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int i = 0; i < nargs && i < 8; ++i) a[i] = args[i];
  // Extra trailing arguments are ignored by the callee under the SysV ABI.
  ((fn8)func)(a[0], a[1], a[2], a[3], a[4], a[5], a[6], a[7]);
}

}  // extern "C"

namespace {

// Entry points of libxtc_hip_pmu.so (include/xtc_hip_pmu.h), found in the
// process when it was loaded with global symbols and its tool initialised.
struct PmuHooks {
  int (*ready)(void);
  int (*open)(int, int, const char**, int*);
  int (*start)(void);
  int (*stop)(double*, int);
  void (*close)(void);
};

bool pmu_hooks(PmuHooks* h) {
  h->ready = (int (*)(void))dlsym(RTLD_DEFAULT, "xtc_hip_pmu_ready");
  h->open = (int (*)(int, int, const char**, int*))dlsym(RTLD_DEFAULT, "xtc_hip_pmu_open");
  h->start = (int (*)(void))dlsym(RTLD_DEFAULT, "xtc_hip_pmu_start");
  h->stop = (int (*)(double*, int))dlsym(RTLD_DEFAULT, "xtc_hip_pmu_stop");
  h->close = (void (*)(void))dlsym(RTLD_DEFAULT, "xtc_hip_pmu_close");
  return h->ready && h->open && h->start && h->stop && h->close && h->ready();
}

constexpr int kMaxEvents = 64;
thread_local int g_eval_status = 0;

// Host counters of the reference's perf_event backend, by the names of
// perf_event_linux.c:37-54 (generic hardware and software events of
// perf_event_open; names that need libpfm are not known here).
struct HostEventDecl {
  const char* name;
  uint32_t type;
  uint64_t config;
};
const HostEventDecl kHostEvents[] = {
    {"cycles", PERF_TYPE_HARDWARE, PERF_COUNT_HW_CPU_CYCLES},
    {"clocks", PERF_TYPE_SOFTWARE, PERF_COUNT_SW_CPU_CLOCK},
    {"instructions", PERF_TYPE_HARDWARE, PERF_COUNT_HW_INSTRUCTIONS},
    {"migrations", PERF_TYPE_SOFTWARE, PERF_COUNT_SW_CPU_MIGRATIONS},
    {"context_switches", PERF_TYPE_SOFTWARE, PERF_COUNT_SW_CONTEXT_SWITCHES},
    {"cache_access", PERF_TYPE_HARDWARE, PERF_COUNT_HW_CACHE_REFERENCES},
    {"cache_misses", PERF_TYPE_HARDWARE, PERF_COUNT_HW_CACHE_MISSES},
    {"branches", PERF_TYPE_HARDWARE, PERF_COUNT_HW_BRANCH_INSTRUCTIONS},
    {"branches_misses", PERF_TYPE_HARDWARE, PERF_COUNT_HW_BRANCH_MISSES},
};

// A counting perf event for `name` on the calling process, user space only,
// inherited by threads it creates later (the attributes of
// perf_event_linux.c:72-81); -1 if the name is unknown or the kernel refuses
// it (no hardware PMU, perf_event_paranoid).
int open_host_event(const char* name) {
  for (const HostEventDecl& d : kHostEvents) {
    if (strcmp(name, d.name)) continue;
    struct perf_event_attr attr;
    memset(&attr, 0, sizeof(attr));
    attr.size = sizeof(attr);
    attr.type = d.type;
    attr.config = d.config;
    attr.exclude_kernel = 1;
    attr.exclude_hv = 1;
    attr.exclude_idle = 1;
    attr.inherit = 1;
    return (int)syscall(SYS_perf_event_open, &attr, 0, -1, -1, 0);
  }
  return -1;
}

uint64_t read_host_event(int fd) {
  uint64_t v = 0;
  if (read(fd, &v, sizeof(v)) != (ssize_t)sizeof(v)) return 0;
  return v;
}

}  // namespace

extern "C" {

void xtc_hip_evaluate_perf(double* results, int events_num, const char* events_names[],
                           int repeat, int number, int min_repeat_ms, void (*func)(void),
                           void** args, int nargs) {
  g_eval_status = 0;
  g_last_error.clear();
  if (!results || repeat <= 0 || number < 0 || min_repeat_ms < 0 || !func || nargs < 0 || nargs > 8 ||
      events_num < 0 || (events_num > 0 && !events_names)) {
    g_eval_status = 1;
    fail("evaluate_perf: invalid arguments");
    return;
  }
  if (events_num > kMaxEvents) {
    g_eval_status = 1;
    fail("evaluate_perf: %d events requested, at most %d", events_num, kMaxEvents);
    return;
  }
  // event kinds: 0 unknown, 1 gpu.time (s), 2 gpu.clocks (ns), 3 hardware
  // counter gpu.<name> (gpu.cycles = GRBM_GUI_ACTIVE, the GPU's busy cycles)
  // read through libxtc_hip_pmu when the process loaded and enabled it, 4 a
  // host counter of perf_event_open (perf_event_linux.c:37-54 names)
  int kinds[kMaxEvents] = {0};
  const char* pmu_names[kMaxEvents];
  int pmu_of_event[kMaxEvents];
  int pmu_slot[kMaxEvents];
  int host_fd[kMaxEvents];
  uint64_t host_start[kMaxEvents] = {0};
  double host_delta[kMaxEvents] = {0};
  int npmu = 0;
  for (int e = 0; e < events_num; ++e) {
    const char* n = events_names[e];
    host_fd[e] = -1;
    kinds[e] = (n && !strcmp(n, "gpu.time")) ? 1 : (n && !strcmp(n, "gpu.clocks")) ? 2 : 0;
    if (kinds[e] == 0 && n && !strncmp(n, "gpu.", 4)) {
      kinds[e] = 3;
      pmu_of_event[e] = npmu;
      pmu_names[npmu++] = !strcmp(n + 4, "cycles") ? "GRBM_GUI_ACTIVE" : n + 4;
    } else if (kinds[e] == 0 && n) {
      host_fd[e] = open_host_event(n);
      if (host_fd[e] >= 0) kinds[e] = 4;
    }
  }
  PmuHooks pmu;
  const bool pmu_on = npmu > 0 && pmu_hooks(&pmu) && pmu.open(g_current, npmu, pmu_names, pmu_slot) == 0;
  double pmu_sums[kMaxEvents] = {0};
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  bool use_events = false;
  for (int e = 0; e < events_num; ++e) use_events = use_events || kinds[e] == 1 || kinds[e] == 2;
  use_events = use_events && current_state();
  if (use_events) {
    hipEventCreate(&ev0);
    hipEventCreate(&ev1);
  }
  if (number > 0) {
    call_payload(func, args, nargs);
  } else {
    number = 1;
  }
  for (int r = 0; r < repeat; ++r) {
    int attempts = number;
    double elapsed;
    float dev_ms = 0.f;
    bool pmu_ok = pmu_on;
    while (1) {
      if (pmu_on) pmu_ok = pmu.start() == 0;
      if (use_events) hipEventRecord(ev0, current_state()->stream);
      for (int e = 0; e < events_num; ++e)
        if (kinds[e] == 4) host_start[e] = read_host_event(host_fd[e]);
      double t0 = now_s();
      for (int a = 0; a < attempts; ++a) call_payload(func, args, nargs);
      elapsed = now_s() - t0;
      for (int e = 0; e < events_num; ++e)
        if (kinds[e] == 4) host_delta[e] = (double)(read_host_event(host_fd[e]) - host_start[e]);
      if (use_events) {
        hipEventRecord(ev1, current_state()->stream);
        hipEventSynchronize(ev1);
        hipEventElapsedTime(&dev_ms, ev0, ev1);
      }
      if (pmu_on) {
        hipDeviceSynchronize();  // every dispatch of the window has completed
        pmu_ok = pmu.stop(pmu_sums, kMaxEvents) == 0 && pmu_ok;
      }
      if (elapsed * 1000.0 >= (double)min_repeat_ms) break;
      attempts *= 2;
    }
    if (events_num > 0) {
      for (int e = 0; e < events_num; ++e) {
        double v = -1.0;
        if (use_events && kinds[e] == 1) v = (double)dev_ms * 1e-3 / attempts;
        if (use_events && kinds[e] == 2) v = (double)dev_ms * 1e6 / attempts;
        if (kinds[e] == 3 && pmu_ok && pmu_slot[pmu_of_event[e]] >= 0)
          v = pmu_sums[pmu_slot[pmu_of_event[e]]] / attempts;
        if (kinds[e] == 4) v = host_delta[e] / attempts;
        results[r * events_num + e] = v;
      }
    } else {
      results[r] = elapsed / attempts;
    }
  }
  for (int e = 0; e < events_num; ++e)
    if (host_fd[e] >= 0) close(host_fd[e]);
  if (pmu_on) pmu.close();
  if (use_events) {
    hipEventDestroy(ev0);
    hipEventDestroy(ev1);
  }
}

int xtc_hip_evaluate_status(void) { return g_eval_status; }

void xtc_hip_evaluate(double* results, int repeat, int number, int min_repeat_ms,
                      void (*func)(void), void** args, int nargs) {
  xtc_hip_evaluate_perf(results, 0, nullptr, repeat, number, min_repeat_ms, func, args, nargs);
}

double xtc_hip_datasheet_flops(const char* dtype) {
  // Published dense MFMA peaks of MI355X (256 CUs at 2.4 GHz), in FMA/s.
  if (!dtype) return 0.0;
  if (!strcmp(dtype, "float32")) return 157.3e12 / 2.0;
  if (!strcmp(dtype, "bfloat16") || !strcmp(dtype, "float16")) return 2516.6e12 / 2.0;
  if (!strcmp(dtype, "float64")) return 78.6e12 / 2.0;
  return 0.0;
}

double xtc_hip_evaluate_flops_operands(const char* dtype, int operands) {
  DeviceState* d = current_state();
  if (!d) {
    fail("evaluate_flops: xtc_hip_init not called");
    return 0.0;
  }
  const bool bf16 = dtype && !strcmp(dtype, "bfloat16");
  const bool f32 = dtype && !strcmp(dtype, "float32");
  const bool f64 = dtype && !strcmp(dtype, "float64");
  if ((!bf16 && !f32 && !f64) || operands < 0 || operands > 2) {
    fail("evaluate_flops: unsupported dtype %s or operands %d", dtype ? dtype : "(null)", operands);
    return 0.0;
  }
  using namespace peak;
  const int blocks = 2 * (d->cus > 0 ? d->cus : 256);
  const size_t waves = (size_t)blocks * (kThreads / 64);
  const size_t words = waves * 64 * (bf16 ? kBf16Frags * 8 : f64 ? kF64Frags : kF32Frags);  // bf16 halves, floats, doubles
  // operand words: the reference's integers 1 + i % 127 (evaluate_flops.c:466-469),
  // zeros, or uniform [-1, 1) from a fixed LCG (bf16: rounded to nearest even)
  std::vector<uint16_t> h16(bf16 ? words : 0);
  std::vector<float> h32(bf16 || f64 ? 0 : words);
  std::vector<double> h64(f64 ? words : 0);
  uint64_t lcg = 0x9e3779b97f4a7c15ull;
  for (size_t i = 0; i < words; ++i) {
    float v = 0.f;
    if (operands == 0) {
      v = (float)(1 + i % 127);
    } else if (operands == 2) {
      lcg = lcg * 6364136223846793005ull + 1442695040888963407ull;
      v = (float)((lcg >> 40) * (1.0 / 16777216.0)) * 2.f - 1.f;
    }
    if (bf16) {
      unsigned u;
      memcpy(&u, &v, 4);
      h16[i] = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    } else if (f64) {
      h64[i] = v;
    } else {
      h32[i] = v;
    }
  }
  const size_t in_bytes = words * (bf16 ? 2 : f64 ? 8 : 4);
  void *in = nullptr, *out = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  double best = 0.0;
  // ~20 ms per launch at the datasheet rate
  const int iters = bf16 ? 48000 : 12000;
  const double fmas = (double)waves * iters * (bf16 ? kBf16FmaPerRound : f64 ? kF64FmaPerRound : kF32FmaPerRound);
  auto launch = [&]() {
    if (f64)
      hipLaunchKernelGGL(mfma_peak_f64, dim3(blocks), dim3(kThreads), 0, d->stream, (const double*)in, (float*)out,
                         iters);
    else if (bf16)
      hipLaunchKernelGGL(mfma_peak_bf16, dim3(blocks), dim3(kThreads), 0, d->stream, (const u32x4*)in,
                         (float*)out, iters);
    else
      hipLaunchKernelGGL(mfma_peak_f32, dim3(blocks), dim3(kThreads), 0, d->stream, (const float*)in,
                         (float*)out, iters);
  };
  bool ok = hipMalloc(&in, in_bytes) == hipSuccess && hipMalloc(&out, (size_t)blocks * kThreads * 4) == hipSuccess &&
            hipMemcpyAsync(in, bf16 ? (const void*)h16.data() : f64 ? (const void*)h64.data() : (const void*)h32.data(), in_bytes,
                           hipMemcpyHostToDevice, d->stream) == hipSuccess &&
            hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess;
  if (ok) {
    launch();  // cold run
    // three batches of 5 launches back to back (~100 ms each, long enough for
    // the clock to settle at the power limit); the best batch's rate
    for (int rep = 0; ok && rep < 3; ++rep) {
      ok = hipEventRecord(e0, d->stream) == hipSuccess;
      for (int l = 0; l < 5; ++l) launch();
      ok = ok && hipGetLastError() == hipSuccess && hipEventRecord(e1, d->stream) == hipSuccess &&
           hipEventSynchronize(e1) == hipSuccess;
      float ms = 0.f;
      ok = ok && hipEventElapsedTime(&ms, e0, e1) == hipSuccess && ms > 0.f;
      if (ok && 5 * fmas / (ms * 1e-3) > best) best = 5 * fmas / (ms * 1e-3);
    }
  }
  if (e0) hipEventDestroy(e0);
  if (e1) hipEventDestroy(e1);
  hipStreamSynchronize(d->stream);
  if (in) hipFree(in);
  if (out) hipFree(out);
  if (!ok) {
    fail("evaluate_flops: the MFMA probe failed");
    return 0.0;
  }
  return best;
}

double xtc_hip_evaluate_flops(const char* dtype) { return xtc_hip_evaluate_flops_operands(dtype, 0); }

}  // extern "C"
