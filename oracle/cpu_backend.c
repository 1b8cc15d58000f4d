/*
 * SPDX-License-Identifier: BSD-3-Clause
 *
 * TEST INFRASTRUCTURE -- the CPU baseline, not part of the product.
 *
 * C restatement of what XTC's MLIR `llvmir` CPU backend compiles a scheduled
 * matmul / conv2d into (the MLIR toolchain it shells out to is not installable
 * offline).  The loop structure is the `tile_oo` scheme of the reference's
 * strategies (src/xtc/search/strategies.py:351-758, order i, k, j, i1, k1, j1
 * with the outer i loop parallel, j1 vectorised and the inner tiles unrolled),
 * lowered the way the reference lowers it:
 *   - tile extents as sub-loop extents, parent loops stepping by them
 *     (src/xtc/backends/mlir/MlirCompilerPasses.py:414-457);
 *   - parallel outer loop -> OpenMP (MlirLLVMTarget.py:279-332,
 *     convert-scf-to-openmp);
 *   - linalg.fill(0) then accumulate (MlirOps.py:189-270);
 *   - -O3 -march=native with FP contraction, as `opt -O2 --fp-contract=fast`
 *     + `cc -O3 -march=native` (src/xtc/utils/ext_tools.py:56-67).
 * Tile sizes are compile-time constants of each variant, as in the code MLIR
 * emits for one schedule; the driver (cpu_baseline.py) "auto-schedules" by
 * timing every variant and keeping the best, like loop-explore does.
 *
 * Conv2d: NHWC x RSCF -> NHWC, direct loop nest b, h, w, r, s, c, f with the
 * (b, h) loops parallel and f vectorised (MlirOps.py:349-404 index map); the
 * input is taken already padded, as XTC's conv2d has no implicit padding
 * (src/xtc/graphs/xtc/operators.py:326-347).
 */
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define MIN(a, b) ((a) < (b) ? (a) : (b))

/* C[M,N] = A[M,K] @ B[K,N], fp32, row-major.  One variant per (TI, TK, TJ). */
#define DEFINE_MATMUL(TI, TK, TJ) DEFINE_MATMUL_FN(matmul_##TI##_##TK##_##TJ, TI, TK, TJ)
#define DEFINE_MATMUL_FN(NAME, TI, TK, TJ)                                               \
  static void NAME(const float *restrict A, const float *restrict B,                     \
                   float *restrict C, int M, int N, int K) {                             \
    _Pragma("omp parallel for schedule(static)") for (int i0 = 0; i0 < M; i0 += TI) {    \
      const int ie = MIN(i0 + TI, M);                                                    \
      for (int i = i0; i < ie; ++i) memset(C + (int64_t)i * N, 0, sizeof(float) * N);    \
      for (int k0 = 0; k0 < K; k0 += TK) {                                               \
        const int ke = MIN(k0 + TK, K);                                                  \
        for (int j0 = 0; j0 < N; j0 += TJ) {                                             \
          const int je = MIN(j0 + TJ, N);                                                \
          for (int i = i0; i < ie; ++i) {                                                \
            float *restrict c = C + (int64_t)i * N;                                      \
            for (int k = k0; k < ke; ++k) {                                              \
              const float a = A[(int64_t)i * K + k];                                     \
              const float *restrict b = B + (int64_t)k * N;                              \
              _Pragma("omp simd") for (int j = j0; j < je; ++j) c[j] += a * b[j];        \
            }                                                                            \
          }                                                                              \
        }                                                                                \
      }                                                                                  \
    }                                                                                    \
  }

#if defined(XTC_CPU_PPRPRP)
/* One sampled schedule of the reference's tile_pprprp strategies
 * (src/xtc/search/strategies.py:772-826: order i, j, i1, j1, k, i2, j2, k1,
 * i3, j3; i and j parallel, j3 vectorised, the inner tiles i3, k1, j3
 * unrolled), built alone with its tile extents as compile-time constants:
 * -DXTC_CPU_I1/I2/I3 (extents of the i1, i2, i3 tiles), J1/J2/J3, K1.  Loop
 * i steps by I1 and i1 walks it by I2, i2 by I3, as XTC lowers tiles
 * (MlirCompilerPasses.py:414-457); the two parallel outer loops form one
 * OpenMP iteration space (scf.forall over both, convert-scf-to-openmp).
 * The fill node (linalg.fill 0) runs over each (i, j) block before its
 * accumulation.  The extents divide the matrix sizes, as the strategy
 * samples divisors. */
#define XI1 XTC_CPU_I1
#define XI2 XTC_CPU_I2
#define XI3 XTC_CPU_I3
#define XJ1 XTC_CPU_J1
#define XJ2 XTC_CPU_J2
#define XJ3 XTC_CPU_J3
#define XK1 XTC_CPU_K1

static void matmul_sched(const float *restrict A, const float *restrict B, float *restrict C, int M, int N,
                         int K) {
  const int nbi = M / XI1, nbj = N / XJ1;
#pragma omp parallel for collapse(2) schedule(static)
  for (int bi = 0; bi < nbi; ++bi) {
    for (int bj = 0; bj < nbj; ++bj) {
      const int i0 = bi * XI1, j0 = bj * XJ1;
      for (int i = i0; i < i0 + XI1; ++i) memset(C + (int64_t)i * N + j0, 0, sizeof(float) * XJ1);
      for (int i1 = i0; i1 < i0 + XI1; i1 += XI2) {
        for (int j1 = j0; j1 < j0 + XJ1; j1 += XJ2) {
          for (int k = 0; k < K; k += XK1) {
            for (int i2 = i1; i2 < i1 + XI2; i2 += XI3) {
              for (int j2 = j1; j2 < j1 + XJ2; j2 += XJ3) {
                float acc[XI3][XJ3];
#pragma GCC unroll 64
                for (int i3 = 0; i3 < XI3; ++i3)
#pragma omp simd
                  for (int j3 = 0; j3 < XJ3; ++j3) acc[i3][j3] = C[(int64_t)(i2 + i3) * N + j2 + j3];
#pragma GCC unroll 16
                for (int k1 = 0; k1 < XK1; ++k1) {
                  const float *restrict b = B + (int64_t)(k + k1) * N + j2;
#pragma GCC unroll 64
                  for (int i3 = 0; i3 < XI3; ++i3) {
                    const float a = A[(int64_t)(i2 + i3) * K + k + k1];
#pragma omp simd
                    for (int j3 = 0; j3 < XJ3; ++j3) acc[i3][j3] += a * b[j3];
                  }
                }
#pragma GCC unroll 64
                for (int i3 = 0; i3 < XI3; ++i3)
#pragma omp simd
                  for (int j3 = 0; j3 < XJ3; ++j3) C[(int64_t)(i2 + i3) * N + j2 + j3] = acc[i3][j3];
              }
            }
          }
        }
      }
    }
  }
}

static int g_sched_m, g_sched_n, g_sched_k;

void xtc_cpu_sched_configure(int M, int N, int K) {
  g_sched_m = M;
  g_sched_n = N;
  g_sched_k = K;
}

/* The scheduled matmul called like an XTC module: void f(A, B, C). */
void xtc_cpu_sched_payload(void *A, void *B, void *C) {
  matmul_sched((const float *)A, (const float *)B, (float *)C, g_sched_m, g_sched_n, g_sched_k);
}

int xtc_cpu_sched_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
#elif defined(XTC_CPU_TI) && defined(XTC_CPU_TK) && defined(XTC_CPU_TJ)
/* One sampled schedule, built alone with its tile sizes as compile-time
 * constants (-DXTC_CPU_TI=.. -DXTC_CPU_TK=.. -DXTC_CPU_TJ=..), as the code
 * MLIR emits for one loop-explore sample: i1 = TI, k1 = TK, j1 = TJ of the
 * tile_oo order i, k, j, i1, k1, j1 (oracle/cpu_baseline.py builds one per
 * sample). */
DEFINE_MATMUL_FN(matmul_sched, XTC_CPU_TI, XTC_CPU_TK, XTC_CPU_TJ)

static int g_sched_m, g_sched_n, g_sched_k;

void xtc_cpu_sched_configure(int M, int N, int K) {
  g_sched_m = M;
  g_sched_n = N;
  g_sched_k = K;
}

/* The scheduled matmul called like an XTC module: void f(A, B, C). */
void xtc_cpu_sched_payload(void *A, void *B, void *C) {
  matmul_sched((const float *)A, (const float *)B, (float *)C, g_sched_m, g_sched_n, g_sched_k);
}

int xtc_cpu_sched_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
#else
DEFINE_MATMUL(4, 64, 64)
DEFINE_MATMUL(4, 128, 128)
DEFINE_MATMUL(4, 256, 256)
DEFINE_MATMUL(8, 64, 128)
DEFINE_MATMUL(8, 128, 256)
DEFINE_MATMUL(8, 256, 64)
DEFINE_MATMUL(16, 128, 128)
DEFINE_MATMUL(32, 256, 512)

typedef void (*matmul_fn)(const float *, const float *, float *, int, int, int);

static const struct {
  int ti, tk, tj;
  matmul_fn fn;
} g_variants[] = {
    {4, 64, 64, matmul_4_64_64},      {4, 128, 128, matmul_4_128_128},
    {4, 256, 256, matmul_4_256_256},  {8, 64, 128, matmul_8_64_128},
    {8, 128, 256, matmul_8_128_256},  {8, 256, 64, matmul_8_256_64},
    {16, 128, 128, matmul_16_128_128}, {32, 256, 512, matmul_32_256_512},
};

int xtc_cpu_matmul_variants(void) { return (int)(sizeof(g_variants) / sizeof(g_variants[0])); }

/* Tile sizes (i1, k1, j1) of variant v; returns 0 on success. */
int xtc_cpu_matmul_variant_tiles(int v, int *ti, int *tk, int *tj) {
  if (v < 0 || v >= xtc_cpu_matmul_variants()) return 1;
  *ti = g_variants[v].ti;
  *tk = g_variants[v].tk;
  *tj = g_variants[v].tj;
  return 0;
}

int xtc_cpu_matmul(int v, const float *A, const float *B, float *C, int M, int N, int K) {
  if (v < 0 || v >= xtc_cpu_matmul_variants() || M < 0 || N < 0 || K < 0) return 1;
  g_variants[v].fn(A, B, C, M, N, K);
  return 0;
}

/* O[b,oh,ow,f] = relu?(sum_{r,s,c} I[b, oh*sh+r, ow*sw+s, c] * W[r,s,c,f]),
 * I already padded to (NB, H, W, C). */
int xtc_cpu_conv2d(const float *restrict I, const float *restrict Wt, float *restrict O, int NB,
                   int H, int W, int C, int F, int R, int S, int sh, int sw, int relu) {
  if (NB < 0 || H < R || W < S || sh <= 0 || sw <= 0) return 1;
  const int OH = (H - R) / sh + 1;
  const int OW = (W - S) / sw + 1;
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < NB; ++b) {
    for (int oh = 0; oh < OH; ++oh) {
      for (int ow = 0; ow < OW; ++ow) {
        float *restrict o = O + (((int64_t)b * OH + oh) * OW + ow) * F;
        for (int f = 0; f < F; ++f) o[f] = 0.0f;
        for (int r = 0; r < R; ++r) {
          for (int s = 0; s < S; ++s) {
            const float *restrict in = I + (((int64_t)b * H + oh * sh + r) * W + ow * sw + s) * C;
            const float *restrict w = Wt + ((int64_t)r * S + s) * C * F;
            for (int c = 0; c < C; ++c) {
              const float a = in[c];
              const float *restrict wr = w + (int64_t)c * F;
#pragma omp simd
              for (int f = 0; f < F; ++f) o[f] += a * wr[f];
            }
          }
        }
        if (relu)
          for (int f = 0; f < F; ++f) o[f] = o[f] > 0.0f ? o[f] : (o[f] != o[f] ? o[f] : 0.0f);
      }
    }
  }
  return 0;
}

int xtc_cpu_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void xtc_cpu_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* A configured matmul with the shape baked in, called like an XTC module
 * payload `void matmul(float *A, float *B, float *C)` so the reference's own
 * evaluate_perf harness can time it. */
static int g_cfg_variant, g_cfg_m, g_cfg_n, g_cfg_k;

int xtc_cpu_configure_matmul(int v, int M, int N, int K) {
  if (v < 0 || v >= xtc_cpu_matmul_variants() || M <= 0 || N <= 0 || K <= 0) return 1;
  g_cfg_variant = v;
  g_cfg_m = M;
  g_cfg_n = N;
  g_cfg_k = K;
  return 0;
}

void xtc_cpu_matmul_payload(void *A, void *B, void *C) {
  g_variants[g_cfg_variant].fn((const float *)A, (const float *)B, (float *)C, g_cfg_m, g_cfg_n, g_cfg_k);
}
#endif /* single-schedule build */
