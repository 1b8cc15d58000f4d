/*
 * SPDX-License-Identifier: BSD-3-Clause
 *
 * xtc_hip.h -- C-ABI of libxtc_hip.so, the MI355X (gfx950) execution backend
 * of XTC.  Plain pointers and sizes only; every entry point returns 0 on
 * success and a non-zero status otherwise, with the message available from
 * xtc_hip_last_error().
 *
 * The library has three groups of entry points:
 *
 *  1. Device runtime.  Replaces the mgpu* calls that the reference's
 *     GPUDevice binds through ctypes
 *     (src/xtc/runtimes/accelerator/gpu/GPUDevice.py:36-63,131-207:
 *     mgpuStreamCreate, mgpuMemAlloc, mgpuMemFree, mgpuMemcpy,
 *     mgpuStreamSynchronize).  Host buffers are never registered for
 *     zero-copy access (GPUDevice.py:327-347 mgpuMemHostRegister): tensors are
 *     copied to HBM explicitly, so kernels always read device memory.
 *
 *  2. Operator entry points.  A compiled XTC module is a shared object that
 *     exports `void <graph.name>(void *in0, ..., void *out0, ...)`
 *     (src/xtc/backends/mlir/MlirGraphBackend.py:125-171,
 *     src/xtc/backends/mlir/MlirTarget/MlirLLVMTarget.py:311).  The HIP
 *     compiler emits that function as a few calls to the entry points below,
 *     one per scheduled graph node, followed by xtc_hip_synchronize(), since
 *     callers time the payload with a wall clock around the call
 *     (src/xtc/csrcs/runtimes/host/evaluate_perf.c:92-120).  All operands are
 *     device pointers to dense row-major (C-contiguous) buffers.
 *
 *  3. Timing harness.  Same protocol and signature as the reference runtime's
 *     evaluate_perf / evaluate (src/xtc/csrcs/runtimes/host/evaluate_perf.c:
 *     187-248, bound in src/xtc/runtimes/host/runtime.py:41-145) and the
 *     peak estimate evaluate_flops (evaluate_flops.c:461-494).
 */
#ifndef XTC_HIP_H
#define XTC_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- status */

/* Message of the last failing call on this thread ("" if none). */
const char *xtc_hip_last_error(void);

/* ---------------------------------------------------------- device runtime */

/* Number of visible GPUs (0 when no GPU/driver); never initialises a device. */
int xtc_hip_device_count(void);

/* Selects `device` on the calling thread and creates the library stream
 * (default priority).  Idempotent.  Replaces GPUDevice.__init_once__
 * (GPUDevice.py:45-63). */
int xtc_hip_init(int device);

/* gcnArchName ("gfx950:sramecc+:xnack-") and marketing name of the device. */
int xtc_hip_device_arch(char *buf, int len);
int xtc_hip_device_name(char *buf, int len);

/* The library stream (hipStream_t) used when a descriptor's stream is NULL. */
void *xtc_hip_stream(void);

/* Waits for all work on the library stream (mgpuStreamSynchronize). */
int xtc_hip_synchronize(void);

/* A caller-owned stream of default priority on the current device
 * (mgpuStreamCreate, GPUDevice.py:54-62), for the descriptors' `stream`
 * field; waiting on one (mgpuStreamSynchronize, GPUDevice.py:171-178,
 * NULL = the library stream); destroying one after its work is done, which
 * also frees its scratch.  Split-K partial sums and counters and the
 * staging copies of transposed operands are kept per stream, so calls on
 * different streams may overlap; calls on one stream run in order. */
void *xtc_hip_stream_create(void);
int xtc_hip_stream_synchronize(void *stream);
int xtc_hip_stream_destroy(void *stream);

/* Frees the scratch the library holds for `stream` (split-K workspace and
 * counters, transpose staging) once the stream's queued work is done,
 * without destroying the stream: for streams the caller created itself and
 * destroys with hipStreamDestroy.  A later call on the stream allocates its
 * scratch again.  A stream's scratch is grown while the call that needs it
 * is being queued, so one stream is driven by one host thread at a time. */
int xtc_hip_stream_release(void *stream);

/* Device memory (mgpuMemAlloc / mgpuMemFree). NULL on failure. */
void *xtc_hip_malloc(uint64_t bytes);
int xtc_hip_free(void *ptr);

/* Synchronous copies on the library stream (mgpuMemcpy + sync). */
int xtc_hip_memcpy_h2d(void *dst_device, const void *src_host, uint64_t bytes);
int xtc_hip_memcpy_d2h(void *dst_host, const void *src_device, uint64_t bytes);
int xtc_hip_memcpy_d2d(void *dst_device, const void *src_device, uint64_t bytes);

/* Zero-fills device memory with a kernel (AcceleratorDevice.memory_fill_zero,
 * src/xtc/itf/runtime/accelerator.py:104-112). */
int xtc_hip_memset_zero(void *ptr, uint64_t bytes);

/* Events on the library stream, for kernel-only timing. */
void *xtc_hip_event_create(void);
int xtc_hip_event_record(void *event, void *stream);
int xtc_hip_event_elapsed_ms(void *start, void *stop, float *ms);
int xtc_hip_event_destroy(void *event);

/* ------------------------------------------------------ operator entry points */

/* Operand types.  fp32 and bf16 operands accumulate and store fp32; fp64
 * operands accumulate and store fp64 (the float64 graphs that the reference's
 * MLIR backend lowers, MlirOps.py:194-195,234,339). */
enum xtc_hip_dtype { XTC_HIP_F32 = 0, XTC_HIP_BF16 = 1, XTC_HIP_F64 = 2 };

/* Kernel template parameters a schedule maps to (block tile BM x BN, K slab
 * BK, WGM x WGN waves).  All zero means "library default for the shape". */
typedef struct {
  int bm, bn, bk, wgm, wgn;
} xtc_hip_tile;

/* C[M,N] = relu?( op(A)[M,K] @ op(B)[K,N] + bias[N]? ): fp32 output (and fp32
 * bias) for fp32 / bf16 operands, fp64 output and bias for fp64 operands.
 * Replaces the scheduled linalg.fill + linalg.matmul pair of
 * MlirOperatorMatmul.generate_op (src/xtc/backends/mlir/MlirOps.py:189-270),
 * with XTCOperMatmul semantics (src/xtc/graphs/xtc/operators.py:159-221):
 * A is the input viewed as (shape[0], prod(rest)), B as (prod(rest[:-1]),
 * last).  The relu node of XTCOperRelu (operators.py:224-249) may be fused
 * as the epilogue: out = max(out, relu_threshold), NaN preserved.
 * trans_a / trans_b are the operand layouts of XTC tensor types: layout
 * [1, 0] stores the operand transposed (MlirOperatorMatmul.args_from_operation
 * and its transposed indexing maps, MlirOps.py:171-178,213-254; NDArray's
 * transposed storage, src/xtc/runtimes/types/ndarray.py:70-102).  With
 * trans_a, A is read from At[K][lda >= M]; with trans_b, B from Bt[N][ldb >= K]. */
typedef struct {
  int dtype;             /* xtc_hip_dtype of A and B; C is fp64 for XTC_HIP_F64, else fp32 */
  int M, N, K;
  int lda, ldb, ldc;     /* row strides in elements of the stored matrices, 0 = dense */
  xtc_hip_tile tile;
  int split_k;           /* >= 1: K partitions, summed inside the launch */
  int group_m;           /* raster group height in tiles, 0 = default */
  int xcd_remap;         /* 1 = map consecutive tiles onto one XCD */
  int relu;
  float relu_threshold;
  void *stream;          /* hipStream_t, NULL = library stream */
  int trans_a;           /* 1: A stored transposed, [K][lda] */
  int trans_b;           /* 1: B stored transposed, [N][ldb] */
  int stages;            /* pipeline depth (LDS stages), 0 = the kernel's default;
                            xtc_hip_matmul_pipeline_depths lists the legal ones */
  double relu_threshold_f64; /* the relu threshold of XTC_HIP_F64 calls (an fp32
                                threshold cannot hold every fp64 value) */
} xtc_hip_matmul_desc;

int xtc_hip_matmul(const xtc_hip_matmul_desc *desc, const void *A, const void *B,
                   void *C, const void *bias);

/* Per-device scratch of xtc_hip_matmul_noalloc: 64 MiB. */
#define XTC_HIP_NOALLOC_SCRATCH_BYTES (64u << 20)

/* xtc_hip_matmul that allocates nothing (no hipMalloc/hipFree, no library
 * allocation).  It has no counterpart in the reference: it is for callers
 * that cannot allocate device memory, such as code under HIP graph capture,
 * tight serving loops and harnesses that forbid allocation.  Same arguments,
 * kernels and results as xtc_hip_matmul.  Its scratch -- split-K partial sums
 * ([splits][M][N] fp32, or [splits][16][N] for the skinny kernel), one
 * arrival counter per output tile, and dense copies of transposed operands
 * that the kernels cannot read in place -- comes from one static array per
 * device of XTC_HIP_NOALLOC_SCRATCH_BYTES, set up by xtc_hip_init.  A call
 * that needs more fails with a message instead of launching its GEMM.  The
 * counters are cleared by a kernel on the call's stream before the GEMM.
 * Every call on a device shares that device's array, whatever its stream:
 * calls that overlap on one device race, so callers order them (one stream,
 * or a wait between streams). */
int xtc_hip_matmul_noalloc(const xtc_hip_matmul_desc *desc, const void *A,
                           const void *B, void *C, const void *bias);

/* O[b,oh,ow,f] = relu?( sum_{r,s,c} Ipad[b,oh*sh+r,ow*sw+s,c] * W[r,s,c,f] )
 * NHWC x RSCF -> NHWC (XTCOperConv2D, operators.py:252-347;
 * MlirOperatorConv2D, MlirOps.py:304-441).  Ipad is I padded by
 * (pad_top, pad_bottom, pad_left, pad_right) with pad_value: the XTCOperPad2D
 * producer (operators.py:350-591, MlirOps.py:719-735) fused into the loader.
 * Output and bias are fp32 for fp32 / bf16 operands and fp64 for fp64 ones.
 * Channel counts that are not whole 16-byte vectors are staged with zero
 * channels (or run on a scalar kernel when the filters are not either). */
typedef struct {
  int dtype;
  int N, H, W, C;        /* unpadded input */
  int F, R, S;
  int stride_h, stride_w;
  int pad_top, pad_bottom, pad_left, pad_right;
  float pad_value;
  xtc_hip_tile tile;
  int split_k;
  int group_m;
  int xcd_remap;
  int relu;
  float relu_threshold;
  void *stream;
  double relu_threshold_f64; /* XTC_HIP_F64 calls: the relu threshold ... */
  double pad_value_f64;      /* ... and the pad value, in fp64 */
} xtc_hip_conv2d_desc;

int xtc_hip_conv2d(const xtc_hip_conv2d_desc *desc, const void *input,
                   const void *weight, void *out, const void *bias);

/* y[i] = max(x[i], threshold) over n fp32 elements (XTCOperRelu forward,
 * operators.py:224-249); x == y allowed. */
int xtc_hip_relu(const float *x, float *y, uint64_t n, float threshold,
                 void *stream);

/* The same over fp64 elements. */
int xtc_hip_relu_f64(const double *x, double *y, uint64_t n, double threshold,
                     void *stream);

/* Constant padding of a row-major fp32 tensor of rank <= 8: out has shape
 * shape[d] + before[d] + after[d]; border = value, interior = input
 * (_OperPadImpl.forward / np.pad, operators.py:413-433). */
int xtc_hip_pad(const float *x, float *y, int ndim, const int64_t *shape,
                const int64_t *before, const int64_t *after, float value,
                void *stream);

/* The same over fp64 elements. */
int xtc_hip_pad_f64(const double *x, double *y, int ndim, const int64_t *shape,
                    const int64_t *before, const int64_t *after, double value,
                    void *stream);

/* Crop of a row-major tensor of rank <= 8 and elem_bytes-byte elements
 * (2: bf16 words, 4: fp32, 8: fp64): shape is the input's, out has shape
 * shape[d] - before[d] - after[d] and out[o] = x[o + before] (the slice of
 * XTCOperUnpad.forward, operators.py:683-702; the subview copy of
 * MlirOperatorUnpad, MlirOps.py:784-887).  A crop larger than its dim fails. */
int xtc_hip_unpad(const void *x, void *y, int elem_bytes, int ndim,
                  const int64_t *shape, const int64_t *before,
                  const int64_t *after, void *stream);

/* Round-to-nearest-even fp32 -> bf16 (stored as uint16) and back. */
int xtc_hip_cast_f32_to_bf16(const float *x, uint16_t *y, uint64_t n, void *stream);
int xtc_hip_cast_bf16_to_f32(const uint16_t *x, float *y, uint64_t n, void *stream);

/* sizeof(xtc_hip_matmul_desc) and sizeof(xtc_hip_conv2d_desc) as this library
 * was compiled: a binding that declares the descriptors itself (ctypes, cgo)
 * checks its own struct sizes against these before the first call, so a
 * field it lacks fails loudly instead of being read past the end of its
 * struct.  No counterpart in the reference, whose mgpu* calls
 * (GPUDevice.py:131-207) take no structs. */
int xtc_hip_matmul_desc_size(void);
int xtc_hip_conv2d_desc_size(void);

/* Compiled kernel instances.  A schedule maps onto one of these; the HIP
 * Scheduler rejects schedules that map to none. */
typedef struct {
  int dtype;
  int conv;              /* 1: implicit-GEMM conv loader */
  xtc_hip_tile tile;
  int lds_bytes;
  int threads;
} xtc_hip_gemm_instance;

int xtc_hip_gemm_instance_count(void);
int xtc_hip_gemm_instance_get(int index, xtc_hip_gemm_instance *out);

/* Tile the library picks when a descriptor leaves `tile` zeroed. */
int xtc_hip_default_tile(int dtype, int conv, int M, int N, int K, xtc_hip_tile *out,
                         int *split_k);

/* Tile a conv2d descriptor gets when it leaves `tile` zeroed.  Unlike
 * xtc_hip_default_tile(dtype, 1, ...) it sees the window, strides and pads:
 * for a window wider than 1x1 the direct conv kernel's wider 1x4-wave block
 * replaces the 8x8 one when its input halo fits and its blocks fit in one
 * wave of 256 CUs, 7x14 pixels (tile 98x64x16) first, else 8x14 (tile
 * 112x64x16). */
int xtc_hip_conv2d_default_tile(const xtc_hip_conv2d_desc *desc, xtc_hip_tile *out, int *split_k);

/* Pipeline depths the kernel that runs `desc` (with 256-byte aligned
 * operands) is compiled for: the LDS stages of the LDS-DMA kernels, 2 for
 * the register-staged generic template (and 4 for its 64x64 tiles, with
 * three register sets of loads in flight: the default when K is split), 1
 * for the scalar kernel.  Writes up
 * to max_depths of them, the default first, and returns their count (-1 on
 * error).  A schedule's unroll of the K-slab loop selects one
 * (MlirCompilerPasses.py:579-596 unrolls loops by the scheduled factor; here
 * the factor of the loop that walks the LDS slabs is how many slabs are in
 * flight).  The conv2d kernels are compiled for one depth each. */
int xtc_hip_matmul_pipeline_depths(const xtc_hip_matmul_desc *desc, int *depths, int max_depths);
int xtc_hip_conv2d_pipeline_depths(const xtc_hip_conv2d_desc *desc, int *depths, int max_depths);

/* ---------------------------------------------------------- timing harness */

/* Same protocol as evaluate_perf (evaluate_perf.c:63-125): one warm-up call
 * when number > 0, then for each of `repeat` repeats the call count doubles
 * from `number` until a batch lasts >= min_repeat_ms; results[r] = batch
 * seconds / calls.  With events, results[r * events_num + e] is event e's
 * count for the final batch of repeat r divided by its calls:
 *   "gpu.time"   device seconds, from events bracketing the batch on the
 *                library stream; "gpu.clocks" the same in nanoseconds;
 *   "gpu.<name>" a GPU hardware counter through libxtc_hip_pmu.so
 *                (include/xtc_hip_pmu.h; "gpu.cycles" = GRBM_GUI_ACTIVE),
 *                as perf_event_gpu.cpp:56-233 reads CUPTI metrics;
 *   "cycles", "clocks", "instructions", "migrations", "context_switches",
 *   "cache_access", "cache_misses", "branches", "branches_misses"
 *                host counters of the calling process through
 *                perf_event_open (perf_event_linux.c:37-54,72-81).
 * A name that cannot be opened yields -1, as in the reference.  At most 64
 * events; func is called with nargs (<= 8) pointer arguments. */
void xtc_hip_evaluate_perf(double *results, int events_num, const char *events_names[],
                           int repeat, int number, int min_repeat_ms,
                           void (*func)(void), void **args, int nargs);

/* Status of the calling thread's last xtc_hip_evaluate_perf / evaluate:
 * 0 when it ran, non-zero when it rejected its arguments (message in
 * xtc_hip_last_error()).  The reference's evaluate_perf returns nothing and
 * asserts instead. */
int xtc_hip_evaluate_status(void);

/* evaluate_perf without events (evaluate_perf.c:240-248). */
void xtc_hip_evaluate(double *results, int repeat, int number, int min_repeat_ms,
                      void (*func)(void), void **args, int nargs);

/* Measured peak multiply-accumulates per second of the current device for
 * dtype ("float32", "bfloat16", "float64"), the device counterpart of the reference's
 * evaluate_flops microbenchmark (evaluate_flops.c:431-494): a register-only
 * loop of independent MFMAs (v_mfma_f32_16x16x4_f32, v_mfma_f32_16x16x32_bf16,
 * v_mfma_f64_16x16x4_f64)
 * on every CU, one wave per SIMD and two workgroups per CU, timed with events
 * over three batches of five ~20 ms launches, best batch.  XTC counts one op
 * per FMA (operation.py:76-82), so this is half the FLOP/s figure.  Operands
 * are the reference's integers 1 + i % 127.  0.0 on error (no device,
 * unsupported dtype; message in xtc_hip_last_error()). */
double xtc_hip_evaluate_flops(const char *dtype);

/* The same probe with operand pattern `operands`: 0 the integers 1 + i % 127,
 * 1 zeros, 2 uniform [-1, 1) (bf16: rounded to nearest even).  Under the
 * board's power limit the rate depends on the operands' switching activity:
 * this is the ceiling a GEMM on such data can reach. */
double xtc_hip_evaluate_flops_operands(const char *dtype, int operands);

/* Published dense MFMA peak of MI355X for dtype, in FMA/s (fp32 157.3,
 * bf16/fp16 2516.6, fp64 78.6 TFLOP/s halved); 0.0 for others. */
double xtc_hip_datasheet_flops(const char *dtype);

#ifdef __cplusplus
}
#endif

#endif /* XTC_HIP_H */
