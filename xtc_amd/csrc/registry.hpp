// SPDX-License-Identifier: BSD-3-Clause
// Table of compiled GEMM/conv kernel instances.  The instance list is
// generated at build time (xtc_amd/csrc/build.py) into several translation
// units compiled in parallel; each contributes one array of GemmEntry.
#pragma once
#include "gemm.hpp"

namespace xtc_hip {

typedef void (*GemmLaunch)(const GemmArgs&, dim3, hipStream_t);

struct GemmEntry {
  int dtype;   // 0 fp32, 1 bf16
  int conv;    // implicit-GEMM conv loader
  int bm, bn, bk, wgm, wgn;
  int lds_bytes;
  int threads;
  GemmLaunch launch;       // one register set of loads in flight (depth 2)
  GemmLaunch launch_ring;  // three register sets (depth 4), or null
};

template <typename T, int BM, int BN, int BK, int WGM, int WGN, bool CONV, int RING>
void launch_gemm(const GemmArgs& a, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((gemm_kernel<T, BM, BN, BK, WGM, WGN, CONV, RING>), grid,
                     dim3(WGM * WGN * 64), 0, s, a);
}

template <typename T, int BM, int BN, int BK, int WGM, int WGN, bool CONV, bool WITH_RING>
inline GemmEntry make_entry() {
  using P = GemmTile<T, BM, BN, BK, WGM, WGN, CONV>;
  return GemmEntry{P::F32 ? 0 : 1, CONV ? 1 : 0, BM, BN, BK, WGM, WGN,
                   (int)(2 * P::STAGE_ELEMS * sizeof(T)), P::NT,
                   &launch_gemm<T, BM, BN, BK, WGM, WGN, CONV, 1>,
                   WITH_RING ? &launch_gemm<T, BM, BN, BK, WGM, WGN, CONV, 3> : nullptr};
}

// Entry tables exist in the host pass only; the device pass compiles the
// explicitly instantiated kernels.
// Provided by the generated registry translation unit.
const GemmEntry* gemm_registry(int* count);

}  // namespace xtc_hip
