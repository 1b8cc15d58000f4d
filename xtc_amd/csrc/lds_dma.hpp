// SPDX-License-Identifier: BSD-3-Clause
// LDS DMA (global_load_lds_dwordx4) issued from inline asm.
//
// The compiler builtin marks an LDS write of unknown order in its wait-count
// model, so while any such DMA is in flight every LDS wait it inserts becomes
// lgkmcnt(0): each read waits for every read issued after it.  Issued from
// asm, the DMA is invisible to that model and the compiler's own LDS waits
// stay exact (lgkmcnt(n)).  The caller must then order the DMA itself: an
// explicit s_waitcnt vmcnt for the DMA before the barrier that publishes its
// data.  (LDS reads return in order, so an extra unordered LGKM event could
// only make such waits longer, never release a read early.)  The LDS buffer
// passed here must be one the compiler sees escape to the asm (its address is
// the M0 operand), so it treats the asm as writing it.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace xtc_hip {

// 16 bytes per lane from src into the 1 KB block at lds_dst (wave-uniform):
// lane l writes lds_dst + 16 l.
__device__ __forceinline__ void lds_dma16(const void* src, void* lds_dst) {
  typedef __attribute__((address_space(3))) void lds_void_t;
  const unsigned m0 = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(lds_void_t*)lds_dst);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0) : "memory", "m0");
}

}  // namespace xtc_hip
