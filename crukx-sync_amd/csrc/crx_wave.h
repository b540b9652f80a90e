// Wave-level primitives of the gfx950 kernels that are written as inline assembly or need a
// declaration form of their own.  Everything else the kernels use at wave level (ballots, mbcnt,
// lane reads, shuffles) goes through the compiler's builtins.
//
// The kernels include this file as <crx_wave.h> (the library's Makefile puts csrc/ on the include
// path); the CPU model of the kernels (tests/model/) supplies its own definitions under the same name.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace crx {

// Orders this wavefront's LDS accesses in the compiler's view without waiting on outstanding memory
// operations (LDS instructions of one wavefront execute in order).  The streaming kernels run one
// wavefront per workgroup, so a workgroup barrier would only drain the rows loaded ahead.  It also
// marks every point where lanes read what other lanes of the wavefront wrote to LDS.
__device__ __forceinline__ void wave_fence() { asm volatile("" ::: "memory"); }

// m with bit k (uniform) cleared, in one scalar instruction
__device__ __forceinline__ void clear_bit(uint64_t &m, uint32_t k) { asm("s_bitset0_b64 %0, %1" : "+s"(m) : "s"(k)); }

}  // namespace crx

// The dynamically sized LDS array of a kernel (its size is the launch's shared-memory argument).
#define CRX_DYNAMIC_LDS(type, name) extern __shared__ __attribute__((aligned(16))) type name[]
