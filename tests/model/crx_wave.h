// The CPU model's definitions of the wave-level primitives that the library's kernels take from
// crukx-sync_amd/csrc/crx_wave.h (inline assembly there): the same meaning, on the wave64 emulator
// of tests/model/simt.cpp.  wave_fence is a meeting point of the wavefront's live lanes, which is
// where the kernels read what other lanes wrote.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace crx {

__forceinline__ void wave_fence() { simt_fence(); }

// m with bit k (uniform) cleared
__forceinline__ void clear_bit(uint64_t &m, uint32_t k) { m &= ~(1ULL << k); }

}  // namespace crx

#define CRX_DYNAMIC_LDS(type, name) type *const name = static_cast<type *>(::simt::dynamic_lds())
