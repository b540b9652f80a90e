// A host stand-in for <hip/hip_runtime.h>, used only to build the CPU model of the library
// (tests/model/): the library's own sources (kernels.hip, engine.cpp, format.cpp) compile against it
// as plain C++ and run on the CPU, each kernel under the wave64 emulator of tests/model/simt.cpp.
//
// Device memory is host memory, every runtime call completes before it returns (streams and events
// only order what is already ordered), and a kernel launch runs its workgroups one after another.
// Within a workgroup every work-item is a fiber; they run one at a time and meet at each wave-level
// collective (ballot, shuffle, lane read, fence) and at each workgroup barrier, where the emulator
// checks that every live lane of the wavefront reached the same point.
#pragma once

#include <sanitizer/allocator_interface.h>
#include <sanitizer/asan_interface.h>

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <type_traits>

// ------------------------------------------------------------------ qualifiers
#define __global__
#define __device__
#define __host__
// LDS variables live in one section, so that the emulator can refill them at every workgroup's start
// (LDS holds no values from earlier workgroups on the GPU either)
#define __shared__ static __attribute__((section("simt_lds")))
#define __constant__ static
#define __launch_bounds__(...)
#define __forceinline__ inline __attribute__((always_inline))
#define __align__(n) __attribute__((aligned(n)))

struct dim3 {
    uint32_t x, y, z;
    constexpr dim3(uint32_t x_ = 1, uint32_t y_ = 1, uint32_t z_ = 1) : x(x_), y(y_), z(z_) {}
};

struct alignas(8) uint2 {
    uint32_t x, y;
};
struct alignas(16) uint4 {
    uint32_t x, y, z, w;
};
inline uint2 make_uint2(uint32_t x, uint32_t y) { return uint2{x, y}; }
inline uint4 make_uint4(uint32_t x, uint32_t y, uint32_t z, uint32_t w) { return uint4{x, y, z, w}; }

// ------------------------------------------------------------------ runtime types
typedef int hipError_t;
enum : int {
    hipSuccess = 0,
    hipErrorInvalidValue = 1,
    hipErrorOutOfMemory = 2,
    hipErrorInvalidDevice = 101,
    hipErrorNotReady = 600,
};
typedef void *hipDeviceptr_t;
typedef struct simt_stream *hipStream_t;
typedef struct simt_event *hipEvent_t;
enum hipMemcpyKind {
    hipMemcpyHostToHost = 0,
    hipMemcpyHostToDevice = 1,
    hipMemcpyDeviceToHost = 2,
    hipMemcpyDeviceToDevice = 3,
    hipMemcpyDefault = 4,
};
#define hipStreamNonBlocking 0x1u
#define hipEventDisableTiming 0x2u
#define hipHostMallocDefault 0x0u
#define HIP_SYMBOL(x) (reinterpret_cast<const void *>(&(x)))

hipError_t hipGetDevice(int *dev);
hipError_t hipStreamCreateWithFlags(hipStream_t *s, unsigned flags);
hipError_t hipEventCreate(hipEvent_t *e);
hipError_t hipEventCreateWithFlags(hipEvent_t *e, unsigned flags);
hipError_t hipEventDestroy(hipEvent_t e);
hipError_t hipEventRecord(hipEvent_t e, hipStream_t s);
hipError_t hipEventQuery(hipEvent_t e);
hipError_t hipEventSynchronize(hipEvent_t e);
hipError_t hipEventElapsedTime(float *ms, hipEvent_t a, hipEvent_t b);
hipError_t hipStreamWaitEvent(hipStream_t s, hipEvent_t e, unsigned flags);
hipError_t hipStreamSynchronize(hipStream_t s);
hipError_t hipHostMalloc(void **p, size_t bytes, unsigned flags);
hipError_t hipHostFree(void *p);
hipError_t hipMemcpyAsync(void *dst, const void *src, size_t bytes, hipMemcpyKind kind, hipStream_t s);
hipError_t hipMemsetAsync(void *dst, int value, size_t bytes, hipStream_t s);
hipError_t hipGetLastError();
// the allocation holding an address: the model's memory is the host's, and the sanitizer's allocator
// knows its blocks (an address outside every block: not known, as the runtime answers for memory it
// did not allocate)
inline hipError_t hipMemGetAddressRange(hipDeviceptr_t *base, size_t *size, hipDeviceptr_t p) {
    const void *b = __sanitizer_get_allocated_begin(p);
    if (!b) {
        *base = nullptr;
        *size = 0;
        return hipErrorInvalidValue;
    }
    *base = const_cast<void *>(b);
    *size = __sanitizer_get_allocated_size(b);
    return hipSuccess;
}
hipError_t hipGetSymbolAddress(void **p, const void *symbol);
const char *hipGetErrorString(hipError_t e);

// ------------------------------------------------------------------ the emulator's interface
namespace simt {

struct Idx {
    uint32_t x, y, z;
};
Idx thread_idx();
Idx block_idx();
Idx grid_dim();
Idx block_dim();
uint32_t lane_id();

enum Op : int { kSync, kBallot, kReadlane, kReadfirst, kShflIdx, kShflUp, kShflXor };
// The calling lane's part in a collective of its wavefront: returns the lane's result.
uint64_t collective(Op op, uint64_t value, uint32_t arg, const void *site);
void block_barrier(const void *site);
void *dynamic_lds();

// Runs body() as every work-item of every workgroup of the launch.
void run(dim3 grid, dim3 block, size_t dynamic_lds_bytes, void (*body)(void *), void *ctx);

template <typename K, typename... P>
void launch(K kernel, dim3 grid, dim3 block, size_t shmem, hipStream_t, P... args) {
    auto closure = [&]() { kernel(args...); };
    using C = decltype(closure);
    run(grid, block, shmem, [](void *c) { (*static_cast<C *>(c))(); }, &closure);
}

template <typename T>
uint64_t to_bits(T v) {
    static_assert(sizeof(T) <= 8 && std::is_trivially_copyable<T>::value, "collective operand");
    uint64_t b = 0;
    std::memcpy(&b, &v, sizeof(T));
    return b;
}
template <typename T>
T from_bits(uint64_t b) {
    T v;
    std::memcpy(&v, &b, sizeof(T));
    return v;
}

}  // namespace simt

#define hipLaunchKernelGGL(kernel, grid, block, shmem, stream, ...) \
    ::simt::launch(kernel, dim3(grid), dim3(block), (size_t)(shmem), stream, ##__VA_ARGS__)

#define threadIdx (::simt::thread_idx())
#define blockIdx (::simt::block_idx())
#define gridDim (::simt::grid_dim())
#define blockDim (::simt::block_dim())

// ------------------------------------------------------------------ device functions
#define SIMT_SITE __builtin_return_address(0)

__attribute__((noinline)) inline uint32_t __lane_id() { return ::simt::lane_id(); }
__attribute__((noinline)) inline unsigned long long __ballot(int p) {
    return ::simt::collective(::simt::kBallot, p ? 1 : 0, 0, SIMT_SITE);
}
__attribute__((noinline)) inline int __any(int p) {
    return ::simt::collective(::simt::kBallot, p ? 1 : 0, 0, SIMT_SITE) != 0;
}
template <typename T>
__attribute__((noinline)) T __shfl(T v, int src, int width = 64) {
    (void)width;
    return ::simt::from_bits<T>(::simt::collective(::simt::kShflIdx, ::simt::to_bits(v), (uint32_t)src, SIMT_SITE));
}
template <typename T>
__attribute__((noinline)) T __shfl_up(T v, unsigned delta, int width = 64) {
    (void)width;
    return ::simt::from_bits<T>(::simt::collective(::simt::kShflUp, ::simt::to_bits(v), delta, SIMT_SITE));
}
template <typename T>
__attribute__((noinline)) T __shfl_xor(T v, int mask, int width = 64) {
    (void)width;
    return ::simt::from_bits<T>(::simt::collective(::simt::kShflXor, ::simt::to_bits(v), (uint32_t)mask, SIMT_SITE));
}
__attribute__((noinline)) inline uint32_t simt_readlane(uint32_t v, uint32_t l) {
    return (uint32_t)::simt::collective(::simt::kReadlane, v, l, SIMT_SITE);
}
__attribute__((noinline)) inline uint32_t simt_readfirstlane(uint32_t v) {
    return (uint32_t)::simt::collective(::simt::kReadfirst, v, 0, SIMT_SITE);
}
__attribute__((noinline)) inline void simt_fence() { ::simt::collective(::simt::kSync, 0, 0, SIMT_SITE); }
__attribute__((noinline)) inline void __syncthreads() { ::simt::block_barrier(SIMT_SITE); }

inline int __popcll(unsigned long long x) { return __builtin_popcountll(x); }

// number of set bits of m among the lanes below this one, lanes 0-31 (lo) / 32-63 (hi), plus acc
inline uint32_t simt_mbcnt_lo(uint32_t m, uint32_t acc) {
    const uint32_t l = ::simt::lane_id();
    const uint32_t below = l >= 32 ? m : (m & ((1u << l) - 1u));
    return acc + (uint32_t)__builtin_popcount(below);
}
inline uint32_t simt_mbcnt_hi(uint32_t m, uint32_t acc) {
    const uint32_t l = ::simt::lane_id();
    const uint32_t below = l < 32 ? 0u : (m & ((1u << (l - 32)) - 1u));
    return acc + (uint32_t)__builtin_popcount(below);
}
#define __builtin_amdgcn_mbcnt_lo(m, acc) simt_mbcnt_lo((m), (acc))
#define __builtin_amdgcn_mbcnt_hi(m, acc) simt_mbcnt_hi((m), (acc))
#define __builtin_amdgcn_readlane(v, l) simt_readlane((v), (l))
#define __builtin_amdgcn_readfirstlane(v) simt_readfirstlane((v))
#define __builtin_amdgcn_fence(order, scope) simt_fence()
// the emulator's memory operations complete when issued: a wait for them has nothing to wait for
#define __builtin_amdgcn_s_waitcnt(imm) ((void)(imm))

// Raw buffer loads: the hardware range check returns 0 for a load that does not lie wholly below
// num_records bytes.
struct simt_rsrc {
    const uint8_t *base;
    uint32_t num_records;
};
typedef simt_rsrc __amdgpu_buffer_rsrc_t;
inline simt_rsrc simt_make_rsrc(void *p, short stride, int num, int flags) {
    (void)stride;
    (void)flags;
    return simt_rsrc{static_cast<const uint8_t *>(p), (uint32_t)num};
}
// A 32-bit word holding the first or last element of a tensor whose ends are not 32-bit aligned also
// holds 16 bits outside the tensor, and the kernels read such words (or their halves) and ignore the
// outside part.  On the GPU such a read cannot fault (an aligned word never crosses a page), so the
// model allows a load that stays inside one aligned word of which some bytes are addressable: the
// bytes outside the allocation read as 0xEE.  Any other load outside an allocation is left to
// AddressSanitizer.
template <typename T>
inline T simt_buffer_load(simt_rsrc r, uint32_t voff, uint32_t soff) {
    static_assert(sizeof(T) <= 4, "loads of at most one word");
    const uint64_t off = (uint64_t)voff + soff;
    if (off + sizeof(T) > r.num_records) return T(0);
    const uint8_t *p = r.base + off;
    uint8_t *w = reinterpret_cast<uint8_t *>((uintptr_t)p & ~uintptr_t(3));
    T v;
    // (a granule's addressable bytes are a prefix of it: the ends of the load decide)
    const bool whole = !__asan_address_is_poisoned(p) && !__asan_address_is_poisoned(p + sizeof(T) - 1);
    if (!whole && p + sizeof(T) <= w + 4 && __asan_region_is_poisoned(w, 4) != w) {
        // straddles the end of an allocation within one word
        uint8_t b[sizeof(T)];
        for (size_t k = 0; k < sizeof(T); ++k)
            b[k] = __asan_address_is_poisoned(p + k) ? 0xEE : p[k];
        std::memcpy(&v, b, sizeof(T));
        return v;
    }
    std::memcpy(&v, p, sizeof(T));
    return v;
}
// Raw buffer stores: the hardware range check drops a store that does not lie wholly below
// num_records bytes.
template <typename T>
inline void simt_buffer_store(T v, simt_rsrc r, uint32_t voff, uint32_t soff) {
    const uint64_t off = (uint64_t)voff + soff;
    if (off + sizeof(T) > r.num_records) return;
    std::memcpy(const_cast<uint8_t *>(r.base) + off, &v, sizeof(T));
}
#define __builtin_amdgcn_raw_buffer_store_b16(v, r, voff, soff, aux) simt_buffer_store<uint16_t>((uint16_t)(v), (r), (voff), (soff))
#define __builtin_amdgcn_raw_buffer_store_b32(v, r, voff, soff, aux) simt_buffer_store<uint32_t>((uint32_t)(v), (r), (voff), (soff))
#define __builtin_amdgcn_make_buffer_rsrc(p, stride, num, flags) simt_make_rsrc((p), (stride), (num), (flags))
#define __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, aux) simt_buffer_load<uint32_t>((r), (voff), (soff))
#define __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, aux) simt_buffer_load<uint16_t>((r), (voff), (soff))

// Atomics: the work-items of the model never run at the same time.
template <typename T, typename U>
inline T atomicAdd(T *p, U v) {
    const T o = *p;
    *p = (T)(o + (T)v);
    return o;
}
template <typename T, typename U>
inline T atomicSub(T *p, U v) {
    const T o = *p;
    *p = (T)(o - (T)v);
    return o;
}
template <typename T, typename U>
inline T atomicOr(T *p, U v) {
    const T o = *p;
    *p = (T)(o | (T)v);
    return o;
}
template <typename T, typename U>
inline T atomicMax(T *p, U v) {
    const T o = *p;
    if ((T)v > o) *p = (T)v;
    return o;
}

// HIP's device min and max
template <typename A, typename B>
inline typename std::common_type<A, B>::type min(A a, B b) {
    typedef typename std::common_type<A, B>::type C;
    return (C)a < (C)b ? (C)a : (C)b;
}
template <typename A, typename B>
inline typename std::common_type<A, B>::type max(A a, B b) {
    typedef typename std::common_type<A, B>::type C;
    return (C)a < (C)b ? (C)b : (C)a;
}
