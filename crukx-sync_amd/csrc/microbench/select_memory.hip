// The apply's select pass without its arithmetic: what its memory traffic alone costs on this GPU.
//
// 7,616,000,000 bf16 weights (15.2 GB, a 7B-shaped state dict) in 65,536-element slabs, one wave per
// slab, streamed the way the select pass streams them: each lane loads elements l and l + 64 of every
// 128-element row as two 16-bit loads, 8 rows in flight, non-temporal.  About 1% of the elements are
// "targets" (positions from a hash of slab and element).  Variants:
//   read                 the stream alone
//   read, 2 B at end     the stream, then each target written as a 2-byte store, 64 per instruction in
//                        ascending order, after the slab's last row (the select pass's write-through)
//   2 B only             those writes without the stream
//   read + 128 B lines   during the stream, every 128-byte line holding a target stored whole (all 64
//                        lanes of the half-row), new bits for the targets, old bits for the rest
//   read + 64 B / 32 B   the same for the 64-byte half-line or 32-byte sector holding a target
//   read, load+2 B at end  the end-of-slab writes, each preceded by a load of its element (all the
//                        slab's loads first), so the line is in L2 when the partial write reaches it
//   read, xor at end     the end-of-slab writes as 32-bit atomic XORs of (old ^ new) into the word
// Build and run: make -C crukx-sync_amd/csrc microbench && crukx-sync_amd/csrc/_build/select_memory
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

#define CHECK(x)                                                                             \
    do {                                                                                     \
        const hipError_t e_ = (x);                                                           \
        if (e_ != hipSuccess) {                                                              \
            std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);       \
            return 1;                                                                        \
        }                                                                                    \
    } while (0)

namespace {

constexpr uint64_t kN = 7616000000ull;
constexpr uint32_t kSlab = 65536, kRows = kSlab / 128, kBatch = 8;
constexpr uint32_t kSlabs = (uint32_t)((kN + kSlab - 1) / kSlab);

// about 1% of the elements, for the variants that test every element as it streams by: a hash of
// (slab, element) below 164 / 16384
__device__ __forceinline__ bool is_target(uint32_t slab, uint32_t x) { return ((x * 40503u + slab * 9973u) & 0x3FFFu) < 164u; }

// the same density for the end-of-slab writes, generated in ascending order: the i-th target of a slab
// lies at a hashed place in the i-th stretch of 99 elements (656 per slab)
constexpr uint32_t kStretch = 99, kPerSlab = 656;
__device__ __forceinline__ uint32_t target_at(uint32_t slab, uint32_t i) {
    uint32_t h = (slab * 0x9E3779B1u) ^ (i * 0x85EBCA77u);
    h ^= h >> 15;
    h *= 0x2C1B3C6Du;
    h ^= h >> 12;
    return i * kStretch + h % kStretch;
}

enum Mode { kRead, kReadEndWrites, kEndWritesOnly, kLines128, kLines64, kSectors32, kReadEndLoadStore, kReadEndXor };

template <int MODE>
__global__ __launch_bounds__(64) void k_stream(uint16_t *w, uint32_t *out) {
    const uint32_t ln = __lane_id(), slab = blockIdx.x;
    const uint64_t first = (uint64_t)slab * kSlab;
    const uint32_t n = (uint32_t)(first + kSlab <= kN ? kSlab : kN - first);
    // range-checked loads over the slab: rows fetched past its end read as zero
    const __amdgpu_buffer_rsrc_t src = __builtin_amdgcn_make_buffer_rsrc(w + first, (short)0, (int)(n * 2), 0x00020000);
    uint32_t acc = 0;
    if (MODE != kEndWritesOnly) {
        uint16_t clo[kBatch], chi[kBatch], nlo[kBatch], nhi[kBatch];
        auto load = [&](uint16_t(&lo)[kBatch], uint16_t(&hi)[kBatch], uint32_t r0) {
#pragma unroll
            for (uint32_t u = 0; u < kBatch; ++u) {
                lo[u] = __builtin_amdgcn_raw_buffer_load_b16(src, (r0 + u) * 256 + ln * 2, 0, 2);
                hi[u] = __builtin_amdgcn_raw_buffer_load_b16(src, (r0 + u) * 256 + ln * 2 + 128, 0, 2);
            }
        };
        load(clo, chi, 0);
        for (uint32_t r0 = 0; r0 < kRows; r0 += kBatch) {
            load(nlo, nhi, r0 + kBatch);
#pragma unroll
            for (uint32_t u = 0; u < kBatch; ++u) {
                acc = acc * 3 + (clo[u] | ((uint32_t)chi[u] << 16));
                if (MODE >= kLines128 && MODE <= kSectors32) {
                    const uint32_t x0 = (r0 + u) * 128 + ln, x1 = x0 + 64;
                    const bool t0 = x0 < n && is_target(slab, x0), t1 = x1 < n && is_target(slab, x1);
                    const uint64_t b0 = __ballot(t0), b1 = __ballot(t1);
                    // lanes sharing the written unit: 64 (128 B), 32 (64 B) or 16 (32 B)
                    const uint32_t width = MODE == kLines128 ? 64 : MODE == kLines64 ? 32 : 16;
                    const uint64_t unit = width == 64 ? ~0ull : ((1ull << width) - 1) << ((ln / width) * width);
                    if ((b0 & unit) && x0 < n) w[first + x0] = (uint16_t)(clo[u] + (t0 ? 1 : 0));
                    if ((b1 & unit) && x1 < n) w[first + x1] = (uint16_t)(chi[u] + (t1 ? 1 : 0));
                }
            }
#pragma unroll
            for (uint32_t u = 0; u < kBatch; ++u) {
                clo[u] = nlo[u];
                chi[u] = nhi[u];
            }
        }
    }
    if (MODE == kReadEndWrites || MODE == kEndWritesOnly) {
        // the slab's targets in ascending order, 64 per store instruction
        for (uint32_t i = ln; i < kPerSlab; i += 64) {
            const uint32_t x = target_at(slab, i);
            if (x < n) w[first + x] = (uint16_t)(acc | 1);
        }
    }
    if (MODE == kReadEndLoadStore) {
        constexpr uint32_t kPer = (kPerSlab + 63) / 64;  // targets per lane
        uint16_t old[kPer];
#pragma unroll
        for (uint32_t q = 0; q < kPer; ++q) {  // every load before any store
            const uint32_t i = ln + 64 * q, x = i < kPerSlab ? target_at(slab, i) : n;
            old[q] = x < n ? w[first + x] : (uint16_t)0;
        }
#pragma unroll
        for (uint32_t q = 0; q < kPer; ++q) {
            const uint32_t i = ln + 64 * q, x = i < kPerSlab ? target_at(slab, i) : n;
            if (x < n) w[first + x] = (uint16_t)(old[q] + 1);
        }
    }
    if (MODE == kReadEndXor) {
        uint32_t *const w32 = reinterpret_cast<uint32_t *>(w);
        for (uint32_t i = ln; i < kPerSlab; i += 64) {
            const uint32_t x = target_at(slab, i);
            const uint64_t e = first + x;  // the element's word and half
            if (x < n) atomicXor(&w32[e >> 1], 1u << (16 * (uint32_t)(e & 1)));
        }
    }
    if (ln == 0) out[slab] = acc;
}

template <int MODE>
float run(uint16_t *w, uint32_t *out) {
    hipEvent_t a, b;
    (void)hipEventCreate(&a);
    (void)hipEventCreate(&b);
    hipLaunchKernelGGL(k_stream<MODE>, dim3(kSlabs), dim3(64), 0, 0, w, out);  // warm-up
    (void)hipEventRecord(a);
    for (int i = 0; i < 5; ++i) hipLaunchKernelGGL(k_stream<MODE>, dim3(kSlabs), dim3(64), 0, 0, w, out);
    (void)hipEventRecord(b);
    (void)hipEventSynchronize(b);
    float ms = 0;
    (void)hipEventElapsedTime(&ms, a, b);
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    return ms / 5;
}

}  // namespace

int main() {
    uint16_t *w = nullptr;
    uint32_t *out = nullptr;
    CHECK(hipMalloc(&w, kN * 2));
    CHECK(hipMalloc(&out, (size_t)kSlabs * 4));
    CHECK(hipMemset(w, 0x3c, kN * 2));
    CHECK(hipDeviceSynchronize());
    std::printf("%llu bf16 weights (%.1f GB), %u slabs of %u, about 1%% targets; mean of 5 launches\n",
                (unsigned long long)kN, kN * 2 / 1e9, kSlabs, kSlab);
    std::printf("read                   %7.3f ms\n", run<kRead>(w, out));
    std::fflush(stdout);
    std::printf("read, 2 B at end       %7.3f ms\n", run<kReadEndWrites>(w, out));
    std::fflush(stdout);
    std::printf("2 B only               %7.3f ms\n", run<kEndWritesOnly>(w, out));
    std::fflush(stdout);
    std::printf("read + 128 B lines     %7.3f ms\n", run<kLines128>(w, out));
    std::fflush(stdout);
    std::printf("read + 64 B half-lines %7.3f ms\n", run<kLines64>(w, out));
    std::fflush(stdout);
    std::printf("read + 32 B sectors    %7.3f ms\n", run<kSectors32>(w, out));
    std::fflush(stdout);
    std::printf("read, load+2 B at end  %7.3f ms\n", run<kReadEndLoadStore>(w, out));
    std::fflush(stdout);
    std::printf("read, xor at end       %7.3f ms\n", run<kReadEndXor>(w, out));
    std::fflush(stdout);
    CHECK(hipDeviceSynchronize());
    CHECK(hipFree(w));
    CHECK(hipFree(out));
    return 0;
}
