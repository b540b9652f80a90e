// Host orchestration of the gfx950 update codec and the C ABI (include/crukx.h).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <new>
#include <string>
#include <system_error>
#include <thread>
#include <vector>

#include <sys/mman.h>

#include "../../include/crukx.h"
#include "format.h"
#include "kernels.h"

namespace crx {

#define HIP_OK(call)                                                                              \
    do {                                                                                          \
        hipError_t e_ = (call);                                                                   \
        if (e_ != hipSuccess)                                                                     \
            throw DeviceError(std::string(#call) + ": " + hipGetErrorString(e_));                 \
    } while (0)

// ------------------------------------------------------------------ timing
namespace {
struct Pending {
    std::string name;
    hipEvent_t a, b;
};
struct Stat {
    int64_t calls = 0;
    double ms = 0;
};
std::mutex g_tmu;
bool g_timing = false;
hipEvent_t g_open = nullptr;
std::vector<Pending> g_pending;
std::vector<hipEvent_t> g_free;  // events reused across launches (creating one per launch costs host time)
std::map<std::string, Stat> g_stats;

hipEvent_t take_event() {  // under g_tmu
    if (!g_free.empty()) {
        hipEvent_t e = g_free.back();
        g_free.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    return hipEventCreate(&e) == hipSuccess ? e : nullptr;
}

// Adds the launches that have finished to the statistics; with `wait`, waits for all of them first
// (a call may return with work still on its stream: apply's writes).
void timing_collect(bool wait) {
    std::lock_guard<std::mutex> lk(g_tmu);
    std::vector<Pending> running;
    for (Pending &p : g_pending) {
        if (wait) {
            (void)hipEventSynchronize(p.b);
        } else if (hipEventQuery(p.b) == hipErrorNotReady) {
            running.push_back(p);
            continue;
        }
        float ms = 0;
        if (hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
            g_stats[p.name].calls++;
            g_stats[p.name].ms += ms;
        }
        g_free.push_back(p.a);
        g_free.push_back(p.b);
    }
    g_pending.swap(running);
}
}  // namespace

// the kernel names crx_timing_only selected (under g_tmu; empty: every kernel)
std::vector<std::string> g_only;

bool timed(const char *name) {  // under g_tmu
    if (g_only.empty()) return true;
    for (const std::string &n : g_only)
        if (n == name) return true;
    return false;
}

void timing_begin(const char *name, hipStream_t s) {
    if (!g_timing) return;
    std::lock_guard<std::mutex> lk(g_tmu);
    if (!timed(name)) return;
    hipEvent_t e = take_event();
    if (!e) return;
    (void)hipEventRecord(e, s);
    g_open = e;
}

void timing_end(const char *name, hipStream_t s) {
    if (!g_timing) return;
    std::lock_guard<std::mutex> lk(g_tmu);
    if (!g_open || !timed(name)) return;
    hipEvent_t e = take_event();
    if (!e) return;
    (void)hipEventRecord(e, s);
    g_pending.push_back(Pending{name, g_open, e});
    g_open = nullptr;
}

// Host phases of a call: wall time between marks, accumulated as "host:<name>" when timing is on.
// A phase that ends at a stream synchronisation includes the wait for the device.
struct HostClock {
    std::chrono::steady_clock::time_point t = std::chrono::steady_clock::now();
    void mark(const char *name) {
        if (!g_timing) return;
        const auto n = std::chrono::steady_clock::now();
        std::lock_guard<std::mutex> lk(g_tmu);
        Stat &st = g_stats[std::string("host:") + name];
        st.calls++;
        st.ms += std::chrono::duration<double, std::milli>(n - t).count();
        t = n;
    }
};

// ------------------------------------------------------------------ auxiliary stream
// Extra streams for work of a call that can overlap the caller's stream: a fixed pool of kAuxStreams
// per device (default priority, created on first use, kept for the process), the caller's stream
// choosing one by its address, so a caller that makes a new stream per step does not make the pool
// grow.  Calls on different caller streams rarely share one (and then only queue behind each other's
// auxiliary work).  A Fork makes it wait for everything enqueued on the caller's stream so far; join()
// makes the caller's stream wait for what was enqueued on it.
constexpr int kAuxStreams = 8, kAuxDevices = 64;
hipStream_t aux_stream(hipStream_t caller) {
    static std::mutex mu;
    static hipStream_t pool[kAuxDevices][kAuxStreams] = {};
    int dev = 0;
    HIP_OK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kAuxDevices) throw DeviceError("device index out of range");
    const uintptr_t h = reinterpret_cast<uintptr_t>(caller);
    const int k = (int)((h ^ (h >> 7) ^ (h >> 13)) % kAuxStreams);
    std::lock_guard<std::mutex> lk(mu);
    hipStream_t &st = pool[dev][k];
    if (!st) HIP_OK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    return st;
}

struct Fork {
    hipStream_t main, aux;
    hipEvent_t ev[2] = {nullptr, nullptr};
    bool joined = false;
    explicit Fork(hipStream_t s) : main(s), aux(aux_stream(s)) {
        HIP_OK(hipEventCreateWithFlags(&ev[0], hipEventDisableTiming));
        HIP_OK(hipEventCreateWithFlags(&ev[1], hipEventDisableTiming));
        HIP_OK(hipEventRecord(ev[0], main));
        HIP_OK(hipStreamWaitEvent(aux, ev[0], 0));
    }
    void join() {
        HIP_OK(hipEventRecord(ev[1], aux));
        HIP_OK(hipStreamWaitEvent(main, ev[1], 0));
        joined = true;
    }
    ~Fork() {
        // an exception before join(): the caller's stream still waits for the auxiliary work, which
        // uses buffers the caller frees after the call
        if (!joined && hipEventRecord(ev[1], aux) == hipSuccess) (void)hipStreamWaitEvent(main, ev[1], 0);
        (void)hipEventDestroy(ev[0]);
        (void)hipEventDestroy(ev[1]);
    }
};

// ------------------------------------------------------------------ host copies of large buffers
// Copies between device memory and pageable host memory (an update's bytes) go through pinned
// chunks.  The runtime stages a pageable copy through its own buffers with one thread: 3.2 ms for a
// 92 MB payload, where the DMA from pinned memory takes 1.6 ms.  Here up to kCopyThreads threads
// each take every kCopyThreads-th chunk through two pinned buffers of their own and enqueue the
// chunk's DMA on the call's stream themselves, so the host-side copies overlap each other and the
// transfers.  The buffers are allocated once per process and direction.
constexpr uint64_t kChunk = 4ULL << 20;
constexpr int kCopyThreads = 4;

struct PinnedRing {
    struct Slot {
        uint8_t *buf[2] = {nullptr, nullptr};
        hipEvent_t ev[2] = {nullptr, nullptr};
        bool used[2] = {false, false};  // an upload DMA from the buffer may still be running
    } slot[kCopyThreads];
    std::mutex mu;
    int dev = -1;  // the device the events were created on

    // with mu held: buffers, and events for the current device (recorded on its streams)
    void ready() {
        int d = 0;
        HIP_OK(hipGetDevice(&d));
        for (Slot &u : slot)
            for (int k = 0; k < 2; ++k) {
                if (u.ev[k] && d != dev) {
                    HIP_OK(hipEventSynchronize(u.ev[k]));
                    (void)hipEventDestroy(u.ev[k]);
                    u.ev[k] = nullptr;
                    u.used[k] = false;
                }
                if (!u.buf[k]) HIP_OK(hipHostMalloc(reinterpret_cast<void **>(&u.buf[k]), kChunk, hipHostMallocDefault));
                if (!u.ev[k]) HIP_OK(hipEventCreateWithFlags(&u.ev[k], hipEventDisableTiming));
            }
        dev = d;
    }
};
PinnedRing g_up, g_down;

// work(w) for w in [0, workers): on threads of their own, w = 0 on the calling thread.  A worker's
// error is rethrown once all have finished, after the stream has drained (no DMA may still use the
// pinned buffers then).
template <typename F>
void run_workers(int workers, hipStream_t s, F &&work) {
    std::string errs[kCopyThreads];
    auto guard = [&](int w) {
        try {
            work(w);
        } catch (const std::exception &e) {
            errs[w] = e.what();
        }
    };
    std::vector<std::thread> threads;
    std::vector<int> here{0};
    for (int w = 1; w < workers; ++w) {
        try {
            threads.emplace_back(guard, w);
        } catch (const std::system_error &) {  // no thread: the calling one takes that share too
            here.push_back(w);
        }
    }
    for (int w : here) guard(w);
    for (std::thread &t : threads) t.join();
    for (const std::string &e : errs)
        if (!e.empty()) {
            (void)hipStreamSynchronize(s);
            throw DeviceError(e);
        }
}

// Fresh host memory (a new Python bytes object, say) costs a page fault and a page of zeroing per
// 4 KiB on its first write: 20 ms for a 92 MB update, where the copy into mapped pages takes 2.4 ms.
// A large destination is therefore marked for huge pages (one fault per 2 MiB), and the copy's
// threads take those faults in parallel: 3.3-4 ms.  (Populating the pages ahead of the copy on
// extra threads measured slower: 3.8-5.5 ms.)  Without transparent huge pages this does nothing.
void hint_huge_pages(uint8_t *p, uint64_t n) {
    constexpr uintptr_t kHuge = 2ULL << 20;
    if (n < 4 * kHuge) return;
    const uintptr_t lo = (reinterpret_cast<uintptr_t>(p) + kHuge - 1) & ~(kHuge - 1);
    const uintptr_t hi = (reinterpret_cast<uintptr_t>(p) + n) & ~(kHuge - 1);
    if (hi > lo) (void)madvise(reinterpret_cast<void *>(lo), hi - lo, MADV_HUGEPAGE);
}

// Device to pageable host memory; complete on return.
void copy_to_host(uint8_t *dst, const uint8_t *src, uint64_t n, hipStream_t s) {
    if (!n) return;
    hint_huge_pages(dst, n);
    std::lock_guard<std::mutex> lk(g_down.mu);
    g_down.ready();
    const uint64_t chunks = (n + kChunk - 1) / kChunk;
    const int workers = (int)std::min<uint64_t>(kCopyThreads, chunks);
    run_workers(workers, s, [&](int w) {
        PinnedRing::Slot &u = g_down.slot[w];
        uint64_t prev_off = 0, prev_m = 0;
        int k = 0;
        for (uint64_t c = (uint64_t)w; c < chunks; c += (uint64_t)workers, k ^= 1) {
            const uint64_t off = c * kChunk, m = std::min(kChunk, n - off);
            HIP_OK(hipMemcpyAsync(u.buf[k], src + off, m, hipMemcpyDeviceToHost, s));
            HIP_OK(hipEventRecord(u.ev[k], s));
            if (prev_m) {  // the previous chunk, in the other buffer
                HIP_OK(hipEventSynchronize(u.ev[k ^ 1]));
                std::memcpy(dst + prev_off, u.buf[k ^ 1], prev_m);
            }
            prev_off = off;
            prev_m = m;
        }
        if (prev_m) {
            HIP_OK(hipEventSynchronize(u.ev[k ^ 1]));
            std::memcpy(dst + prev_off, u.buf[k ^ 1], prev_m);
        }
    });
}

// Pageable host memory to the device.  On return the source has been read and every DMA is
// enqueued on `s`; a buffer is reused only after its last DMA has completed.
void copy_from_host(uint8_t *dst, const uint8_t *src, uint64_t n, hipStream_t s) {
    if (n < 4 * kChunk) {  // small: the runtime's staging is as fast
        if (n) HIP_OK(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, s));
        return;
    }
    std::lock_guard<std::mutex> lk(g_up.mu);
    g_up.ready();
    const uint64_t chunks = (n + kChunk - 1) / kChunk;
    run_workers(kCopyThreads, s, [&](int w) {
        PinnedRing::Slot &u = g_up.slot[w];
        int k = 0;
        for (uint64_t c = (uint64_t)w; c < chunks; c += kCopyThreads, k ^= 1) {
            const uint64_t off = c * kChunk, m = std::min(kChunk, n - off);
            if (u.used[k]) HIP_OK(hipEventSynchronize(u.ev[k]));  // its previous DMA is done
            std::memcpy(u.buf[k], src + off, m);
            HIP_OK(hipMemcpyAsync(dst + off, u.buf[k], m, hipMemcpyHostToDevice, s));
            HIP_OK(hipEventRecord(u.ev[k], s));
            u.used[k] = true;
        }
    });
}

// ------------------------------------------------------------------ workspace
// Device buffers of one call.  Small buffers are carved from chunks of kArenaChunk bytes so that a
// call makes few trips through the caller's allocator; large ones are allocated on their own unless
// a reserved block (reserve) still has room for them.
constexpr uint64_t kArenaChunk = 8ULL << 20;

// Every buffer an allocation of its own, of exactly the size asked for (no chunks, no reserved
// block): set by the CPU model of the library, so that a memory checker sees each buffer's bounds.
bool g_arena_unpooled = false;

struct Arena {
    crx_alloc_fn fn;
    void *ctx;
    uint8_t *chunk = nullptr;
    uint64_t used = 0, size = 0;
    uint64_t total = 0;  // bytes handed out by get()
    // Scoped buffers (the parts of a chunked update, one after another): within a scope every buffer is
    // an allocation of its own, and at its end they become spares that the next scope's buffers reuse
    // (the smallest spare large enough).  A scope ends only once the device is done with its buffers.
    bool scoped = false;
    std::vector<std::pair<void *, uint64_t>> live, spare;

    void *raw(uint64_t bytes) {
        void *p = fn(ctx, bytes);
        if (!p) throw std::bad_alloc();
        return p;
    }
    void begin_scope() { scoped = true; }
    void end_scope() {
        spare.insert(spare.end(), live.begin(), live.end());
        live.clear();
        scoped = false;
    }
    void *scoped_get(uint64_t bytes) {
        if (g_arena_unpooled) {  // exact bounds for a memory checker: no reuse
            total += bytes;
            return raw(std::max<uint64_t>(bytes, 1));
        }
        bytes = (std::max<uint64_t>(bytes, 1) + 255) & ~uint64_t(255);
        total += bytes;
        size_t best = spare.size();
        for (size_t i = 0; i < spare.size(); ++i)
            if (spare[i].second >= bytes && (best == spare.size() || spare[i].second < spare[best].second)) best = i;
        if (best < spare.size()) {
            live.push_back(spare[best]);
            spare.erase(spare.begin() + (ptrdiff_t)best);
            return live.back().first;
        }
        live.emplace_back(raw(bytes), bytes);
        return live.back().first;
    }
    // one block of `bytes` for the buffers that follow
    void reserve(uint64_t bytes) {
        if (g_arena_unpooled) return;
        bytes = (bytes + 255) & ~uint64_t(255);
        if (bytes <= size - used) return;
        chunk = static_cast<uint8_t *>(raw(bytes));
        used = 0;
        size = bytes;
    }
    template <typename T>
    T *get(uint64_t count) {
        if (scoped) return static_cast<T *>(scoped_get(count * sizeof(T)));
        if (g_arena_unpooled) {
            total += count * sizeof(T);
            return static_cast<T *>(raw(std::max<uint64_t>(count * sizeof(T), 1)));
        }
        uint64_t bytes = std::max<uint64_t>(count * sizeof(T), 16);
        bytes = (bytes + 255) & ~uint64_t(255);
        total += bytes;
        if (used + bytes > size) {
            if (bytes > kArenaChunk / 4) return static_cast<T *>(raw(bytes));
            chunk = static_cast<uint8_t *>(raw(kArenaChunk));
            used = 0;
            size = kArenaChunk;
        }
        T *p = reinterpret_cast<T *>(chunk + used);
        used += bytes;
        return p;
    }
};

// Workspace bytes of the last call of one kind and its size key (e.g. its slab count): a following
// call with a key within 1/16 of it reserves that much (plus 1/32) in one allocation, instead of one
// trip through the caller's allocator per large buffer.  Only a hint: a call that needs more
// allocates the rest buffer by buffer.
struct ArenaHint {
    std::mutex m;
    uint64_t key = 0, bytes = 0;

    uint64_t get(uint64_t k) {
        std::lock_guard<std::mutex> g(m);
        if (!key || k + k / 16 < key || key + key / 16 < k) return 0;
        return bytes + bytes / 32;
    }
    void put(uint64_t k, uint64_t b) {
        std::lock_guard<std::mutex> g(m);
        key = k;
        bytes = b;
    }
};
ArenaHint g_apply_hint, g_encode_hint;

// The small transfers of a call go through pinned host memory, so each is a plain asynchronous DMA (a
// copy from or to pageable memory is staged by the runtime and holds the host thread until it is
// done).  Uploads are copied in when issued; downloads land in the arena and are copied out by
// sync(), which every call runs before it reads them.  One arena per host thread; its memory is
// reused only after the stream it served was synchronized (or its last copy waited for).  The
// blocks only grow and are never freed: hipHostFree waits for the whole device, which would hold a
// call until work it left on its stream (apply's writes) had finished.
struct PinnedStage {
    std::vector<std::pair<uint8_t *, uint64_t>> blocks;  // each twice the size of the one before
    size_t cur = 0;                                      // the block in use
    uint64_t used = 0;                                   // bytes handed out from it
    struct Out {
        void *dst;
        const uint8_t *src;
        uint64_t n;
    };
    std::vector<Out> out;  // downloads to copy out at the next sync
    hipEvent_t ev = nullptr;
    bool pending = false;  // the pinned blocks and the event are kept until the process ends: no HIP
                           // call from a destructor that may run after the runtime's own teardown

    uint8_t *get(uint64_t n) {
        n = (n + 63) & ~uint64_t(63);
        while (cur < blocks.size() && used + n > blocks[cur].second) {
            ++cur;
            used = 0;
        }
        if (cur == blocks.size()) {
            const uint64_t size = std::max<uint64_t>({n, uint64_t(4) << 20, blocks.empty() ? 0 : 2 * blocks.back().second});
            uint8_t *p = nullptr;
            HIP_OK(hipHostMalloc(reinterpret_cast<void **>(&p), size, hipHostMallocDefault));
            blocks.emplace_back(p, size);
        }
        uint8_t *p = blocks[cur].first + used;
        used += n;
        return p;
    }
    void copied(hipStream_t s) {
        if (!ev) HIP_OK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
        HIP_OK(hipEventRecord(ev, s));
        pending = true;
    }
    void wait() {
        if (pending) HIP_OK(hipEventSynchronize(ev));
        pending = false;
    }
    // after the stream is synchronized: deliver the downloads, reuse the blocks from the first
    void finish() {
        wait();
        for (const Out &o : out) std::memcpy(o.dst, o.src, o.n);
        out.clear();
        restart();
    }
    // at the start of a call: whatever an interrupted call left is dropped, once no DMA can still use it
    void abandon() {
        if (pending) (void)hipEventSynchronize(ev);
        pending = false;
        out.clear();
        restart();
    }
    void restart() {
        cur = 0;
        used = 0;
    }
};
thread_local PinnedStage t_stage;

template <typename T>
void h2d(T *dst, const T *src, uint64_t n, hipStream_t s) {
    if (!n) return;
    uint8_t *p = t_stage.get(n * sizeof(T));
    std::memcpy(p, src, n * sizeof(T));
    HIP_OK(hipMemcpyAsync(dst, p, n * sizeof(T), hipMemcpyHostToDevice, s));
    t_stage.copied(s);
}
template <typename T>
void d2h(T *dst, const T *src, uint64_t n, hipStream_t s) {
    if (!n) return;
    uint8_t *p = t_stage.get(n * sizeof(T));
    HIP_OK(hipMemcpyAsync(p, src, n * sizeof(T), hipMemcpyDeviceToHost, s));
    t_stage.copied(s);
    t_stage.out.push_back({dst, p, n * sizeof(T)});
}
template <typename T>
void zero(T *dst, uint64_t n, hipStream_t s) {
    if (n) HIP_OK(hipMemsetAsync(dst, 0, n * sizeof(T), s));
}
void sync(hipStream_t s) {
    HIP_OK(hipStreamSynchronize(s));
    t_stage.finish();
}

// Small uploads issued as one copy: add() places each host array in one pinned range and its device
// buffer at the same offset of one allocation (each copy issued costs the device several microseconds
// between kernels, and the host a runtime call).  at<T>(i) is item i's device address after commit().
struct UploadBatch {
    struct Item {
        const void *src;  // nullptr: zeros
        uint64_t off, bytes;
    };
    std::vector<Item> items;
    uint64_t total = 0;
    uint8_t *dev = nullptr;

    template <typename T>
    size_t add(const T *src, uint64_t n) {
        items.push_back({src, total, n * sizeof(T)});
        total += (std::max<uint64_t>(n * sizeof(T), 1) + 255) & ~uint64_t(255);
        return items.size() - 1;
    }
    template <typename T>
    size_t add_zeros(uint64_t n) { return add(static_cast<const T *>(nullptr), n); }
    void commit(Arena &ar, hipStream_t s) {
        dev = ar.get<uint8_t>(total);
        uint8_t *p = t_stage.get(total);
        for (const Item &it : items) {
            if (it.src) std::memcpy(p + it.off, it.src, it.bytes);
            else std::memset(p + it.off, 0, it.bytes);
        }
        HIP_OK(hipMemcpyAsync(dev, p, total, hipMemcpyHostToDevice, s));
        t_stage.copied(s);
    }
    template <typename T>
    T *at(size_t i) const { return reinterpret_cast<T *>(dev + items[i].off); }
};

// The caller's `slab` is the reference's _SLAB (codec.py:30): tensors of more elements get the exact
// group-size check before decoding (codec.py:598-604); 0 or less means its default, 2^24.
uint64_t group_check_numel(int32_t slab) { return slab > 0 ? (uint64_t)slab : (1ULL << 24); }

// Elements per slab: the caller's `slab` as a multiple of kRow, at most 65536 (slab ranks and offsets
// are kept in 16 bits).
uint32_t slab_size(int32_t slab) {
    if (slab <= 0) return 65536;
    uint32_t s = (uint32_t)slab;
    s = std::max<uint32_t>(kRow, std::min<uint32_t>(s, 65536u));
    return s / kRow * kRow;
}

// Slab layout and the chunking of the per-tensor histogram scan.
struct Layout {
    std::vector<TensorDesc> descs;
    std::vector<int32_t> call_index;  // descriptor -> caller's tensor index
    uint32_t tiles = 0;
    std::vector<ScanChunk> chunks;
    std::vector<uint32_t> tensor_chunk_begin;
};

void finish_layout(Layout &L, uint32_t slab) {
    L.tiles = 0;
    L.chunks.clear();
    L.tensor_chunk_begin.assign(1, 0);
    for (uint32_t t = 0; t < L.descs.size(); ++t) {
        TensorDesc &d = L.descs[t];
        uint64_t nt = (d.numel + slab - 1) / slab;
        if ((uint64_t)L.tiles + nt >= (1ULL << 31)) throw Invalid("too many slabs; raise the slab size");
        d.tile_begin = L.tiles;
        d.n_tiles = (uint32_t)nt;
        L.tiles += (uint32_t)nt;
        for (uint32_t c = 0; c < nt; c += kScanTiles)
            L.chunks.push_back(
                ScanChunk{d.tile_begin + c, d.tile_begin + std::min<uint32_t>(c + kScanTiles, (uint32_t)nt), t, 0});
        L.tensor_chunk_begin.push_back((uint32_t)L.chunks.size());
    }
}

TensorDesc make_desc(const uint16_t *p, uint64_t numel) {
    if (((uintptr_t)p) & 1) throw Invalid("tensor data must be 2-byte aligned");
    if (numel >= (1ULL << 32)) throw Invalid("tensors of 2^32 or more elements are not supported");
    TensorDesc d{};
    d.frame = reinterpret_cast<const uint32_t *>((uintptr_t)p & ~uintptr_t(3));
    d.lead = (uint32_t)(((uintptr_t)p & 3) >> 1);
    d.base = const_cast<uint16_t *>(p);
    d.numel = numel;
    return d;
}

// Device copies of the scan chunking.
struct ScanDev {
    ScanChunk *chunks;
    uint32_t *tcb, *csum;
    uint32_t n_chunks;
    uint32_t *tile_tensor;  // [tiles]
};

// The scan's tables on the device, with its chunk list and the tensors' first chunks already uploaded
// (chunks, tcb); the slab-to-tensor map is built here.
ScanDev scan_buffers(Arena &ar, const Layout &L, const TensorDesc *d_descs, ScanChunk *chunks, uint32_t *tcb,
                     hipStream_t s) {
    ScanDev sd;
    sd.tile_tensor = ar.get<uint32_t>(L.tiles);
    launch_tile_map(d_descs, (uint32_t)L.descs.size(), sd.tile_tensor, s);
    sd.n_chunks = (uint32_t)L.chunks.size();
    sd.chunks = chunks;
    sd.tcb = tcb;
    sd.csum = ar.get<uint32_t>((uint64_t)sd.n_chunks * 256);
    return sd;
}

}  // namespace crx

using namespace crx;

// ------------------------------------------------------------------ handles
struct crx_update {
    Update u;  // refers to the caller's bytes (block table, payload)
};

struct crx_encoded {
    int32_t n = 0;
    std::vector<int32_t> present;
    std::vector<uint64_t> checksum;
    std::vector<uint64_t> numel;
    std::vector<Table> tables;
    std::vector<std::vector<Group>> groups;  // per caller tensor
    uint64_t n_blocks = 0;
    const uint32_t *d_block_bits = nullptr;
    uint64_t payload_len = 0;
    const uint8_t *d_payload = nullptr;
    uint64_t total_changes = 0;
    // the serialised header, built once for crx_encoded_size and crx_encoded_write (with the names it
    // was built for: a call with other names builds it again)
    std::mutex hdr_mu;
    std::vector<uint8_t> hdr;
    std::vector<std::string> hdr_names;
    bool hdr_valid = false;
};

namespace crx {
namespace {

// LEB128 varint at p (at most 10 bytes); returns the end
inline uint8_t *varint_at(uint8_t *p, uint64_t v) {
    while (v >= 0x80) {
        *p++ = (uint8_t)(v | 0x80);
        v >>= 7;
    }
    *p++ = (uint8_t)v;
    return p;
}

// The header (wire.py:64-85): magic, version, tables, then the tensors with changes.  Written through
// a pointer into a buffer sized for the longest varints, then cut to length.
void write_header(const crx_encoded &e, const char *const *names, const uint64_t *name_lens, std::vector<uint8_t> &out) {
    uint64_t cap = 5 + 10 + 10;
    for (const Table &t : e.tables) cap += 1 + 10 + 11 * t.symbols.size();
    for (int32_t t = 0; t < e.n; ++t)
        if (e.present[t]) cap += 10 + name_lens[t] + 10 + 8 + 10 + 12 * e.groups[t].size();
    out.resize(cap);
    uint8_t *p = out.data();
    *p++ = 'C', *p++ = 'R', *p++ = 'X', *p++ = 'S', *p++ = kVersion;
    p = varint_at(p, e.tables.size());
    for (const Table &t : e.tables) {
        *p++ = (uint8_t)t.exponent;
        p = varint_at(p, t.symbols.size());
        for (size_t k = 0; k < t.symbols.size(); ++k) {
            p = varint_at(p, t.symbols[k]);
            *p++ = t.lengths[k];
        }
    }
    uint64_t n_present = 0;
    for (int32_t t = 0; t < e.n; ++t) n_present += e.present[t] ? 1 : 0;
    p = varint_at(p, n_present);
    for (int32_t t = 0; t < e.n; ++t) {
        if (!e.present[t]) continue;
        p = varint_at(p, name_lens[t]);
        std::memcpy(p, names[t], name_lens[t]);
        p += name_lens[t];
        p = varint_at(p, e.numel[t]);
        for (int k = 0; k < 8; ++k) *p++ = (uint8_t)(e.checksum[t] >> (8 * k));
        p = varint_at(p, e.groups[t].size());
        for (const Group &g : e.groups[t]) {
            *p++ = (uint8_t)g.exponent;
            p = varint_at(p, g.count);
            *p++ = (uint8_t)g.rice;
        }
    }
    out.resize((uint64_t)(p - out.data()));
}

// The header for these names, copied from the handle's when that was built for the same names (a copy:
// another thread may rebuild the handle's for other names).
std::vector<uint8_t> header_of(crx_encoded &e, const char *const *names, const uint64_t *name_lens) {
    std::lock_guard<std::mutex> lock(e.hdr_mu);
    bool same = e.hdr_valid && e.hdr_names.size() == (size_t)e.n;
    for (int32_t t = 0; same && t < e.n; ++t)
        same = e.hdr_names[t].size() == name_lens[t] && std::memcmp(e.hdr_names[t].data(), names[t], name_lens[t]) == 0;
    if (!same) {
        write_header(e, names, name_lens, e.hdr);
        e.hdr_names.assign(e.n, std::string());
        for (int32_t t = 0; t < e.n; ++t) e.hdr_names[t].assign(names[t], name_lens[t]);
        e.hdr_valid = true;
    }
    return e.hdr;
}

// Python's repr() of a str, for names quoted in messages as the reference's f-strings do: single
// quotes unless the name holds a single quote and no double quote; backslashes, the quote and
// control characters escaped.
std::string py_repr(const std::string &s) {
    const char q = (s.find('\'') != std::string::npos && s.find('"') == std::string::npos) ? '"' : '\'';
    std::string out(1, q);
    for (unsigned char c : s) {
        if (c == '\\' || c == (unsigned char)q) {
            out += '\\';
            out += (char)c;
        } else if (c == '\n') {
            out += "\\n";
        } else if (c == '\r') {
            out += "\\r";
        } else if (c == '\t') {
            out += "\\t";
        } else if (c < 0x20 || c == 0x7F) {
            char buf[8];
            std::snprintf(buf, sizeof buf, "\\x%02x", c);
            out += buf;
        } else {
            out += (char)c;
        }
    }
    return out + q;
}

// ------------------------------------------------------------------ encode
// codec.encode (codec.py:278-420) on the device.
// rare symbols downloaded with the symbol counts, before their number is known
constexpr uint64_t kRareFirst = 16384;

// Elements of the tensors of a layout.
uint64_t layout_elements(const Layout &L) {
    uint64_t n = 0;
    for (const TensorDesc &d : L.descs) n += d.numel;
    return n;
}

// Elements per part of an update encoded or applied part by part (an update of 2^32 or more changes):
// each part's changes stay below 2^31, so that every per-part index fits 32 bits; a tensor larger than
// this is a part of its own (fewer than 2^32 changes).  CRX_PART_ELEMENTS (> 0) sets the size and splits
// every update larger than it, for tests of the part-wise path at sizes an oracle can check.
constexpr uint64_t kPartElements = 1ULL << 31;
uint64_t part_elements_override() {
    const char *v = std::getenv("CRX_PART_ELEMENTS");
    return v ? std::strtoull(v, nullptr, 10) : 0;
}

// Consecutive tensors of the layout in parts of at most `limit` elements (a larger tensor alone).
std::vector<std::pair<uint32_t, uint32_t>> split_parts(const Layout &L, uint64_t limit) {
    std::vector<std::pair<uint32_t, uint32_t>> out;
    uint32_t b = 0;
    uint64_t acc = 0;
    for (uint32_t i = 0; i < (uint32_t)L.descs.size(); ++i) {
        if (i > b && acc + L.descs[i].numel > limit) {
            out.emplace_back(b, i);
            b = i;
            acc = 0;
        }
        acc += L.descs[i].numel;
    }
    if (b < (uint32_t)L.descs.size()) out.emplace_back(b, (uint32_t)L.descs.size());
    return out;
}

// The layout of tensors [d0, d1) of L.
Layout sub_layout(const Layout &L, uint32_t d0, uint32_t d1, uint32_t slab) {
    Layout P;
    P.descs.assign(L.descs.begin() + d0, L.descs.begin() + d1);
    P.call_index.assign(L.call_index.begin() + d0, L.call_index.begin() + d1);
    finish_layout(P, slab);
    return P;
}

// The changes of the tensors of L ranked (codec.py:124-147,278-341): per slab exponent counts of all
// elements and of the changed ones, their scans, the groups (tensor, exponent) with their counts, and
// each slab's change records.  Stops before the records' second pass when the update has `stop_at` or
// more changes (C says how many; nothing else is then valid).
struct Ranked {
    TensorDesc *d_descs = nullptr;
    ScanDev sd{};
    EncRankArgs a{};
    uint32_t *hall = nullptr, *hchg = nullptr, *gbase = nullptr;
    GroupDev *d_groups = nullptr;
    uint64_t *delta = nullptr, *full = nullptr;  // [tiles] checksum parts
    uint64_t G = 0, C = 0;
};

Ranked rank_changes(const Layout &L, uint32_t slab, hipStream_t s, Arena &ar, HostClock *hc, uint64_t stop_at) {
    const uint32_t T = (uint32_t)L.descs.size(), tiles = L.tiles;
    Ranked R;
    UploadBatch ub;  // the tensors, the scan's chunks and a zeroed overflow flag in one copy
    const size_t i_descs = ub.add(L.descs.data(), T), i_chunks = ub.add(L.chunks.data(), L.chunks.size()),
                 i_tcb = ub.add(L.tensor_chunk_begin.data(), L.tensor_chunk_begin.size()),
                 i_ovf = ub.add_zeros<unsigned int>(1);
    ub.commit(ar, s);
    R.d_descs = ub.at<TensorDesc>(i_descs);
    R.hall = ar.get<uint32_t>((uint64_t)tiles * 256);
    R.hchg = ar.get<uint32_t>((uint64_t)tiles * 256);
    R.delta = ar.get<uint64_t>(tiles);
    R.full = ar.get<uint64_t>(tiles);
    R.sd = scan_buffers(ar, L, R.d_descs, ub.at<ScanChunk>(i_chunks), ub.at<uint32_t>(i_tcb), s);
    uint32_t *tot_all = ar.get<uint32_t>((uint64_t)T * 256), *tot_chg = ar.get<uint32_t>((uint64_t)T * 256);
    uint32_t *csum_chg = ar.get<uint32_t>((uint64_t)R.sd.n_chunks * 256);  // the change counts' chunk sums
    R.d_groups = ar.get<GroupDev>((uint64_t)T * 256);
    R.gbase = ar.get<uint32_t>((uint64_t)T * 256);
    unsigned long long *gcnt = ar.get<unsigned long long>(2);

    // Each slab stores its change records in a region of its own, sized for 1/24 of its elements
    // (+64).  If one overflows, the exact counts of that pass give exact regions for a second pass.
    const uint64_t per_slab = slab / 24 + 64;
    uint32_t *rec_count = ar.get<uint32_t>(tiles);
    unsigned int *ovf = ub.at<unsigned int>(i_ovf);
    R.a = EncRankArgs{R.d_descs, R.sd.tile_tensor, T, slab, R.hall, R.hchg, ar.get<uint64_t>((uint64_t)tiles * per_slab),
                      nullptr, per_slab, rec_count, ovf, R.delta, R.full};
    launch_enc_rank(R.a, tiles, s);
    if (hc) hc->mark("enc_setup");
    // the scans and groups need only the counts, which are exact even when a slab's records overflowed
    // their region; the overflow flag is read with the group totals, and on overflow the rank pass runs
    // again into exact regions (rewriting the counts, so they are scanned again)
    unsigned int hovf1 = 0;
    unsigned long long gc[2];
    for (int pass = 0;; ++pass) {
        const ScanTabs tabs{{R.hall, R.hchg}, {R.sd.csum, csum_chg}, {tot_all, tot_chg}};
        launch_scan_tables(R.d_descs, tabs, 2, R.sd.chunks, R.sd.n_chunks, R.sd.tcb, T, s);
        launch_enc_groups(tot_chg, T, R.d_groups, R.gbase, gcnt, s);
        d2h(&hovf1, ovf, 1, s);
        d2h(gc, gcnt, 2, s);
        sync(s);
        R.G = gc[0];
        R.C = gc[1];
        if (!hovf1 || R.C >= stop_at) break;
        if (pass) throw DeviceError("change records overflowed exact regions");
        unsigned long long *rec_base = ar.get<unsigned long long>(tiles + 1);
        launch_scan_u32(rec_count, tiles, rec_base, ar.get<unsigned long long>(scan_parts(tiles)), s);
        unsigned long long total = 0;
        d2h(&total, rec_base + tiles, 1, s);
        sync(s);
        R.a.rec = ar.get<uint64_t>(total);
        R.a.rec_base = rec_base;
        zero(ovf, 1, s);
        launch_enc_rank(R.a, tiles, s);
    }
    return R;
}

// Rice parameters of the groups, chosen from their three candidate costs (codec.py:354-360), and their
// first blocks; returns the bits of their gap codes.
uint64_t choose_rice(std::vector<GroupDev> &groups, const std::vector<unsigned long long> &hcost) {
    uint64_t blk = 0, bits = 0;
    for (uint64_t g = 0; g < groups.size(); ++g) {
        GroupDev &gr = groups[g];
        const int c[3] = {(int)(gr.r0 ? gr.r0 - 1 : 0), (int)gr.r0, (int)std::min<uint32_t>(gr.r0 + 1, kMaxRice)};
        const uint64_t sh[3] = {hcost[g * 3], hcost[g * 3 + 1], hcost[g * 3 + 2]};
        gr.rice = (uint32_t)rice_choose(gr.count, c, sh);
        const int k = gr.rice == (uint32_t)c[0] ? 0 : gr.rice == (uint32_t)c[1] ? 1 : 2;
        bits += sh[k] + (uint64_t)gr.count * (1 + gr.rice);
        gr.blk_base = (uint32_t)blk;
        blk += n_blocks(gr.count);
    }
    return bits;
}

// One canonical Huffman table per exponent with residuals (codec.py:369-392), symbols ascending, from
// the counts of the dense symbols ([256][kDense]) and of the rare ones ((exponent << 17 | zz, count),
// keys ascending); appended to E.tables.  lut gets (code << 5) | length of the dense symbols, rkeys and
// rvals those of the rare ones.  Returns the bits of all residual codes.
uint64_t build_tables(const std::vector<uint64_t> &dense, const std::vector<std::pair<uint32_t, uint64_t>> &rare,
                      crx_encoded &E, std::vector<uint32_t> &lut, std::vector<uint32_t> &rkeys,
                      std::vector<uint32_t> &rvals) {
    lut.assign(256 * kDense, 0);
    rkeys.clear();
    rvals.clear();
    uint64_t bits = 0;
    std::vector<uint32_t> syms;
    std::vector<uint64_t> counts;
    size_t ri = 0;
    for (int e = 0; e < 256; ++e) {
        syms.clear();
        counts.clear();
        for (int z = 0; z < kDense; ++z)
            if (dense[e * kDense + z]) {
                syms.push_back(z);
                counts.push_back(dense[e * kDense + z]);
            }
        for (; ri < rare.size() && (int)(rare[ri].first >> 17) == e; ++ri) {
            syms.push_back(rare[ri].first & 0x1FFFF);
            counts.push_back(rare[ri].second);
        }
        if (syms.empty()) continue;
        const std::vector<int> len = huffman_lengths(counts);
        const std::vector<uint32_t> code = canonical_codes(len);
        Table tb;
        tb.exponent = e;
        tb.symbols = syms;
        tb.lengths.resize(syms.size());
        for (size_t k = 0; k < syms.size(); ++k) {
            tb.lengths[k] = (uint8_t)len[k];
            bits += counts[k] * (uint64_t)len[k];
            const uint32_t v = (code[k] << 5) | (uint32_t)len[k];
            if (syms[k] < (uint32_t)kDense) lut[e * kDense + syms[k]] = v;
            else {
                rkeys.push_back(((uint32_t)e << 17) | syms[k]);
                rvals.push_back(v);
            }
        }
        E.tables.push_back(std::move(tb));
    }
    return bits;
}

// An update encoded part by part (more changes than one pass indexes in 32 bits, or parts asked for):
// the tensors in parts of at most `limit` elements.  Pass 1 ranks each part for its groups, symbol
// counts and checksum parts; the tables are built from the whole update's counts (codec.py:362-392);
// pass 2 ranks each part again and codes it at its bit offset in the one payload (the reference's
// batches join mid-byte the same way, codec.py:394-410).  The bytes are those of a single pass.  A
// part's buffers are reused by the next part's (Arena scopes).
void encode_parts(const Layout &L, uint64_t limit, uint32_t slab, const int32_t *has_cache, const uint64_t *cache_vals,
                  hipStream_t s, Arena &ar, crx_encoded &E) {
    const std::vector<std::pair<uint32_t, uint32_t>> ranges = split_parts(L, limit);
    struct Part {
        Layout L;
        std::vector<GroupDev> groups;  // Rice parameters and part-relative first blocks chosen on the host
        std::vector<uint32_t> dense;   // [256][kDense] symbol counts
        std::vector<std::pair<uint32_t, uint64_t>> rare;  // (exponent << 17 | zz, count), keys ascending
        uint64_t C = 0, B = 0, blk0 = 0, bits = 0, bit0 = 0;
    };
    std::vector<Part> parts(ranges.size());
    std::vector<uint64_t> dense(256 * kDense, 0);
    std::vector<std::pair<uint32_t, uint64_t>> rare;
    uint64_t C_all = 0, B_all = 0;
    for (size_t k = 0; k < parts.size(); ++k) {
        Part &p = parts[k];
        p.L = sub_layout(L, ranges[k].first, ranges[k].second, slab);
        const uint32_t T = (uint32_t)p.L.descs.size();
        std::vector<uint64_t> hdelta(T), hfull(T);
        std::vector<unsigned long long> hcost;
        ar.begin_scope();
        const Ranked R = rank_changes(p.L, slab, s, ar, nullptr, UINT64_MAX);
        p.C = R.C;
        uint64_t *t_delta = ar.get<uint64_t>(T), *t_full = ar.get<uint64_t>(T);
        launch_tensor_sums(R.d_descs, T, R.delta, t_delta, s);
        launch_tensor_sums(R.d_descs, T, R.full, t_full, s);
        d2h(hdelta.data(), t_delta, T, s);
        d2h(hfull.data(), t_full, T, s);
        unsigned long long hs[2] = {0, 0};
        uint32_t *d_rare = nullptr;
        if (R.C) {
            uint64_t *sorted = ar.get<uint64_t>(R.C);
            launch_place(R.a, p.L.tiles, R.sd.tile_tensor, R.hall, R.hchg, R.gbase, sorted, R.C, s);
            uint32_t *cmap = ar.get<uint32_t>((R.C + kElemsPerThread - 1) / kElemsPerThread);
            launch_chunk_map(R.d_groups, (uint32_t)R.G, cmap, s);
            launch_r0(R.d_groups, (uint32_t)R.G, sorted, s);
            uint32_t *d_dense = ar.get<uint32_t>(256 * kDense);
            d_rare = ar.get<uint32_t>(R.C);
            unsigned long long *scnt = ar.get<unsigned long long>(2), *cost = ar.get<unsigned long long>(R.G * 3);
            zero(d_dense, 256 * kDense, s);
            zero(scnt, 2, s);
            zero(cost, R.G * 3, s);
            StatsArgs st{sorted, R.C, R.d_groups, (uint32_t)R.G, cmap, d_dense, d_rare, R.C, scnt, cost};
            launch_stats(st, s);
            p.groups.resize(R.G);
            hcost.resize(R.G * 3);
            p.dense.resize(256 * kDense);
            d2h(p.groups.data(), R.d_groups, R.G, s);
            d2h(hcost.data(), cost, R.G * 3, s);
            d2h(p.dense.data(), d_dense, 256 * kDense, s);
            d2h(hs, scnt, 2, s);
        }
        sync(s);
        if (hs[1]) throw DeviceError("rare symbol list overflowed");
        std::vector<uint32_t> hrare(hs[0]);
        if (hs[0]) {
            d2h(hrare.data(), d_rare, hs[0], s);
            sync(s);
        }
        ar.end_scope();
        std::sort(hrare.begin(), hrare.end());
        for (size_t i = 0; i < hrare.size();) {
            size_t j = i;
            while (j < hrare.size() && hrare[j] == hrare[i]) ++j;
            p.rare.emplace_back(hrare[i], (uint64_t)(j - i));
            i = j;
        }
        if (p.C) {
            p.bits = choose_rice(p.groups, hcost);
            p.B = p.groups.back().blk_base + n_blocks(p.groups.back().count);
        }
        for (uint32_t d = 0; d < T; ++d) {  // checksums (codec.py:344-352) and groups of the part's tensors
            const int32_t t = p.L.call_index[d];
            E.checksum[t] = (has_cache && has_cache[t]) ? cache_vals[t] + hdelta[d] : hfull[d];
        }
        for (const GroupDev &gr : p.groups) {
            const int32_t t = p.L.call_index[gr.tensor];
            E.present[t] = 1;
            E.groups[t].push_back(Group{(int)gr.exponent, gr.count, (int)gr.rice});
        }
        p.blk0 = B_all;
        B_all += p.B;
        C_all += p.C;
        for (size_t i = 0; i < p.dense.size(); ++i) dense[i] += p.dense[i];
        rare.insert(rare.end(), p.rare.begin(), p.rare.end());
    }
    E.total_changes = C_all;
    if (!C_all) return;
    // one table per exponent from the whole update's symbol counts
    std::sort(rare.begin(), rare.end());
    size_t w = 0;
    for (size_t i = 0; i < rare.size(); ++i) {
        if (w && rare[w - 1].first == rare[i].first) rare[w - 1].second += rare[i].second;
        else rare[w++] = rare[i];
    }
    rare.resize(w);
    std::vector<uint32_t> lut, rkeys, rvals;
    build_tables(dense, rare, E, lut, rkeys, rvals);
    // each part's bits: its gap codes (chosen above) and its residual codes; then its first bit
    uint64_t total_bits = 0;
    for (Part &p : parts) {
        for (size_t i = 0; i < p.dense.size(); ++i) p.bits += (uint64_t)p.dense[i] * (lut[i] & 31u);
        for (const auto &kc : p.rare) {
            const size_t at = (size_t)(std::lower_bound(rkeys.begin(), rkeys.end(), kc.first) - rkeys.begin());
            p.bits += kc.second * (rvals[at] & 31u);
        }
        p.bit0 = total_bits;
        total_bits += p.bits;
    }

    // the payload and the block table of the whole update, written part by part
    const uint64_t n_words = (total_bits + 31) / 32 + 4;
    uint32_t *words = ar.get<uint32_t>(n_words);
    uint32_t *bb = ar.get<uint32_t>(B_all);
    uint32_t *d_lut = ar.get<uint32_t>(256 * kDense);
    uint32_t *d_rk = ar.get<uint32_t>(rkeys.size()), *d_rv = ar.get<uint32_t>(rvals.size());
    h2d(d_lut, lut.data(), lut.size(), s);
    h2d(d_rk, rkeys.data(), rkeys.size(), s);
    h2d(d_rv, rvals.data(), rvals.size(), s);
    zero(words, n_words, s);
    for (Part &p : parts) {
        if (!p.C) continue;
        const uint64_t G = p.groups.size();
        ar.begin_scope();
        const Ranked R = rank_changes(p.L, slab, s, ar, nullptr, UINT64_MAX);
        if (R.C != p.C || R.G != G) throw DeviceError("a part of the update ranked differently the second time");
        uint64_t *sorted = ar.get<uint64_t>(p.C);
        launch_place(R.a, p.L.tiles, R.sd.tile_tensor, R.hall, R.hchg, R.gbase, sorted, p.C, s);
        GroupDev *d_groups = ar.get<GroupDev>(G);
        h2d(d_groups, p.groups.data(), G, s);
        const uint64_t n_thr = (p.C + kElemsPerThread - 1) / kElemsPerThread;
        uint32_t *cmap = ar.get<uint32_t>(n_thr);
        launch_chunk_map(d_groups, (uint32_t)G, cmap, s);
        unsigned long long *tsum = ar.get<unsigned long long>(n_thr), *toff = ar.get<unsigned long long>(n_thr + 1);
        unsigned long long *bstart = ar.get<unsigned long long>(p.B + 1);
        unsigned int *bovf = ar.get<unsigned int>(1);
        CodeArgs ca{sorted, p.C, d_groups, (uint32_t)G, d_lut, d_rk, d_rv, (uint32_t)rkeys.size(), cmap, tsum, toff,
                    words, bstart, n_words, bovf, p.bit0};
        launch_code_lengths(ca, s);
        launch_scan_u64(tsum, n_thr, toff, ar.get<unsigned long long>(scan_parts(n_thr)), s);
        zero(bovf, 1, s);
        const unsigned long long end = p.bit0 + p.bits;  // the block starts are payload bits: so is the end
        h2d(bstart + p.B, &end, 1, s);
        launch_pack(ca, s);
        launch_block_bits(bstart, p.B, bb + p.blk0, bovf, s);
        unsigned int hovf = 0;
        unsigned long long dev_bits = 0;
        d2h(&hovf, bovf, 1, s);
        d2h(&dev_bits, toff + n_thr, 1, s);
        sync(s);
        ar.end_scope();
        if (hovf & 2u || dev_bits != p.bits) throw DeviceError("the packed payload's size differs from its codes' lengths");
        if (hovf) throw Invalid("a block exceeds 2^32 bits; the update cannot be represented");
    }
    E.n_blocks = B_all;
    E.d_block_bits = bb;
    E.payload_len = (total_bits + 7) / 8;
    E.d_payload = reinterpret_cast<const uint8_t *>(words);
}

void encode(int32_t n, const uint16_t *const *olds, const uint16_t *const *news, const uint64_t *numels,
            const int32_t *has_cache, const uint64_t *cache_vals, int32_t slab_req, hipStream_t s, Arena &ar,
            crx_encoded &E) {
    const uint32_t slab = slab_size(slab_req);
    E.n = n;
    E.present.assign(n, 0);
    E.checksum.assign(n, 0);
    E.numel.assign(numels, numels + n);
    E.groups.assign(n, {});
    HostClock hc;
    Layout L;
    for (int32_t t = 0; t < n; ++t) {
        if (!numels[t]) continue;
        TensorDesc d = make_desc(olds[t], numels[t]);
        TensorDesc dn = make_desc(news[t], numels[t]);
        if (dn.lead != d.lead) throw Invalid("old and new must have the same 4-byte alignment");
        d.frame_new = dn.frame;
        d.cold = (has_cache && has_cache[t]) ? 0u : 1u;
        L.descs.push_back(d);
        L.call_index.push_back(t);
    }
    if (L.descs.empty()) return;
    finish_layout(L, slab);
    const uint64_t forced = part_elements_override();
    if (forced && layout_elements(L) > forced) {  // parts asked for (tests of the part-wise path)
        encode_parts(L, forced, slab, has_cache, cache_vals, s, ar, E);
        return;
    }
    const uint32_t T = (uint32_t)L.descs.size(), tiles = L.tiles;
    const uint64_t hint_key = tiles;
    ar.reserve(g_encode_hint.get(hint_key));
    hc.mark("enc_layout");

    Ranked R = rank_changes(L, slab, s, ar, &hc, 1ULL << 32);
    hc.mark("enc_wait_groups");
    if (R.C >= (1ULL << 32)) {  // too many changes for one pass: the update is encoded part by part
        encode_parts(L, kPartElements, slab, has_cache, cache_vals, s, ar, E);
        return;
    }
    const uint64_t G = R.G, C = R.C;
    E.total_changes = C;
    if (C == 0) return;
    TensorDesc *const d_descs = R.d_descs;
    GroupDev *const d_groups = R.d_groups;
    uint64_t *const delta = R.delta, *const full = R.full;
    const EncRankArgs &a = R.a;
    const ScanDev &sd = R.sd;
    uint32_t *const hall = R.hall, *const hchg = R.hchg, *const gbase = R.gbase;

    uint64_t *sorted = ar.get<uint64_t>(C);
    launch_place(a, tiles, sd.tile_tensor, hall, hchg, gbase, sorted, C, s);
    const uint64_t n_thr = (C + kElemsPerThread - 1) / kElemsPerThread;  // threads of the walking kernels
    uint32_t *cmap = ar.get<uint32_t>(n_thr);
    launch_chunk_map(d_groups, (uint32_t)G, cmap, s);
    launch_r0(d_groups, (uint32_t)G, sorted, s);
    // what the host reads back after the symbol counts, in one block so that one copy brings it (the
    // first kRareFirst rare symbols with it): cost | dense | scnt | t_delta | t_full | rare
    const uint64_t o_dense = G * 3 * 8, o_scnt = o_dense + 256 * kDense * 4, o_delta = o_scnt + 16,
                   o_full = o_delta + 8 * (uint64_t)T, o_rare = o_full + 8 * (uint64_t)T;
    uint8_t *dl = ar.get<uint8_t>(o_rare + 4 * C);
    unsigned long long *cost = reinterpret_cast<unsigned long long *>(dl);
    uint32_t *dense = reinterpret_cast<uint32_t *>(dl + o_dense);
    unsigned long long *scnt = reinterpret_cast<unsigned long long *>(dl + o_scnt);
    uint64_t *t_delta = reinterpret_cast<uint64_t *>(dl + o_delta), *t_full = reinterpret_cast<uint64_t *>(dl + o_full);
    uint32_t *rare = reinterpret_cast<uint32_t *>(dl + o_rare);
    zero(dl, o_delta, s);  // cost, dense and scnt; the sums are written whole
    StatsArgs st{sorted, C, d_groups, (uint32_t)G, cmap, dense, rare, C, scnt, cost};
    launch_stats(st, s);
    launch_tensor_sums(d_descs, T, delta, t_delta, s);
    launch_tensor_sums(d_descs, T, full, t_full, s);

    std::vector<GroupDev> groups(G);
    d2h(groups.data(), d_groups, G, s);
    // the first rare symbols in the same wait (an update has few); the rest, if any, after it
    const uint64_t rare_first = std::min<uint64_t>(C, kRareFirst);
    std::vector<uint8_t> hdl(o_rare + 4 * rare_first);
    d2h(hdl.data(), dl, hdl.size(), s);
    sync(s);
    hc.mark("enc_wait_stats");
    std::vector<unsigned long long> hcost(G * 3);
    std::vector<uint32_t> hdense(256 * kDense);
    std::vector<uint64_t> hdelta(T), hfull(T);
    unsigned long long hs[2];
    std::memcpy(hcost.data(), hdl.data(), o_dense);
    std::memcpy(hdense.data(), hdl.data() + o_dense, 256 * kDense * 4);
    std::memcpy(hs, hdl.data() + o_scnt, 16);
    std::memcpy(hdelta.data(), hdl.data() + o_delta, 8 * (uint64_t)T);
    std::memcpy(hfull.data(), hdl.data() + o_full, 8 * (uint64_t)T);
    if (hs[1]) throw DeviceError("rare symbol list overflowed");
    std::vector<uint32_t> hrare(hs[0]);
    if (hs[0]) std::memcpy(hrare.data(), hdl.data() + o_rare, 4 * std::min<uint64_t>(hs[0], rare_first));
    if (hs[0] > rare_first) {
        d2h(hrare.data() + rare_first, rare + rare_first, hs[0] - rare_first, s);
        sync(s);
    }
    hc.mark("enc_wait_rare");
    std::sort(hrare.begin(), hrare.end());
    std::vector<std::pair<uint32_t, uint64_t>> rare_runs;
    for (size_t i = 0; i < hrare.size();) {
        size_t j = i;
        while (j < hrare.size() && hrare[j] == hrare[i]) ++j;
        rare_runs.emplace_back(hrare[i], (uint64_t)(j - i));
        i = j;
    }

    // What the code kernels need first: Rice parameters and first blocks of the groups (codec.py:354-360),
    // and one canonical Huffman table per exponent, symbols ascending (codec.py:369-392).  The payload's
    // length follows from them: a group's gap codes take its chosen cost, its symbols their code lengths.
    uint64_t total_bits = choose_rice(groups, hcost);
    const uint64_t B = groups.empty() ? 0 : groups.back().blk_base + n_blocks(groups.back().count);
    std::vector<uint64_t> dense64(hdense.begin(), hdense.end());
    std::vector<uint32_t> lut, rkeys, rvals;
    total_bits += build_tables(dense64, rare_runs, E, lut, rkeys, rvals);
    hc.mark("enc_tables");

    // the code lengths, their offsets and the bits, with no wait: the payload's size is known
    UploadBatch ub;  // the groups with their Rice parameters, the code tables, a zeroed overflow flag
    const size_t i_groups = ub.add(groups.data(), G), i_lut = ub.add(lut.data(), lut.size()),
                 i_rk = ub.add(rkeys.data(), rkeys.size()), i_rv = ub.add(rvals.data(), rvals.size()),
                 i_ovf = ub.add_zeros<unsigned int>(1);
    ub.commit(ar, s);
    GroupDev *d_groups2 = ub.at<GroupDev>(i_groups);
    uint32_t *d_lut = ub.at<uint32_t>(i_lut), *d_rk = ub.at<uint32_t>(i_rk), *d_rv = ub.at<uint32_t>(i_rv);
    unsigned long long *tsum = ar.get<unsigned long long>(n_thr), *toff = ar.get<unsigned long long>(n_thr + 1);
    const uint64_t n_words = (total_bits + 31) / 32 + 4;
    uint32_t *words = ar.get<uint32_t>(n_words);
    unsigned long long *bstart = ar.get<unsigned long long>(B + 1);
    uint32_t *bb = ar.get<uint32_t>(B);
    unsigned int *bovf = ub.at<unsigned int>(i_ovf);
    CodeArgs ca{sorted, C, d_groups2, (uint32_t)G, d_lut, d_rk, d_rv, (uint32_t)rkeys.size(), cmap, tsum, toff,
                words, bstart, n_words, bovf};
    launch_code_lengths(ca, s);
    launch_scan_u64(tsum, n_thr, toff, ar.get<unsigned long long>(scan_parts(n_thr)), s);
    zero(words, n_words, s);
    HIP_OK(hipMemcpyAsync(bstart + B, toff + n_thr, sizeof(unsigned long long), hipMemcpyDeviceToDevice, s));
    launch_pack(ca, s);
    launch_block_bits(bstart, B, bb, bovf, s);
    unsigned int hovf = 0;
    unsigned long long dev_bits = 0;
    d2h(&hovf, bovf, 1, s);
    d2h(&dev_bits, toff + n_thr, 1, s);

    // the rest of the host's part while the device packs: checksums (codec.py:344-352), the groups
    for (uint32_t d = 0; d < T; ++d) {
        const int32_t t = L.call_index[d];
        E.checksum[t] = (has_cache && has_cache[t]) ? cache_vals[t] + hdelta[d] : hfull[d];
    }
    for (uint64_t g = 0; g < G; ++g) {
        const GroupDev &gr = groups[g];
        const int32_t t = L.call_index[gr.tensor];
        E.present[t] = 1;
        E.groups[t].push_back(Group{(int)gr.exponent, gr.count, (int)gr.rice});
    }
    E.n_blocks = B;
    sync(s);
    hc.mark("enc_wait_pack");
    if (hovf & 2u || dev_bits != total_bits) throw DeviceError("the packed payload's size differs from its codes' lengths");
    if (hovf) throw Invalid("a block exceeds 2^32 bits; the update cannot be represented");
    g_encode_hint.put(hint_key, ar.total);
    E.d_block_bits = bb;
    E.payload_len = (total_bits + 7) / 8;
    E.d_payload = reinterpret_cast<const uint8_t *>(words);
}

// ------------------------------------------------------------------ apply
// codec.apply (codec.py:578-717) on the device: decode, locate, verify, then write.
uint32_t apply_slab(int32_t slab_req) { return slab_size(slab_req); }

// The update's device state that its parts share: the decoding tables, the payload, the block table and
// each block's first payload bit.
struct ApplyShared {
    uint32_t *lim = nullptr, *off = nullptr, *syms = nullptr;
    uint32_t n_syms = 0, n_tables = 0;
    const uint64_t *pay = nullptr;  // the words holding the payload, from bit bit0 of the first
    uint64_t pay_words = 0;
    uint32_t bit0 = 0;
    uint32_t *bb = nullptr;            // [blocks] bits of each block
    unsigned long long *boff = nullptr;  // [blocks + 1] first payload bit of each block
};

// A part of an update: tensors [t0, t1) of the update, their groups with element and block bases
// counted from the part's first change and block, and the part's blocks [b0, b0 + B) of the update.
struct ApplyPart {
    uint32_t t0 = 0, t1 = 0;
    std::vector<GroupDev> groups;
    std::vector<int32_t> group_of;  // [tensors of the part][256]: group of (tensor, exponent), or -1
    uint64_t C = 0, B = 0, b0 = 0;
};

// What one part's pass found: error flags, and per tensor of the part the checksum delta and (for
// tensors without a cached checksum) the full checksum of the receiver's weights before the update.
struct PartCheck {
    unsigned int bad = 0;
    std::vector<uint64_t> delta, full;
};

// One part of an update, or the whole of it (codec.py:578-717): decode, locate, verify, then write.
// dry: the part is only verified; nothing is written (no write-through, no commit, and the receiver's
// exponent counts are not kept up to date).
PartCheck apply_part(const Update &u, const Layout &L, const ApplyPart &P, const ApplyShared &sh,
                     const int32_t *has_cache, const uint64_t *cache_vals, uint32_t slab, int32_t slab_req, bool dry,
                     hipStream_t s, Arena &ar, HostClock &hc) {
    const uint32_t T = (uint32_t)L.descs.size(), tiles = L.tiles;
    const uint64_t G = P.groups.size(), B = P.B, C = P.C;
    std::vector<uint32_t> tensor_chg(T + 1, (uint32_t)C);  // first change of each tensor (its changes are contiguous)
    for (int64_t gi = (int64_t)G - 1; gi >= 0; --gi) tensor_chg[P.groups[gi].tensor] = P.groups[gi].elem_base;
    for (int64_t t = (int64_t)T - 1; t >= 0; --t) tensor_chg[t] = std::min(tensor_chg[t], tensor_chg[t + 1]);
    std::vector<TensorDesc> descs = L.descs;
    if (dry)
        for (TensorDesc &d : descs) d.hist_out = nullptr;
    // the verdict's inputs (unused by a dry pass, which uploads them all the same: its write pass then
    // asks for exactly the buffers the dry pass had)
    std::vector<uint64_t> want(T), cached(T, 0);
    std::vector<int32_t> has(T, 0);
    for (uint32_t d = 0; d < T; ++d) {
        const uint32_t t = P.t0 + d;
        want[d] = u.tensors[t].checksum;
        has[d] = (has_cache && has_cache[t]) ? 1 : 0;
        if (has[d]) cached[d] = cache_vals[t];
    }

    // every small upload of the part in one copy, ahead of the decoder, which starts at once
    UploadBatch ub;
    const size_t i_descs = ub.add(descs.data(), T), i_groups = ub.add(P.groups.data(), G),
                 i_gof = ub.add(P.group_of.data(), P.group_of.size()), i_tchg = ub.add(tensor_chg.data(), T + 1),
                 i_chunks = ub.add(L.chunks.data(), L.chunks.size()),
                 i_tcb = ub.add(L.tensor_chunk_begin.data(), L.tensor_chunk_begin.size()),
                 i_want = ub.add(want.data(), T), i_cached = ub.add(cached.data(), T), i_has = ub.add(has.data(), T),
                 i_bad = ub.add_zeros<unsigned int>(1), i_nmore = ub.add_zeros<unsigned int>(1);
    ub.commit(ar, s);
    TensorDesc *d_descs = ub.at<TensorDesc>(i_descs);
    GroupDev *d_groups = ub.at<GroupDev>(i_groups);
    unsigned int *bad = ub.at<unsigned int>(i_bad);
    uint32_t *bmap = ar.get<uint32_t>(B);
    BlockInfo *binfo = ar.get<BlockInfo>(B);
    launch_block_map(d_groups, (uint32_t)G, bmap, binfo, s);

    // The decoder needs nothing from the receiver's weights: it runs on the auxiliary stream while
    // the main stream takes the exponent counts (pass A) and their scans.
    unsigned long long *dz = ar.get<unsigned long long>(C);
    unsigned long long *blk_sum = ar.get<unsigned long long>(B), *blk_prefix = ar.get<unsigned long long>(B + 1);
    hc.mark("apply_upload");
    Fork fork(s);
    DecodeArgs da{d_descs, sh.pay, sh.pay_words, sh.bb + P.b0, sh.boff + P.b0, B, d_groups, (uint32_t)G, bmap,
                  sh.lim, sh.off, sh.syms, sh.n_syms, dz, blk_sum, bad, sh.n_tables, sh.bit0};
    launch_decode(da, fork.aux);
    launch_scan_u64(blk_sum, B, blk_prefix, ar.get<unsigned long long>(scan_parts(B)), fork.aux);

    uint32_t *hall = ar.get<uint32_t>((uint64_t)tiles * 256);
    uint64_t *full = ar.get<uint64_t>(tiles), *t_full = ar.get<uint64_t>(T);
    ScanDev sd = scan_buffers(ar, L, d_descs, ub.at<ScanChunk>(i_chunks), ub.at<uint32_t>(i_tcb), s);
    uint32_t *sizes = ar.get<uint32_t>((uint64_t)T * 256);
    int32_t *d_gof = ub.at<int32_t>(i_gof);
    uint32_t *local = ar.get<uint32_t>(C);
    unsigned long long *rec = ar.get<unsigned long long>(C);  // the select pass's records, slab by slab
    uint32_t *pn = ar.get<uint32_t>(C);                       // offset in the slab | new bits << 16
    uint32_t *rstart = ar.get<uint32_t>((uint64_t)tiles + 1);
    uint64_t *sdelta = ar.get<uint64_t>(tiles), *tdelta = ar.get<uint64_t>(T);
    uint32_t *tchg = ub.at<uint32_t>(i_tchg);
    uint32_t *lb = ar.get<uint32_t>((uint64_t)(tiles + 1) * 256);  // row tiles: read, never used

    // pass A: slabs of tensors without cached counts are streamed for their counts (and the even rows
    // of old checksums not cached: the select pass sums the rest as it streams the weights); cached
    // counts are read by the scan in place (copied only to a separate hist_out)
    std::vector<uint32_t> hist_list;
    for (const TensorDesc &d : descs) {
        const bool cached = d.hist_in != nullptr;
        if (!cached || (d.hist_out && d.hist_out != d.hist_in))
            for (uint32_t i = 0; i < d.n_tiles; ++i) hist_list.push_back(d.tile_begin + i);
    }
    HistArgs ha{d_descs, sd.tile_tensor, T, slab, hall, full, nullptr};
    if (hist_list.size() == tiles) {
        launch_hist(ha, tiles, s);
    } else if (!hist_list.empty()) {
        uint32_t *d_list = ar.get<uint32_t>(hist_list.size());
        h2d(d_list, hist_list.data(), hist_list.size(), s);
        ha.list = d_list;
        launch_hist(ha, (uint32_t)hist_list.size(), s);
    }
    const ScanTabs tabs{{hall, nullptr}, {sd.csum, nullptr}, {sizes, nullptr}};
    launch_scan_tables(d_descs, tabs, 1, sd.chunks, sd.n_chunks, sd.tcb, T, s);
    fork.join();
    hc.mark("apply_pass_a");

    BlockArgs ba{d_groups, (uint32_t)G, slab, binfo, d_descs, sizes, blk_prefix, local, dz, bad, B,
                 group_check_numel(slab_req)};
    launch_local_fix(ba, B, s);
    uint2 *more = ar.get<uint2>((uint64_t)kSelMoreWindows * tiles);  // windows after the first, per slab
    unsigned int *n_more = ub.at<unsigned int>(i_nmore);
    uint8_t *multi = ar.get<uint8_t>(tiles);
    uint32_t *done = ar.get<uint32_t>(tiles);
    // the verdict's inputs, set up before the select pass writes anything: between its writes and the
    // commit that can undo them, the host only launches
    // (allocated in a dry pass too: a part's write pass then asks for exactly the buffers its dry pass had)
    uint64_t *d_want = ub.at<uint64_t>(i_want), *d_cached = ub.at<uint64_t>(i_cached);
    int32_t *d_has = ub.at<int32_t>(i_has);
    unsigned int *ok = ar.get<unsigned int>(1);
    SelectArgs sa{d_descs, sd.tile_tensor, T, slab, hall, lb, d_gof, d_groups, local, rec, rstart, tchg, bad, more,
                  n_more, (uint32_t)std::min<uint64_t>(1024, (uint64_t)kSelMoreWindows * tiles), dz, sdelta, multi,
                  done, (uint32_t)C, blk_prefix, full};
    launch_locate(sa, tiles, s);
    // a dry pass marks every slab as one of several windows: the select pass then writes nothing, and
    // the verify pass takes every slab's checksum delta
    if (dry) HIP_OK(hipMemsetAsync(multi, 1, tiles, s));
    // slabs streamed in one window are written through by the select pass, before the verdict: the
    // commit below undoes those writes if the update does not verify
    bool any_cold = false;
    for (const TensorDesc &d : descs) any_cold |= d.cold != 0;
    launch_select(sa, tiles, C > kSelectDenseTargets * tiles, any_cold, s);
    SlabArgs sla{d_descs, sd.tile_tensor, slab, rstart, rec, dz, pn, sdelta, bad, nullptr, (uint32_t)C, multi, done};
    launch_verify(sla, tiles, s);
    launch_tensor_sums(d_descs, T, sdelta, tdelta, s);
    launch_tensor_sums(d_descs, T, full, t_full, s);  // the select pass summed the cold slabs
    if (!dry) {
        // the verdict on the device too, and the commit behind it (the remaining writes if the update
        // verifies, the undoing of the select pass's if not); the host waits for the verdict's data only
        launch_verdict(T, reinterpret_cast<const unsigned long long *>(tdelta), t_full, d_has, d_cached, d_want, bad,
                       ok, s);
        sla.ok = ok;
        launch_commit(sla, tiles, s);  // next to the verdict: nothing on the host can fail in between
    }
    hc.mark("apply_launch");

    PartCheck r;
    r.delta.resize(T);
    r.full.resize(T);
    d2h(&r.bad, bad, 1, s);
    d2h(r.delta.data(), tdelta, T, s);
    d2h(r.full.data(), t_full, T, s);
    t_stage.finish();  // the downloads above (behind the commit, which exits at once when the update verifies)
    hc.mark("apply_wait_verify");
    return r;
}

// The reference's verdict (codec.py:598-604,696-712) from the passes' findings over the whole update:
// the group-size check first, then any checksum mismatch (naming up to three tensors), then any other
// inconsistency.  Returns when the whole update verifies.
void raise_verdict(const Update &u, unsigned int bad, const std::vector<uint64_t> &delta,
                   const std::vector<uint64_t> &full, const int32_t *has_cache, const uint64_t *cache_vals) {
    if (bad & kBadGroup) throw Corrupt("group has more changes than elements");
    std::vector<std::string> wrong;
    for (uint32_t t = 0; t < (uint32_t)u.tensors.size(); ++t) {
        const uint64_t old = (has_cache && has_cache[t]) ? cache_vals[t] : full[t];
        if (old + delta[t] != u.tensors[t].checksum) wrong.push_back(u.tensors[t].name);
    }
    if (!wrong.empty()) {
        std::string m = "update does not verify (checksum mismatch: [";
        for (size_t i = 0; i < std::min<size_t>(3, wrong.size()); ++i) m += (i ? ", " : "") + py_repr(wrong[i]);
        throw Corrupt(m + "])");
    }
    if (bad) throw Corrupt("payload positions outside their exponent groups");
}

void apply(const Update &u, const uint8_t *payload_dev, uint16_t *const *targets, const uint64_t *numels,
           const int32_t *has_cache, const uint64_t *cache_vals, uint32_t *const *hist_in, uint32_t *const *hist_out,
           int32_t slab_req, hipStream_t s, Arena &ar, uint64_t *changed) {
    *changed = 0;
    const uint32_t T = (uint32_t)u.tensors.size();
    if (!T) return;
    HostClock hc;
    const uint32_t slab = apply_slab(slab_req);
    const uint64_t C = u.total_changes;
    Layout L;
    for (uint32_t t = 0; t < T; ++t) {
        if (numels[t] != u.tensors[t].numel) throw Invalid(u.tensors[t].name + ": numel mismatch");
        TensorDesc d = make_desc(targets[t], numels[t]);
        d.cold = (has_cache && has_cache[t]) ? 0u : 1u;
        d.hist_in = hist_in ? hist_in[t] : nullptr;
        d.hist_out = hist_out ? hist_out[t] : nullptr;
        L.descs.push_back(d);
        L.call_index.push_back((int32_t)t);
    }
    finish_layout(L, slab);
    // an update of 2^32 or more changes is applied part by part (each part's changes indexed in 32 bits)
    const uint64_t forced = part_elements_override();
    const bool split = C >= (1ULL << 32) || (forced && layout_elements(L) > forced);
    const std::vector<std::pair<uint32_t, uint32_t>> ranges =
        split ? split_parts(L, forced ? forced : kPartElements) : std::vector<std::pair<uint32_t, uint32_t>>{{0, T}};
    const uint32_t tiles = L.tiles;
    const uint64_t hint_key = (uint64_t)tiles + C / 256;
    if (!split) ar.reserve(g_apply_hint.get(hint_key));
    hc.mark("apply_layout");

    // groups, decoding tables and the group lookup (codec.py:594-625)
    int table_of[256];
    std::fill(table_of, table_of + 256, -1);
    // per table and code length l: lim = end of the length-l codes left-justified to 17 bits (the
    // canonical ranges are consecutive, so the length of a 17-bit peek p is 1 + #{l : lim[l] <= p}),
    // off = symbol index of the length-l code 0
    std::vector<uint32_t> lim(u.tables.size() * 17, 0), off(u.tables.size() * 17, 0), syms;
    for (size_t ti = 0; ti < u.tables.size(); ++ti) {
        const Table &tb = u.tables[ti];
        table_of[tb.exponent] = (int)ti;
        uint32_t per_len[kMaxCodeLen + 1] = {};
        for (uint8_t l : tb.lengths) per_len[l]++;
        std::vector<uint32_t> order(tb.symbols.size());
        for (size_t k = 0; k < order.size(); ++k) order[k] = (uint32_t)k;
        std::stable_sort(order.begin(), order.end(), [&](uint32_t a, uint32_t b) { return tb.lengths[a] < tb.lengths[b]; });
        uint32_t code = 0, idx = (uint32_t)syms.size();
        for (int l = 1; l <= kMaxCodeLen; ++l) {
            lim[ti * 17 + l - 1] = (code + per_len[l]) << (kMaxCodeLen - l);
            off[ti * 17 + l - 1] = idx - code;
            code = (code + per_len[l]) << 1;
            idx += per_len[l];
        }
        for (uint32_t k : order) syms.push_back(tb.symbols[k]);
    }
    std::vector<ApplyPart> parts(ranges.size());
    uint64_t B_all = 0;
    for (size_t k = 0; k < ranges.size(); ++k) {
        ApplyPart &P = parts[k];
        P.t0 = ranges[k].first;
        P.t1 = ranges[k].second;
        P.group_of.assign((uint64_t)(P.t1 - P.t0) * 256, -1);
        uint64_t elem = 0, blk = 0;
        for (uint32_t t = P.t0; t < P.t1; ++t)
            for (const Group &g : u.tensors[t].groups) {
                GroupDev gd{};
                gd.tensor = t - P.t0;
                gd.exponent = (uint32_t)g.exponent;
                gd.count = (uint32_t)g.count;
                gd.elem_base = (uint32_t)elem;
                gd.blk_base = (uint32_t)blk;
                gd.rice = (uint32_t)g.rice;
                gd.table = (uint32_t)table_of[g.exponent];
                P.group_of[(uint64_t)(t - P.t0) * 256 + g.exponent] = (int32_t)P.groups.size();
                P.groups.push_back(gd);
                elem += g.count;
                blk += n_blocks(g.count);
            }
        // a part's changes are at most its elements (the parser checks each tensor's), below 2^32
        if (elem >= (1ULL << 32)) throw Invalid("a part of the update has 2^32 or more changes");
        P.C = elem;
        P.B = blk;
        P.b0 = B_all;
        B_all += blk;
    }
    hc.mark("apply_tables");

    ApplyShared sh;
    UploadBatch tb;  // the decoding tables, in one copy
    const size_t i_lim = tb.add(lim.data(), lim.size()), i_off = tb.add(off.data(), off.size()),
                 i_syms = tb.add(syms.data(), syms.size());
    tb.commit(ar, s);
    sh.lim = tb.at<uint32_t>(i_lim);
    sh.off = tb.at<uint32_t>(i_off);
    sh.syms = tb.at<uint32_t>(i_syms);
    sh.n_syms = (uint32_t)syms.size();
    sh.n_tables = (uint32_t)(lim.size() / 17);
    sh.bb = ar.get<uint32_t>(B_all);
    if (payload_dev)  // the update is in device memory: its block table precedes the payload there
        HIP_OK(hipMemcpyAsync(sh.bb, payload_dev - (u.payload_offset - u.block_table_offset), 4 * B_all,
                              hipMemcpyDeviceToDevice, s));
    else
        HIP_OK(hipMemcpyAsync(sh.bb, u.block_table, 4 * B_all, hipMemcpyHostToDevice, s));
    // A device-resident payload is read in place, in the 8-byte aligned words that hold it, when those
    // words lie inside the allocation the update is in (the first one does: the update's header precedes
    // the payload; the last one may reach past the update's end).  Otherwise, and from the host, it is
    // copied into words of its own, zero-padded.
    bool in_place = false;
    if (payload_dev && u.payload_len) {
        const uintptr_t at = reinterpret_cast<uintptr_t>(payload_dev), lead = at & 7;
        const uint64_t words = (lead + u.payload_len + 7) / 8;
        hipDeviceptr_t base = nullptr;
        size_t size = 0;
        if (hipMemGetAddressRange(&base, &size, reinterpret_cast<hipDeviceptr_t>(at)) == hipSuccess &&
            at - lead >= reinterpret_cast<uintptr_t>(base) &&
            at - lead + 8 * words <= reinterpret_cast<uintptr_t>(base) + size) {
            in_place = true;
            sh.pay = reinterpret_cast<const uint64_t *>(at - lead);
            sh.bit0 = 8 * (uint32_t)lead;
            sh.pay_words = words;
        } else {
            (void)hipGetLastError();  // an address the runtime does not know: copied instead
        }
    }
    if (!in_place) {
        sh.pay_words = (u.payload_len + 7) / 8 + 2;
        uint64_t *pay = ar.get<uint64_t>(sh.pay_words);
        // the copy fills whole words up to payload_len / 8; the rest (partial last word, two pad words) is zeroed
        zero(pay + u.payload_len / 8, sh.pay_words - u.payload_len / 8, s);
        if (u.payload_len) {
            if (payload_dev)
                HIP_OK(hipMemcpyAsync(pay, payload_dev, u.payload_len, hipMemcpyDeviceToDevice, s));
            else
                copy_from_host(reinterpret_cast<uint8_t *>(pay), u.payload_host, u.payload_len, s);
        }
        sh.pay = pay;
    }
    sh.boff = ar.get<unsigned long long>(B_all + 1);
    launch_scan_u32(sh.bb, B_all, sh.boff, ar.get<unsigned long long>(scan_parts(B_all)), s);

    if (!split) {
        const PartCheck r = apply_part(u, L, parts[0], sh, has_cache, cache_vals, slab, slab_req, false, s, ar, hc);
        raise_verdict(u, r.bad, r.delta, r.full, has_cache, cache_vals);
        g_apply_hint.put(hint_key, ar.total);
        // the verdict is final, and the writes behind it are done (the downloads above followed them)
        *changed = C;
        return;
    }
    // Part by part: every part verified first without writing, the verdict taken on the whole update,
    // then each part applied (its own verification passes again: the same inputs).  Each part's buffers
    // are reused by the next part's.
    unsigned int bad = 0;
    std::vector<uint64_t> delta(T, 0), full(T, 0);
    std::vector<Layout> layouts;
    for (const ApplyPart &P : parts) layouts.push_back(sub_layout(L, P.t0, P.t1, slab));
    for (size_t k = 0; k < parts.size(); ++k) {
        ar.begin_scope();
        const PartCheck r = apply_part(u, layouts[k], parts[k], sh, has_cache, cache_vals, slab, slab_req, true, s, ar, hc);
        ar.end_scope();
        bad |= r.bad;
        std::copy(r.delta.begin(), r.delta.end(), delta.begin() + parts[k].t0);
        std::copy(r.full.begin(), r.full.end(), full.begin() + parts[k].t0);
    }
    raise_verdict(u, bad, delta, full, has_cache, cache_vals);
    for (size_t k = 0; k < parts.size(); ++k) {
        ar.begin_scope();
        PartCheck r;
        try {
            r = apply_part(u, layouts[k], parts[k], sh, has_cache, cache_vals, slab, slab_req, false, s, ar, hc);
        } catch (const std::bad_alloc &) {
            if (!k) throw;  // nothing written yet
            throw DeviceError("out of memory while writing a part of the update; the parts before it are written");
        }
        ar.end_scope();
        bool same = r.bad == 0;
        for (uint32_t d = 0; same && d < (uint32_t)r.delta.size(); ++d) same = r.delta[d] == delta[parts[k].t0 + d];
        if (!same)  // the receiver's weights changed between the passes (another writer)
            throw DeviceError("a part of the update did not verify when written after the whole update had; the "
                              "parts before it are written");
    }
    *changed = C;
}

void full_checksum(const uint16_t *p, uint64_t n, hipStream_t s, Arena &ar, uint64_t *out) {
    *out = 0;
    if (!n) return;
    TensorDesc d = make_desc(p, n);
    const uint64_t words = (n + d.lead + 1) >> 1;
    const uint32_t parts = (uint32_t)std::min<uint64_t>(2048, (words + 65535) / 65536);
    uint64_t *partial = ar.get<uint64_t>(parts);
    launch_checksum(d.frame, d.lead, n, partial, parts, s);
    std::vector<uint64_t> h(parts);
    d2h(h.data(), partial, parts, s);
    sync(s);
    for (uint64_t v : h) *out += v;
}

template <typename F>
int32_t guarded(char *err, uint64_t errlen, F &&f) {
    auto put = [&](const char *m) {
        if (err && errlen) std::snprintf(err, (size_t)errlen, "%s", m);
    };
    try {
        t_stage.abandon();
        f();
        if (g_timing) timing_collect(false);
        return CRX_OK;
    } catch (const Corrupt &e) {
        put(e.what());
        if (g_timing) timing_collect(false);
        return CRX_CORRUPT;
    } catch (const Invalid &e) {
        put(e.what());
        return CRX_INVALID;
    } catch (const DeviceError &e) {
        put(e.what());
        return CRX_DEVICE;
    } catch (const NeedMore &) {
        put("need more bytes");
        return CRX_INVALID;
    } catch (const std::bad_alloc &) {
        put("out of memory");
        return CRX_NOMEM;
    } catch (const std::exception &e) {
        put(e.what());
        return CRX_DEVICE;
    }
}

}  // namespace
}  // namespace crx

// ------------------------------------------------------------------ C ABI
extern "C" {

int32_t crx_abi_version(void) { return CRX_ABI_VERSION; }

int32_t crx_parse(const uint8_t *data, uint64_t len, crx_update **out, char *err, uint64_t errlen) {
    *out = nullptr;
    return guarded(err, errlen, [&] {
        auto *h = new crx_update();
        try {
            parse(data, len, len, len ? data[len - 1] : 0, h->u);
        } catch (...) {
            delete h;
            throw;
        }
        h->u.payload_host = data + h->u.payload_offset;
        *out = h;
    });
}

int32_t crx_parse_prefix(const uint8_t *prefix, uint64_t prefix_len, uint64_t total_len, uint8_t last_byte,
                         crx_update **out, uint64_t *need, char *err, uint64_t errlen) {
    *out = nullptr;
    *need = 0;
    try {
        const uint64_t want = prefix_need(prefix, prefix_len, total_len);
        if (want > prefix_len && prefix_len < total_len) {  // ask for more without an exception
            *need = std::min(want, total_len);
            if (err && errlen) std::snprintf(err, (size_t)errlen, "need %llu bytes", (unsigned long long)*need);
            return CRX_INVALID;
        }
        auto *h = new crx_update();
        try {
            parse(prefix, prefix_len, total_len, last_byte, h->u);
        } catch (...) {
            delete h;
            throw;
        }
        h->u.payload_host = nullptr;
        *out = h;
        return CRX_OK;
    } catch (const NeedMore &m) {
        *need = m.need;
        if (err && errlen) std::snprintf(err, (size_t)errlen, "need %llu bytes", (unsigned long long)m.need);
        return CRX_INVALID;
    } catch (const Corrupt &e) {
        if (err && errlen) std::snprintf(err, (size_t)errlen, "%s", e.what());
        return CRX_CORRUPT;
    } catch (const std::bad_alloc &) {
        return CRX_NOMEM;
    } catch (const std::exception &e) {
        if (err && errlen) std::snprintf(err, (size_t)errlen, "%s", e.what());
        return CRX_INVALID;
    }
}

void crx_update_free(crx_update *u) { delete u; }
int64_t crx_update_n_tables(const crx_update *u) { return (int64_t)u->u.tables.size(); }

int32_t crx_update_table(const crx_update *u, int64_t i, int32_t *exponent, int64_t *n_sym, uint32_t *symbols,
                         uint8_t *lengths) {
    if (i < 0 || (size_t)i >= u->u.tables.size()) return CRX_INVALID;
    const Table &t = u->u.tables[i];
    *exponent = t.exponent;
    *n_sym = (int64_t)t.symbols.size();
    if (symbols) std::copy(t.symbols.begin(), t.symbols.end(), symbols);
    if (lengths) std::copy(t.lengths.begin(), t.lengths.end(), lengths);
    return CRX_OK;
}

int64_t crx_update_n_tensors(const crx_update *u) { return (int64_t)u->u.tensors.size(); }

int32_t crx_update_tensor(const crx_update *u, int64_t i, const uint8_t **name, uint64_t *name_len, uint64_t *numel,
                          uint64_t *checksum, int32_t *n_groups) {
    if (i < 0 || (size_t)i >= u->u.tensors.size()) return CRX_INVALID;
    const TensorHeader &t = u->u.tensors[i];
    *name = reinterpret_cast<const uint8_t *>(t.name.data());
    *name_len = t.name.size();
    *numel = t.numel;
    *checksum = t.checksum;
    *n_groups = (int32_t)t.groups.size();
    return CRX_OK;
}

int32_t crx_update_group(const crx_update *u, int64_t i, int32_t g, int32_t *exponent, uint64_t *count, int32_t *rice) {
    if (i < 0 || (size_t)i >= u->u.tensors.size()) return CRX_INVALID;
    const TensorHeader &t = u->u.tensors[i];
    if (g < 0 || (size_t)g >= t.groups.size()) return CRX_INVALID;
    *exponent = t.groups[g].exponent;
    *count = t.groups[g].count;
    *rice = t.groups[g].rice;
    return CRX_OK;
}

int32_t crx_update_headers(const crx_update *u, char *names, uint64_t names_cap, uint64_t *names_len,
                           uint64_t *name_ends, uint64_t *numels, uint64_t *checksums) {
    uint64_t total = 0;
    for (const TensorHeader &t : u->u.tensors) total += t.name.size();
    *names_len = total;
    if (total > names_cap) return CRX_INVALID;
    uint64_t off = 0;
    for (size_t i = 0; i < u->u.tensors.size(); ++i) {
        const TensorHeader &t = u->u.tensors[i];
        std::memcpy(names + off, t.name.data(), t.name.size());
        off += t.name.size();
        name_ends[i] = off;
        numels[i] = t.numel;
        checksums[i] = t.checksum;
    }
    return CRX_OK;
}

uint64_t crx_update_n_blocks(const crx_update *u) { return u->u.n_blocks; }

int32_t crx_update_block_bits(const crx_update *u, uint32_t *out) {
    if (u->u.n_blocks) std::memcpy(out, u->u.block_table, 4 * u->u.n_blocks);
    return CRX_OK;
}

uint64_t crx_update_payload_offset(const crx_update *u) { return u->u.payload_offset; }
uint64_t crx_update_payload_len(const crx_update *u) { return u->u.payload_len; }
uint64_t crx_update_total_changes(const crx_update *u) { return u->u.total_changes; }

int32_t crx_apply(const crx_update *u, const uint8_t *payload_dev, uint16_t *const *targets, const uint64_t *numels,
                  const int32_t *has_cache, const uint64_t *cache_vals, int32_t slab, void *stream, crx_alloc_fn alloc,
                  void *alloc_ctx, uint64_t *changed, char *err, uint64_t errlen) {
    *changed = 0;
    return guarded(err, errlen, [&] {
        if (!payload_dev && u->u.payload_len && !u->u.payload_host) throw Invalid("payload is not on the host");
        Arena ar{alloc, alloc_ctx};
        apply(u->u, payload_dev, targets, numels, has_cache, cache_vals, nullptr, nullptr, slab, (hipStream_t)stream, ar,
              changed);
    });
}

int32_t crx_apply_cached(const crx_update *u, const uint8_t *payload_dev, uint16_t *const *targets,
                         const uint64_t *numels, const int32_t *has_cache, const uint64_t *cache_vals,
                         uint32_t *const *hist_in, uint32_t *const *hist_out, int32_t slab, void *stream,
                         crx_alloc_fn alloc, void *alloc_ctx, uint64_t *changed, char *err, uint64_t errlen) {
    *changed = 0;
    return guarded(err, errlen, [&] {
        if (!payload_dev && u->u.payload_len && !u->u.payload_host) throw Invalid("payload is not on the host");
        Arena ar{alloc, alloc_ctx};
        apply(u->u, payload_dev, targets, numels, has_cache, cache_vals, hist_in, hist_out, slab, (hipStream_t)stream,
              ar, changed);
    });
}

uint64_t crx_apply_hist_words(uint64_t numel, int32_t slab) {
    const uint32_t sl = apply_slab(slab);
    return (numel + sl - 1) / sl * 256;
}

int32_t crx_encode(int32_t n, const uint16_t *const *olds, const uint16_t *const *news, const uint64_t *numels,
                   const int32_t *has_cache, const uint64_t *cache_vals, int32_t slab, void *stream, crx_alloc_fn alloc,
                   void *alloc_ctx, crx_encoded **out, char *err, uint64_t errlen) {
    *out = nullptr;
    return guarded(err, errlen, [&] {
        auto *e = new crx_encoded();
        try {
            Arena ar{alloc, alloc_ctx};
            encode(n, olds, news, numels, has_cache, cache_vals, slab, (hipStream_t)stream, ar, *e);
        } catch (...) {
            delete e;
            throw;
        }
        *out = e;
    });
}

int32_t crx_encoded_present(const crx_encoded *e, int32_t t) { return (t >= 0 && t < e->n) ? e->present[t] : 0; }
uint64_t crx_encoded_checksum(const crx_encoded *e, int32_t t) { return (t >= 0 && t < e->n) ? e->checksum[t] : 0; }
void crx_encoded_checksums(const crx_encoded *e, int32_t *present, uint64_t *checksums) {
    for (int32_t t = 0; t < e->n; ++t) {
        present[t] = e->present[t];
        checksums[t] = e->checksum[t];
    }
}
uint64_t crx_encoded_total_changes(const crx_encoded *e) { return e->total_changes; }

uint64_t crx_encoded_size(const crx_encoded *e, const char *const *names, const uint64_t *name_lens) {
    const std::vector<uint8_t> hdr = header_of(*const_cast<crx_encoded *>(e), names, name_lens);
    std::vector<uint8_t> pl;
    put_varint(pl, e->payload_len);
    return hdr.size() + 4 * e->n_blocks + pl.size() + e->payload_len;
}

int32_t crx_encoded_write(const crx_encoded *e, const char *const *names, const uint64_t *name_lens, uint8_t *dst,
                          int32_t dst_on_device, void *stream, char *err, uint64_t errlen) {
    return guarded(err, errlen, [&] {
        hipStream_t s = (hipStream_t)stream;
        const std::vector<uint8_t> hdr = header_of(*const_cast<crx_encoded *>(e), names, name_lens);
        std::vector<uint8_t> pl;
        put_varint(pl, e->payload_len);
        const hipMemcpyKind from_dev = dst_on_device ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost;
        const uint64_t off_bt = hdr.size(), off_pl = off_bt + 4 * e->n_blocks, off_pay = off_pl + pl.size();
        if (dst_on_device) {
            // the host bytes go through the pinned arena: every copy is left ordered on the stream
            h2d(dst, hdr.data(), hdr.size(), s);
            h2d(dst + off_pl, pl.data(), pl.size(), s);
        } else {
            std::memcpy(dst, hdr.data(), hdr.size());
            std::memcpy(dst + off_pl, pl.data(), pl.size());
        }
        if (dst_on_device) {
            if (e->n_blocks) HIP_OK(hipMemcpyAsync(dst + off_bt, e->d_block_bits, 4 * e->n_blocks, from_dev, s));
            if (e->payload_len) HIP_OK(hipMemcpyAsync(dst + off_pay, e->d_payload, e->payload_len, from_dev, s));
        } else {
            HIP_OK(hipStreamSynchronize(s));  // the encode's work, before the staged copies below
            copy_to_host(dst + off_bt, reinterpret_cast<const uint8_t *>(e->d_block_bits), 4 * e->n_blocks, s);
            copy_to_host(dst + off_pay, e->d_payload, e->payload_len, s);
        }
    });
}

int64_t crx_encoded_n_tables(const crx_encoded *e) { return (int64_t)e->tables.size(); }

int32_t crx_encoded_table(const crx_encoded *e, int64_t i, int32_t *exponent, int64_t *n_sym, uint32_t *symbols,
                          uint8_t *lengths) {
    if (i < 0 || (size_t)i >= e->tables.size()) return CRX_INVALID;
    const Table &t = e->tables[i];
    *exponent = t.exponent;
    *n_sym = (int64_t)t.symbols.size();
    if (symbols) std::copy(t.symbols.begin(), t.symbols.end(), symbols);
    if (lengths) std::copy(t.lengths.begin(), t.lengths.end(), lengths);
    return CRX_OK;
}

int32_t crx_encoded_n_groups(const crx_encoded *e, int32_t t) {
    return (t >= 0 && t < e->n) ? (int32_t)e->groups[t].size() : 0;
}

int32_t crx_encoded_group(const crx_encoded *e, int32_t t, int32_t g, int32_t *exponent, uint64_t *count, int32_t *rice) {
    if (t < 0 || t >= e->n || g < 0 || (size_t)g >= e->groups[t].size()) return CRX_INVALID;
    *exponent = e->groups[t][g].exponent;
    *count = e->groups[t][g].count;
    *rice = e->groups[t][g].rice;
    return CRX_OK;
}

uint64_t crx_encoded_n_blocks(const crx_encoded *e) { return e->n_blocks; }

int32_t crx_encoded_block_bits(const crx_encoded *e, uint32_t *out, void *stream) {
    return guarded(nullptr, 0, [&] {
        if (e->n_blocks)
            HIP_OK(hipMemcpyAsync(out, e->d_block_bits, 4 * e->n_blocks, hipMemcpyDeviceToHost, (hipStream_t)stream));
        HIP_OK(hipStreamSynchronize((hipStream_t)stream));
    });
}

uint64_t crx_encoded_payload_len(const crx_encoded *e) { return e->payload_len; }

int32_t crx_encoded_payload(const crx_encoded *e, uint8_t *out, void *stream) {
    return guarded(nullptr, 0, [&] {
        if (e->payload_len)
            HIP_OK(hipMemcpyAsync(out, e->d_payload, e->payload_len, hipMemcpyDeviceToHost, (hipStream_t)stream));
        HIP_OK(hipStreamSynchronize((hipStream_t)stream));
    });
}

void crx_encoded_free(crx_encoded *e) { delete e; }

int32_t crx_checksum(const uint16_t *data, uint64_t n, void *stream, crx_alloc_fn alloc, void *alloc_ctx, uint64_t *out,
                     char *err, uint64_t errlen) {
    *out = 0;
    return guarded(err, errlen, [&] {
        Arena ar{alloc, alloc_ctx};
        full_checksum(data, n, (hipStream_t)stream, ar, out);
    });
}

int32_t crx_checksum_noalloc(const uint16_t *data, uint64_t n, void *stream, uint64_t *out, char *err,
                             uint64_t errlen) {
    // no exceptions, containers or pinned staging here: nothing on this path allocates
    *out = 0;
    auto fail = [&](int32_t rc, const char *m) {
        if (err && errlen) std::snprintf(err, (size_t)errlen, "%s", m);
        return rc;
    };
    if (!n) return CRX_OK;
    if (reinterpret_cast<uintptr_t>(data) & 1) return fail(CRX_INVALID, "tensor data must be 2-byte aligned");
    if (n >= (1ULL << 32)) return fail(CRX_INVALID, "crx_checksum_noalloc takes at most 2^32 - 1 elements");
    const uint32_t *frame = reinterpret_cast<const uint32_t *>(reinterpret_cast<uintptr_t>(data) & ~uintptr_t(3));
    const uint32_t lead = (uint32_t)((reinterpret_cast<uintptr_t>(data) & 3) >> 1);
    const hipError_t e = checksum_noalloc(frame, lead, n, (hipStream_t)stream, out);
    if (e != hipSuccess) return fail(CRX_DEVICE, hipGetErrorString(e));
    return CRX_OK;
}

int32_t crx_huffman_lengths(const uint64_t *counts, int64_t n, int32_t *lengths) {
    if (n <= 0) return CRX_INVALID;
    try {
        std::vector<int> L = huffman_lengths(std::vector<uint64_t>(counts, counts + n));
        std::copy(L.begin(), L.end(), lengths);
        return CRX_OK;
    } catch (const std::bad_alloc &) {
        return CRX_NOMEM;
    }
}

int32_t crx_canonical_codes(const int32_t *lengths, int64_t n, uint32_t *codes) {
    if (n <= 0) return CRX_INVALID;
    try {
        std::vector<uint32_t> c = canonical_codes(std::vector<int>(lengths, lengths + n));
        std::copy(c.begin(), c.end(), codes);
        return CRX_OK;
    } catch (const std::bad_alloc &) {
        return CRX_NOMEM;
    }
}

void crx_rice_candidates(uint64_t count, uint64_t gap_sum, int32_t cand[3]) {
    int c[3];
    rice_candidates(count, gap_sum, c);
    for (int k = 0; k < 3; ++k) cand[k] = c[k];
}

int32_t crx_rice_choose(uint64_t count, const int32_t cand[3], const uint64_t shifted[3]) {
    const int c[3] = {cand[0], cand[1], cand[2]};
    return rice_choose(count, c, shifted);
}

void crx_timing_enable(int32_t on) { g_timing = on != 0; }

void crx_timing_only(const char *names) {
    std::lock_guard<std::mutex> lk(g_tmu);
    g_only.clear();
    if (!names) return;
    std::string cur;
    for (const char *c = names;; ++c) {
        if (*c == ',' || *c == 0) {
            if (!cur.empty()) g_only.push_back(cur);
            cur.clear();
            if (!*c) break;
        } else {
            cur += *c;
        }
    }
}

void crx_timing_reset(void) {
    timing_collect(true);
    std::lock_guard<std::mutex> lk(g_tmu);
    g_stats.clear();
}

int32_t crx_timing_read(char *buf, uint64_t len) {
    timing_collect(true);
    std::lock_guard<std::mutex> lk(g_tmu);
    std::string out;
    char line[256];
    for (const auto &kv : g_stats) {
        std::snprintf(line, sizeof line, "%s %lld %.6f\n", kv.first.c_str(), (long long)kv.second.calls, kv.second.ms);
        out += line;
    }
    if (buf && len) std::snprintf(buf, (size_t)len, "%s", out.c_str());
    return (int32_t)out.size();
}

}  // extern "C"
