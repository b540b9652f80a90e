// The wave64 emulator and host runtime behind tests/model/hip/hip_runtime.h: the library's kernels,
// compiled as plain C++, run on the CPU with every memory access checked by AddressSanitizer.
//
// A launch runs its workgroups one after another.  Each work-item of a workgroup is a fiber with its
// own stack; fibers run one at a time, in work-item order, until they reach a collective of their
// wavefront (ballot, lane read, shuffle, fence) or a workgroup barrier.  When every fiber waits, a
// wavefront whose live lanes (those that have not returned) all wait on a collective is resolved: the
// lanes must have reached the same call site the same number of times and asked for the same thing,
// otherwise the model stops and reports the divergence.  Lanes that returned take no part, as inactive
// lanes take no part on the GPU; a lane read or shuffle from a lane that returned is reported too.
// Between two collectives a lane's reads see the writes of the lanes that ran before it, so every
// place where the kernels read what other lanes wrote must be a collective (the kernels mark those with
// wave_fence); a missing one shows as a wrong result.
#include <hip/hip_runtime.h>
#include <sanitizer/asan_interface.h>
#include <sanitizer/common_interface_defs.h>
#include <pthread.h>
#include <sys/mman.h>
#include <unistd.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <memory>
#include <vector>

extern "C" void simt_switch(void **save_sp, void *load_sp);
// x86-64 System V: saves the callee-saved registers and the stack pointer of the running context in
// *save_sp, then resumes the context whose stack pointer is load_sp.
asm(R"(
    .text
    .globl simt_switch
    .type simt_switch,@function
simt_switch:
    pushq %rbp
    pushq %rbx
    pushq %r12
    pushq %r13
    pushq %r14
    pushq %r15
    movq %rsp, (%rdi)
    movq %rsi, %rsp
    popq %r15
    popq %r14
    popq %r13
    popq %r12
    popq %rbx
    popq %rbp
    ret
    .size simt_switch, .-simt_switch
)");

namespace crx {
extern bool g_arena_unpooled;
}

// the LDS variables of the library's kernels (the section of the stand-in's __shared__)
extern "C" uint8_t __start_simt_lds[], __stop_simt_lds[];

namespace simt {
namespace {

enum State { kRunnable, kWaitWave, kWaitBlock, kDone };

struct Fiber {
    void *sp = nullptr;
    uint8_t *stack = nullptr;  // usable stack [stack, stack + size), a guard page below
    size_t size = 0;
    void *fake = nullptr;
    uint32_t tid = 0;
    State st = kDone;
    uint64_t seq = 0, bseq = 0;  // wave collectives and workgroup barriers passed
    const void *site = nullptr;
    Op op = kSync;
    uint64_t val = 0, res = 0;
    uint32_t arg = 0;
};

constexpr size_t kStackBytes = 128 << 10;
Fiber g_pool[1024];  // the work-items of the running workgroup
uint32_t g_n = 0;
Fiber *g_cur = nullptr;
void *g_sched_sp = nullptr, *g_sched_fake = nullptr;
const void *g_main_bottom = nullptr;
size_t g_main_size = 0;
Idx g_block{0, 0, 0}, g_grid{1, 1, 1}, g_bdim{1, 1, 1};
void (*g_body)(void *) = nullptr;
void *g_ctx = nullptr;
uint8_t *g_dyn = nullptr;
uint64_t g_launches = 0;
uint64_t g_resolves = 0, g_switches = 0;
const int g_stack_fill = std::getenv("SIMT_STACK_FILL") ? (int)std::strtol(std::getenv("SIMT_STACK_FILL"), nullptr, 0) : -1;
constexpr size_t kStackFill = 32 << 10;
const int g_lds_fill = std::getenv("SIMT_LDS_FILL") ? (int)std::strtol(std::getenv("SIMT_LDS_FILL"), nullptr, 0) : 0xA5;

[[noreturn]] void fail(const char *what) {
    std::fprintf(stderr, "simt: %s (launch %llu, workgroup %u)\n", what, (unsigned long long)g_launches, g_block.x);
    for (uint32_t t = 0; t < g_n; ++t) {
        const Fiber &f = g_pool[t];
        std::fprintf(stderr, "  item %3u state %d op %d seq %llu bseq %llu site %p arg %u\n", t, (int)f.st, (int)f.op,
                     (unsigned long long)f.seq, (unsigned long long)f.bseq, f.site, f.arg);
    }
    std::fflush(stderr);
    std::abort();
}

// Switches from the running fiber to `to` (the scheduler's context when null); returns when some
// context switches back to `from`.
void switch_to(Fiber *from, Fiber *to) {
    ++g_switches;
    g_cur = to;
    if (to) {
        __sanitizer_start_switch_fiber(from ? &from->fake : &g_sched_fake, to->stack, to->size);
    } else {
        __sanitizer_start_switch_fiber(&from->fake, g_main_bottom, g_main_size);
    }
    simt_switch(from ? &from->sp : &g_sched_sp, to ? to->sp : g_sched_sp);
    __sanitizer_finish_switch_fiber(from ? from->fake : g_sched_fake, nullptr, nullptr);
}

void resolve(uint32_t w);

// The context to run once the running work-item f has stopped (it waits, or it has returned): the
// next runnable work-item after it; else, once a wavefront's live lanes all wait on a collective, that
// collective is resolved and its lowest lane runs; else the scheduler (workgroup barrier, end).
Fiber *next_after(const Fiber *f) {
    for (uint32_t t = f->tid + 1; t < g_n; ++t)
        if (g_pool[t].st == kRunnable) return &g_pool[t];
    for (uint32_t w = 0; 64 * w < g_n; ++w) {
        bool any = false, all_wave = true;
        const uint32_t hi = std::min<uint32_t>(64 * w + 64, g_n);
        for (uint32_t t = 64 * w; t < hi; ++t) {
            const State st = g_pool[t].st;
            if (st == kDone) continue;
            any = true;
            if (st != kWaitWave) {
                all_wave = false;
                break;
            }
        }
        if (any && all_wave) resolve(w);
    }
    for (uint32_t t = 0; t < g_n; ++t)
        if (g_pool[t].st == kRunnable) return &g_pool[t];
    return nullptr;
}

[[noreturn]] void fiber_main() {
    Fiber *f = g_cur;
    __sanitizer_finish_switch_fiber(nullptr, nullptr, nullptr);
    g_body(g_ctx);
    f->st = kDone;
    Fiber *to = next_after(f);
    g_cur = to;
    __sanitizer_start_switch_fiber(nullptr, to ? to->stack : g_main_bottom, to ? to->size : g_main_size);
    simt_switch(&f->sp, to ? to->sp : g_sched_sp);
    __builtin_trap();
}

void prepare(Fiber &f, uint32_t tid) {
    if (!f.stack) {
        const size_t page = (size_t)sysconf(_SC_PAGESIZE);
        void *m = mmap(nullptr, kStackBytes + page, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
        if (m == MAP_FAILED) fail("no memory for a fiber stack");
        mprotect(m, page, PROT_NONE);  // an overflow faults instead of writing past the stack
        f.stack = static_cast<uint8_t *>(m) + page;
        f.size = kStackBytes;
        __asan_unpoison_memory_region(f.stack, f.size);
    }
    // (a work-item that returned left its stack as it found it: every frame it entered was left)
    uintptr_t top = ((uintptr_t)f.stack + f.size) & ~uintptr_t(15);
    // private variables start as what the previous work-item left, as registers do on the GPU;
    // SIMT_STACK_FILL fills the top of the stack with a byte instead
    if (g_stack_fill >= 0) std::memset(reinterpret_cast<void *>(top - kStackFill), g_stack_fill, kStackFill);
    void **sp = reinterpret_cast<void **>(top);
    *--sp = nullptr;                                    // fiber_main's return address (never used)
    *--sp = reinterpret_cast<void *>(&fiber_main);      // where simt_switch's ret goes
    for (int i = 0; i < 6; ++i) *--sp = nullptr;        // rbp rbx r12 r13 r14 r15
    f.sp = sp;
    f.fake = nullptr;
    f.tid = tid;
    f.st = kRunnable;
    f.seq = f.bseq = 0;
    f.site = nullptr;
}

// The running work-item stops (its state is set): the next context runs.
void stop() {
    Fiber *f = g_cur;
    Fiber *to = next_after(f);
    if (to == f) return;  // it was the last of its wavefront to arrive, and runs first
    switch_to(f, to);
}

// The live lanes of wavefront w all wait on a collective: check they agree, compute every result.
void resolve(uint32_t w) {
    ++g_resolves;
    const uint32_t lo = 64 * w, hi = std::min<uint32_t>(lo + 64, g_n);
    Fiber *lane[64] = {};
    uint64_t live = 0;
    Fiber *first = nullptr;
    for (uint32_t t = lo; t < hi; ++t) {
        Fiber *f = &g_pool[t];
        if (f->st == kDone) continue;
        lane[t - lo] = f;
        live |= 1ULL << (t - lo);
        if (!first) first = f;
    }
    const Op op = first->op;
    uint64_t ballot = 0;
    for (uint32_t l = 0; l < 64; ++l) {
        Fiber *f = lane[l];
        if (!f) continue;
        if (f->site != first->site || f->seq != first->seq || f->op != op)
            fail("lanes of a wavefront reached different collectives (divergence)");
        if (op == kReadlane && f->arg != first->arg) fail("readlane with a lane index that is not uniform");
        ballot |= (f->val & 1) << l;
    }
    for (uint32_t l = 0; l < 64; ++l) {
        Fiber *f = lane[l];
        if (!f) continue;
        uint32_t src = l;
        switch (op) {
        case kSync: f->res = 0; break;
        case kBallot: f->res = ballot; break;
        case kReadlane: src = f->arg & 63; break;
        case kReadfirst: src = (uint32_t)__builtin_ctzll(live); break;
        case kShflIdx: src = f->arg & 63; break;
        case kShflUp: src = l >= f->arg ? l - f->arg : l; break;
        case kShflXor: src = (l ^ f->arg) & 63; break;
        }
        if (op >= kReadlane) {
            if (!((live >> src) & 1)) fail("a lane read or shuffle from a lane that has returned");
            f->res = lane[src]->val;
        }
    }
    for (uint32_t l = 0; l < 64; ++l)
        if (lane[l]) {
            lane[l]->st = kRunnable;
            lane[l]->seq++;
        }
}

// Runs the workgroup's work-items to their end: the scheduler's context is entered only when no
// work-item can run and no collective can be resolved.
void schedule() {
    for (;;) {
        Fiber *to = nullptr;
        for (uint32_t t = 0; t < g_n && !to; ++t)
            if (g_pool[t].st == kRunnable) to = &g_pool[t];
        if (to) {
            switch_to(nullptr, to);
            continue;
        }
        bool done = true;
        const Fiber *first = nullptr;
        for (uint32_t t = 0; t < g_n; ++t) {
            const Fiber *f = &g_pool[t];
            if (f->st == kDone) continue;
            done = false;
            if (f->st != kWaitBlock) fail("work-items wait on different things (deadlock)");
            if (!first) first = f;
            if (f->site != first->site || f->bseq != first->bseq) fail("a workgroup barrier reached from different places");
        }
        if (done) return;
        for (uint32_t t = 0; t < g_n; ++t) {
            Fiber *f = &g_pool[t];
            if (f->st == kWaitBlock) {
                f->st = kRunnable;
                f->bseq++;
            }
        }
    }
}

}  // namespace

Idx thread_idx() { return Idx{g_cur->tid, 0, 0}; }
Idx block_idx() { return g_block; }
Idx grid_dim() { return g_grid; }
Idx block_dim() { return g_bdim; }
uint32_t lane_id() { return g_cur->tid & 63u; }
void *dynamic_lds() { return g_dyn; }

uint64_t collective(Op op, uint64_t value, uint32_t arg, const void *site) {
    Fiber *f = g_cur;
    f->op = op;
    f->val = value;
    f->arg = arg;
    f->site = site;
    f->st = kWaitWave;
    stop();
    return f->res;
}

void block_barrier(const void *site) {
    Fiber *f = g_cur;
    f->site = site;
    f->st = kWaitBlock;
    stop();
}

void run(dim3 grid, dim3 block, size_t dyn_bytes, void (*body)(void *), void *ctx) {
    if (g_cur) fail("a launch from inside a kernel");
    if (grid.y != 1 || grid.z != 1 || block.y != 1 || block.z != 1 || block.x == 0 || block.x > 1024)
        fail("only one-dimensional launches of 1 to 1024 work-items are modelled");
    ++g_launches;
    static thread_local const void *t_bottom = nullptr;
    static thread_local size_t t_size = 0;
    if (!t_bottom) {  // the calling thread's stack, where the scheduler runs
        pthread_attr_t at;
        void *lo = nullptr;
        if (pthread_getattr_np(pthread_self(), &at) == 0) {
            pthread_attr_getstack(&at, &lo, &t_size);
            pthread_attr_destroy(&at);
        }
        t_bottom = lo;
    }
    g_main_bottom = t_bottom;
    g_main_size = t_size;
    g_n = block.x;
    g_grid = Idx{grid.x, 1, 1};
    g_bdim = Idx{block.x, 1, 1};
    g_body = body;
    g_ctx = ctx;
    // the dynamic LDS of the launch, exactly as large as asked (and never zeroed, as on the GPU)
    std::unique_ptr<uint8_t[]> dyn(new uint8_t[dyn_bytes ? dyn_bytes : 1]);
    std::memset(dyn.get(), 0xA5, dyn_bytes ? dyn_bytes : 1);
    g_dyn = dyn_bytes ? dyn.get() : nullptr;
    static const bool profile = std::getenv("SIMT_PROFILE") != nullptr;
    const auto t0 = std::chrono::steady_clock::now();
    const uint64_t r0 = g_resolves, s0 = g_switches;
    for (uint32_t b = 0; b < grid.x; ++b) {
        g_block = Idx{b, 0, 0};
        // what a workgroup finds in LDS: not what an earlier one left (SIMT_LDS_FILL: the byte)
        std::memset(__start_simt_lds, g_lds_fill, (size_t)(__stop_simt_lds - __start_simt_lds));
        if (dyn_bytes) std::memset(g_dyn, g_lds_fill, dyn_bytes);
        for (uint32_t t = 0; t < g_n; ++t) prepare(g_pool[t], t);
        schedule();
    }
    g_dyn = nullptr;
    if (profile)
        std::fprintf(stderr, "simt: launch %llu body %p grid %u block %u: %llu collectives, %llu switches: %.1f ms\n",
                     (unsigned long long)g_launches, (void *)body, grid.x, block.x,
                     (unsigned long long)(g_resolves - r0), (unsigned long long)(g_switches - s0),
                     std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count());
}

}  // namespace simt

// ------------------------------------------------------------------ host runtime
struct simt_stream {
    int unused;
};
struct simt_event {
    int unused;
};

hipError_t hipGetDevice(int *dev) {
    *dev = 0;
    return hipSuccess;
}
hipError_t hipStreamCreateWithFlags(hipStream_t *s, unsigned) {
    *s = new simt_stream{0};
    return hipSuccess;
}
hipError_t hipEventCreate(hipEvent_t *e) {
    *e = new simt_event{0};
    return hipSuccess;
}
hipError_t hipEventCreateWithFlags(hipEvent_t *e, unsigned) { return hipEventCreate(e); }
hipError_t hipEventDestroy(hipEvent_t e) {
    delete e;
    return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t, hipStream_t) { return hipSuccess; }
hipError_t hipEventQuery(hipEvent_t) { return hipSuccess; }
hipError_t hipEventSynchronize(hipEvent_t) { return hipSuccess; }
hipError_t hipEventElapsedTime(float *ms, hipEvent_t, hipEvent_t) {
    *ms = 0.0f;
    return hipSuccess;
}
hipError_t hipStreamWaitEvent(hipStream_t, hipEvent_t, unsigned) { return hipSuccess; }
hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
hipError_t hipHostMalloc(void **p, size_t bytes, unsigned) {
    return posix_memalign(p, 64, bytes ? bytes : 1) == 0 ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t hipHostFree(void *p) {
    free(p);
    return hipSuccess;
}
hipError_t hipMemcpyAsync(void *dst, const void *src, size_t bytes, hipMemcpyKind, hipStream_t) {
    if (bytes) std::memcpy(dst, src, bytes);
    return hipSuccess;
}
hipError_t hipMemsetAsync(void *dst, int value, size_t bytes, hipStream_t) {
    if (bytes) std::memset(dst, value, bytes);
    return hipSuccess;
}
hipError_t hipGetLastError() { return hipSuccess; }
hipError_t hipGetSymbolAddress(void **p, const void *symbol) {
    *p = const_cast<void *>(symbol);
    return hipSuccess;
}
const char *hipGetErrorString(hipError_t) { return "error of the emulated HIP runtime"; }

// Every device buffer of a call is an allocation of its own, so that AddressSanitizer knows its bounds.
static struct ModelInit {
    ModelInit() { crx::g_arena_unpooled = true; }
} g_model_init;
