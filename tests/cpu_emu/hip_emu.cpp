// hip_emu.cpp -- CPU emulation of the HIP features the forge-sort kernels and
// host runtime use (TEST INFRASTRUCTURE ONLY; see hip/hip_runtime.h).
//
// Execution model:
//  * a launch runs its blocks on a pool of OS threads, several blocks resident
//    at once so that the look-back between tiles is a real cross-thread race.
//    As on the device, blocks are dealt round-robin to EMU_XCDS queues (default
//    8, block b to queue b % EMU_XCDS) and every queue starts its blocks in
//    increasing order; EMU_WORKERS threads (default 8, rounded up to a
//    multiple of the queues) serve the queues;
//  * inside a block every GPU thread is a ucontext fiber, scheduled round-robin;
//  * __syncthreads waits for every live thread of the block;
//  * a wave64 operation completes once no lane of the wave is still runnable:
//    the lanes waiting at it are the active lanes, lanes that diverged to a
//    barrier or finished are inactive (the SIMT meaning of EXEC);
//  * s_sleep yields; a block whose runnable threads all sleep yields its OS thread;
//  * device allocations end on a PROT_NONE guard page (and start after one), so
//    an out-of-bounds access becomes SIGSEGV, reported with the faulting
//    kernel, block and thread.
#include <hip/hip_runtime.h>
#include <sched.h>
#include <signal.h>
#include <stdio.h>
#include <stdlib.h>
#include <sys/mman.h>
#include <time.h>
#include <ucontext.h>
#include <execinfo.h>
#include <unistd.h>

#include <atomic>
#include <chrono>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "fs_params.h"

namespace emu {

enum State { RUNNABLE, AT_BARRIER, AT_WAVEOP, DONE };
enum WaveKind { WK_BALLOT, WK_ALL, WK_SHFL_UP, WK_FIRSTLANE, WK_BARRIER, WK_READLANE };

struct Fiber {
    ucontext_t ctx;
    char* stack = nullptr;
    State state = RUNNABLE;
    bool sleeping = false;
    int pred = 0;
    int wkind = 0;
    uint64_t wval = 0, warg = 0, wres = 0;
};

static size_t stack_bytes() {
    const char* e = getenv("EMU_STACK_KB");
    return (size_t)(e ? atoi(e) : 1024) * 1024;
}

struct Block {
    uint64_t magic = 0xB10C0B10C0ull;
    int nthreads = 0;
    std::vector<Fiber> f;
    ucontext_t sched;
    int cur = -1;
    emu_dim3 bidx{}, bdim{}, gdim{};
    void (*entry)(void**) = nullptr;
    void** params = nullptr;
    int barrier_result = 0;
};

thread_local Block* B = nullptr;
static const char* g_kernel = "";

emu_dim3 thread_idx() { return emu_dim3{(uint32_t)B->cur, 0, 0}; }
emu_dim3 block_idx() { return B->bidx; }
emu_dim3 block_dim() { return B->bdim; }
emu_dim3 grid_dim() { return B->gdim; }
unsigned lane() { return (unsigned)B->cur & 63u; }

[[noreturn]] static void die(const char* why);

static void check_block() {
    if (!B || B->magic != 0xB10C0B10C0ull || B->cur < 0 || B->cur >= B->nthreads) die("emulator state corrupted");
}

static void yield_to_sched() {
    check_block();
    swapcontext(&B->f[B->cur].ctx, &B->sched);
    check_block();
}

void syncthreads() {
    check_block();
    Fiber& me = B->f[B->cur];
    me.state = AT_BARRIER;
    me.pred = 0;
    yield_to_sched();
}

int syncthreads_or(int p) {
    Fiber& me = B->f[B->cur];
    me.state = AT_BARRIER;
    me.pred = p != 0;
    yield_to_sched();
    return B->barrier_result;
}

static uint64_t wave_op(int kind, uint64_t val, uint64_t arg) {
    Fiber& me = B->f[B->cur];
    me.state = AT_WAVEOP;
    me.wkind = kind;
    me.wval = val;
    me.warg = arg;
    yield_to_sched();
    return me.wres;
}

uint64_t ballot(int p) { return wave_op(WK_BALLOT, p != 0, 0); }
int all(int p) { return (int)wave_op(WK_ALL, p != 0, 0); }
uint32_t shfl_up(uint32_t v, unsigned off) { return (uint32_t)wave_op(WK_SHFL_UP, v, off); }
uint32_t readfirstlane(uint32_t v) { return (uint32_t)wave_op(WK_FIRSTLANE, v, 0); }
uint32_t readlane(uint32_t v, uint32_t src) { return (uint32_t)wave_op(WK_READLANE, v, src); }
// Lockstep point: lanes of a wave run one after another between wave
// operations here, while on the GPU they execute each instruction together;
// the kernels mark the places where that matters with a wave barrier.
void wave_barrier() { (void)wave_op(WK_BARRIER, 0, 0); }

void sleep_hint() {
    Fiber& me = B->f[B->cur];
    me.sleeping = true;
    yield_to_sched();
}

static void fiber_main() {
    B->entry(B->params);
    B->f[B->cur].state = DONE;
    swapcontext(&B->f[B->cur].ctx, &B->sched);
}

[[noreturn]] static void die(const char* why) {
    fprintf(stderr, "hip_emu: %s (kernel %s, B=%p)\n", why, g_kernel, (void*)B);
    fflush(stderr);
    abort();
}

static bool resolve_wave(int w) {
    Block& b = *B;
    const int lo = w * 64, hi = std::min(b.nthreads, lo + 64);
    int waiting = 0, kind = -1;
    for (int i = lo; i < hi; ++i) {
        if (b.f[i].state == RUNNABLE) return false;     // a lane may still arrive
        if (b.f[i].state == AT_WAVEOP) {
            if (kind >= 0 && kind != b.f[i].wkind) die("divergent wave operations in one wave");
            kind = b.f[i].wkind;
            ++waiting;
        }
    }
    if (!waiting) return false;
    uint64_t mask = 0;
    int first = -1;
    bool allp = true;
    for (int i = lo; i < hi; ++i)
        if (b.f[i].state == AT_WAVEOP) {
            if (first < 0) first = i;
            if (b.f[i].wval) mask |= 1ull << (i - lo);
            allp = allp && b.f[i].wval;
        }
    for (int i = lo; i < hi; ++i) {
        Fiber& f = b.f[i];
        if (f.state != AT_WAVEOP) continue;
        switch (kind) {
            case WK_BALLOT: f.wres = mask; break;
            case WK_ALL: f.wres = allp; break;
            case WK_FIRSTLANE: f.wres = b.f[first].wval; break;
            case WK_BARRIER: f.wres = 0; break;
            case WK_READLANE: {
                // the source lane must take part (the kernels only read lanes they know are active)
                const int src = lo + (int)(f.warg & 63u);
                if (src >= hi || b.f[src].state != AT_WAVEOP) die("readlane of a lane outside the operation");
                f.wres = b.f[src].wval;
                break;
            }
            case WK_SHFL_UP: {
                const int src = (i - lo) - (int)f.warg;
                f.wres = (src >= 0 && b.f[lo + src].state == AT_WAVEOP) ? b.f[lo + src].wval : f.wval;
                break;
            }
        }
    }
    for (int i = lo; i < hi; ++i)
        if (b.f[i].state == AT_WAVEOP) b.f[i].state = RUNNABLE;
    return true;
}

static void run_block(uint32_t bid, uint32_t grid, uint32_t nthreads, void (*entry)(void**), void** params) {
    Block b;
    b.nthreads = (int)nthreads;
    b.f.resize(nthreads);
    b.bidx = {bid, 0, 0};
    b.bdim = {nthreads, 1, 1};
    b.gdim = {grid, 1, 1};
    b.entry = entry;
    b.params = params;
    B = &b;
    for (uint32_t i = 0; i < nthreads; ++i) {
        Fiber& f = b.f[i];
        f.stack = (char*)malloc(stack_bytes());
        getcontext(&f.ctx);
        f.ctx.uc_stack.ss_sp = f.stack;
        f.ctx.uc_stack.ss_size = stack_bytes();
        f.ctx.uc_link = nullptr;
        makecontext(&f.ctx, fiber_main, 0);
    }
    // EMU_SCHED=wave / wave_rev: waves one at a time (in increasing or
    // decreasing order), each run - its wave operations resolved at once -
    // until every lane waits at a block barrier, has finished or spins; a wave
    // then gets ahead of the others as far as the barriers allow, which shows
    // a missing barrier between the waves' LDS accesses as a wrong result.
    // Default: every runnable thread once per round, wave operations resolved
    // after the round.
    static const int sched_mode = [] {
        const char* e = getenv("EMU_SCHED");
        return !e ? 0 : strcmp(e, "wave") == 0 ? 1 : strcmp(e, "wave_rev") == 0 ? 2 : 0;
    }();
    const int nwaves = (b.nthreads + 63) / 64;
    for (;;) {
        bool ran = false, awake = false;
        bool resolved = false;
        if (sched_mode == 0) {
            for (int i = 0; i < b.nthreads; ++i) {
                if (b.f[i].state != RUNNABLE) continue;
                if (!b.f[i].sleeping) awake = true;
                b.f[i].sleeping = false;
                b.cur = i;
                swapcontext(&b.sched, &b.f[i].ctx);
                ran = true;
            }
            b.cur = -1;
            for (int w = 0; w < nwaves; ++w) resolved |= resolve_wave(w);
        } else {
            for (int k = 0; k < nwaves; ++k) {
                const int w = sched_mode == 1 ? k : nwaves - 1 - k;
                const int lo = w * 64, hi = std::min(b.nthreads, lo + 64);
                for (;;) {                               // this wave until it blocks or only spins
                    bool wran = false, wawake = false;
                    for (int i = lo; i < hi; ++i) {
                        if (b.f[i].state != RUNNABLE) continue;
                        if (!b.f[i].sleeping) wawake = true;
                        b.f[i].sleeping = false;
                        b.cur = i;
                        swapcontext(&b.sched, &b.f[i].ctx);
                        wran = true;
                    }
                    b.cur = -1;
                    const bool wres = resolve_wave(w);
                    ran |= wran;
                    awake |= wawake;
                    resolved |= wres;
                    if (!wres && (!wran || !wawake)) break;
                }
            }
        }
        int live = 0, at_bar = 0, orv = 0;
        for (auto& f : b.f) {
            if (f.state == DONE) continue;
            ++live;
            if (f.state == AT_BARRIER) { ++at_bar; orv |= f.pred; }
        }
        if (live == 0) break;
        if (at_bar == live) {
            b.barrier_result = orv;
            for (auto& f : b.f)
                if (f.state == AT_BARRIER) f.state = RUNNABLE;
            resolved = true;
        }
        if (!ran && !resolved) die("deadlock: every live thread waits and nothing can resolve");
        if (ran && !awake && !resolved) sched_yield();   // the whole block is spin-waiting
    }
    for (auto& f : b.f) free(f.stack);
    B = nullptr;
}

static int xcds() {
    const char* e = getenv("EMU_XCDS");
    int x = e ? atoi(e) : 8;
    return x > 0 ? x : 1;
}

static int workers() {
    const char* e = getenv("EMU_WORKERS");
    int w = e ? atoi(e) : 8;
    const int x = xcds();
    if (w < x) w = x;
    return (w + x - 1) / x * x;
}

void launch(const char* name, void (*entry)(void**), uint32_t grid, uint32_t block, void** params) {
    g_kernel = name;
    if (getenv("EMU_TRACE")) fprintf(stderr, "hip_emu: launch %s grid=%u block=%u\n", name, grid, block);
    const int nx = xcds();
    int hold_queue = -1, hold_ms = 0;
    bool hold_until_timeout = false;
    static std::atomic<bool> held{false};
    if (const char* h = getenv("EMU_HOLD_QUEUE"))
        if (strncmp(name, "fs_onesweep", 11) == 0 && !held.exchange(true)) {
            char until[16] = {0};
            if (sscanf(h, "%d:%15s", &hold_queue, until) == 2 && strcmp(until, "timeout") == 0) hold_until_timeout = true;
            else if (sscanf(h, "%d:%d", &hold_queue, &hold_ms) != 2) hold_ms = 0;
        }
    std::vector<std::atomic<uint32_t>> next(nx);           // per-queue position
    for (auto& c : next) c = 0;
    auto worker = [&](int queue) {
        if (!getenv("EMU_NO_SEGV_HANDLER")) {
            stack_t ss;                   // the signal handler's stack; kept for the process
            ss.ss_size = 1 << 16;
            ss.ss_sp = malloc(ss.ss_size);
            ss.ss_flags = 0;
            sigaltstack(&ss, nullptr);
        }
        // EMU_HOLD_QUEUE=q:ms holds queue q of the first digit-pass launch of
        // the process back for ms milliseconds, as if another stream's work
        // occupied that XCD; q:timeout holds it until a look-back wait of the
        // launch has ended at its spin bound (the status word says so), so
        // that the outcome does not depend on timing
        if (hold_ms > 0 && queue == hold_queue) std::this_thread::sleep_for(std::chrono::milliseconds(hold_ms));
        if (hold_until_timeout && queue == hold_queue) {
            const volatile uint32_t* status = (const volatile uint32_t*)(uintptr_t)(*(FsArgs*)params[0]).status;
            for (int ms = 0; !(*status & FS_DEVERR_LOOKBACK_TIMEOUT); ++ms) {
                if (ms > 600000) {
                    fprintf(stderr, "hip_emu: held queue %d: no look-back timeout within 600 s\n", queue);
                    abort();
                }
                std::this_thread::sleep_for(std::chrono::milliseconds(1));
            }
        }
        for (;;) {
            const uint64_t b = (uint64_t)queue + (uint64_t)nx * next[queue].fetch_add(1);
            if (b >= grid) break;
            run_block((uint32_t)b, grid, block, entry, params);
        }
    };
    std::vector<std::thread> pool;
    const int nw = workers();
    for (int i = 0; i < nw; ++i) pool.emplace_back(worker, i % nx);
    for (auto& t : pool) t.join();
}

}  // namespace emu

// ---------------------------------------------------------------------------
// kernels of radix_kernels.hip (compiled into the same library) and their
// argument unpacking
// ---------------------------------------------------------------------------
extern "C" {
void fs_upsweep_k32(FsArgs);
void fs_upsweep_k64(FsArgs);
void fs_onesweep_k32(FsArgs, uint32_t);
void fs_onesweep_k32_v(FsArgs, uint32_t);
void fs_onesweep_k64(FsArgs, uint32_t);
void fs_onesweep_k64_v(FsArgs, uint32_t);
void fs_onesweep_any_k32(FsArgs, uint32_t);
void fs_onesweep_any_k64(FsArgs, uint32_t);
void fs_first_k32(FsArgs);
void fs_first_k64(FsArgs);
void fs_local_k32(FsArgs);
void fs_local_k64(FsArgs);
void fs_local_deferred_k64(FsArgs);
void fs_local_deferred_k32(FsArgs);
void fs_onesweep_k32_s(FsArgs, uint32_t);
void fs_onesweep_any_k32_s(FsArgs, uint32_t);
void fs_onesweep_k32_vs(FsArgs, uint32_t);
void fs_onesweep_k64_s(FsArgs, uint32_t);
void fs_onesweep_any_k64_s(FsArgs, uint32_t);
void fs_onesweep_k64_vs(FsArgs, uint32_t);
void fs_local_k32_w(FsArgs);
void fs_local_deferred_k32_w(FsArgs);
void fs_local_k64_w(FsArgs);
void fs_local_deferred_k64_w(FsArgs);
void fs_rescatter_k32(FsArgs);
void fs_rescatter_k64(FsArgs);
void fs_onesweep_loop_k64(FsArgs, uint32_t);
void fs_region_sample_k32(FsArgs);
void fs_region_sample_k64(FsArgs);
void fs_iota(uint32_t*, uint64_t);
void fs_scratch_address(uint64_t*);
void fs_gather_elems(uint64_t, uint64_t, uint64_t, uint64_t, uint64_t, uint32_t, uint64_t);
extern uint32_t fs_kernel_tile_keys[FS_VARIANTS];
extern uint32_t fs_kernel_block_threads[FS_VARIANTS];
extern uint32_t fs_kernel_local_geometry[9];
}

struct emu_function {
    const char* name;
    void (*entry)(void**);
};

#define A0 (*(FsArgs*)p[0])
#define D1 (*(uint32_t*)p[1])
static emu_function g_funcs[] = {
    {"fs_upsweep_k32", [](void** p) { fs_upsweep_k32(A0); }},
    {"fs_upsweep_k64", [](void** p) { fs_upsweep_k64(A0); }},
    {"fs_onesweep_k32", [](void** p) { fs_onesweep_k32(A0, D1); }},
    {"fs_onesweep_k32_v", [](void** p) { fs_onesweep_k32_v(A0, D1); }},
    {"fs_onesweep_k64", [](void** p) { fs_onesweep_k64(A0, D1); }},
    {"fs_onesweep_k64_v", [](void** p) { fs_onesweep_k64_v(A0, D1); }},
    {"fs_onesweep_any_k32", [](void** p) { fs_onesweep_any_k32(A0, D1); }},
    {"fs_onesweep_any_k64", [](void** p) { fs_onesweep_any_k64(A0, D1); }},
    {"fs_first_k32", [](void** p) { fs_first_k32(A0); }},
    {"fs_first_k64", [](void** p) { fs_first_k64(A0); }},
    {"fs_local_k32", [](void** p) { fs_local_k32(A0); }},
    {"fs_local_k64", [](void** p) { fs_local_k64(A0); }},
    {"fs_local_deferred_k64", [](void** p) { fs_local_deferred_k64(A0); }},
    {"fs_local_deferred_k32", [](void** p) { fs_local_deferred_k32(A0); }},
    {"fs_onesweep_k32_s", [](void** p) { fs_onesweep_k32_s(A0, D1); }},
    {"fs_onesweep_any_k32_s", [](void** p) { fs_onesweep_any_k32_s(A0, D1); }},
    {"fs_onesweep_k32_vs", [](void** p) { fs_onesweep_k32_vs(A0, D1); }},
    {"fs_onesweep_k64_s", [](void** p) { fs_onesweep_k64_s(A0, D1); }},
    {"fs_onesweep_any_k64_s", [](void** p) { fs_onesweep_any_k64_s(A0, D1); }},
    {"fs_onesweep_k64_vs", [](void** p) { fs_onesweep_k64_vs(A0, D1); }},
    {"fs_local_k32_w", [](void** p) { fs_local_k32_w(A0); }},
    {"fs_local_deferred_k32_w", [](void** p) { fs_local_deferred_k32_w(A0); }},
    {"fs_local_k64_w", [](void** p) { fs_local_k64_w(A0); }},
    {"fs_local_deferred_k64_w", [](void** p) { fs_local_deferred_k64_w(A0); }},
    {"fs_rescatter_k32", [](void** p) { fs_rescatter_k32(A0); }},
    {"fs_rescatter_k64", [](void** p) { fs_rescatter_k64(A0); }},
    {"fs_onesweep_loop_k64", [](void** p) { fs_onesweep_loop_k64(A0, D1); }},
    {"fs_region_sample_k32", [](void** p) { fs_region_sample_k32(A0); }},
    {"fs_region_sample_k64", [](void** p) { fs_region_sample_k64(A0); }},
    {"fs_iota", [](void** p) { fs_iota(*(uint32_t**)p[0], *(uint64_t*)p[1]); }},
    {"fs_scratch_address", [](void** p) { fs_scratch_address(*(uint64_t**)p[0]); }},
    {"fs_gather_elems", [](void** p) {
         fs_gather_elems(*(uint64_t*)p[0], *(uint64_t*)p[1], *(uint64_t*)p[2], *(uint64_t*)p[3],
                         *(uint64_t*)p[4], *(uint32_t*)p[5], *(uint64_t*)p[6]);
     }},
};

struct emu_module { int dummy; };
struct emu_stream { bool capturing = false; };
struct emu_event { std::chrono::steady_clock::time_point t; };

// ---------------------------------------------------------------------------
// guard-page device memory
// ---------------------------------------------------------------------------
namespace {
std::mutex g_mu;
std::map<void*, std::pair<char*, size_t>> g_allocs;   // user ptr -> (mapping, length)
const size_t kPage = 4096;

void on_segv(int, siginfo_t* si, void*) {
    char msg[256];
    snprintf(msg, sizeof msg, "hip_emu: device memory fault at %p (kernel %s, block %d, thread %d)\n",
             si->si_addr, emu::g_kernel, emu::B ? (int)emu::B->bidx.x : -1, emu::B ? emu::B->cur : -1);
    if (write(2, msg, strlen(msg)) < 0) {}
    void* frames[64];
    const int nf = backtrace(frames, 64);
    backtrace_symbols_fd(frames, nf, 2);
    _exit(86);
}

struct SegvInstaller {
    SegvInstaller() {
        if (getenv("EMU_NO_SEGV_HANDLER")) return;
        struct sigaction sa;
        memset(&sa, 0, sizeof sa);
        sa.sa_sigaction = on_segv;
        sa.sa_flags = SA_SIGINFO | SA_ONSTACK;
        sigaction(SIGSEGV, &sa, nullptr);
    }
} g_segv;
}  // namespace

hipError_t hipMalloc(void** p, size_t n) {
    const size_t body = (n + kPage - 1) / kPage * kPage;
    const size_t len = body + 2 * kPage;
    char* m = (char*)mmap(nullptr, len, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
    if (m == MAP_FAILED) return hipErrorOutOfMemory;
    mprotect(m, kPage, PROT_NONE);
    mprotect(m + kPage + body, kPage, PROT_NONE);
    const size_t n16 = (n + 15) / 16 * 16;
    char* user = m + kPage + body - n16;       // ends on the trailing guard page (16-byte aligned)
    std::lock_guard<std::mutex> g(g_mu);
    g_allocs[user] = {m, len};
    *p = user;
    return hipSuccess;
}

namespace { void flush_copies(); }
hipError_t hipFree(void* p) {
    if (!p) return hipSuccess;
    flush_copies();
    std::lock_guard<std::mutex> g(g_mu);
    auto it = g_allocs.find(p);
    if (it == g_allocs.end()) return hipErrorInvalidValue;
    munmap(it->second.first, it->second.second);
    g_allocs.erase(it);
    return hipSuccess;
}

// Asynchronous copies are deferred, as a DMA engine may run them late: they
// take place, in issue order, at the next point that waits for the stream or
// runs stream-ordered work (a launch, a synchronous copy or memset, an event
// or stream wait, a free).  Host code that reuses a source buffer, or reads a
// destination, before waiting then sees what real hardware may show it.
namespace {
struct emu_copy { void* d; const void* s; size_t n; };
std::mutex g_copy_mu;
std::vector<emu_copy> g_pending;
void flush_copies() {
    std::lock_guard<std::mutex> lk(g_copy_mu);
    for (const emu_copy& c : g_pending) memmove(c.d, c.s, c.n);
    g_pending.clear();
}
}  // namespace
hipError_t hipHostMalloc(void** p, size_t n, unsigned) { return hipMalloc(p, n); }
hipError_t hipHostFree(void* p) { flush_copies(); return hipFree(p); }
hipError_t hipMemset(void* p, int v, size_t n) { flush_copies(); memset(p, v, n); return hipSuccess; }
hipError_t hipMemcpy(void* d, const void* s, size_t n, hipMemcpyKind) { flush_copies(); memmove(d, s, n); return hipSuccess; }
hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind, hipStream_t) {
    std::lock_guard<std::mutex> lk(g_copy_mu);
    g_pending.push_back({d, s, n});
    return hipSuccess;
}
hipError_t hipMemcpyDtoH(void* d, hipDeviceptr_t s, size_t n) { flush_copies(); memcpy(d, s, n); return hipSuccess; }

hipError_t hipGetDeviceCount(int* c) { *c = 1; return hipSuccess; }
hipError_t hipSetDevice(int d) { return d == 0 ? hipSuccess : hipErrorInvalidValue; }
hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t, int) {
    const char* e = getenv("EMU_CUS");
    *v = e ? atoi(e) : 2;
    return hipSuccess;
}
hipError_t hipGetLastError(void) { return hipSuccess; }
const char* hipGetErrorString(hipError_t e) { return e == hipSuccess ? "success" : "emulated HIP error"; }
hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned) { *s = new emu_stream(); return hipSuccess; }
// Capture is a state flag only: launches on a capturing stream still run at
// once (enough for the host runtime's capture rules, which is what the
// emulator tests); the default stream (nullptr) never captures.
hipError_t hipStreamBeginCapture(hipStream_t s, int) {
    if (!s) return hipErrorInvalidValue;
    s->capturing = true;
    return hipSuccess;
}
hipError_t hipStreamEndCapture(hipStream_t s, void** graph) {
    if (!s || !s->capturing) return hipErrorInvalidValue;
    s->capturing = false;
    if (graph) *graph = nullptr;
    return hipSuccess;
}
hipError_t hipStreamIsCapturing(hipStream_t s, hipStreamCaptureStatus* st) {
    *st = (s && s->capturing) ? hipStreamCaptureStatusActive : hipStreamCaptureStatusNone;
    return hipSuccess;
}
hipError_t hipStreamDestroy(hipStream_t s) { delete s; return hipSuccess; }
hipError_t hipStreamSynchronize(hipStream_t) { flush_copies(); return hipSuccess; }
hipError_t hipDeviceSynchronize(void) { flush_copies(); return hipSuccess; }

hipError_t hipModuleLoad(hipModule_t* m, const char*) { *m = new emu_module(); return hipSuccess; }
hipError_t hipModuleUnload(hipModule_t m) { delete m; return hipSuccess; }
hipError_t hipModuleGetFunction(hipFunction_t* f, hipModule_t, const char* name) {
    for (auto& e : g_funcs)
        if (!strcmp(e.name, name)) { *f = &e; return hipSuccess; }
    return hipErrorNotFound;
}
hipError_t hipModuleGetGlobal(hipDeviceptr_t* p, size_t* sz, hipModule_t, const char* name) {
    if (!strcmp(name, "fs_kernel_tile_keys")) { *p = fs_kernel_tile_keys; *sz = sizeof fs_kernel_tile_keys; return hipSuccess; }
    if (!strcmp(name, "fs_kernel_block_threads")) { *p = fs_kernel_block_threads; *sz = sizeof fs_kernel_block_threads; return hipSuccess; }
    if (!strcmp(name, "fs_kernel_local_geometry")) { *p = fs_kernel_local_geometry; *sz = sizeof fs_kernel_local_geometry; return hipSuccess; }
    return hipErrorNotFound;
}
hipError_t hipModuleLaunchKernel(hipFunction_t f, unsigned gx, unsigned, unsigned, unsigned bx, unsigned,
                                 unsigned, unsigned, hipStream_t, void** params, void**) {
    flush_copies();
    emu::launch(f->name, f->entry, gx, bx, params);
    return hipSuccess;
}
hipError_t hipEventCreate(hipEvent_t* e) { *e = new emu_event(); return hipSuccess; }
hipError_t hipEventDestroy(hipEvent_t e) { delete e; return hipSuccess; }
hipError_t hipEventRecord(hipEvent_t e, hipStream_t) { e->t = std::chrono::steady_clock::now(); return hipSuccess; }
// launches complete before their call returns; deferred copies run here
hipError_t hipEventSynchronize(hipEvent_t) { flush_copies(); return hipSuccess; }
hipError_t hipEventElapsedTime(float* ms, hipEvent_t a, hipEvent_t b) {
    *ms = std::chrono::duration<float, std::milli>(b->t - a->t).count();
    return hipSuccess;
}

// Test helpers the emulator tests call through ctypes (TEST INFRASTRUCTURE).
extern "C" void* emu_test_stream_create() { hipStream_t s = nullptr; hipStreamCreateWithFlags(&s, 0); return s; }
extern "C" int emu_test_begin_capture(void* s) { return hipStreamBeginCapture((hipStream_t)s, 0); }
extern "C" int emu_test_end_capture(void* s) { return hipStreamEndCapture((hipStream_t)s, nullptr); }
