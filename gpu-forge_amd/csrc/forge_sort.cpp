// forge_sort.cpp -- host runtime behind include/forge_sort.h.
//
// Replaces forge-sort's Metal plumbing (src/metal_helpers.rs: device/queue
// init :206-217, PSO cache :78-146, shared buffers :194-202) and the encoders
// of src/lib.rs (dispatch_sort :285-409, encode_sort_pipeline_full
// :1520-1639, encode_sort_pipeline_64 :1302-1478) with HIP: one device, one
// stream, the gfx950 code object loaded by hipModuleLoad, grow-only scratch
// in HBM, and a fixed launch sequence per sort:
//   fs_upsweep (its last block writes the schedule) -> fs_onesweep x digits
// The sequence never reads anything back to the host, so fs_encode is fully
// asynchronous; which digit passes really run is decided on the device.
//
// Every HIP error is mapped to a status code and a message; nothing panics or
// throws across the C ABI.
#include <dlfcn.h>
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "../../include/forge_sort.h"
#include "fs_params.h"

namespace {

struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;
};

struct ProfEntry {
    const char* name;
    hipEvent_t start, stop;
};

const char* const kKernelNames[] = {
    "fs_upsweep_k32", "fs_upsweep_k64", "fs_onesweep_k32", "fs_onesweep_k32_v",
    "fs_onesweep_k64", "fs_onesweep_k64_v", "fs_iota", "fs_onesweep_any_k32", "fs_onesweep_any_k64",
    "fs_scratch_address", "fs_first_k32", "fs_first_k64", "fs_region_sample_k32", "fs_region_sample_k64",
    "fs_local_k32", "fs_rescatter_k32", "fs_rescatter_k64", "fs_local_k64",
    "fs_local_deferred_k64", "fs_onesweep_loop_k64", "fs_local_deferred_k32", "fs_local_k32_w",
    "fs_local_deferred_k32_w", "fs_local_k64_w", "fs_local_deferred_k64_w", "fs_onesweep_k32_s",
    "fs_onesweep_any_k32_s", "fs_onesweep_k32_vs", "fs_onesweep_k64_s", "fs_onesweep_any_k64_s", "fs_onesweep_k64_vs",
};
enum {
    K_UP32, K_UP64, K_OS32, K_OS32V, K_OS64, K_OS64V, K_IOTA, K_ANY32, K_ANY64, K_SCRATCH_ADDR, K_FIRST32, K_FIRST64,
    K_SAMPLE32, K_SAMPLE64, K_LOCAL32, K_RESCATTER32, K_RESCATTER64, K_LOCAL64, K_DEFER64, K_LOOP64, K_DEFER32,
    K_LOCAL32W, K_DEFER32W, K_LOCAL64W, K_DEFER64W, K_OS32S, K_ANY32S, K_OS32VS, K_OS64S, K_ANY64S, K_OS64VS,
    K_COUNT
};
// the stable digit-pass kernel and the keys-only first-pass kernel of each variant (FS_VAR_*)
const int kPassKernel[FS_VARIANTS] = {K_OS32, K_OS32V, K_OS64, K_OS64V, K_OS32S, K_OS32VS, K_OS64S, K_OS64VS};
const int kAnyKernel[FS_VARIANTS] = {K_ANY32, -1, K_ANY64, -1, K_ANY32S, -1, K_ANY64S, -1};

}  // namespace

struct fs_sorter {
    int device = 0;
    hipStream_t stream = nullptr;
    bool own_stream = false;
    hipModule_t module = nullptr;
    hipFunction_t fn[K_COUNT] = {};
    uint32_t tile[FS_VARIANTS] = {};    // keys per tile of each digit-pass variant (FS_VAR_*)
    uint32_t block[FS_VARIANTS] = {};   // threads per block of each variant
    // keys a block of the local sort holds and its threads per block, by
    // [wide][64-bit keys] (fs_local_k32, fs_local_k64, fs_local_k32_w, fs_local_k64_w)
    uint32_t local_keys[2][2] = {};
    uint32_t local_block[2][2] = {};
    uint32_t local_min_bits32 = 8;  // fewest segment bits whose 32-bit segments fs_local_k32 sorts itself
    int num_cus = 256;

    DevBuf s1k, s2k, s1v, s2v, lb0, lb1, iok, iov, tilemap;
    uint32_t* hist = nullptr;       // [FS_HIST_SLOTS][8][256], zero between sorts
    uint32_t* binbase = nullptr;    // [8][256]
    uint32_t* cursors = nullptr;    // [FS_REGIONS] region cursors of the fused pass, zero between sorts
    uint32_t* rstart = nullptr;     // [FS_REGIONS + 1] region starts
    uint32_t* rtable = nullptr;     // [FS_RTABLE_WORDS] region bases, total and caps of the fused pass
    uint32_t* plan = nullptr;       // u32[FS_PLAN_WORDS] device-side schedule
    uint32_t* segc = nullptr;       // u32[FS_SEGC_WORDS] segment counters and deferred-segment list of the top-16 path
    uint32_t* status = nullptr;     // pinned host word written by kernels on device errors
    unsigned long long* stats = nullptr;   // device u64[FS_STAT_COUNT]
    bool stats_on = false;

    hipStream_t last_stream = nullptr;   // stream of the last enqueued sort
    bool pending = false;
    // A sort was enqueued on a capturing stream: a HIP graph may hold the
    // addresses of the scratch buffers, so they must not be reallocated.
    bool captured = false;

    // Device address of the code object's static scratch array (fs_encode_no_alloc),
    // reported by fs_scratch_address once, when the module is loaded.
    void* na_scratch = nullptr;

    // Test options (fs_sorter_set_test_option); defaults give the product layout.
    bool force_wide = false;             // 64-bit look-back entries for any n
    uint32_t fused_mode = 0;             // FS_TEST_FUSED: 0 by size, 1 never, 2 always
    uint32_t top16_mode = 0;             // FS_TEST_TOP16: 0 by size, 1 never, 2 always (even skewed), 3 sampled
    uint32_t seg_bits = 0;               // FS_TEST_SEG_BITS: 0 by size, else the segment bits
    uint32_t local_wide_mode = 0;        // FS_TEST_LOCAL_WIDE: 0 by size, 1 wide local-sort blocks
    // the last sort's schedule (the sorter's, or the static scratch's) and
    // whether it began with the fused first pass
    uint32_t* last_plan = nullptr;
    bool last_fused = false;
    bool last_top16 = false;
    uint32_t up_blocks_per_cu = 0;       // upsweep blocks per CU (0: by key width)
    uint32_t fault = FS_FAULT_NONE;      // injected fault (FS_FAULT_INJECTION builds only)

    bool profiling = false;
    std::vector<ProfEntry> prof;         // launches since profiling was enabled or reset
    std::vector<hipEvent_t> event_pool;

    // Slice API staging: two pinned host chunks, copied by the CPU while the
    // DMA engine moves the other (allocated on the first slice call).
    // pin_busy[b]: a copy that reads or writes pin[b] was enqueued and
    // pin_ev[b] (recorded after it) has not been waited on since.
    void* pin[2] = {nullptr, nullptr};
    hipEvent_t pin_ev[2] = {nullptr, nullptr};
    bool pin_busy[2] = {false, false};

    std::string err;
};

// ---------------------------------------------------------------------------
// helpers
// ---------------------------------------------------------------------------

// Message of the last failed construction on this thread (there is no sorter
// to hold it); fs_last_error(NULL) returns it.
static thread_local std::string g_create_err;

static std::string display(fs_status st, const char* detail) {
    // Display strings of SortError (lib.rs:94-104)
    switch (st) {
        case FS_ERR_DEVICE_NOT_FOUND: return "no HIP GPU device found";
        case FS_ERR_SHADER_COMPILATION: return std::string("shader compilation failed: ") + detail;
        case FS_ERR_GPU_EXECUTION: return std::string("GPU execution failed: ") + detail;
        default: return detail;
    }
}

static fs_status set_err(fs_sorter* s, fs_status st, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (s) s->err = display(st, buf);
    return st;
}

#define HIP_TRY(s, call)                                                                  \
    do {                                                                                  \
        hipError_t e_ = (call);                                                           \
        if (e_ != hipSuccess)                                                             \
            return set_err((s), FS_ERR_GPU_EXECUTION, "%s: %s", #call, hipGetErrorString(e_)); \
    } while (0)

static bool key64(fs_key_type t) { return t == FS_KEY_U64 || t == FS_KEY_I64 || t == FS_KEY_F64; }
static size_t key_bytes(fs_key_type t) { return key64(t) ? 8 : 4; }
static uint32_t xform_of(fs_key_type t) {
    switch (t) {
        case FS_KEY_I32: case FS_KEY_I64: return FS_XF_SIGN;     // lib.rs:52-57, :78-79
        case FS_KEY_F32: case FS_KEY_F64: return FS_XF_FLOAT;    // lib.rs:60-65, :82-87
        default: return FS_XF_NONE;
    }
}
static bool valid_type(int t) { return t >= FS_KEY_U32 && t <= FS_KEY_F64; }

static std::string code_object_path() {
    const char* env = getenv("FORGE_SORT_CODE_OBJECT");
    if (env && *env) return env;
    Dl_info info;
    if (dladdr((void*)&fs_sorter_new, &info) && info.dli_fname) {
        std::string p(info.dli_fname);
        size_t slash = p.rfind('/');
        std::string dir = slash == std::string::npos ? "." : p.substr(0, slash);
        return dir + "/forge_sort_gfx950.hsaco";
    }
    return "forge_sort_gfx950.hsaco";
}

static void free_buf(DevBuf& b) {
    if (b.p) (void)hipFree(b.p);
    b.p = nullptr;
    b.bytes = 0;
}

// Wait for any sort still in flight on a stream other than the sorter's own.
static fs_status drain(fs_sorter* s) {
    if (s->pending) {
        HIP_TRY(s, hipStreamSynchronize(s->last_stream));
        HIP_TRY(s, hipStreamSynchronize(s->stream));
        s->pending = false;
    }
    return FS_OK;
}

// Grow-only device buffer (ensure_buffers*, lib.rs:1120-1289).  Growing waits
// for in-flight work first, since that work may still use the old buffer.
// graph_visible: kernels a caller may capture use the buffer (everything but
// the slice API's staging buffers, which only synchronous calls use).
static fs_status ensure(fs_sorter* s, DevBuf& b, size_t bytes, bool graph_visible = true) {
    if (b.bytes >= bytes) return FS_OK;
    if (s->captured && graph_visible)
        return set_err(s, FS_ERR_INVALID_ARGUMENT,
                       "scratch must grow to %zu bytes, but a sort of this sorter was captured into a HIP graph that "
                       "may still use it: reserve capacity (fs_reserve) before capturing, or call "
                       "fs_allow_scratch_growth once those graphs are destroyed", bytes);
    fs_status st = drain(s);
    if (st != FS_OK) return st;
    free_buf(b);
    size_t want = bytes + (bytes >> 3);   // headroom against repeated small growth
    hipError_t e = hipMalloc(&b.p, want);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        b.p = nullptr;
        return set_err(s, FS_ERR_OUT_OF_MEMORY, "hipMalloc(%zu bytes) failed: %s", want,
                       hipGetErrorString(e));
    }
    b.bytes = want;
    return FS_OK;
}

static hipEvent_t take_event(fs_sorter* s) {
    if (!s->event_pool.empty()) {
        hipEvent_t e = s->event_pool.back();
        s->event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

static void recycle_profile(fs_sorter* s) {
    for (auto& p : s->prof) {
        if (p.start) s->event_pool.push_back(p.start);
        if (p.stop) s->event_pool.push_back(p.stop);
    }
    s->prof.clear();
}

static fs_status launch(fs_sorter* s, int k, unsigned grid, unsigned block, void** args,
                        hipStream_t st, bool no_events = false) {
    ProfEntry pe{kKernelNames[k], nullptr, nullptr};
    const bool profiling = s->profiling && !no_events;
    if (profiling) {
        pe.start = take_event(s);
        pe.stop = take_event(s);
        if (pe.start) HIP_TRY(s, hipEventRecord(pe.start, st));
    }
    HIP_TRY(s, hipModuleLaunchKernel(s->fn[k], grid, 1, 1, block, 1, 1, 0, st, args, nullptr));
    if (profiling) {
        if (pe.stop) HIP_TRY(s, hipEventRecord(pe.stop, st));
        s->prof.push_back(pe);
    }
    return FS_OK;
}

// After a device error the histogram and the schedule (with the upsweep's
// ticket) are cleared, so the next sort starts from the state every sort
// leaves behind.  The whole device is drained first: a sort enqueued on
// another stream (fs_encode with a caller's stream, a graph replay) may still
// be using these tables.
static void reset_device_tables(fs_sorter* s) {
    (void)hipDeviceSynchronize();
    (void)hipMemset(s->hist, 0, (size_t)FS_HIST_WORDS * 4);
    (void)hipMemset(s->plan, 0, FS_PLAN_WORDS * sizeof(uint32_t));
    (void)hipMemset(s->cursors, 0, FS_REGIONS * sizeof(uint32_t));
    if (s->na_scratch) (void)hipMemset(s->na_scratch, 0, FS_NA_ZERO_BYTES);
    (void)hipDeviceSynchronize();
}

static fs_status check_device_status(fs_sorter* s) {
    uint32_t st = __atomic_load_n(s->status, __ATOMIC_ACQUIRE);
    if (st) {
        __atomic_store_n(s->status, 0u, __ATOMIC_RELEASE);
        reset_device_tables(s);
        if (st & FS_DEVERR_BAD_TILE)
            return set_err(s, FS_ERR_GPU_EXECUTION, "digit pass drew a tile id beyond the grid");
        if (st & FS_DEVERR_BAD_DIGITS)
            return set_err(s, FS_ERR_GPU_EXECUTION, "digit count does not match the key width");
        if (st & FS_DEVERR_BAD_PLAN)
            return set_err(s, FS_ERR_GPU_EXECUTION, "device schedule named an unknown buffer");
        if (st & FS_DEVERR_LOOKBACK_TIMEOUT)
            return set_err(s, FS_ERR_GPU_EXECUTION, "look-back wait exceeded its spin bound");
        return set_err(s, FS_ERR_GPU_EXECUTION, "device status 0x%x", st);
    }
    return FS_OK;
}

// ---------------------------------------------------------------------------
// the launch sequence
// ---------------------------------------------------------------------------

static int variant_of(fs_op op, fs_key_type t) {
    return key64(t) ? (op == FS_OP_SORT ? FS_VAR_K64 : FS_VAR_K64V) : (op == FS_OP_SORT ? FS_VAR_K32 : FS_VAR_K32V);
}

// Look-back tile entries are 64-bit once an inclusive prefix may need more
// than 30 bits, or when a test forces that layout.
static bool wide_lookback(const fs_sorter* s, uint64_t n) { return n >= FS_LB_WIDE_KEYS || s->force_wide; }

// Keys of the fullest region group of the fused first pass (fs_params.h):
// tile t writes the regions of group (t / FS_XCD_TILES) % FS_SUBS.  The
// regions of a group share its keys by digit value; fs_region_sample_* sizes
// them from a sample, within FS_FUSED_S1_KEYS of S1.
static uint64_t fused_sub_keys(uint64_t n, uint32_t tile) {
    const uint64_t tiles = (n + tile - 1) / tile;
    const uint64_t runs = (tiles + FS_XCD_TILES - 1) / FS_XCD_TILES;    // runs of FS_XCD_TILES tiles
    const uint64_t most = (runs + FS_SUBS - 1) / FS_SUBS;              // group 0 has the most runs
    uint64_t keys = most * FS_XCD_TILES * tile;
    if (keys > n) keys = n;
    return keys;
}

// Keys-only sorts (32- and 64-bit keys) start with the fused first pass (no
// histogram read); S1 then holds FS_REGIONS regions, which must stay below
// 2^32 keys (n <= 2^31 keeps them below 1.875 n + 2^17).
static bool fused_path(const fs_sorter* s, fs_op op, fs_key_type t, uint64_t n) {
    if (op != FS_OP_SORT || n > (1ull << 31) || s->fused_mode == 1u) return false;
    if (FS_FUSED_S1_KEYS(fused_sub_keys(n, s->tile[variant_of(op, t)])) >= (1ull << 32)) return false;
    return s->fused_mode == 2u || n >= FS_FUSED_MIN_KEYS;
}

// Keys a block of the local sort (wide: its wide blocks) holds for keys of this type.
static uint32_t local_keys_of(const fs_sorter* s, fs_key_type t, bool wide) {
    return s->local_keys[wide ? 1 : 0][key64(t) ? 1 : 0];
}

// The most keys a segment of a uniform input may hold on average for nearly
// every segment to fit one block of the local sort: a block's keys less five
// standard deviations (their square root).
static uint64_t local_mean_max(const fs_sorter* s, fs_key_type t, bool wide) {
    const uint64_t lk = local_keys_of(s, t, wide);
    uint64_t root = 0;
    while ((root + 1) * (root + 1) <= lk) ++root;
    return lk > 5 * root ? lk - 5 * root : 0;
}

// Keys-only integer sorts (u32, i32 from FS_TOP16_MIN_KEYS32 keys, u64, i64
// from FS_TOP16_MIN_KEYS64 keys) take the top-16 path (fused pass on the digit below the top byte, stable
// pass on the top digit, local sort of each segment); it needs the fused
// pass's regions, hence the fused range.  Float keys keep the LSD passes:
// their top 16 bits (sign, exponent, a few mantissa bits) are concentrated
// in a few values for most data, which the region sample would refuse.
static bool top16_path(const fs_sorter* s, fs_op op, fs_key_type t, uint64_t n) {
    if (op != FS_OP_SORT || s->top16_mode == 1u || n < 2) return false;
    if (t != FS_KEY_U32 && t != FS_KEY_I32 && t != FS_KEY_U64 && t != FS_KEY_I64) return false;
    if (n > (1ull << 31) || s->fused_mode == 1u) return false;
    if (FS_FUSED_S1_KEYS(fused_sub_keys(n, s->tile[variant_of(op, t)])) >= (1ull << 32)) return false;
    if (s->top16_mode >= 2u) return true;
    // By size: the 2^16 segments of a uniform input must fit a block (a wide
    // one from the sizes local_wide names on) with a margin of five standard
    // deviations, so that hardly any takes the big-segment path.
    return n >= (key64(t) ? FS_TOP16_MIN_KEYS64 : FS_TOP16_MIN_KEYS32) && n <= (local_mean_max(s, t, true) << 16);
}

// The digit-pass variant a sort runs: by key width and op, and its small
// tiles (FS_VAR_K32S ... FS_VAR_K64VS) below FS_SMALL_TILE_KEYS (32-bit keys)
// or FS_SMALL_TILE_KEYS64 (64-bit keys) keys on the LSD passes (the fused and
// top-16 sequences and the static scratch keep the larger tiles).
static int sort_variant(const fs_sorter* s, fs_op op, fs_key_type t, uint64_t n, bool no_alloc) {
    const int v = variant_of(op, t);
    if (no_alloc || n >= (key64(t) ? FS_SMALL_TILE_KEYS64 : FS_SMALL_TILE_KEYS)) return v;
    if (op == FS_OP_SORT && (fused_path(s, op, t, n) || top16_path(s, op, t, n))) return v;
    return v + (FS_VAR_K32S - FS_VAR_K32);    // the small variant of each (FS_VAR_* order)
}

// The top-16 path's local sort runs on wide blocks (twice the keys) where
// the 2^16 segments of a uniform input would outgrow the other blocks.
static bool local_wide(const fs_sorter* s, fs_key_type t, uint64_t n) {
    return s->local_wide_mode == 1u || n > (local_mean_max(s, t, false) << 16);
}

// Bits that name a segment of the local sort: the fewest whose segments of
// a uniform input hold at most mean_max keys on average (local_mean_max), so
// that nearly every segment fits one block, but at least the top byte and at
// most the top 16 bits the two digit passes order.  (Between a half and all
// of mean_max keys each: fewer segment bits leave fewer bits to the local
// sort.)
static uint32_t seg_bits_for(uint64_t n, uint64_t mean_max) {
    uint32_t b = 8;
    while (b < 16 && n > (mean_max << b)) ++b;
    return b;
}

// Grows the scratch a sort of n keys needs (grow-only, like ensure_buffers*,
// lib.rs:1120-1289): ping-pong buffers for keys (and values), and two
// look-back arrays of tile entries followed by one 32-bit group entry per
// FS_LB_GROUP tiles.
static fs_status reserve(fs_sorter* s, fs_op op, fs_key_type t, uint64_t n) {
    if (n <= 1) return FS_OK;
    const size_t kb = key_bytes(t);
    const uint32_t tile = s->tile[sort_variant(s, op, t, n, false)];
    const uint64_t num_tiles = (n + tile - 1) / tile;
    fs_status r;
    const bool fused = fused_path(s, op, t, n) || top16_path(s, op, t, n);
    if ((r = ensure(s, s->s1k, (fused ? FS_FUSED_S1_KEYS(fused_sub_keys(n, tile)) : n) * kb)) != FS_OK) return r;
    if ((r = ensure(s, s->s2k, n * kb)) != FS_OK) return r;
    if (fused && (r = ensure(s, s->tilemap, num_tiles * FS_TILE_DESC_WORDS * 4)) != FS_OK) return r;
    if (op != FS_OP_SORT) {
        if ((r = ensure(s, s->s1v, n * 4)) != FS_OK) return r;
        if (op == FS_OP_PAIRS && (r = ensure(s, s->s2v, n * 4)) != FS_OK) return r;
    }
    const size_t lb_bytes = (size_t)num_tiles * FS_RADIX * (wide_lookback(s, n) ? 8 : 4) +
                            (size_t)((num_tiles + FS_LB_GROUP - 1) / FS_LB_GROUP) * FS_RADIX * 4;
    if ((r = ensure(s, s->lb0, lb_bytes)) != FS_OK) return r;
    return ensure(s, s->lb1, lb_bytes);
}

// Device addresses of the scratch a sort uses: the sorter's own grow-only
// buffers, or the static array of fs_encode_no_alloc.
struct ScratchSet {
    uint64_t s1k, s2k, s1v, s2v, lb0, lb1, hist, binbase, plan, cursors, rstart, tilemap, rtable, segc;
};

static ScratchSet sorter_scratch(const fs_sorter* s) {
    return ScratchSet{(uint64_t)(uintptr_t)s->s1k.p, (uint64_t)(uintptr_t)s->s2k.p,
                      (uint64_t)(uintptr_t)s->s1v.p, (uint64_t)(uintptr_t)s->s2v.p,
                      (uint64_t)(uintptr_t)s->lb0.p, (uint64_t)(uintptr_t)s->lb1.p,
                      (uint64_t)(uintptr_t)s->hist, (uint64_t)(uintptr_t)s->binbase,
                      (uint64_t)(uintptr_t)s->plan, (uint64_t)(uintptr_t)s->cursors,
                      (uint64_t)(uintptr_t)s->rstart, (uint64_t)(uintptr_t)s->tilemap.p,
                      (uint64_t)(uintptr_t)s->rtable, (uint64_t)(uintptr_t)s->segc};
}

static ScratchSet static_scratch(const fs_sorter* s) {
    const uint64_t p = (uint64_t)(uintptr_t)s->na_scratch;
    return ScratchSet{p + FS_NA_OFF_S1K, p + FS_NA_OFF_S2K, p + FS_NA_OFF_S1V, p + FS_NA_OFF_S2V,
                      p + FS_NA_OFF_LB0, p + FS_NA_OFF_LB1, p + FS_NA_OFF_HIST, p + FS_NA_OFF_BINBASE,
                      p + FS_NA_OFF_PLAN, p + FS_NA_OFF_CURSORS, p + FS_NA_OFF_RSTART, p + FS_NA_OFF_TILEMAP,
                      p + FS_NA_OFF_RTABLE, 0};   // (no top-16 path on the static scratch)
}

// no_alloc: the sort runs on the static scratch (fs_encode_no_alloc): nothing
// is allocated, the scratch is not grown and no profiling events are created.
static fs_status enqueue(fs_sorter* s, fs_op op, fs_key_type t, void* keys, uint32_t* vals,
                         uint64_t n, hipStream_t st, bool no_alloc = false) {
    if (!valid_type(t)) return set_err(s, FS_ERR_INVALID_ARGUMENT, "unknown key type %d", (int)t);
    if (op != FS_OP_SORT && op != FS_OP_ARGSORT && op != FS_OP_PAIRS)
        return set_err(s, FS_ERR_INVALID_ARGUMENT, "unknown op %d", (int)op);
    if (n >= (1ull << 32))
        return set_err(s, FS_ERR_INVALID_ARGUMENT, "n = %llu exceeds 2^32 - 1", (unsigned long long)n);
    if (n > 0 && !keys) return set_err(s, FS_ERR_INVALID_ARGUMENT, "null keys");
    if (n > 0 && op != FS_OP_SORT && !vals) return set_err(s, FS_ERR_INVALID_ARGUMENT, "null values");

    if (n <= 1) {
        // lib.rs:710-712 / :1677-1682: nothing to sort; argsort of one key is [0]
        if (n == 1 && op == FS_OP_ARGSORT) {
            uint64_t one = 1;
            void* args[] = {&vals, &one};
            fs_status r = launch(s, K_IOTA, 1, 64, args, st, no_alloc);
            if (r != FS_OK) return r;
        }
        return FS_OK;
    }

    const size_t kb = key_bytes(t);
    if ((uintptr_t)keys % kb != 0 || (vals && (uintptr_t)vals % 4 != 0))
        return set_err(s, FS_ERR_INVALID_ARGUMENT, "misaligned key or value pointer");
    const int var = sort_variant(s, op, t, n, no_alloc);
    const uint32_t tile = s->tile[var];
    const uint32_t num_tiles = (uint32_t)((n + tile - 1) / tile);
    // the static scratch holds narrow look-back entries (n < 2^30 there)
    const bool wide = !no_alloc && wide_lookback(s, n);
    fs_status r;
    if (no_alloc) {
        if (n > FS_NA_MAX_KEYS)
            return set_err(s, FS_ERR_INVALID_ARGUMENT,
                           "n = %llu exceeds the %u keys the no-allocation scratch holds (use fs_encode)",
                           (unsigned long long)n, (unsigned)FS_NA_MAX_KEYS);
        if (num_tiles > FS_NA_MAX_TILES)      // every variant's tile is at least FS_NA_MIN_TILE keys
            return set_err(s, FS_ERR_INVALID_ARGUMENT, "tile geometry exceeds the no-allocation scratch layout");
    } else if ((r = reserve(s, op, t, n)) != FS_OK) {
        return r;
    }
    const ScratchSet sc = no_alloc ? static_scratch(s) : sorter_scratch(s);
    // the fused first pass, when its regions fit the scratch (the static
    // scratch's S1 holds FS_NA_MAX_KEYS 8-byte keys)
    const uint64_t sub_keys = fused_sub_keys(n, tile);
    const bool top16 = !no_alloc && top16_path(s, op, t, n);
    const bool fused = top16 || (fused_path(s, op, t, n) &&
                                 (!no_alloc || FS_FUSED_S1_KEYS(sub_keys) * kb <= (uint64_t)FS_NA_MAX_KEYS * 8));

    FsArgs a;
    memset(&a, 0, sizeof a);
    a.n = n;
    a.key64 = key64(t) ? 1u : 0u;
    a.xform = xform_of(t);
    a.op = op == FS_OP_SORT ? FSK_OP_KEYS : (op == FS_OP_ARGSORT ? FSK_OP_ARGSORT : FSK_OP_PAIRS);
    a.digits = key64(t) ? 8u : 4u;     // one 8-bit digit per key byte
    a.num_tiles = num_tiles;
    a.wide = wide ? 1u : 0u;
    a.tile = tile;
    a.vec_ok = ((uintptr_t)keys % 16 == 0) ? 1u : 0u;
    // upsweep: 1 block per CU for 32-bit keys (measured faster than 2: fewer
    // counter clears, folds and histogram atomics for the same keys), 2 for
    // 64-bit keys (the blocks' 64 KiB of counters allow two resident); fewer
    // when the keys give each block less than one step of FS_UPSWEEP_UNROLL
    // units per thread (a test option can set the blocks per CU)
    const uint64_t up_per_cu = s->up_blocks_per_cu ? s->up_blocks_per_cu : (key64(t) ? 2u : 1u);
    const uint64_t up_units = a.vec_ok ? n / (16u / key_bytes(t)) : n;
    const uint64_t up_span = (uint64_t)FS_UPSWEEP_UNROLL * FS_HIST_BLOCK;
    uint64_t up_blocks = (up_units + up_span - 1) / up_span;
    if (up_blocks > (uint64_t)s->num_cus * up_per_cu) up_blocks = (uint64_t)s->num_cus * up_per_cu;
    if (up_blocks == 0) up_blocks = 1;
    a.keys = (uint64_t)(uintptr_t)keys;
    a.vals = (uint64_t)(uintptr_t)vals;
    a.s1k = sc.s1k;
    a.s2k = sc.s2k;
    a.s1v = sc.s1v;
    a.s2v = sc.s2v;
    a.hist = sc.hist;
    a.binbase = sc.binbase;
    a.lookback0 = sc.lb0;
    a.lookback1 = sc.lb1;
    a.plan = sc.plan;
    a.cursors = sc.cursors;
    a.rstart = sc.rstart;
    a.tilemap = sc.tilemap;
    a.rtable = sc.rtable;
    a.fused = fused ? 1u : 0u;
    a.sub_keys = fused ? (uint32_t)sub_keys : 0u;
    a.s1_keys = fused ? (uint32_t)FS_FUSED_S1_KEYS(sub_keys) : 0u;
    a.segc = top16 ? sc.segc : 0u;
    const bool wide_local = top16 && local_wide(s, t, n);
    a.seg_bits = !top16 ? 0u : s->seg_bits ? s->seg_bits : seg_bits_for(n, local_mean_max(s, t, wide_local));
    // 32-bit keys: at least the segment bits whose segments the local sort's
    // first launch sorts itself, where that leaves a uniform input's segments
    // a quarter of a block or more on average (from 2^25 keys on; smaller
    // sorts, which take the top-16 path only when a test forces it, defer
    // their segments to the second launch)
    if (top16 && !s->seg_bits && !key64(t) && a.seg_bits < s->local_min_bits32 &&
        (n >> s->local_min_bits32) >= local_keys_of(s, t, wide_local) / 4u)
        a.seg_bits = s->local_min_bits32;
    // a segment the region sample estimates above 16 blocks' keys sends the
    // sort to the LSD passes (unless a test forces the top-16 path)
    a.seg_limit = s->top16_mode == 2u ? 0xFFFFFFFFu : 16u * local_keys_of(s, t, wide_local);
    a.status = (uint64_t)(uintptr_t)s->status;
    a.stats = s->stats_on ? (uint64_t)(uintptr_t)s->stats : 0u;
#ifdef FS_FAULT_INJECTION
    a.fault = s->fault;
    if (s->fault == FS_FAULT_BAD_DIGITS) a.digits = 5u;
    if (s->fault == FS_FAULT_SMALL_S1) a.s1_keys /= 2u;
#endif

    void* args1[] = {&a};
    if (fused) {
        // region sample (it picks the scatter digit: 2 on the top-16 path
        // unless the sample shows oversized segments, else 0) -> fused pass ->
        // its re-scatter launch (works only after an overflow) -> the digit
        // passes in launch slots 0 .. digits-2 -> (top-16 launch sequence) the
        // local sort, one block per segment
        if ((r = launch(s, key64(t) ? K_SAMPLE64 : K_SAMPLE32, 1, FS_HIST_BLOCK, args1, st, no_alloc)) != FS_OK)
            return r;
        unsigned grid = num_tiles;
#ifdef FS_FAULT_INJECTION
        if (s->fault == FS_FAULT_EXTRA_BLOCK) grid += 1u;
#endif
        // a small grid for the launches that usually have nothing to do (one
        // block per CU: the loop kernels' occupancy), so that they cost a few
        // blocks instead of one per tile
        const unsigned small = num_tiles < (uint32_t)s->num_cus ? num_tiles : (unsigned)s->num_cus;
        if ((r = launch(s, key64(t) ? K_FIRST64 : K_FIRST32, grid, s->block[var], args1, st, no_alloc)) != FS_OK)
            return r;
        if ((r = launch(s, key64(t) ? K_RESCATTER64 : K_RESCATTER32, small, s->block[var], args1, st, no_alloc)) != FS_OK)
            return r;
        for (uint32_t sl = 0; sl + 1 < a.digits; ++sl) {
            uint32_t slot = sl;
            void* args2[] = {&a, &slot};
            // top-16 launch sequence: slot 0 is the top digit's pass, or on
            // the LSD passes the first of them; the other slots run only for
            // those.  They launch one block per tile (an idle launch: ~14 µs)
            // so that inputs the sample sends to the LSD passes (narrow or
            // skewed keys) run every pass at full speed; only 64-bit slots
            // from FS_LOOP_SLOT64 on (keys with more than 40 varying bits
            // whose top 16 bits the sample refused) take the loop kernel's
            // small grid (idle: ~5 µs; working: one block per CU, slower).
            const bool loop = top16 && key64(t) && sl >= FS_LOOP_SLOT64;
            if ((r = launch(s, loop ? K_LOOP64 : kPassKernel[var], loop ? small : num_tiles, s->block[var], args2, st,
                            no_alloc)) != FS_OK)
                return r;
        }
        const uint32_t lthreads = s->local_block[wide_local ? 1 : 0][key64(t) ? 1 : 0];
        const int klocal = wide_local ? (key64(t) ? K_LOCAL64W : K_LOCAL32W) : (key64(t) ? K_LOCAL64 : K_LOCAL32);
        const int kdefer = wide_local ? (key64(t) ? K_DEFER64W : K_DEFER32W) : (key64(t) ? K_DEFER64 : K_DEFER32);
        if (top16 && (r = launch(s, klocal, 1u << a.seg_bits, lthreads, args1, st, no_alloc)) != FS_OK)
            return r;
        // the segments the local sort deferred (larger than a block; 64-bit
        // keys: many equal keys; 32-bit keys: fewer segment bits than it
        // sorts in one stable pass), on a small grid
        if (top16 && (r = launch(s, kdefer, small, key64(t) ? FS_LD64_BLOCK : FS_LD32_BLOCK, args1, st, no_alloc)) !=
                         FS_OK)
            return r;
        s->last_stream = st;
        s->pending = true;
        s->last_plan = (uint32_t*)(uintptr_t)sc.plan;
        s->last_fused = true;
        s->last_top16 = top16;
        return FS_OK;
    }
    {
        const unsigned up_grid = (unsigned)up_blocks;
        if ((r = launch(s, key64(t) ? K_UP64 : K_UP32, up_grid, FS_HIST_BLOCK, args1, st, no_alloc)) != FS_OK) return r;
    }
    const int os = kPassKernel[var];
    for (uint32_t d = 0; d < a.digits; ++d) {
        uint32_t digit = d;
        void* args2[] = {&a, &digit};
        // digit 0 of a keys-only sort: its pass, when it runs, is the first,
        // which needs no stability (same tiles as the stable kernel)
        const int k = (d == 0 && op == FS_OP_SORT) ? kAnyKernel[var] : os;
        unsigned grid = num_tiles;
#ifdef FS_FAULT_INJECTION
        if (s->fault == FS_FAULT_EXTRA_BLOCK && d == 0) grid += 1u;
#endif
        if ((r = launch(s, k, grid, s->block[var], args2, st, no_alloc)) != FS_OK) return r;
    }
    s->last_stream = st;
    s->pending = true;
    s->last_plan = (uint32_t*)(uintptr_t)sc.plan;
    s->last_fused = false;
    s->last_top16 = false;
    return FS_OK;
}

static fs_status sync_and_check(fs_sorter* s) {
    if (s->pending) {
        hipError_t e = hipStreamSynchronize(s->last_stream);
        s->pending = false;
        if (e != hipSuccess)
            return set_err(s, FS_ERR_GPU_EXECUTION, "hipStreamSynchronize: %s", hipGetErrorString(e));
    }
    return check_device_status(s);
}

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------

extern "C" {

const char* fs_status_str(fs_status st) {
    switch (st) {
        case FS_OK: return "ok";
        case FS_ERR_DEVICE_NOT_FOUND: return "no HIP GPU device found";
        case FS_ERR_SHADER_COMPILATION: return "shader compilation failed";
        case FS_ERR_GPU_EXECUTION: return "GPU execution failed";
        case FS_ERR_LENGTH_MISMATCH: return "length mismatch";
        case FS_ERR_INVALID_ARGUMENT: return "invalid argument";
        case FS_ERR_OUT_OF_MEMORY: return "out of memory";
    }
    return "unknown status";
}

fs_status fs_tile_config(const fs_sorter* s, uint32_t keys_per_tile[4]) {
    if (!s || !keys_per_tile) return FS_ERR_INVALID_ARGUMENT;
    for (int i = 0; i < 4; ++i) keys_per_tile[i] = s->tile[i];
    return FS_OK;
}

const char* fs_last_error(const fs_sorter* s) { return s ? s->err.c_str() : g_create_err.c_str(); }

// Frees a partly built sorter and records why construction failed.
static fs_status create_failed(fs_sorter* s, fs_status st, const std::string& detail) {
    g_create_err = display(st, detail.c_str());
    if (s) fs_sorter_free(s);
    return st;
}

static fs_status create(int device, hipStream_t stream, bool own, fs_sorter** out) {
    if (!out) return create_failed(nullptr, FS_ERR_INVALID_ARGUMENT, "null output pointer");
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0 || device < 0 || device >= count) {
        (void)hipGetLastError();
        return create_failed(nullptr, FS_ERR_DEVICE_NOT_FOUND, "");
    }
    fs_sorter* s = new (std::nothrow) fs_sorter();
    if (!s) return create_failed(nullptr, FS_ERR_OUT_OF_MEMORY, "host allocation of the sorter");
    s->device = device;
    hipError_t e = hipSetDevice(device);
    if (e != hipSuccess) {
        delete s;
        return create_failed(nullptr, FS_ERR_DEVICE_NOT_FOUND, "");
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && cus > 0)
        s->num_cus = cus;
    if (own) {
        e = hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking);
        if (e != hipSuccess) {
            delete s;
            return create_failed(nullptr, FS_ERR_GPU_EXECUTION, std::string("hipStreamCreate: ") + hipGetErrorString(e));
        }
        s->own_stream = true;
    } else {
        s->stream = stream;
    }
    s->last_stream = s->stream;

    const std::string path = code_object_path();
    e = hipModuleLoad(&s->module, path.c_str());
    if (e != hipSuccess)
        return create_failed(s, FS_ERR_SHADER_COMPILATION,
                             "hipModuleLoad(" + path + "): " + hipGetErrorString(e));
    for (int k = 0; k < K_COUNT; ++k) {
        e = hipModuleGetFunction(&s->fn[k], s->module, kKernelNames[k]);
        if (e != hipSuccess)
            return create_failed(s, FS_ERR_SHADER_COMPILATION, std::string("kernel ") + kKernelNames[k] +
                                 " missing from the code object");
    }
    {
        // tile geometry compiled into the code object
        hipDeviceptr_t gp = nullptr, bp = nullptr;
        size_t gsz = 0, bsz = 0;
        if (hipModuleGetGlobal(&gp, &gsz, s->module, "fs_kernel_tile_keys") != hipSuccess || gsz != sizeof s->tile ||
            hipModuleGetGlobal(&bp, &bsz, s->module, "fs_kernel_block_threads") != hipSuccess ||
            bsz != sizeof s->block || hipMemcpyDtoH(s->tile, gp, sizeof s->tile) != hipSuccess ||
            hipMemcpyDtoH(s->block, bp, sizeof s->block) != hipSuccess) {
            return create_failed(s, FS_ERR_SHADER_COMPILATION,
                                 "code object lacks fs_kernel_tile_keys/fs_kernel_block_threads");
        }
        for (int i = 0; i < FS_VARIANTS; ++i)
            if (s->tile[i] == 0 || s->block[i] < FS_RADIX)
                return create_failed(s, FS_ERR_SHADER_COMPILATION, "code object has an invalid tile geometry");
        hipDeviceptr_t lp = nullptr;
        size_t lsz = 0;
        uint32_t lg[9] = {};
        if (hipModuleGetGlobal(&lp, &lsz, s->module, "fs_kernel_local_geometry") != hipSuccess ||
            lsz != sizeof(lg) || hipMemcpyDtoH(lg, lp, sizeof(lg)) != hipSuccess || lg[4] < 8 || lg[4] > 16)
            return create_failed(s, FS_ERR_SHADER_COMPILATION, "code object lacks a valid fs_kernel_local_geometry");
        for (int w = 0; w < 2; ++w)
            for (int i = 0; i < 2; ++i) {
                const uint32_t keys = lg[w ? 5 + 2 * i : 2 * i], threads = lg[w ? 6 + 2 * i : 2 * i + 1];
                if (keys == 0 || threads < FS_RADIX)
                    return create_failed(s, FS_ERR_SHADER_COMPILATION, "code object has an invalid local geometry");
                s->local_keys[w][i] = keys;
                s->local_block[w][i] = threads;
            }
        s->local_min_bits32 = lg[4];
    }
    const size_t tab = (size_t)FS_MAX_DIGITS * FS_RADIX * 4;
    if (hipMalloc(&s->hist, (size_t)FS_HIST_WORDS * 4) != hipSuccess || hipMalloc(&s->binbase, tab) != hipSuccess ||
        hipMalloc(&s->cursors, FS_REGIONS * 4) != hipSuccess || hipMalloc(&s->rstart, (FS_REGIONS + 1) * 4) != hipSuccess ||
        hipMalloc(&s->rtable, FS_RTABLE_WORDS * 4) != hipSuccess ||
        hipMalloc(&s->plan, FS_PLAN_WORDS * sizeof(uint32_t)) != hipSuccess ||
        hipMalloc(&s->segc, FS_SEGC_WORDS * sizeof(uint32_t)) != hipSuccess ||
        hipMalloc(&s->stats, FS_STAT_SLOTS * FS_STAT_COUNT * sizeof(unsigned long long)) != hipSuccess ||
        hipHostMalloc(&s->status, sizeof(uint32_t), hipHostMallocDefault) != hipSuccess)
        return create_failed(s, FS_ERR_OUT_OF_MEMORY, "device tables of the sorter");
    *s->status = 0;
    {
        // The static scratch of fs_encode_no_alloc: its address in this
        // module, from the kernel (the module API has no symbol for a
        // file-scope static); its tables must start at zero.
        uint64_t* out = (uint64_t*)s->stats;
        void* args[] = {&out};
        uint64_t got[2] = {0, 0};
        if (hipModuleLaunchKernel(s->fn[K_SCRATCH_ADDR], 1, 1, 1, 64, 1, 1, 0, s->stream, args, nullptr) != hipSuccess ||
            hipStreamSynchronize(s->stream) != hipSuccess ||
            hipMemcpy(got, s->stats, sizeof got, hipMemcpyDeviceToHost) != hipSuccess)
            return create_failed(s, FS_ERR_GPU_EXECUTION, "querying the no-allocation scratch address");
        if (got[0] == 0 || got[0] % 256 != 0 || got[1] != FS_NA_SCRATCH_BYTES)
            return create_failed(s, FS_ERR_SHADER_COMPILATION, "code object's no-allocation scratch has an unexpected "
                                 "address or size (rebuild the code object and the library together)");
        s->na_scratch = (void*)(uintptr_t)got[0];
        if (hipMemset(s->na_scratch, 0, FS_NA_ZERO_BYTES) != hipSuccess)
            return create_failed(s, FS_ERR_GPU_EXECUTION, "clearing the no-allocation scratch tables");
    }
    // The histogram table and the upsweep's ticket must start at zero; the
    // upsweep's last block re-zeroes both after every sort.
    if (hipMemset(s->hist, 0, (size_t)FS_HIST_WORDS * 4) != hipSuccess ||
        hipMemset(s->cursors, 0, FS_REGIONS * 4) != hipSuccess ||
        hipMemset(s->stats, 0, FS_STAT_SLOTS * FS_STAT_COUNT * sizeof(unsigned long long)) != hipSuccess ||
        hipMemset(s->plan, 0, FS_PLAN_WORDS * sizeof(uint32_t)) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess)
        return create_failed(s, FS_ERR_GPU_EXECUTION, "clearing the device tables");
    *out = s;
    return FS_OK;
}

fs_status fs_sorter_new(int device, fs_sorter** out) { return create(device, nullptr, true, out); }

fs_status fs_sorter_with_context(int device, void* hip_stream, fs_sorter** out) {
    return create(device, (hipStream_t)hip_stream, false, out);
}

void fs_sorter_free(fs_sorter* s) {
    if (!s) return;
    (void)hipSetDevice(s->device);
    if (s->pending) (void)hipStreamSynchronize(s->last_stream);
    if (s->stream || s->own_stream) (void)hipStreamSynchronize(s->stream);
    recycle_profile(s);
    for (hipEvent_t e : s->event_pool) (void)hipEventDestroy(e);
    DevBuf* bufs[] = {&s->s1k, &s->s2k, &s->s1v, &s->s2v, &s->lb0, &s->lb1, &s->iok, &s->iov, &s->tilemap};
    for (DevBuf* b : bufs) free_buf(*b);
    if (s->hist) (void)hipFree(s->hist);
    if (s->cursors) (void)hipFree(s->cursors);
    if (s->rstart) (void)hipFree(s->rstart);
    if (s->rtable) (void)hipFree(s->rtable);
    if (s->binbase) (void)hipFree(s->binbase);
    if (s->plan) (void)hipFree(s->plan);
    if (s->segc) (void)hipFree(s->segc);
    if (s->stats) (void)hipFree(s->stats);
    if (s->status) (void)hipHostFree(s->status);
    for (int b = 0; b < 2; ++b) {
        if (s->pin[b]) (void)hipHostFree(s->pin[b]);
        if (s->pin_ev[b]) (void)hipEventDestroy(s->pin_ev[b]);
    }
    if (s->module) (void)hipModuleUnload(s->module);
    if (s->own_stream && s->stream) (void)hipStreamDestroy(s->stream);
    delete s;
}

fs_status fs_alloc_sort_buffer(fs_sorter* s, fs_key_type type, size_t capacity, void** device_ptr) {
    if (!s || !device_ptr) return FS_ERR_INVALID_ARGUMENT;
    if (!valid_type(type)) return set_err(s, FS_ERR_INVALID_ARGUMENT, "unknown key type %d", (int)type);
    *device_ptr = nullptr;
    HIP_TRY(s, hipSetDevice(s->device));
    size_t bytes = capacity * key_bytes(type);
    if (bytes == 0) bytes = key_bytes(type);
    hipError_t e = hipMalloc(device_ptr, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        *device_ptr = nullptr;
        return set_err(s, FS_ERR_OUT_OF_MEMORY, "hipMalloc(%zu bytes) failed: %s", bytes, hipGetErrorString(e));
    }
    return FS_OK;
}

fs_status fs_free_sort_buffer(fs_sorter* s, void* device_ptr) {
    if (!s) return FS_ERR_INVALID_ARGUMENT;
    if (!device_ptr) return FS_OK;
    fs_status r = drain(s);
    if (r != FS_OK) return r;
    HIP_TRY(s, hipFree(device_ptr));
    return FS_OK;
}

fs_status fs_copy_to_device(fs_sorter* s, void* dst, const void* src, size_t bytes) {
    if (!s || (bytes && (!dst || !src))) return FS_ERR_INVALID_ARGUMENT;
    if (!bytes) return FS_OK;
    fs_status r = drain(s);
    if (r != FS_OK) return r;
    HIP_TRY(s, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s->stream));
    HIP_TRY(s, hipStreamSynchronize(s->stream));
    return FS_OK;
}

fs_status fs_copy_to_host(fs_sorter* s, void* dst, const void* src, size_t bytes) {
    if (!s || (bytes && (!dst || !src))) return FS_ERR_INVALID_ARGUMENT;
    if (!bytes) return FS_OK;
    fs_status r = drain(s);
    if (r != FS_OK) return r;
    HIP_TRY(s, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s->stream));
    HIP_TRY(s, hipStreamSynchronize(s->stream));
    return FS_OK;
}

fs_status fs_copy_device(fs_sorter* s, void* dst, const void* src, size_t bytes) {
    if (!s || (bytes && (!dst || !src))) return FS_ERR_INVALID_ARGUMENT;
    if (!bytes) return FS_OK;
    fs_status r = drain(s);
    if (r != FS_OK) return r;
    HIP_TRY(s, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s->stream));
    HIP_TRY(s, hipStreamSynchronize(s->stream));
    return FS_OK;
}

fs_status fs_device_synchronize(fs_sorter* s) {
    if (!s) return FS_ERR_INVALID_ARGUMENT;
    HIP_TRY(s, hipSetDevice(s->device));
    HIP_TRY(s, hipDeviceSynchronize());
    s->pending = false;
    return check_device_status(s);
}

fs_status fs_encode(fs_sorter* s, fs_op op, fs_key_type type, void* device_keys, uint32_t* device_values,
                    uint64_t n, void* hip_stream) {
    if (!s) return FS_ERR_INVALID_ARGUMENT;
    HIP_TRY(s, hipSetDevice(s->device));
    hipStream_t st = hip_stream ? (hipStream_t)hip_stream : s->stream;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cap) != hipSuccess) {
        (void)hipGetLastError();
        cap = hipStreamCaptureStatusNone;
    }
    if (cap == hipStreamCaptureStatusActive) {
        // The graph being captured will hold the scratch addresses: from now
        // on the scratch may not be reallocated (ensure refuses to grow it,
        // including for this sort, which must fit what was reserved).
        s->captured = true;
    } else if (s->pending && s->last_stream != st) {
        fs_status r = drain(s);   // scratch is shared: serialise sorts issued on different streams
        if (r != FS_OK) return r;
    }
    return enqueue(s, op, type, device_keys, op == FS_OP_SORT ? nullptr : device_values, n, st);
}

fs_status fs_encode_no_alloc(fs_sorter* s, fs_op op, fs_key_type type, void* device_keys,
                             uint32_t* device_values, uint64_t n, void* hip_stream) {
    if (!s) return FS_ERR_INVALID_ARGUMENT;
    HIP_TRY(s, hipSetDevice(s->device));
    hipStream_t st = hip_stream ? (hipStream_t)hip_stream : s->stream;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cap) != hipSuccess) {
        (void)hipGetLastError();
        cap = hipStreamCaptureStatusNone;
    }
    // The static scratch is shared by every call through this sorter: a sort
    // on another stream must be done before this one starts (not waited for
    // while capturing, where the caller orders the work).
    if (cap != hipStreamCaptureStatusActive && s->pending && s->last_stream != st) {
        fs_status r = drain(s);
        if (r != FS_OK) return r;
    }
    return enqueue(s, op, type, device_keys, op == FS_OP_SORT ? nullptr : device_values, n, st, true);
}

fs_status fs_reserve(fs_sorter* s, fs_op op, fs_key_type type, uint64_t n) {
    if (!s) return FS_ERR_INVALID_ARGUMENT;
    if (!valid_type(type)) return set_err(s, FS_ERR_INVALID_ARGUMENT, "unknown key type %d", (int)type);
    if (op != FS_OP_SORT && op != FS_OP_ARGSORT && op != FS_OP_PAIRS)
        return set_err(s, FS_ERR_INVALID_ARGUMENT, "unknown op %d", (int)op);
    if (n >= (1ull << 32))
        return set_err(s, FS_ERR_INVALID_ARGUMENT, "n = %llu exceeds 2^32 - 1", (unsigned long long)n);
    HIP_TRY(s, hipSetDevice(s->device));
    return reserve(s, op, type, n);
}

fs_status fs_allow_scratch_growth(fs_sorter* s) {
    if (!s) return FS_ERR_INVALID_ARGUMENT;
    s->captured = false;
    return FS_OK;
}

fs_status fs_sorter_set_test_option(fs_sorter* s, fs_test_option opt, uint64_t value) {
    if (!s) return FS_ERR_INVALID_ARGUMENT;
    fs_status r = drain(s);
    if (r != FS_OK) return r;
    switch (opt) {
        case FS_TEST_WIDE_LOOKBACK: s->force_wide = value != 0; return FS_OK;
        case FS_TEST_FUSED:
            if (value > 2) return set_err(s, FS_ERR_INVALID_ARGUMENT, "fused mode %llu > 2", (unsigned long long)value);
            s->fused_mode = (uint32_t)value;
            return FS_OK;
        case FS_TEST_TOP16:
            if (value > 3) return set_err(s, FS_ERR_INVALID_ARGUMENT, "top-16 mode %llu > 3", (unsigned long long)value);
            s->top16_mode = (uint32_t)value;
            return FS_OK;
        case FS_TEST_LOCAL_WIDE:
            if (value > 1) return set_err(s, FS_ERR_INVALID_ARGUMENT, "local-sort block choice %llu > 1",
                                          (unsigned long long)value);
            s->local_wide_mode = (uint32_t)value;
            return FS_OK;
        case FS_TEST_SEG_BITS:
            if (value != 0 && (value < 8 || value > 16))
                return set_err(s, FS_ERR_INVALID_ARGUMENT, "segment bits %llu outside 8..16", (unsigned long long)value);
            s->seg_bits = (uint32_t)value;
            return FS_OK;
        case FS_TEST_UPSWEEP_BLOCKS_PER_CU:
            if (value > 64) return set_err(s, FS_ERR_INVALID_ARGUMENT, "upsweep blocks per CU %llu > 64",
                                           (unsigned long long)value);
            s->up_blocks_per_cu = (uint32_t)value;
            return FS_OK;
        case FS_TEST_INJECT_FAULT:
#ifdef FS_FAULT_INJECTION
            if (value > FS_FAULT_SMALL_S1) return set_err(s, FS_ERR_INVALID_ARGUMENT, "unknown fault %llu",
                                                           (unsigned long long)value);
            s->fault = (uint32_t)value;
            return FS_OK;
#else
            return set_err(s, FS_ERR_INVALID_ARGUMENT, "fault injection is not compiled into this library");
#endif
    }
    return set_err(s, FS_ERR_INVALID_ARGUMENT, "unknown test option %d", (int)opt);
}

fs_status fs_synchronize(fs_sorter* s) {
    if (!s) return FS_ERR_INVALID_ARGUMENT;
    HIP_TRY(s, hipSetDevice(s->device));
    return sync_and_check(s);
}

fs_status fs_sort_buffer(fs_sorter* s, fs_key_type type, void* device_keys, uint64_t n) {
    fs_status r = fs_encode(s, FS_OP_SORT, type, device_keys, nullptr, n, nullptr);
    if (r != FS_OK) return r;
    return sync_and_check(s);
}

fs_status fs_argsort_buffer(fs_sorter* s, fs_key_type type, const void* device_keys, uint64_t n,
                            uint32_t* device_indices) {
    fs_status r = fs_encode(s, FS_OP_ARGSORT, type, (void*)device_keys, device_indices, n, nullptr);
    if (r != FS_OK) return r;
    return sync_and_check(s);
}

fs_status fs_sort_pairs_buffer(fs_sorter* s, fs_key_type type, void* device_keys, uint32_t* device_values,
                               uint64_t n) {
    fs_status r = fs_encode(s, FS_OP_PAIRS, type, device_keys, device_values, n, nullptr);
    if (r != FS_OK) return r;
    return sync_and_check(s);
}

// Slice API staging: chunks of FS_PIN_CHUNK bytes through two pinned host
// buffers, so that the CPU copy of one chunk overlaps the DMA of the other (a
// pageable hipMemcpy stages through the runtime's own buffers one piece at a
// time).
#ifndef FS_PIN_CHUNK
#define FS_PIN_CHUNK (8u << 20)
#endif
static fs_status ensure_pinned(fs_sorter* s) {
    for (int b = 0; b < 2; ++b) {
        if (!s->pin[b]) HIP_TRY(s, hipHostMalloc(&s->pin[b], FS_PIN_CHUNK, hipHostMallocDefault));
        if (!s->pin_ev[b]) HIP_TRY(s, hipEventCreate(&s->pin_ev[b]));
    }
    return FS_OK;
}
static fs_status stage_to_device(fs_sorter* s, void* dev, const void* host, size_t bytes) {
    for (size_t off = 0, i = 0; off < bytes; off += FS_PIN_CHUNK, ++i) {
        const size_t len = bytes - off < FS_PIN_CHUNK ? bytes - off : FS_PIN_CHUNK;
        const int b = (int)(i & 1);
        // The last DMA out of pin[b] (this call's or an earlier staging call's)
        // must be done before the CPU overwrites it.
        if (s->pin_busy[b]) HIP_TRY(s, hipEventSynchronize(s->pin_ev[b]));
        s->pin_busy[b] = false;
        memcpy(s->pin[b], (const char*)host + off, len);
        HIP_TRY(s, hipMemcpyAsync((char*)dev + off, s->pin[b], len, hipMemcpyHostToDevice, s->stream));
        HIP_TRY(s, hipEventRecord(s->pin_ev[b], s->stream));
        s->pin_busy[b] = true;
    }
    return FS_OK;
}
static fs_status stage_to_host(fs_sorter* s, void* host, const void* dev, size_t bytes) {
    const size_t chunks = (bytes + FS_PIN_CHUNK - 1) / FS_PIN_CHUNK;
    auto issue = [&](size_t i) -> fs_status {
        const size_t off = i * FS_PIN_CHUNK;
        const size_t len = bytes - off < FS_PIN_CHUNK ? bytes - off : FS_PIN_CHUNK;
        // stream order puts this DMA after any earlier one that reads pin[i & 1]
        HIP_TRY(s, hipMemcpyAsync(s->pin[i & 1], (const char*)dev + off, len, hipMemcpyDeviceToHost, s->stream));
        HIP_TRY(s, hipEventRecord(s->pin_ev[i & 1], s->stream));
        s->pin_busy[i & 1] = true;
        return FS_OK;
    };
    fs_status r;
    for (size_t i = 0; i < chunks && i < 2; ++i)
        if ((r = issue(i)) != FS_OK) return r;
    for (size_t i = 0; i < chunks; ++i) {
        const size_t off = i * FS_PIN_CHUNK;
        const size_t len = bytes - off < FS_PIN_CHUNK ? bytes - off : FS_PIN_CHUNK;
        HIP_TRY(s, hipEventSynchronize(s->pin_ev[i & 1]));
        s->pin_busy[i & 1] = false;
        memcpy((char*)host + off, s->pin[i & 1], len);
        if (i + 2 < chunks && (r = issue(i + 2)) != FS_OK) return r;
    }
    return FS_OK;
}

// Slice API: stage through the sorter's own device buffers, like the
// reference's memcpy into buf_a (lib.rs:800-806) and back (:828-834).
static fs_status host_op(fs_sorter* s, fs_op op, fs_key_type type, void* keys, uint32_t* vals, uint64_t n) {
    if (!s) return FS_ERR_INVALID_ARGUMENT;
    if (!valid_type(type)) return set_err(s, FS_ERR_INVALID_ARGUMENT, "unknown key type %d", (int)type);
    if (n >= (1ull << 32))
        return set_err(s, FS_ERR_INVALID_ARGUMENT, "n = %llu exceeds 2^32 - 1", (unsigned long long)n);
    if (n == 0) return FS_OK;
    if (!keys || (op != FS_OP_SORT && !vals)) return set_err(s, FS_ERR_INVALID_ARGUMENT, "null pointer");
    if (n == 1) {
        if (op == FS_OP_ARGSORT) vals[0] = 0;
        return FS_OK;
    }
    HIP_TRY(s, hipSetDevice(s->device));
    fs_status r = drain(s);
    if (r != FS_OK) return r;
    const size_t kb = key_bytes(type);
    if ((r = ensure(s, s->iok, n * kb, false)) != FS_OK) return r;
    if (op != FS_OP_SORT && (r = ensure(s, s->iov, n * 4, false)) != FS_OK) return r;
    if ((r = ensure_pinned(s)) != FS_OK) return r;
    if ((r = stage_to_device(s, s->iok.p, keys, n * kb)) != FS_OK) return r;
    if (op == FS_OP_PAIRS && (r = stage_to_device(s, s->iov.p, vals, n * 4)) != FS_OK) return r;
    if ((r = enqueue(s, op, type, s->iok.p, (uint32_t*)s->iov.p, n, s->stream)) != FS_OK) return r;
    if (op != FS_OP_ARGSORT && (r = stage_to_host(s, keys, s->iok.p, n * kb)) != FS_OK) return r;
    if (op != FS_OP_SORT && (r = stage_to_host(s, vals, s->iov.p, n * 4)) != FS_OK) return r;
    return sync_and_check(s);
}

fs_status fs_sort(fs_sorter* s, fs_key_type type, void* host_keys, uint64_t n) {
    return host_op(s, FS_OP_SORT, type, host_keys, nullptr, n);
}

fs_status fs_argsort(fs_sorter* s, fs_key_type type, const void* host_keys, uint64_t n, uint32_t* host_indices) {
    return host_op(s, FS_OP_ARGSORT, type, (void*)host_keys, host_indices, n);
}

fs_status fs_sort_pairs(fs_sorter* s, fs_key_type type, void* host_keys, uint64_t n_keys, uint32_t* host_values,
                        uint64_t n_values) {
    if (!s) return FS_ERR_INVALID_ARGUMENT;
    if (n_keys != n_values)   // lib.rs:1928-1934, checked before any GPU work
        return set_err(s, FS_ERR_LENGTH_MISMATCH, "length mismatch: keys=%llu, values=%llu",
                       (unsigned long long)n_keys, (unsigned long long)n_values);
    return host_op(s, FS_OP_PAIRS, type, host_keys, host_values, n_keys);
}

fs_status fs_last_pass_info(fs_sorter* s, uint32_t* n_passes, uint32_t* digit_mask) {
    if (!s) return FS_ERR_INVALID_ARGUMENT;
    fs_status r = drain(s);
    if (r != FS_OK) return r;
    uint32_t w[FS_PLAN_WORDS];
    HIP_TRY(s, hipMemcpy(w, s->last_plan ? s->last_plan : s->plan, sizeof w, hipMemcpyDeviceToHost));
    if (n_passes) *n_passes = w[FS_PLAN_NPASSES];
    if (digit_mask) *digit_mask = w[FS_PLAN_MASK] & ((1u << FS_MAX_DIGITS) - 1u);
    return FS_OK;
}

fs_status fs_sorter_first_pass(fs_sorter* s, uint32_t* kind) {
    if (!s || !kind) return FS_ERR_INVALID_ARGUMENT;
    fs_status r = drain(s);
    if (r != FS_OK) return r;
    uint32_t w[FS_PLAN_WORDS];
    HIP_TRY(s, hipMemcpy(w, s->last_plan ? s->last_plan : s->plan, sizeof w, hipMemcpyDeviceToHost));
    const uint32_t mask = w[FS_PLAN_MASK];
    if (s->last_top16 && (mask & FS_MASK_TOP16))
        *kind = w[FS_PLAN_RESCATTER] ? 4u : 3u;
    else
        *kind = !s->last_fused ? 0u : ((mask & FS_MASK_FUSED) && !w[FS_PLAN_RESCATTER]) ? 1u : 2u;
    return FS_OK;
}

fs_status fs_set_lookback_stats(fs_sorter* s, int enable) {
    if (!s) return FS_ERR_INVALID_ARGUMENT;
    fs_status r = drain(s);
    if (r != FS_OK) return r;
    s->stats_on = enable != 0;
    return FS_OK;
}

fs_status fs_read_lookback_stats(fs_sorter* s, uint64_t out[4]) {
    if (!s || !out) return FS_ERR_INVALID_ARGUMENT;
    fs_status r = drain(s);
    if (r != FS_OK) return r;
    uint64_t slots[FS_STAT_SLOTS * FS_STAT_COUNT];
    HIP_TRY(s, hipMemcpy(slots, s->stats, sizeof slots, hipMemcpyDeviceToHost));
    HIP_TRY(s, hipMemset(s->stats, 0, sizeof slots));
    for (int c = 0; c < FS_STAT_COUNT; ++c) {
        out[c] = 0;
        for (int k = 0; k < FS_STAT_SLOTS; ++k) out[c] += slots[k * FS_STAT_COUNT + c];
    }
    return FS_OK;
}

fs_status fs_set_profiling(fs_sorter* s, int enable) {
    if (!s) return FS_ERR_INVALID_ARGUMENT;
    fs_status r = drain(s);
    if (r != FS_OK) return r;
    recycle_profile(s);
    s->profiling = enable != 0;
    return FS_OK;
}

fs_status fs_profile_reset(fs_sorter* s) {
    if (!s) return FS_ERR_INVALID_ARGUMENT;
    fs_status r = drain(s);
    if (r != FS_OK) return r;
    recycle_profile(s);
    return FS_OK;
}

int fs_profile_count(fs_sorter* s) { return s ? (int)s->prof.size() : 0; }

fs_status fs_profile_read(fs_sorter* s, int index, const char** kernel_name, float* ms) {
    if (!s || index < 0 || index >= (int)s->prof.size()) return FS_ERR_INVALID_ARGUMENT;
    fs_status r = drain(s);
    if (r != FS_OK) return r;
    const ProfEntry& p = s->prof[index];
    if (kernel_name) *kernel_name = p.name;
    if (ms) {
        *ms = 0.f;
        if (p.start && p.stop) HIP_TRY(s, hipEventElapsedTime(ms, p.start, p.stop));
    }
    return FS_OK;
}

// ---------------------------------------------------------------------------
// GpuGather (forge-runtime/src/gather.rs:26-173): output[i] = source[indices[i]]
// for u32 or u64 elements, with its own stream (or the caller's) and the same
// code object as the sorter.
// ---------------------------------------------------------------------------

struct fs_gather {
    int device = 0;
    hipStream_t stream = nullptr;
    bool own_stream = false;
    hipModule_t module = nullptr;
    hipFunction_t fn = nullptr;
    uint32_t* status = nullptr;     // host-visible error bits (hipHostMalloc)
    int num_cus = 256;
    hipStream_t last_stream = nullptr;
    bool pending = false;
    std::string err;
};

static fs_status gather_err(fs_gather* g, fs_status st, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (g) g->err = display(st, buf);
    return st;
}

#define GATHER_TRY(g, call)                                                                \
    do {                                                                                   \
        hipError_t e_ = (call);                                                            \
        if (e_ != hipSuccess)                                                              \
            return gather_err((g), FS_ERR_GPU_EXECUTION, "%s: %s", #call, hipGetErrorString(e_)); \
    } while (0)

static fs_status gather_create(int device, hipStream_t stream, bool own, fs_gather** out) {
    if (!out) return create_failed(nullptr, FS_ERR_INVALID_ARGUMENT, "null output pointer");
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0 || device < 0 || device >= count) {
        (void)hipGetLastError();
        return create_failed(nullptr, FS_ERR_DEVICE_NOT_FOUND, "");
    }
    fs_gather* g = new (std::nothrow) fs_gather();
    if (!g) return create_failed(nullptr, FS_ERR_OUT_OF_MEMORY, "host allocation of the gather");
    g->device = device;
    hipError_t e = hipSetDevice(device);
    int cus = 0;
    if (e == hipSuccess && hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess &&
        cus > 0)
        g->num_cus = cus;
    if (e == hipSuccess && own) {
        e = hipStreamCreateWithFlags(&g->stream, hipStreamNonBlocking);
        g->own_stream = e == hipSuccess;
    } else if (e == hipSuccess) {
        g->stream = stream;
    }
    g->last_stream = g->stream;
    const std::string path = code_object_path();
    if (e == hipSuccess) e = hipModuleLoad(&g->module, path.c_str());
    if (e == hipSuccess) e = hipModuleGetFunction(&g->fn, g->module, "fs_gather_elems");
    if (e == hipSuccess) e = hipHostMalloc((void**)&g->status, sizeof(uint32_t), hipHostMallocDefault);
    if (e != hipSuccess) {
        const std::string msg = "loading " + path + ": " + hipGetErrorString(e);
        fs_gather_free(g);
        return create_failed(nullptr, FS_ERR_SHADER_COMPILATION, msg);
    }
    *g->status = 0;
    *out = g;
    return FS_OK;
}

fs_status fs_gather_new(int device, fs_gather** out) { return gather_create(device, nullptr, true, out); }

fs_status fs_gather_with_context(int device, void* hip_stream, fs_gather** out) {
    return gather_create(device, (hipStream_t)hip_stream, false, out);
}

void fs_gather_free(fs_gather* g) {
    if (!g) return;
    (void)hipSetDevice(g->device);
    if (g->pending) (void)hipStreamSynchronize(g->last_stream);
    if (g->status) (void)hipHostFree(g->status);
    if (g->module) (void)hipModuleUnload(g->module);
    if (g->own_stream && g->stream) (void)hipStreamDestroy(g->stream);
    delete g;
}

const char* fs_gather_last_error(const fs_gather* g) { return g ? g->err.c_str() : g_create_err.c_str(); }

fs_status fs_gather_alloc_buffer(fs_gather* g, size_t bytes, void** device_ptr) {
    if (!g || !device_ptr) return FS_ERR_INVALID_ARGUMENT;
    *device_ptr = nullptr;
    GATHER_TRY(g, hipSetDevice(g->device));
    if (hipMalloc(device_ptr, bytes ? bytes : 1) != hipSuccess) {
        (void)hipGetLastError();
        *device_ptr = nullptr;
        return gather_err(g, FS_ERR_OUT_OF_MEMORY, "hipMalloc(%zu) failed", bytes);
    }
    return FS_OK;
}

fs_status fs_gather_free_buffer(fs_gather* g, void* device_ptr) {
    if (!g) return FS_ERR_INVALID_ARGUMENT;
    if (device_ptr) GATHER_TRY(g, hipFree(device_ptr));
    return FS_OK;
}

fs_status fs_gather_encode(fs_gather* g, int is_64bit, const void* source, uint64_t source_len,
                           const uint32_t* indices, void* output, uint64_t count, void* hip_stream) {
    if (!g) return FS_ERR_INVALID_ARGUMENT;
    if (count == 0) return FS_OK;
    if (!source || !indices || !output)
        return gather_err(g, FS_ERR_INVALID_ARGUMENT, "null device pointer");
    if (count >= (1ull << 32) || source_len > (1ull << 32))
        return gather_err(g, FS_ERR_INVALID_ARGUMENT, "count or source length beyond u32 indices");
    GATHER_TRY(g, hipSetDevice(g->device));
    hipStream_t st = hip_stream ? (hipStream_t)hip_stream : g->stream;
    if (g->pending && g->last_stream != st) GATHER_TRY(g, hipStreamSynchronize(g->last_stream));
    uint64_t blocks = (count + 255) / 256;
    if (blocks > (uint64_t)g->num_cus * 16) blocks = (uint64_t)g->num_cus * 16;
    uint64_t src = (uint64_t)(uintptr_t)source, idx = (uint64_t)(uintptr_t)indices;
    uint64_t dst = (uint64_t)(uintptr_t)output, stat = (uint64_t)(uintptr_t)g->status;
    uint32_t is64 = is_64bit ? 1u : 0u;
    void* args[] = {&src, &source_len, &idx, &dst, &count, &is64, &stat};
    GATHER_TRY(g, hipModuleLaunchKernel(g->fn, (unsigned)blocks, 1, 1, 256, 1, 1, 0, st, args, nullptr));
    g->last_stream = st;
    g->pending = true;
    return FS_OK;
}

fs_status fs_gather_synchronize(fs_gather* g) {
    if (!g) return FS_ERR_INVALID_ARGUMENT;
    GATHER_TRY(g, hipSetDevice(g->device));
    if (g->pending) GATHER_TRY(g, hipStreamSynchronize(g->last_stream));
    g->pending = false;
    const uint32_t st = __atomic_load_n(g->status, __ATOMIC_ACQUIRE);
    if (st) {
        __atomic_store_n(g->status, 0u, __ATOMIC_RELEASE);
        if (st & FS_DEVERR_GATHER_INDEX)
            return gather_err(g, FS_ERR_GPU_EXECUTION, "gather index out of range of the source");
        return gather_err(g, FS_ERR_GPU_EXECUTION, "device status 0x%x", st);
    }
    return FS_OK;
}

fs_status fs_gather_u32(fs_gather* g, const uint32_t* source, uint64_t source_len, const uint32_t* indices,
                        uint32_t* output, uint64_t count) {
    fs_status r = fs_gather_encode(g, 0, source, source_len, indices, output, count, nullptr);
    return r != FS_OK ? r : fs_gather_synchronize(g);
}

fs_status fs_gather_u64(fs_gather* g, const uint64_t* source, uint64_t source_len, const uint32_t* indices,
                        uint64_t* output, uint64_t count) {
    fs_status r = fs_gather_encode(g, 1, source, source_len, indices, output, count, nullptr);
    return r != FS_OK ? r : fs_gather_synchronize(g);
}

}  // extern "C"
