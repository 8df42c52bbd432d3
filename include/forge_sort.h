/*
 * forge_sort.h -- C ABI of the MI355X (gfx950) forge-sort radix sort.
 *
 * Drop-in boundary for forge-sort's GpuSorter
 * (metal-forge-compute/forge-sort/src/lib.rs).  Each entry point names the
 * Rust API it replaces; a Rust/ctypes binding maps them 1:1.  All pointers are
 * plain host or device addresses and all sizes are element counts unless the
 * name says bytes.  No HIP or torch types appear here: a HIP stream is passed
 * as `void*` (a hipStream_t; NULL = the sorter's own stream).
 *
 * Semantics kept from the reference:
 *   - sorts are ascending; floats follow the IEEE total order of Rust's
 *     f32/f64::total_cmp (-NaN < -inf < ... < -0.0 < +0.0 < ... < +inf < +NaN)
 *     by the FloatFlip transform (shaders/sort.metal:812-868);
 *   - n <= 1 returns FS_OK with no GPU work (lib.rs:710-712, :1677-1682);
 *   - pairs check the lengths before any work (lib.rs:1928-1934);
 *   - n is limited to 2^32 - 1 (u32 counts and indices, lib.rs:106-130);
 *   - one call at a time per sorter (&mut self in Rust): not thread-safe.
 * Stronger than the reference: argsort and pairs are stable (ties keep their
 * original index order) and deterministic.
 */
#ifndef FORGE_SORT_H
#define FORGE_SORT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* SortError (lib.rs:94-104) as status codes; the message of the last failure
 * is available from fs_last_error(). */
typedef enum fs_status {
    FS_OK = 0,
    FS_ERR_DEVICE_NOT_FOUND = 1,    /* SortError::DeviceNotFound */
    FS_ERR_SHADER_COMPILATION = 2,  /* SortError::ShaderCompilation: code object missing or not loadable */
    FS_ERR_GPU_EXECUTION = 3,       /* SortError::GpuExecution: any HIP runtime or kernel failure */
    FS_ERR_LENGTH_MISMATCH = 4,     /* SortError::LengthMismatch{keys, values} */
    FS_ERR_INVALID_ARGUMENT = 5,    /* null pointer, n >= 2^32, unknown key type (Rust's types rule these out) */
    FS_ERR_OUT_OF_MEMORY = 6        /* allocation failure (the reference panics, metal_helpers.rs:194-202) */
} fs_status;

/* SortKey implementations (lib.rs:42-88). */
typedef enum fs_key_type {
    FS_KEY_U32 = 0,
    FS_KEY_I32 = 1,
    FS_KEY_F32 = 2,
    FS_KEY_U64 = 3,
    FS_KEY_I64 = 4,
    FS_KEY_F64 = 5
} fs_key_type;

/* Operation for fs_encode (the three families of GpuSorter calls). */
typedef enum fs_op {
    FS_OP_SORT = 0,      /* sort_<t> / sort_buffer: keys in place */
    FS_OP_ARGSORT = 1,   /* argsort_<t>: keys untouched, u32 indices out */
    FS_OP_PAIRS = 2      /* sort_pairs_<t>: keys and u32 values in place */
} fs_op;

/* GpuSorter (lib.rs:132-154): device, stream, loaded code object, grow-only scratch. */
typedef struct fs_sorter fs_sorter;

/* ---- construction ---------------------------------------------------------- */

/* GpuSorter::new (lib.rs:596-599).  Uses HIP device `device` and a stream the
 * sorter owns.  Loads the gfx950 code object (hipModuleLoad). */
fs_status fs_sorter_new(int device, fs_sorter **out);

/* GpuSorter::with_context (lib.rs:606-686).  Uses the caller's HIP stream
 * (`hip_stream`, not owned; NULL = the default stream) on `device`.
 *
 * Forward progress.  A digit pass is one launch of one block per tile whose
 * tiles chain their digit counts through a decoupled look-back: a tile waits
 * (a bounded spin) until the tiles before it have published theirs.  This
 * assumes what the hardware dispatcher does when the launch has the device
 * to itself: on each XCD the launch's blocks start in increasing tile order,
 * so the smallest unfinished tile is always running or next to start, and a
 * wait always ends.  Kernels the caller runs at the same time on other
 * streams that hold every slot of one XCD for long can stall the tiles
 * dealt to that XCD; the tiles waiting on them give up after FS_SPIN_LIMIT
 * polls (2^24, seconds), and the sort then ends with FS_ERR_GPU_EXECUTION
 * ("look-back wait exceeded its spin bound") at the next synchronizing call,
 * its output unspecified.  Sorts of one sorter, and anything ordered with
 * them on one stream, never wait on each other. */
fs_status fs_sorter_with_context(int device, void *hip_stream, fs_sorter **out);

/* Drop for GpuSorter: frees scratch, unloads the module, destroys an owned stream. */
void fs_sorter_free(fs_sorter *s);

/* The message of the last failing call (SortError's Display text, lib.rs:94-104).
 * With s == NULL: why the last fs_sorter_new / fs_sorter_with_context on this
 * thread failed. */
const char *fs_last_error(const fs_sorter *s);

/* Display text of a status code. */
const char *fs_status_str(fs_status st);

/* ---- SortBuffer (lib.rs:160-281, alloc_sort_buffer :694-702) --------------- */

/* alloc_sort_buffer<T>(capacity): device memory for `capacity` keys of `type`. */
fs_status fs_alloc_sort_buffer(fs_sorter *s, fs_key_type type, size_t capacity, void **device_ptr);

/* Drop for SortBuffer<T>. */
fs_status fs_free_sort_buffer(fs_sorter *s, void *device_ptr);

/* SortBuffer::copy_from_slice (lib.rs:213-228): host -> device, synchronous. */
fs_status fs_copy_to_device(fs_sorter *s, void *device_dst, const void *host_src, size_t bytes);

/* SortBuffer::copy_to_slice / as_slice (lib.rs:195-241): device -> host, synchronous. */
fs_status fs_copy_to_host(fs_sorter *s, void *host_dst, const void *device_src, size_t bytes);

/* Device -> device copy of `bytes`, synchronous (staging fresh inputs in HBM). */
fs_status fs_copy_device(fs_sorter *s, void *device_dst, const void *device_src, size_t bytes);

/* ---- slice API: host arrays (copies in and out, like lib.rs:791-838) ------- */
/* The copies stage through two 8 MiB pinned host buffers that the sorter
 * allocates on its first slice call and frees in fs_sorter_free; the caller's
 * arrays need not be pinned or aligned. */

/* sort_u32 :791, sort_i32 :840, sort_f32 :920, sort_u64 :2238, sort_i64 :2348, sort_f64 :2417 */
fs_status fs_sort(fs_sorter *s, fs_key_type type, void *host_keys, uint64_t n);

/* argsort_u32 :1675, argsort_i32 :1754, argsort_f32 :1838, argsort_u64 :2595,
 * argsort_i64 :2669, argsort_f64 :2747.  host_indices receives n u32 indices. */
fs_status fs_argsort(fs_sorter *s, fs_key_type type, const void *host_keys, uint64_t n,
                     uint32_t *host_indices);

/* sort_pairs_u32 :1923, sort_pairs_i32 :2024, sort_pairs_f32 :2132,
 * sort_pairs_u64 :2826, sort_pairs_i64 :2921 (f64 accepted as well). */
fs_status fs_sort_pairs(fs_sorter *s, fs_key_type type, void *host_keys, uint64_t n_keys,
                        uint32_t *host_values, uint64_t n_values);

/* ---- device-resident API ----------------------------------------------------- */

/* sort_buffer :708 (u32), sort_i32_buffer :1060, sort_f32_buffer :1000,
 * sort_u64_buffer :2301, sort_i64_buffer :2486, sort_f64_buffer :2540.
 * Sorts `n` keys at device_keys in place and waits for completion. */
fs_status fs_sort_buffer(fs_sorter *s, fs_key_type type, void *device_keys, uint64_t n);

/* Device-resident argsort (the reference only has the slice form): indices of
 * the stable ascending order into device_indices; keys are not modified. */
fs_status fs_argsort_buffer(fs_sorter *s, fs_key_type type, const void *device_keys, uint64_t n,
                            uint32_t *device_indices);

/* Device-resident pairs sort (the reference only has the slice form). */
fs_status fs_sort_pairs_buffer(fs_sorter *s, fs_key_type type, void *device_keys,
                               uint32_t *device_values, uint64_t n);

/* encode_sort (lib.rs:749-785), generalised to every op and key type: enqueue
 * the sort on `hip_stream` (NULL = the sorter's stream) and return without
 * waiting.  For FS_OP_ARGSORT `device_values` is the index output and
 * `device_keys` is read only; for FS_OP_SORT `device_values` is ignored.
 * Errors detected on the device are reported by the next fs_synchronize.
 * The forward-progress assumption of fs_sorter_with_context holds here too:
 * work on other streams that occupies a whole XCD for long while the sort
 * runs can make it fail with FS_ERR_GPU_EXECUTION after the spin bound.
 *
 * HIP graph capture: fs_encode on a capturing stream records kernel launches
 * only (no memset, no allocation).  The graph then holds the addresses of the
 * sorter's scratch (ping-pong buffers, look-back arrays, histogram, schedule),
 * so from that call on the sorter refuses to grow its scratch
 * (FS_ERR_INVALID_ARGUMENT), the captured sort included: reserve capacity with
 * fs_reserve before capturing.  Graphs must be destroyed before
 * fs_sorter_free, and fs_allow_scratch_growth re-enables growth once they are.
 * A replay uses the same scratch as the sorter's eager sorts: launch replays
 * on the sorter's stream (or order them with its other work). */
fs_status fs_encode(fs_sorter *s, fs_op op, fs_key_type type, void *device_keys,
                    uint32_t *device_values, uint64_t n, void *hip_stream);

/* fs_encode for callers that cannot allocate: code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc.  No counterpart in the
 * reference.  Same arguments and results as fs_encode, but every scratch
 * buffer of the sort (histogram, bin-base and schedule tables, look-back
 * arrays, key and value ping-pong buffers) lives in a static array of the
 * loaded code object (FS_NO_ALLOC_SCRATCH_BYTES, held by each sorter until
 * fs_sorter_free), so the call allocates and frees nothing and never grows
 * anything: n is limited to FS_NO_ALLOC_MAX_KEYS keys of any type and op
 * (FS_ERR_INVALID_ARGUMENT beyond).  Every call through one sorter uses the
 * same array and finds the last call's contents in it (the kernels leave the
 * tables cleared for the next sort): calls through one sorter that overlap on
 * the device race, so issue them on one stream or order them.  fs_encode's
 * scratch is separate. */
#define FS_NO_ALLOC_MAX_KEYS 1048576u
#define FS_NO_ALLOC_SCRATCH_BYTES 25534464u   /* 24.4 MiB with the gfx950 tile geometry */
fs_status fs_encode_no_alloc(fs_sorter *s, fs_op op, fs_key_type type, void *device_keys,
                             uint32_t *device_values, uint64_t n, void *hip_stream);

/* Grow the sorter's scratch for sorts of up to n keys of `type` with `op`
 * (the grow-only ensure_buffers*, lib.rs:1120-1289, done ahead of time), e.g.
 * before capturing a sort into a HIP graph.  Synchronous. */
fs_status fs_reserve(fs_sorter *s, fs_op op, fs_key_type type, uint64_t n);

/* Lift the no-growth rule a captured sort imposes (see fs_encode); call only
 * once every graph that captured a sort of this sorter has been destroyed.
 * No counterpart in the reference (Metal has no graph capture). */
fs_status fs_allow_scratch_growth(fs_sorter *s);

/* Wait for the sorter's stream (and the last encode's stream); report device errors. */
fs_status fs_synchronize(fs_sorter *s);

/* Wait for all work on the sorter's device (hipDeviceSynchronize); report device errors. */
fs_status fs_device_synchronize(fs_sorter *s);

/* ---- introspection -------------------------------------------------------------- */

/* Facts about the last completed sort: number of digit passes that ran and the
 * bitmask of digit positions that were not constant (the rest were skipped). */
fs_status fs_last_pass_info(fs_sorter *s, uint32_t *n_passes, uint32_t *digit_mask);

/* Kernel timing (the role of forge-primitives' GpuTimer, timing.rs:40-48):
 * when enabled, every launch is bracketed by HIP events on the stream it runs
 * on.  Launches accumulate until fs_profile_reset (or re-enabling);
 * fs_profile_read waits for them and returns each launch's kernel symbol and
 * duration in ms. */
fs_status fs_set_profiling(fs_sorter *s, int enable);
fs_status fs_profile_reset(fs_sorter *s);
int fs_profile_count(fs_sorter *s);
fs_status fs_profile_read(fs_sorter *s, int index, const char **kernel_name, float *ms);

/* Decoupled look-back counters of the digit passes, summed over every sort
 * since the last read: {tiles that looked back, round trips (per digit),
 * rounds that met an unpublished predecessor, predecessor entries consumed}.
 * Off by default; reading resets them. */
fs_status fs_set_lookback_stats(fs_sorter *s, int enable);
fs_status fs_read_lookback_stats(fs_sorter *s, uint64_t counters[4]);

/* Keys per tile of the digit-pass kernels compiled into the loaded code
 * object: [u32 keys, u32 keys + values, u64 keys, u64 keys + values]. */
fs_status fs_tile_config(const fs_sorter *s, uint32_t keys_per_tile[4]);

/* ---- testing hooks (no counterpart in the reference) ---------------------------
 * Layout switches that let tests reach code paths the product takes only at
 * sizes too large for a test, and (in CPU-emulator builds compiled with
 * FS_FAULT_INJECTION only) injected faults that drive the device-side error
 * guards.  The product never reads the environment for these; the defaults
 * give the normal layout.  Not for production use. */
typedef enum fs_test_option {
    FS_TEST_WIDE_LOOKBACK = 0,          /* value != 0: 64-bit look-back entries for any n */
    FS_TEST_UPSWEEP_BLOCKS_PER_CU = 1,  /* histogram blocks per CU, 1..64 (0 = by key width) */
    FS_TEST_INJECT_FAULT = 2,           /* FS_FAULT_* (fault-injection builds only) */
    FS_TEST_FUSED = 3,                  /* keys-only sorts begin with the fused first pass:
                                           0 = from FS_FUSED_MIN_KEYS keys on (the default),
                                           1 = never, 2 = at every size */
    FS_TEST_TOP16 = 4,                  /* keys-only u32/i32/u64/i64 sorts take the top-16 launch sequence:
                                           0 = from FS_TOP16_MIN_KEYS32/64 keys on (the default),
                                           1 = never, 2 = at every size of at least 2 keys and
                                           on the top-16 path even where its region sample
                                           estimates oversized segments, 3 = at every size,
                                           the sample choosing as by default */
    FS_TEST_SEG_BITS = 5,               /* top-16 path: 0 = segment bits by size (the default),
                                           8..16 = segments named by that many top bits */
    FS_TEST_LOCAL_WIDE = 6              /* top-16 path: 0 = wide local-sort blocks by size (the
                                           default: beyond the other blocks' size limit),
                                           1 = wide blocks at every size */
} fs_test_option;
fs_status fs_sorter_set_test_option(fs_sorter *s, fs_test_option opt, uint64_t value);

/* Keys-only sorts (any key type) from this many keys on (up to 2^31) begin
 * with the fused first pass; below it the histogram read and the first
 * digit pass cost less than the fused pass and the region read after it
 * (measured for u32 and u64 keys). */
#define FS_FUSED_MIN_KEYS 33554432u

/* Keys-only u32 and i32 sorts from FS_TOP16_MIN_KEYS32 keys on, u64 and i64
 * sorts from FS_TOP16_MIN_KEYS64 keys on, up to 2^16 times the keys a wide
 * local-sort block holds less five standard deviations (gfx950 build:
 * 572,522,496 32-bit keys with 9,216-key blocks, 280,035,328 64-bit keys with
 * 4,608-key blocks; up to 280,035,328 and 135,266,304 keys the blocks of half
 * that size sort the segments, at lower cost per key), take the top-16 path: the fused first pass on the byte
 * below the highest, one stable pass on the highest byte, then a local sort of
 * every segment of keys that share their top bits, in LDS - three reads and
 * writes of the keys instead of four (32-bit keys) or eight (64-bit keys).
 * Float keys keep the LSD passes (their exponent bytes make segments too large
 * for one block), and so does an input whose region sample shows a segment of
 * more than 16 blocks' keys (constant or skewed top bytes): the same launches
 * then run the fused pass on the lowest byte and the stable passes on the
 * others.  The thresholds are where the path measured faster than the LSD
 * passes on one MI355X for uniform keys (32-bit keys: between 41.9M and 46.1M
 * keys; 64-bit keys: between 65,536 and 131,072, taken at 2^21, where the
 * launches of the sequence that a refused input leaves idle cost less than the
 * path gains). */
#define FS_TOP16_MIN_KEYS32 44040192u
#define FS_TOP16_MIN_KEYS64 2097152u

/* How the last completed sort began: 0 = the histogram read (argsort, pairs,
 * and keys-only sorts outside the fused range), 1 = the fused first pass of a
 * keys-only sort, its regions read by the next pass,
 * 2 = the fused first pass after a region overflowed (the keys re-scattered
 * into exact regions by its second launch), or every digit constant (no
 * pass after it),
 * 3 = the top-16 path (fused pass on the second-highest byte, its regions
 * read by the pass on the highest byte, then the local sort),
 * 4 = the top-16 path after a region of its fused pass overflowed (the keys
 * re-scattered into exact regions by a second launch of the fused pass). */
fs_status fs_sorter_first_pass(fs_sorter *s, uint32_t *kind);

/* ---- GpuGather (forge-runtime/src/gather.rs:26-173) --------------------------
 * output[i] = source[indices[i]] for u32 or u64 elements, u32 indices
 * (shaders/gather.metal:5-27).  The reference reads past the source for an
 * index out of range; here the source length is passed, such an element comes
 * out 0, and the next fs_gather_synchronize reports FS_ERR_GPU_EXECUTION. */
typedef struct fs_gather fs_gather;

/* GpuGather::new (gather.rs:38-46): device `device`, a stream of its own. */
fs_status fs_gather_new(int device, fs_gather **out);

/* GpuGather::with_context (gather.rs:49-72): the caller's HIP stream (not owned). */
fs_status fs_gather_with_context(int device, void *hip_stream, fs_gather **out);

/* Drop for GpuGather. */
void fs_gather_free(fs_gather *g);

/* Message of the last failing call (NULL: the last failed fs_gather_new /
 * fs_gather_with_context on this thread). */
const char *fs_gather_last_error(const fs_gather *g);

/* GpuGather::alloc_buffer (gather.rs:169-173): device memory of `bytes`. */
fs_status fs_gather_alloc_buffer(fs_gather *g, size_t bytes, void **device_ptr);
fs_status fs_gather_free_buffer(fs_gather *g, void *device_ptr);

/* encode_gather (gather.rs:81-119): enqueue on hip_stream (NULL = the gather's
 * own) and return without waiting; `is_64bit` selects u64 elements. */
fs_status fs_gather_encode(fs_gather *g, int is_64bit, const void *source, uint64_t source_len,
                           const uint32_t *indices, void *output, uint64_t count, void *hip_stream);

/* Wait for the last encode; report an out-of-range index. */
fs_status fs_gather_synchronize(fs_gather *g);

/* gather_u32 (gather.rs:124-132) and gather_u64 (:135-143): encode and wait. */
fs_status fs_gather_u32(fs_gather *g, const uint32_t *source, uint64_t source_len, const uint32_t *indices,
                        uint32_t *output, uint64_t count);
fs_status fs_gather_u64(fs_gather *g, const uint64_t *source, uint64_t source_len, const uint32_t *indices,
                        uint64_t *output, uint64_t count);

#ifdef __cplusplus
}
#endif

#endif /* FORGE_SORT_H */
