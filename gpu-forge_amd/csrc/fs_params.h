// fs_params.h -- structures shared by the host runtime (forge_sort.cpp) and the
// gfx950 kernels (radix_kernels.hip).  Plain C layout, no HIP types.
#ifndef FS_PARAMS_H
#define FS_PARAMS_H

#include <stdint.h>

// Radix: 8-bit digits, 256 bins; 4 digits for 32-bit keys, 8 for 64-bit.
#define FS_RADIX_BITS 8
#define FS_RADIX 256
#define FS_MAX_DIGITS 8

// Digit-pass tiles: BLOCK threads (BLOCK/64 wave64s) x ITEMS keys per thread,
// per kernel variant.  The host reads the tile sizes from the code object
// (fs_kernel_tile_keys / fs_kernel_block_threads), so they are only defined here.
#ifndef FS_K32_BLOCK
#define FS_K32_BLOCK 768
#endif
#ifndef FS_K32_ITEMS
#define FS_K32_ITEMS 23
#endif
#ifndef FS_K32V_BLOCK
#define FS_K32V_BLOCK 768
#endif
#ifndef FS_K32V_ITEMS
#define FS_K32V_ITEMS 18
#endif
#ifndef FS_K64_BLOCK
#define FS_K64_BLOCK 768
#endif
#ifndef FS_K64_ITEMS
#define FS_K64_ITEMS 11
#endif
#ifndef FS_K64V_BLOCK
#define FS_K64V_BLOCK 768
#endif
#ifndef FS_K64V_ITEMS
#define FS_K64V_ITEMS 10
#endif
// Items whose LDS reads the staging and store loops keep in flight at once
// (0: all of a thread's items).  8 (two batches of the u32 tile's 23 items
// and a third of 7) measured 1% faster per u32 256M sort than all 23 at
// once, 4, 6, 10 and 12 in between.
#ifndef FS_STAGE_BATCH
#define FS_STAGE_BATCH 8
#endif
// Small tiles of the keys-only 32-bit digit pass: keys-only u32/i32/f32 sorts
// below FS_SMALL_TILE_KEYS keys on the LSD passes (not the fused or top-16
// launch sequences, whose kernels share the tiles above, nor the static
// scratch of fs_encode_no_alloc, laid out for them).  Below 2^21 keys a pass
// has too few 768 x 23-key tiles to fill the CUs.  u32 sorts (host-timed
// median, µs) with 768 x 12 / 8 / 6-key tiles: 65,536 keys 62.9 / 58.8 /
// 59.2, 2^18 66.0 / 62.8 / 61.6, 2^20 75.9 / 73.1 / 73.2, 2^21 - 1 87.6 /
// 90.1 / 91.0; 768 x 23 at 2^20 87.0, at 2^21 96.2 (from 2^23 keys on the
// larger tiles are faster).
#ifndef FS_K32S_BLOCK
#define FS_K32S_BLOCK 768
#endif
#ifndef FS_K32S_ITEMS
#define FS_K32S_ITEMS 8
#endif
#ifndef FS_SMALL_TILE_KEYS
#define FS_SMALL_TILE_KEYS (1u << 21)
#endif
// The same for 32-bit argsort and pairs (768 x 6 below 2^21 keys), and for
// 64-bit keys, with and without values (768 x 4 below FS_SMALL_TILE_KEYS64).
// Host-timed medians, µs, large / small tiles: u32 argsort 2^16 keys 81 / 61,
// 2^20 91 / 79, 2^21 - 1 100 / 93; u32 pairs 2^20 97 / 83, 2^21 - 1 104 / 95;
// u64 sort 2^16 108 / 90, 2^18 117 / 100, 2^20 149 / 142, 2^21 - 1 174 / 198;
// u64 argsort 2^18 125 / 106, 2^21 - 1 183 / 202; f64 pairs 2^18 128 / 108.
#ifndef FS_K32VS_ITEMS
#define FS_K32VS_ITEMS 6
#endif
#ifndef FS_K64S_ITEMS
#define FS_K64S_ITEMS 4
#endif
#ifndef FS_K64VS_ITEMS
#define FS_K64VS_ITEMS 4
#endif
#ifndef FS_KS_BLOCK
#define FS_KS_BLOCK 768
#endif
#ifndef FS_SMALL_TILE_KEYS64
#define FS_SMALL_TILE_KEYS64 (1u << 20)
#endif
// index into fs_kernel_tile_keys
#define FS_VAR_K32 0
#define FS_VAR_K32V 1
#define FS_VAR_K64 2
#define FS_VAR_K64V 3
#define FS_VAR_K32S 4      // the small tiles of each of the four
#define FS_VAR_K32VS 5
#define FS_VAR_K64S 6
#define FS_VAR_K64VS 7
#define FS_VARIANTS 8

// Histogram atomics: a wave whose lanes share one digit with at least
// FS_PEEL_MIN others adds that digit's lanes with one atomic.
#ifndef FS_PEEL_MIN
#define FS_PEEL_MIN 8
#endif

// Upsweep (all-digit histogram) block, and 16-byte loads in flight per lane.
#ifndef FS_HIST_BLOCK
#define FS_HIST_BLOCK 1024
#endif
#ifndef FS_UPSWEEP_UNROLL
#define FS_UPSWEEP_UNROLL 4
#endif
// Upsweep counter replicas (lanes with equal lane % replicas share a counter:
// 32 keeps every lane of a half-wave on its own LDS bank) and the vectors per
// lane between two folds of the 16-bit counters into the histogram.  64 KiB
// of LDS for both key widths.
#ifndef FS_UP_REPLICAS_K32
#define FS_UP_REPLICAS_K32 32
#endif
#ifndef FS_UP_REPLICAS_K64
#define FS_UP_REPLICAS_K64 16
#endif
#ifndef FS_UP_CHUNK_STEPS
#define FS_UP_CHUNK_STEPS 256
#endif

// Look-back tile entries, one per (tile, digit), in a single chain over all
// tiles: a 32-bit word [flag:2 | value:30] when n < FS_LB_WIDE_KEYS, else a
// 64-bit word whose high half holds the flag bits and low half the value (an
// inclusive prefix can then exceed 30 bits).  Counts of one tile or group are
// far below 2^30 either way.
#define FS_LB_AGG 0x40000000u
#define FS_LB_INC 0x80000000u
#define FS_LB_FLAGS 0xC0000000u
#define FS_LB_VALUE 0x3FFFFFFFu
#ifndef FS_LB_WIDE_KEYS
#define FS_LB_WIDE_KEYS (1u << 30)
#endif

// XCDs of the device and consecutive tiles given to one XCD by a digit pass's
// block-to-tile mapping.
#ifndef FS_XCDS
#define FS_XCDS 8
#endif
#ifndef FS_XCD_TILES
#define FS_XCD_TILES 8
#endif

// Predecessor tile entries read per look-back round trip.
#ifndef FS_LB_WINDOW
#define FS_LB_WINDOW 4
#endif
// Second look-back level: FS_LB_GROUP consecutive tiles (a power of two)
// share a group entry per digit holding
// (tiles added << FS_LB_GCOUNT_SHIFT) | sum of their counts; FS_LB_GWIN groups
// are read per round trip.  FS_LB_GROUP * tile keys < 2^24 keeps the sum in
// its field.
#ifndef FS_LB_GROUP
#define FS_LB_GROUP 16
#endif
// Two groups per round trip measured 0.5% faster per u32 256M sort than 4
// and 1 (with 8-item staging batches); a tile window of 4 entries against 3
// (equal) and 6 (slower).
#ifndef FS_LB_GWIN
#define FS_LB_GWIN 2
#endif
#define FS_LB_GCOUNT_SHIFT 24
#define FS_LB_GSUM 0x00FFFFFFu

// Bounded spin of a look-back wait (iterations of s_sleep(1), ~64 clocks each).
// A predecessor tile that owns a tile id is resident and finishes in
// microseconds; the bound only guarantees that every wait ends.  (The CPU
// emulator's fault-injection build sets a tiny bound.)
#ifndef FS_SPIN_LIMIT
#define FS_SPIN_LIMIT (1u << 24)
#endif

// Per-pass flags in the device-side schedule.
#define FS_PASS_FIRST 1u   // apply the forward key transform on load; argsort: generate indices
#define FS_PASS_LAST 2u    // apply the inverse transform on store; argsort: do not store keys
#define FS_PASS_REGIONED 4u  // the source is the fused first pass's region layout (see below)
#define FS_PASS_SKEWED 8u    // a bin of the digit holds more than 1/FS_SKEW_SHARE of the keys: the
                             // pass's tile histogram uses replicated counters
#define FS_PASS_SEGCOUNT 16u // the pass (the top digit on the top-16 path, reading keys in the order of
                             // the digit below) adds the keys of every top-16-bit segment to FsArgs.segc
#ifndef FS_SKEW_SHARE
#define FS_SKEW_SHARE 64u
#endif
#define FS_SKEW_BIT (1u << 16)  // schedule steps: bit 16 + j of their constant mask marks digit j skewed

// Operation.
#define FSK_OP_KEYS 0u
#define FSK_OP_ARGSORT 1u
#define FSK_OP_PAIRS 2u

// Key transform (sort.metal:812-868 modes, fused into the passes).
#define FS_XF_NONE 0u
#define FS_XF_SIGN 1u      // i32/i64: xor the sign bit (self-inverse)
#define FS_XF_FLOAT 2u     // f32/f64: FloatFlip forward, IFloatFlip inverse

// Side duty of a digit-pass launch whose digit is constant (bits 24-31 of its
// schedule word 2j; its word 2j+1 then names the buffers):
#define FS_DUTY_NONE 0u
#define FS_DUTY_COPY 1u    // copy keys (and values) between the buffers named, over the grid
#define FS_DUTY_IOTA 2u    // argsort with every digit constant: indices = 0..n-1
#define FS_DUTY_UNREGION 3u  // keys-only, only digit 0 varies: the region layout of S1 -> caller keys,
                             // with the inverse transform

// Fused first pass of keys-only sorts (fs_first_*).  It reads the caller's
// keys once, counts the other digits for the later passes (the histogram read
// a sort otherwise starts with), and scatters the keys by digit 0 into fixed
// regions of scratch S1: FS_SUBS regions per digit value, region
// k = digit * FS_SUBS + sub at S1 + base[k], holding cap[digit] keys, where
// sub is the XCD group of the tile.  The region table (base[k] for every
// region, base[FS_REGIONS] = the regions' total, then cap[d] for every digit
// value) is written just before the pass by fs_region_sample_*, from the
// digit-0 histogram of a sample of the keys: a digit value's regions hold
// 1.5x its estimated share of the fullest region group's keys (the share at
// least a quarter of 1/256), plus a margin.  A tile takes the space of each of
// its digit runs with one atomic on the region's cursor (an LSD sort's first
// pass needs no order among equal digits), so the pass has no look-back.  The
// region start table (virtual position of each region's first key, regions
// in order) lets the next pass read the keys in digit-0 order.  A region that
// would overflow drops its runs, and the schedule step falls back to the
// stable passes over the caller's untouched keys.
#ifndef FS_SUBS
#define FS_SUBS 8
#endif
#define FS_REGIONS (FS_RADIX * FS_SUBS)
// Region table words (bases, total, caps), and the sample: FS_SAMPLE_CHUNKS
// runs of FS_SAMPLE_CHUNK consecutive keys spread evenly over the input (all
// keys when there are fewer).
#define FS_RTABLE_WORDS (FS_REGIONS + 2 + FS_RADIX)
#define FS_RTABLE_CAPS (FS_REGIONS + 1)
#define FS_RTABLE_SDIGIT (FS_REGIONS + 1 + FS_RADIX)   // the digit the fused pass scatters by
#define FS_SAMPLE_CHUNKS 256
#define FS_SAMPLE_CHUNK 128
// S1 keys the fused pass's regions may take for region groups of at most
// sub_keys keys each: 1.5 x (1 + 256 / 1024) of FS_SUBS groups, plus the
// margins and rounding of every region.
#define FS_FUSED_S1_KEYS(sub_keys) ((15ull * (unsigned long long)(sub_keys) * FS_SUBS + 7ull) / 8ull + \
                                    (unsigned long long)FS_REGIONS * 65ull)
// Histogram table: FS_HIST_SLOTS copies of [FS_MAX_DIGITS][FS_RADIX]; the
// fused pass's tiles fold their counts into copy (tile % FS_HIST_SLOTS), so
// that no counter takes more than num_tiles / FS_HIST_SLOTS atomics.  The
// schedule step, in the pass's last tile, reads and clears every copy: 1 to 8
// copies measured alike, 16 slower (u64: +5% fused pass), 32 slower still.
#define FS_HIST_SLOTS 4
// Tile descriptor of the region layout, 4 words {x, y, z, w} per tile of the
// pass after the fused one.  w = region k0 of the tile's first key, with
// FS_TILE_MULTI set when the tile covers more than two regions.  Otherwise
// the S1 index of position p is p + (p < y ? x : z) (y: first position of the
// second region, or 0xFFFFFFFF); with FS_TILE_MULTI, x is the region of the
// tile's last key and indices come from the region start table.
// FS_TILE_ONE_DIGIT: every region of the tile holds the same digit-0 value.
#define FS_TILE_MULTI 0x80000000u
#define FS_TILE_ONE_DIGIT 0x40000000u
#define FS_TILE_DESC_WORDS 4
#define FS_HIST_WORDS (FS_HIST_SLOTS * FS_MAX_DIGITS * FS_RADIX)

// Error bits reported through the host-visible status word.
#define FS_DEVERR_LOOKBACK_TIMEOUT 1u

// Device-side schedule written by the upsweep's last block: FS_PLAN_WORDS u32 words, stored
// and loaded with agent-scope (sc1) accesses.  Buffers are named by id, never
// by address, so a kernel only ever dereferences addresses from its own
// arguments.
#define FS_BUF_NONE 0u
#define FS_BUF_KEYS 1u      // caller keys
#define FS_BUF_VALS 2u      // caller values (pairs) or output indices (argsort)
#define FS_BUF_S1K 3u
#define FS_BUF_S2K 4u
#define FS_BUF_S1V 5u
#define FS_BUF_S2V 6u
// per digit-pass launch slot j (the launch's `slot` argument; in the LSD
// schedules slot j sorts digit j):
//              word 2j   = active | digit << 1 | exec_index << 8 | flags << 16 | duty << 24
//              word 2j+1 = src_k | dst_k << 8 | src_v << 16 | dst_v << 24 (buffer ids)
#define FS_PLAN_PASS_WORDS 2
#define FS_PLAN_NPASSES (FS_MAX_DIGITS * FS_PLAN_PASS_WORDS)      // passes that run
#define FS_PLAN_MASK (FS_PLAN_NPASSES + 1)                         // bit j: digit j sorted
#define FS_MASK_FUSED (1u << 8)     // mask word: the fused first pass's regions were used
#define FS_MASK_TOP16 (1u << 9)     // mask word: the top-16 path ran (digit passes on the two top
                                    // digits, then the local sort of each top-16-bit segment)
#define FS_PLAN_TICKET (FS_PLAN_NPASSES + 2)                       // upsweep blocks finished (0 between sorts)
// Local sort of the top-16 path (fs_local_*): word FS_PLAN_LOCAL = active | seg_bits << 8 |
// flags << 16, word FS_PLAN_LOCAL + 1 = buffer ids as a pass's word 2j+1.
#define FS_PLAN_LOCAL (FS_PLAN_NPASSES + 4)
// 1: the fused pass's second launch re-scatters the keys into exact regions
// (a region of its first launch overflowed); 0: that launch does nothing
#define FS_PLAN_RESCATTER (FS_PLAN_NPASSES + 6)
#define FS_PLAN_WORDS (FS_PLAN_NPASSES + 8)

// Top-16 path of keys-only integer sorts (from FS_TOP16_MIN_KEYS32/64 keys): the
// fused first pass scatters by the digit below the top byte (digit 2 of
// 32-bit keys, 6 of 64-bit keys; the region sample's choice,
// FS_RTABLE_SDIGIT) into its regions, a stable pass on the top digit reads
// the regions in order - so its output is ordered by the top 16 bits - and
// counts the keys of every top-16-bit value (FS_SEGS counters), and the
// local sort (fs_local_*) sorts each segment of keys sharing their top
// seg_bits bits, in LDS, by the bits below: one block per segment, one read
// and one write of every key.  A segment larger than a block holds is sorted
// by that block through scratch, a digit at a time.
// seg_bits is chosen on the host so that a segment of a uniform input fits
// a block.  The region sample estimates the segments from its keys (their
// top seg_bits bits): one estimated above FsArgs.seg_limit keys (skewed or
// constant top bytes) makes it choose digit 0 instead, and the same launches
// run the LSD passes (the stable passes on the other digits in the
// digit-pass launches, the local sort's launch idle).
#define FS_SEGS 65536u
// the segment counters, a count (zero before the local sort) and a list of
// segment ids (the 64-bit local sort's deferred segments)
#define FS_SEGC_WORDS (2u * FS_SEGS + 1u)
// a segment estimate counts only from this many sampled keys on
#define FS_SEG_MIN_SAMPLES 8u
#ifndef FS_L32_BLOCK
#define FS_L32_BLOCK 256
#endif
#ifndef FS_L32_ITEMS
#define FS_L32_ITEMS 18
#endif
// 64-bit keys: 256 x 9 keys per block (an 18 KiB stage holding the group counters
// until it is written, 22 KiB of LDS: seven blocks per CU)
#ifndef FS_L64_BLOCK
#define FS_L64_BLOCK 256
#endif
#ifndef FS_L64_ITEMS
#define FS_L64_ITEMS 9
#endif
// ... grouped by the FS_L64_GBITS bits below the segment's (2^11 LDS
// counters: about one key per group), each key then ranked within its group
// by comparison when no group holds more than FS_L64_GLIM keys
#ifndef FS_L64_GBITS
#define FS_L64_GBITS 11
#endif
#ifndef FS_L64_GLIM
#define FS_L64_GLIM 32u
#endif
// Threads per block of the local sort's deferred launches (the same keys per
// thread, one block per CU): segments up to that many times the keys per
// thread are sorted in LDS there, larger ones a digit at a time through
// scratch.  (Inputs with many copies of each key make segments of a few
// values times their copies: at 2^28 u32 keys with 2^16 distinct values,
// 2-4 times a block of the first launch.)
#ifndef FS_LD32_BLOCK
#define FS_LD32_BLOCK 512
#endif
#ifndef FS_LD64_BLOCK
#define FS_LD64_BLOCK 1024
#endif
// Wide local-sort blocks (the same keys per thread, FS_LW_BLOCK threads):
// sorts too large for 2^16 segments of the blocks above to fit them (more
// than 280M 32-bit or 135M 64-bit keys) take the top-16 path on these, up
// to twice those sizes
#ifndef FS_LW_BLOCK
#define FS_LW_BLOCK 512
#endif
// 64-bit keys on the top-16 launch sequence: the digit-pass slots from this
// one on (their 5th LSD pass and later, after the fused pass) are launched
// on the persistent loop kernel's small grid; the earlier slots, and every
// slot of 32-bit keys, launch one block per tile
#ifndef FS_LOOP_SLOT64
#define FS_LOOP_SLOT64 4u
#endif

// Error bits additionally reported through the status word.
#define FS_DEVERR_BAD_TILE 2u        // a digit pass block mapped to a tile >= num_tiles
#define FS_DEVERR_BAD_PLAN 4u        // a schedule named a buffer the call does not have
#define FS_DEVERR_GATHER_INDEX 8u    // a gather index was >= the source length
#define FS_DEVERR_BAD_DIGITS 16u     // the digit count does not match the key width

// Faults a CPU-emulator test build (FS_FAULT_INJECTION) can inject, so that
// every device-side guard is exercised without a faulty kernel on a GPU.
#define FS_FAULT_NONE 0u
#define FS_FAULT_BAD_DIGITS 1u     // host passes a digit count other than 4/8 -> BAD_PLAN
#define FS_FAULT_BAD_BUFFER 2u     // schedule names an unknown buffer for the first pass -> BAD_PLAN
#define FS_FAULT_EXTRA_BLOCK 3u    // first digit pass launched with one block too many -> BAD_TILE
#define FS_FAULT_STALL_TILE 4u     // tile 1 of the first pass never publishes -> LOOKBACK_TIMEOUT
#define FS_FAULT_SMALL_S1 5u       // the region sample's S1 budget halved: its layout does not fit and
                                   // the regions split the budget evenly (no error; the sort stays exact)

// Scratch of the entry point that allocates nothing (fs_encode_no_alloc): a
// file-scope static device array of FS_NA_SCRATCH_BYTES in the code object,
// laid out as the histogram, bin-base and schedule tables, the two look-back
// arrays and the key/value ping-pong buffers for sorts of up to
// FS_NA_MAX_KEYS keys of any type and op (64-bit keys with values: the
// largest).  Offsets in bytes, each 256-byte aligned.
#define FS_NA_MAX_KEYS (1u << 20)
#define FS_NA_ALIGN(x) ((((x) + 255ull) / 256ull) * 256ull)
#define FS_MIN2(a, b) ((a) < (b) ? (a) : (b))
#define FS_NA_MIN_TILE FS_MIN2(FS_MIN2(FS_K32_BLOCK * FS_K32_ITEMS, FS_K32V_BLOCK * FS_K32V_ITEMS), \
                               FS_MIN2(FS_K64_BLOCK * FS_K64_ITEMS, FS_K64V_BLOCK * FS_K64V_ITEMS))
#define FS_NA_MAX_TILES ((FS_NA_MAX_KEYS + FS_NA_MIN_TILE - 1) / FS_NA_MIN_TILE)
#define FS_NA_TABLE_BYTES FS_NA_ALIGN((unsigned long long)FS_MAX_DIGITS * FS_RADIX * 4)
#define FS_NA_HIST_BYTES FS_NA_ALIGN((unsigned long long)FS_HIST_WORDS * 4)
#define FS_NA_LB_BYTES FS_NA_ALIGN((unsigned long long)FS_NA_MAX_TILES * FS_RADIX * 4 + \
                                   (unsigned long long)((FS_NA_MAX_TILES + FS_LB_GROUP - 1) / FS_LB_GROUP) * FS_RADIX * 4)
#define FS_NA_OFF_HIST 0ull
#define FS_NA_OFF_PLAN (FS_NA_OFF_HIST + FS_NA_HIST_BYTES)
#define FS_NA_OFF_CURSORS (FS_NA_OFF_PLAN + FS_NA_ALIGN(FS_PLAN_WORDS * 4))
#define FS_NA_OFF_BINBASE (FS_NA_OFF_CURSORS + FS_NA_ALIGN(FS_REGIONS * 4))
#define FS_NA_OFF_RSTART (FS_NA_OFF_BINBASE + FS_NA_TABLE_BYTES)
#define FS_NA_OFF_RTABLE (FS_NA_OFF_RSTART + FS_NA_ALIGN((FS_REGIONS + 1) * 4))
#define FS_NA_OFF_TILEMAP (FS_NA_OFF_RTABLE + FS_NA_ALIGN(FS_RTABLE_WORDS * 4))
#define FS_NA_OFF_LB0 (FS_NA_OFF_TILEMAP + FS_NA_ALIGN((unsigned long long)FS_NA_MAX_TILES * FS_TILE_DESC_WORDS * 4))
#define FS_NA_OFF_LB1 (FS_NA_OFF_LB0 + FS_NA_LB_BYTES)
#define FS_NA_OFF_S1K (FS_NA_OFF_LB1 + FS_NA_LB_BYTES)
#define FS_NA_OFF_S2K (FS_NA_OFF_S1K + (unsigned long long)FS_NA_MAX_KEYS * 8)
#define FS_NA_OFF_S1V (FS_NA_OFF_S2K + (unsigned long long)FS_NA_MAX_KEYS * 8)
#define FS_NA_OFF_S2V (FS_NA_OFF_S1V + (unsigned long long)FS_NA_MAX_KEYS * 4)
#define FS_NA_SCRATCH_BYTES (FS_NA_OFF_S2V + (unsigned long long)FS_NA_MAX_KEYS * 4)
// bytes that must be zero before the first sort (histogram copies, the
// schedule with its ticket, the region cursors); every sort leaves them zero
#define FS_NA_ZERO_BYTES FS_NA_OFF_BINBASE

// Kernel argument block, passed by value to every kernel.
typedef struct FsArgs {
    uint64_t n;                 // number of keys (2 <= n < 2^32)
    uint32_t key64;             // 1 for 8-byte keys
    uint32_t xform;             // FS_XF_*
    uint32_t op;                // FSK_OP_*
    uint32_t digits;            // 4 or 8
    uint32_t num_tiles;         // ceil(n / tile)
    uint32_t wide;              // 1: 64-bit look-back tile entries (n >= FS_LB_WIDE_KEYS)
    uint32_t tile;              // keys per tile of the digit-pass variant in use
    uint32_t vec_ok;            // keys pointer is 16-byte aligned
    uint32_t fault;             // FS_FAULT_* to inject (read only by FS_FAULT_INJECTION builds), else 0
    uint64_t keys;              // caller keys (in place for KEYS/PAIRS; read-only for ARGSORT)
    uint64_t vals;              // caller values (PAIRS) or output indices (ARGSORT)
    uint64_t s1k, s2k, s1v, s2v;   // scratch ping-pong buffers
    uint64_t hist;              // u32 [FS_HIST_SLOTS][FS_MAX_DIGITS][256], zero between sorts
    uint64_t binbase;           // u32 [digits][256]
    uint64_t lookback0, lookback1;  // [num_tiles][256] tile entries (u32, or u64 when wide),
                                    // then u32 [groups][256] group entries; alternate per pass
    uint64_t plan;              // u32[FS_PLAN_WORDS] schedule
    uint64_t status;            // u32, host-visible error bits
    uint64_t stats;             // u64[FS_STAT_SLOTS][FS_STAT_COUNT] look-back counters, or 0 when off
    uint64_t cursors;           // u32[FS_REGIONS] region fill cursors of the fused pass (zero between sorts)
    uint64_t rstart;            // u32[FS_REGIONS + 1] virtual start of each region (fused pass's schedule step)
    uint64_t tilemap;           // u32[num_tiles][4] tile descriptors of the region layout (fused pass's schedule step)
    uint64_t rtable;            // u32[FS_RTABLE_WORDS] region bases, total and caps (fs_region_sample_*)
    uint32_t sub_keys;          // keys of the fullest region group (fused path), else 0
    uint32_t fused;             // 1: the sort starts with the fused first pass (keys-only)
    uint32_t s1_keys;           // keys S1 holds (fused path: the regions' budget), else 0
    uint32_t seg_limit;         // top-16 path: the region sample takes the LSD passes instead when it
                                // estimates a segment of more keys than this (0xFFFFFFFF: never)
    uint64_t segc;              // u32[FS_SEGC_WORDS]: keys per top-16-bit value (top-16 path; zero before its
                                // top-digit pass), then the count and list of the segments the 64-bit local
                                // sort leaves to its second launch
    uint32_t seg_bits;          // top-16 launch sequence: bits that name a segment of the local sort
                                // (8..16), else 0
    uint32_t reserved0;
} FsArgs;

// Look-back statistics (accumulated only when FsArgs.stats is set).
#define FS_STAT_TILES 0      // tiles that looked back
#define FS_STAT_ROUNDS 1     // look-back round trips, summed over the 256 digits
#define FS_STAT_STALLS 2     // rounds that found a predecessor not yet published
#define FS_STAT_ENTRIES 3    // predecessor entries consumed
#define FS_STAT_COUNT 4
#define FS_STAT_SLOTS 64     // stats is u64[FS_STAT_SLOTS][FS_STAT_COUNT]

#endif
