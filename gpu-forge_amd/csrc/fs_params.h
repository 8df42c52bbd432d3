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
// (fs_tile_config), so they are only defined here.
#ifndef FS_K32_BLOCK
#define FS_K32_BLOCK 512
#endif
#ifndef FS_K32_ITEMS
#define FS_K32_ITEMS 16
#endif
#ifndef FS_K32V_BLOCK
#define FS_K32V_BLOCK 256
#endif
#ifndef FS_K32V_ITEMS
#define FS_K32V_ITEMS 16
#endif
#ifndef FS_K64_BLOCK
#define FS_K64_BLOCK 256
#endif
#ifndef FS_K64_ITEMS
#define FS_K64_ITEMS 16
#endif
#ifndef FS_K64V_BLOCK
#define FS_K64V_BLOCK 256
#endif
#ifndef FS_K64V_ITEMS
#define FS_K64V_ITEMS 12
#endif
// Ranking inside a wave: 0 = ballot match (8 ballots per key),
// 1 = LDS atomic-OR lane masks.
#ifndef FS_RANK_MODE
#define FS_RANK_MODE 0
#endif
// index into fs_tile_config
#define FS_VAR_K32 0
#define FS_VAR_K32V 1
#define FS_VAR_K64 2
#define FS_VAR_K64V 3

// Upsweep (all-digit histogram) block.
#define FS_HIST_BLOCK 256

// Look-back entries: one 32-bit word per (tile, digit) = [flag:2 | count:30].
// Counts are kept below 2^30 by splitting the input into portions of at most
// 2^30 keys; each portion has its own look-back chain and bin bases.
#define FS_LB_AGG 0x40000000u
#define FS_LB_INC 0x80000000u
#define FS_LB_FLAGS 0xC0000000u
#define FS_LB_VALUE 0x3FFFFFFFu
#define FS_PORTION_KEYS (1u << 30)
#define FS_MAX_PORTIONS 4

// Bounded spin of a look-back wait (iterations of s_sleep(1), ~64 clocks each).
// A predecessor tile that owns a tile id is resident and finishes in
// microseconds; the bound only guarantees that every wait ends.
#define FS_SPIN_LIMIT (1u << 24)

// Per-pass flags in the device-side schedule.
#define FS_PASS_FIRST 1u   // apply the forward key transform on load; argsort: generate indices
#define FS_PASS_LAST 2u    // apply the inverse transform on store; argsort: do not store keys

// Operation.
#define FSK_OP_KEYS 0u
#define FSK_OP_ARGSORT 1u
#define FSK_OP_PAIRS 2u

// Key transform (sort.metal:812-868 modes, fused into the passes).
#define FS_XF_NONE 0u
#define FS_XF_SIGN 1u      // i32/i64: xor the sign bit (self-inverse)
#define FS_XF_FLOAT 2u     // f32/f64: FloatFlip forward, IFloatFlip inverse

// Finish step after the last pass.
#define FS_FIN_NONE 0u
#define FS_FIN_COPY 1u     // copy keys (and values) scratch -> caller buffer
#define FS_FIN_IOTA 2u     // argsort with every digit constant: indices = 0..n-1

// Error bits reported through the host-visible status word.
#define FS_DEVERR_LOOKBACK_TIMEOUT 1u

typedef struct FsPassSched {
    uint32_t active;       // this digit position is sorted (not constant)
    uint32_t exec_index;   // 0..n_passes-1 among active digits
    uint32_t flags;        // FS_PASS_*
    uint32_t pad;
    uint64_t src_k, dst_k, src_v, dst_v;   // device addresses
} FsPassSched;

typedef struct FsPlan {
    FsPassSched pass[FS_MAX_DIGITS];
    uint32_t n_passes;
    uint32_t finish;       // FS_FIN_*
    uint32_t digit_mask;   // bit j set when digit j is active
    uint32_t pad;
    uint64_t fin_src_k, fin_dst_k, fin_src_v, fin_dst_v;
} FsPlan;

// Kernel argument block, passed by value to every kernel.
typedef struct FsArgs {
    uint64_t n;                 // number of keys (2 <= n < 2^32)
    uint32_t key64;             // 1 for 8-byte keys
    uint32_t xform;             // FS_XF_*
    uint32_t op;                // FSK_OP_*
    uint32_t digits;            // 4 or 8
    uint32_t num_tiles;         // ceil(n / tile)
    uint32_t tiles_per_portion; // power of two, tiles_per_portion * tile <= FS_PORTION_KEYS
    uint32_t hist_tiles_per_block;  // power of two dividing tiles_per_portion
    uint32_t tile;              // keys per tile of the digit-pass variant in use
    uint32_t vec_ok;            // keys pointer is 16-byte aligned
    uint32_t pad2;
    uint64_t keys;              // caller keys (in place for KEYS/PAIRS; read-only for ARGSORT)
    uint64_t vals;              // caller values (PAIRS) or output indices (ARGSORT)
    uint64_t s1k, s2k, s1v, s2v;   // scratch ping-pong buffers
    uint64_t hist;              // u32 [FS_MAX_PORTIONS][digits][256], zero between sorts
    uint64_t binbase;           // u32 [FS_MAX_PORTIONS][digits][256]
    uint64_t lookback0, lookback1;  // u32 [num_tiles][256] each
    uint64_t tile_ctr;          // u32 [FS_MAX_DIGITS]
    uint64_t plan;              // FsPlan
    uint64_t status;            // u32, host-visible error bits
} FsArgs;

#endif
