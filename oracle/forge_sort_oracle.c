/*
 * forge_sort_oracle.c -- CPU restatement of forge-sort's GpuSorter radix sort.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP product path:
 * it may be loaded by tests/, by __graft_entry__.smoke() and by bench.py's
 * cpu_baseline leg, and by nothing else.  The product library never links it.
 *
 * What it restates (paths relative to metal-forge-compute/forge-sort/):
 *   - key transforms            shaders/sort.metal:812-832 (32-bit), :848-868 (64-bit)
 *   - type -> transform mode    src/lib.rs:42-88, :875, :955, :2383, :2452
 *                               (i64 uses mode 0 = sign XOR, not FloatFlip)
 *   - 32-bit digit schedule     src/lib.rs:574-578: MSD on byte 3, then the
 *                               inner LSD passes on bytes 0,1,2 inside every bucket
 *   - 64-bit digit schedule     src/lib.rs:1398-1449: MSD on byte 7, then inner
 *                               passes byte 0, bytes 1-3, bytes 4-6 (LSB first)
 *   - edge returns              src/lib.rs:710-712 (n<=1), :1677-1682 (argsort of
 *                               0/1 keys), :1929-1934 (LengthMismatch before work)
 *   - argsort/pairs             src/lib.rs:1838-1917, :1923-2018 (indices carried
 *                               through the sort; pairs = argsort + gather)
 *
 * One deliberate difference from the reference kernels: every counting pass
 * here is stable, so argsort and pairs break ties by original index.  The
 * reference's MSD scatter claims tile slots with device atomics
 * (sort.metal:337-340) and is not stable; the build's contract is the stable
 * order the reference's spec promises (ai/tasks/spec/PM.md:302).
 *
 * Pinning (tests/test_oracle.py): the reference's own known-answer vectors
 * (tests/golden/), numpy's sort / stable argsort on independent encodings
 * (Rust's documented total_cmp formula for floats, not FloatFlip), brute force
 * over every small multiset permutation, and planted mistakes (or_mutation)
 * that each check must catch.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* Key type codes; identical to fs_key_type in include/forge_sort.h. */
enum { OR_U32 = 0, OR_I32 = 1, OR_F32 = 2, OR_U64 = 3, OR_I64 = 4, OR_F64 = 5 };
/* Status codes; identical to fs_status in include/forge_sort.h. */
enum { OR_OK = 0, OR_ERR_LENGTH_MISMATCH = 4, OR_ERR_INVALID_ARGUMENT = 5, OR_ERR_OOM = 6 };

/*
 * Planted-mistake switch, used only by the oracle's own meta-tests to show
 * that the pinning checks fail when a plausible bug is present:
 *   1 = skip the inner LSD pass on byte 1 (a dropped term)
 *   2 = use FloatFlip (mode 1) for i64, as sort.metal:837-840's stale comment says
 *   3 = break ties in reverse index order (unstable)
 *   4 = skip the inverse transform for f32 (wrong output encoding)
 *   5 = MSD on byte 2 instead of byte 3 (wrong index)
 */
int or_mutation = 0;

/* ---- transforms: sort.metal:812-832 / :848-868 ------------------------- */

static inline uint32_t t32(uint32_t v, uint32_t mode) {
    if (mode == 0) return v ^ 0x80000000u;                        /* i32 sign flip */
    if (mode == 1) return (v & 0x80000000u) ? ~v : (v ^ 0x80000000u);  /* FloatFlip */
    return (v & 0x80000000u) ? (v ^ 0x80000000u) : ~v;             /* IFloatFlip */
}

static inline uint64_t t64(uint64_t v, uint32_t mode) {
    const uint64_t s = 0x8000000000000000ull;
    if (mode == 0) return v ^ s;
    if (mode == 1) return (v & s) ? ~v : (v ^ s);
    return (v & s) ? (v ^ s) : ~v;
}

void or_transform_32(uint32_t *d, uint64_t n, uint32_t mode) {
    for (uint64_t i = 0; i < n; ++i) d[i] = t32(d[i], mode);
}

void or_transform_64(uint64_t *d, uint64_t n, uint32_t mode) {
    for (uint64_t i = 0; i < n; ++i) d[i] = t64(d[i], mode);
}

/* ---- stable counting passes ------------------------------------------- */

/* One stable counting pass over [lo,hi) on the byte at `shift`. */
static void pass32(const uint32_t *ks, uint32_t *kd, const uint32_t *vs, uint32_t *vd,
                   uint64_t lo, uint64_t hi, unsigned shift) {
    uint64_t cnt[256] = {0};
    for (uint64_t i = lo; i < hi; ++i) cnt[(ks[i] >> shift) & 0xFFu]++;
    uint64_t off[256], run = lo;
    for (int d = 0; d < 256; ++d) { off[d] = run; run += cnt[d]; }
    if (or_mutation == 3) {
        /* planted mistake: each digit run is filled back to front (unstable) */
        for (int d = 0; d < 256; ++d) off[d] += cnt[d];
        for (uint64_t i = lo; i < hi; ++i) {
            unsigned d = (ks[i] >> shift) & 0xFFu;
            uint64_t p = --off[d];
            kd[p] = ks[i];
            if (vs) vd[p] = vs[i];
        }
        return;
    }
    for (uint64_t i = lo; i < hi; ++i) {
        unsigned d = (ks[i] >> shift) & 0xFFu;
        uint64_t p = off[d]++;
        kd[p] = ks[i];
        if (vs) vd[p] = vs[i];
    }
}

static void pass64(const uint64_t *ks, uint64_t *kd, const uint32_t *vs, uint32_t *vd,
                   uint64_t lo, uint64_t hi, unsigned shift) {
    uint64_t cnt[256] = {0};
    for (uint64_t i = lo; i < hi; ++i) cnt[(ks[i] >> shift) & 0xFFu]++;
    uint64_t off[256], run = lo;
    for (int d = 0; d < 256; ++d) { off[d] = run; run += cnt[d]; }
    if (or_mutation == 3) {
        for (int d = 0; d < 256; ++d) off[d] += cnt[d];
        for (uint64_t i = lo; i < hi; ++i) {
            unsigned d = (ks[i] >> shift) & 0xFFu;
            uint64_t p = --off[d];
            kd[p] = ks[i];
            if (vs) vd[p] = vs[i];
        }
        return;
    }
    for (uint64_t i = lo; i < hi; ++i) {
        unsigned d = (ks[i] >> shift) & 0xFFu;
        uint64_t p = off[d]++;
        kd[p] = ks[i];
        if (vs) vd[p] = vs[i];
    }
}

/*
 * 32-bit sort of already-transformed keys (vals may be NULL).
 * MSD partition on byte 3, then per bucket the inner LSD passes on bytes
 * 0,1,2 (lib.rs:574-578, sort.metal:378-769).  Result in keys/vals.
 */
int or_sort_raw32(uint32_t *keys, uint32_t *vals, uint64_t n) {
    if (n <= 1) return OR_OK;
    uint32_t *kt = (uint32_t *)malloc(n * sizeof(uint32_t));
    uint32_t *vt = vals ? (uint32_t *)malloc(n * sizeof(uint32_t)) : NULL;
    if (!kt || (vals && !vt)) { free(kt); free(vt); return OR_ERR_OOM; }

    const unsigned msd_shift = (or_mutation == 5) ? 16u : 24u;
    /* MSD scatter keys -> kt (sort.metal:64-142 histogram, :153-181 prep, :193-365 scatter) */
    uint64_t cnt[256] = {0}, start[257];
    for (uint64_t i = 0; i < n; ++i) cnt[(keys[i] >> msd_shift) & 0xFFu]++;
    start[0] = 0;
    for (int d = 0; d < 256; ++d) start[d + 1] = start[d] + cnt[d];
    pass32(keys, kt, vals, vt, 0, n, msd_shift);

    /* inner LSD passes per bucket: kt -> keys -> kt -> keys (b->a->b->a, sort.metal:602-608) */
    for (int b = 0; b < 256; ++b) {
        uint64_t lo = start[b], hi = start[b + 1];
        if (hi - lo == 0) continue;
        const uint32_t *src_k = kt; uint32_t *dst_k = keys;
        const uint32_t *src_v = vt; uint32_t *dst_v = vals;
        int passes_done = 0;
        for (unsigned byte = 0; byte < 3; ++byte) {
            unsigned shift = byte * 8u;
            if (or_mutation == 5 && byte == 2) shift = 24u;
            if (or_mutation == 1 && byte == 1) continue;
            pass32(src_k, dst_k, src_v, dst_v, lo, hi, shift);
            const uint32_t *tk = dst_k; dst_k = (uint32_t *)src_k; src_k = tk;
            const uint32_t *tv = dst_v; dst_v = (uint32_t *)src_v; src_v = tv;
            passes_done++;
        }
        if ((passes_done & 1) == 0) {
            /* result currently in kt/vt: move back into keys/vals */
            memcpy(keys + lo, kt + lo, (hi - lo) * sizeof(uint32_t));
            if (vals) memcpy(vals + lo, vt + lo, (hi - lo) * sizeof(uint32_t));
        }
    }
    free(kt); free(vt);
    return OR_OK;
}

/*
 * 64-bit sort of already-transformed keys.  MSD on byte 7, then inner LSD
 * passes byte 0, bytes 1-3, bytes 4-6 inside every bucket (lib.rs:1398-1449).
 */
int or_sort_raw64(uint64_t *keys, uint32_t *vals, uint64_t n) {
    if (n <= 1) return OR_OK;
    uint64_t *kt = (uint64_t *)malloc(n * sizeof(uint64_t));
    uint32_t *vt = vals ? (uint32_t *)malloc(n * sizeof(uint32_t)) : NULL;
    if (!kt || (vals && !vt)) { free(kt); free(vt); return OR_ERR_OOM; }

    const unsigned msd_shift = (or_mutation == 5) ? 48u : 56u;
    uint64_t cnt[256] = {0}, start[257];
    for (uint64_t i = 0; i < n; ++i) cnt[(keys[i] >> msd_shift) & 0xFFu]++;
    start[0] = 0;
    for (int d = 0; d < 256; ++d) start[d + 1] = start[d] + cnt[d];
    pass64(keys, kt, vals, vt, 0, n, msd_shift);

    for (int b = 0; b < 256; ++b) {
        uint64_t lo = start[b], hi = start[b + 1];
        if (hi - lo == 0) continue;
        const uint64_t *src_k = kt; uint64_t *dst_k = keys;
        const uint32_t *src_v = vt; uint32_t *dst_v = vals;
        int passes_done = 0;
        for (unsigned byte = 0; byte < 7; ++byte) {
            unsigned shift = byte * 8u;
            if (or_mutation == 5 && byte == 6) shift = 56u;
            if (or_mutation == 1 && byte == 1) continue;
            pass64(src_k, dst_k, src_v, dst_v, lo, hi, shift);
            const uint64_t *tk = dst_k; dst_k = (uint64_t *)src_k; src_k = tk;
            const uint32_t *tv = dst_v; dst_v = (uint32_t *)src_v; src_v = tv;
            passes_done++;
        }
        if ((passes_done & 1) == 0) {
            memcpy(keys + lo, kt + lo, (hi - lo) * sizeof(uint64_t));
            if (vals) memcpy(vals + lo, vt + lo, (hi - lo) * sizeof(uint32_t));
        }
    }
    free(kt); free(vt);
    return OR_OK;
}

/* ---- type-level entry points mirroring GpuSorter ----------------------- */

static int is64(int kt) { return kt >= OR_U64; }

/* forward / inverse transform modes per type, lib.rs:42-88 (+ :2383 for i64) */
static int needs_transform(int kt) { return kt != OR_U32 && kt != OR_U64; }
static uint32_t fwd_mode(int kt) {
    if (kt == OR_F32 || kt == OR_F64) return 1;
    if (kt == OR_I64 && or_mutation == 2) return 1;
    return 0;
}
static uint32_t inv_mode(int kt) {
    if (kt == OR_F32 || kt == OR_F64) return 2;
    if (kt == OR_I64 && or_mutation == 2) return 2;
    return 0;
}

static void apply(int kt, void *keys, uint64_t n, uint32_t mode) {
    if (is64(kt)) or_transform_64((uint64_t *)keys, n, mode);
    else or_transform_32((uint32_t *)keys, n, mode);
}

/* sort_<t>: lib.rs:791 (u32), :840 (i32), :920 (f32), :2238 (u64), :2348 (i64), :2417 (f64) */
int or_sort(int kt, void *keys, uint64_t n) {
    if (kt < OR_U32 || kt > OR_F64) return OR_ERR_INVALID_ARGUMENT;
    if (n <= 1) return OR_OK;
    if (needs_transform(kt)) apply(kt, keys, n, fwd_mode(kt));
    int rc = is64(kt) ? or_sort_raw64((uint64_t *)keys, NULL, n)
                      : or_sort_raw32((uint32_t *)keys, NULL, n);
    if (rc) return rc;
    if (needs_transform(kt) && !(kt == OR_F32 && or_mutation == 4))
        apply(kt, keys, n, inv_mode(kt));
    return OR_OK;
}

/* argsort_<t>: lib.rs:1675, :1754, :1838, :2595, :2669, :2747.  Input not modified. */
int or_argsort(int kt, const void *keys, uint64_t n, uint32_t *out) {
    if (kt < OR_U32 || kt > OR_F64) return OR_ERR_INVALID_ARGUMENT;
    if (n == 0) return OR_OK;
    if (n == 1) { out[0] = 0; return OR_OK; }
    size_t kb = is64(kt) ? 8 : 4;
    void *tmp = malloc(n * kb);
    if (!tmp) return OR_ERR_OOM;
    memcpy(tmp, keys, n * kb);
    for (uint64_t i = 0; i < n; ++i) out[i] = (uint32_t)i;      /* sort_init_indices, sort.metal:777-783 */
    if (needs_transform(kt)) apply(kt, tmp, n, fwd_mode(kt));
    int rc = is64(kt) ? or_sort_raw64((uint64_t *)tmp, out, n)
                      : or_sort_raw32((uint32_t *)tmp, out, n);
    free(tmp);
    return rc;
}

/*
 * sort_pairs_<t>: lib.rs:1923 (u32), :2024, :2132, :2826, :2921.  LengthMismatch
 * is reported before any work (:1928-1934).  The reference sorts indices and
 * gathers values (sort.metal:792-800); with a stable sort that equals carrying
 * the values, which is what is done here.
 */
int or_sort_pairs(int kt, void *keys, uint64_t n_keys, uint32_t *vals, uint64_t n_vals) {
    if (kt < OR_U32 || kt > OR_F64) return OR_ERR_INVALID_ARGUMENT;
    if (n_keys != n_vals) return OR_ERR_LENGTH_MISMATCH;
    uint64_t n = n_keys;
    if (n <= 1) return OR_OK;
    if (needs_transform(kt)) apply(kt, keys, n, fwd_mode(kt));
    int rc = is64(kt) ? or_sort_raw64((uint64_t *)keys, vals, n)
                      : or_sort_raw32((uint32_t *)keys, vals, n);
    if (rc) return rc;
    if (needs_transform(kt) && !(kt == OR_F32 && or_mutation == 4))
        apply(kt, keys, n, inv_mode(kt));
    return OR_OK;
}

/* GpuGather: output[i] = source[indices[i]] for u32 / u64 elements
 * (metal-forge-compute/forge-runtime/shaders/gather.metal:5-27, driven by
 * src/gather.rs:81-143).  The reference has no bounds check; here an index at
 * or past source_len yields OR_ERR_INVALID_ARGUMENT (the product reports it as
 * a GPU execution error and writes 0 there).  Mutation 6 reads the next
 * element instead. */
int or_gather(int is64, const void *source, uint64_t source_len, const uint32_t *indices, void *output,
              uint64_t count) {
    int bad = 0;
    for (uint64_t i = 0; i < count; ++i) {
        uint64_t j = indices[i];
        if (or_mutation == 6 && j + 1 < source_len) ++j;
        if (j >= source_len) {
            bad = 1;
            if (is64) ((uint64_t *)output)[i] = 0; else ((uint32_t *)output)[i] = 0;
            continue;
        }
        if (is64) ((uint64_t *)output)[i] = ((const uint64_t *)source)[j];
        else ((uint32_t *)output)[i] = ((const uint32_t *)source)[j];
    }
    return bad ? OR_ERR_INVALID_ARGUMENT : OR_OK;
}
