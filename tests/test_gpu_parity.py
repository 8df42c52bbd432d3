"""Parity of the HIP path with the CPU oracle, through the C ABI.

Keys must be bit-identical to the oracle's sort; argsort indices and pair
values must be identical to the oracle's stable order (ties by original
index).  Covers the reference suite's cases (tests/golden/), its edge cases
(empty, single, all-equal, sorted, reversed, non-tile-aligned, sub-tile,
NaN/inf/-0.0/subnormals, byte-isolated 64-bit values) and every
BASELINE.json configuration at full size.
"""
import json
import os

import numpy as np
import pytest

import oracle
from forge_sort import datagen

pytestmark = pytest.mark.gpu

BITS = {"u32": np.uint32, "i32": np.uint32, "f32": np.uint32,
        "u64": np.uint64, "i64": np.uint64, "f64": np.uint64}
NP = oracle.NP_DTYPES
KINDS = ["u32", "i32", "f32", "u64", "i64", "f64"]
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden.json")


@pytest.fixture(scope="module")
def sorter():
    from forge_sort import GpuSorter
    s = GpuSorter.new()
    yield s
    s.close()


def bits_equal(a, b, kind):
    return np.array_equal(np.asarray(a).view(BITS[kind]), np.asarray(b).view(BITS[kind]))


def first_diff(a, b, kind):
    x, y = np.asarray(a).view(BITS[kind]), np.asarray(b).view(BITS[kind])
    idx = np.nonzero(x != y)[0]
    return None if idx.size == 0 else (int(idx[0]), hex(int(x[idx[0]])), hex(int(y[idx[0]])))


def check_sort(sorter, kind, keys):
    exp = oracle.sort(kind, keys)
    got = keys.copy()
    getattr(sorter, f"sort_{kind}")(got)
    assert bits_equal(got, exp, kind), first_diff(got, exp, kind)


def check_argsort(sorter, kind, keys):
    exp = oracle.argsort(kind, keys)
    before = keys.copy()
    got = getattr(sorter, f"argsort_{kind}")(keys)
    assert np.array_equal(got, exp), first_diff(got, exp, "u32")
    assert bits_equal(keys, before, kind), "argsort modified its input"


def check_pairs(sorter, kind, keys, vals):
    ek, ev = oracle.sort_pairs(kind, keys, vals)
    gk, gv = keys.copy(), vals.copy()
    getattr(sorter, f"sort_pairs_{kind}")(gk, gv)
    assert bits_equal(gk, ek, kind), first_diff(gk, ek, kind)
    assert np.array_equal(gv, ev), first_diff(gv, ev, "u32")


def check_buffer(sorter, kind, keys):
    exp = oracle.sort(kind, keys)
    buf = sorter.alloc_sort_buffer(kind, max(1, keys.size))
    buf.copy_from_slice(keys)
    fn = "sort_buffer" if kind == "u32" else f"sort_{kind}_buffer"
    getattr(sorter, fn)(buf)
    got = buf.as_slice()
    buf.free()
    assert bits_equal(got, exp, kind), first_diff(got, exp, kind)


# ---- golden vectors from the reference tests ---------------------------------

def load_golden():
    with open(GOLDEN) as f:
        return json.load(f)["cases"]


def golden_sort_cases():
    return [c for c in load_golden() if c["op"] != "gather"]


@pytest.mark.parametrize("case", golden_sort_cases(), ids=lambda c: c["name"])
def test_golden(sorter, case):
    kind = case["type"]
    keys = np.array(case["keys"], dtype=BITS[kind]).view(NP[kind])
    if case["op"] == "sort":
        got = keys.copy()
        getattr(sorter, f"sort_{kind}")(got)
        assert got.view(BITS[kind]).tolist() == case["expected_keys"]
        check_buffer(sorter, kind, keys)
    elif case["op"] == "argsort":
        assert getattr(sorter, f"argsort_{kind}")(keys).tolist() == case["expected_indices"]
    else:
        k, v = keys.copy(), np.array(case["values"], dtype=np.uint32)
        getattr(sorter, f"sort_pairs_{kind}")(k, v)
        assert k.view(BITS[kind]).tolist() == case["expected_keys"]
        assert v.tolist() == case["expected_values"]


# ---- edge cases and sizes ------------------------------------------------------

def make_keys(kind, n, dist, seed, tile=None):
    g = np.random.Generator(np.random.PCG64(seed))
    wide = BITS[kind] == np.uint64
    hi = 1 << (64 if wide else 32)
    if dist == "uniform":
        b = g.integers(0, hi, size=n, dtype=BITS[kind], endpoint=False)
    elif dist == "zeros":
        b = np.zeros(n, dtype=BITS[kind])
    elif dist == "same":
        b = np.full(n, 0xDEADBEEF, dtype=BITS[kind])
    elif dist == "sorted":
        b = np.sort(g.integers(0, hi, size=n, dtype=BITS[kind], endpoint=False))
    elif dist == "reverse":
        b = np.sort(g.integers(0, hi, size=n, dtype=BITS[kind], endpoint=False))[::-1].copy()
    elif dist == "few":
        b = g.choice(g.integers(0, hi, size=7, dtype=BITS[kind], endpoint=False), size=n)
    elif dist == "lowbits":
        b = g.integers(0, 1 << 12, size=n, dtype=BITS[kind])
    elif dist == "byte0":       # one varying digit, the lowest: single pass, then copy back
        b = g.integers(0, 256, size=n, dtype=BITS[kind])
    elif dist == "byte1":       # one varying digit above it: copy to scratch, then single pass
        b = (g.integers(0, 256, size=n, dtype=BITS[kind]) << BITS[kind](8)).astype(BITS[kind])
    elif dist == "skew0":       # lowest byte 3 or 200, the rest uniform
        b = g.integers(0, hi, size=n, dtype=BITS[kind], endpoint=False)
        b = (b & ~BITS[kind](0xFF)) | np.where(g.integers(0, 2, size=n) == 0, 3, 200).astype(BITS[kind])
    elif dist == "grp0":        # lowest byte 3 in the tiles ((tile / 8) % 8 == 0) of region group 0
        b = g.integers(0, hi, size=n, dtype=BITS[kind], endpoint=False)
        in0 = (np.arange(n) // tile // 8) % 8 == 0
        b[in0] = (b[in0] & ~BITS[kind](0xFF)) | BITS[kind](3)
    elif dist == "grp2":        # the byte below the top one (2; 6 of 64-bit keys) is 3 in the tiles of
        b = g.integers(0, hi, size=n, dtype=BITS[kind], endpoint=False)   # region group 0 (top-16 fused pass)
        in0 = (np.arange(n) // tile // 8) % 8 == 0
        sh = BITS[kind](48 if wide else 16)
        b[in0] = (b[in0] & ~(BITS[kind](0xFF) << sh)) | (BITS[kind](3) << sh)
    elif dist == "top8":        # the top byte only two values: segments far larger than a block holds
        top = 56 if wide else 24
        b = g.integers(0, 1 << top, size=n, dtype=BITS[kind])
        b |= np.where(g.integers(0, 2, size=n) == 0, 0x10, 0xF0).astype(BITS[kind]) << BITS[kind](top)
    elif dist == "dup":         # 2^16 distinct values: every key has ~n / 2^16 equal ones
        b = g.choice(g.integers(0, hi, size=1 << 16, dtype=BITS[kind], endpoint=False), size=n)
    elif dist == "zipf":        # Zipf(1.1) ranks below 2^20: a few huge segments, many tiny ones
        b = np.minimum(g.zipf(1.1, size=n) - 1, (1 << 20) - 1).astype(BITS[kind])
    else:
        raise ValueError(dist)
    keys = b.view(NP[kind])
    if kind in ("f32", "f64") and dist == "uniform" and n >= 16:
        specials = ([0x7FC00000, 0xFFC00001, 0x7F800000, 0xFF800000, 0, 0x80000000, 1, 0x80000001]
                    if kind == "f32" else
                    [0x7FF8000000000000, 0xFFF8000000000001, 0x7FF0000000000000,
                     0xFFF0000000000000, 0, 1 << 63, 1, (1 << 63) | 1])
        pos = g.choice(n, size=min(n, 64), replace=False)
        keys.view(BITS[kind])[pos] = np.array(specials, dtype=BITS[kind])[np.arange(pos.size) % 8]
    return keys


SIZES = [2, 3, 100, 255, 4095, 4096, 4097, 65543, 1_000_000]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n", SIZES)
def test_sort_sizes(sorter, kind, n):
    check_sort(sorter, kind, make_keys(kind, n, "uniform", seed=n))


@pytest.mark.parametrize("kind", ["u32", "i32", "f32"])
@pytest.mark.parametrize("n,dist", [((1 << 21) - 1, "uniform"), (1 << 21, "uniform"), ((1 << 21) - 1, "few"),
                                    (1_500_001, "byte1"), (6_144 * 7 + 5, "uniform")])
def test_small_tile_boundary(sorter, kind, n, dist):
    """Keys-only 32-bit sorts take the digit pass's small tiles below 2^21
    keys (FS_SMALL_TILE_KEYS) and the stable tiles from there: exact against
    the oracle on both sides, a single varying digit (the copy and the pass
    on the small tiles) and a ragged last tile."""
    keys = make_keys(kind, n, dist, seed=140 + n % 91)
    check_sort(sorter, kind, keys)
    check_buffer(sorter, kind, keys)


@pytest.mark.parametrize("kind", ["u32", "f32", "u64", "i64", "f64"])
def test_small_tile_boundary_values_and_64(sorter, kind):
    """Argsort and pairs below and at FS_SMALL_TILE_KEYS (32-bit keys), and
    64-bit sorts, argsort and pairs below and at FS_SMALL_TILE_KEYS64 (2^20):
    exact against the oracle on both tile sizes."""
    limit = (1 << 20) if kind.endswith("64") else (1 << 21)
    for n in (limit - 1, limit):
        keys = make_keys(kind, n, "few" if n % 2 else "uniform", seed=150 + n % 89)
        if kind.endswith("64"):
            check_sort(sorter, kind, keys)
        check_argsort(sorter, kind, keys)
        vals = np.random.Generator(np.random.PCG64(n)).integers(0, 1 << 32, size=n, dtype=np.uint32)
        check_pairs(sorter, kind, keys, vals)


TILE_VARIANT = {("sort", False): "k32", ("sort", True): "k64", ("argsort", False): "k32_v",
                ("argsort", True): "k64_v", ("pairs", False): "k32_v", ("pairs", True): "k64_v"}


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("op", ["sort", "argsort", "pairs"])
def test_tile_boundaries(sorter, kind, op):
    """Sizes at the edges of the kernel's own tile (read from the code object):
    one tile less one key, one tile, one tile plus one, two tiles plus one."""
    tile = sorter.tile_config()[TILE_VARIANT[(op, BITS[kind] == np.uint64)]]
    for n in (tile - 1, tile, tile + 1, 2 * tile + 1):
        keys = make_keys(kind, n, "few" if op == "argsort" else "uniform", seed=300 + n)
        if op == "sort":
            check_sort(sorter, kind, keys)
        elif op == "argsort":
            check_argsort(sorter, kind, keys)
        else:
            check_pairs(sorter, kind, keys, np.arange(n, dtype=np.uint32)[::-1].copy())


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dist", ["zeros", "same", "sorted", "reverse", "few", "lowbits"])
def test_sort_distributions(sorter, kind, dist):
    check_sort(sorter, kind, make_keys(kind, 100_003, dist, seed=7))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n", [2, 100, 4097, 65543, 1_000_000])
def test_argsort_sizes(sorter, kind, n):
    check_argsort(sorter, kind, make_keys(kind, n, "uniform", seed=100 + n))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dist", ["same", "few", "lowbits", "reverse"])
def test_argsort_ties(sorter, kind, dist):
    check_argsort(sorter, kind, make_keys(kind, 70_001, dist, seed=11))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n", [2, 100, 4097, 1_000_000])
@pytest.mark.parametrize("dist", ["uniform", "few"])
def test_pairs(sorter, kind, n, dist):
    keys = make_keys(kind, n, dist, seed=200 + n)
    vals = np.random.Generator(np.random.PCG64(n)).integers(0, 1 << 32, size=n, dtype=np.uint32)
    check_pairs(sorter, kind, keys, vals)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n", [0, 1])
def test_trivial_lengths(sorter, kind, n):
    keys = make_keys(kind, 2, "uniform", seed=1)[:n].copy()
    check_sort(sorter, kind, keys)
    assert getattr(sorter, f"argsort_{kind}")(keys).tolist() == list(range(n))
    vals = np.arange(n, dtype=np.uint32)
    getattr(sorter, f"sort_pairs_{kind}")(keys, vals)
    assert vals.tolist() == list(range(n))


@pytest.mark.parametrize("kind", KINDS)
def test_sort_buffer(sorter, kind):
    for n in (2, 4097, 300_007):
        check_buffer(sorter, kind, make_keys(kind, n, "uniform", seed=n + 3))


def test_length_mismatch_before_gpu_work(sorter):
    from forge_sort import LengthMismatch
    with pytest.raises(LengthMismatch, match="length mismatch: keys=3, values=2"):
        sorter.sort_pairs_u32(np.array([1, 2, 3], np.uint32), np.array([10, 20], np.uint32))


def test_buffer_reuse_and_interleaving(sorter):
    """regression.rs: one sorter across types and sizes, grow-only scratch reused."""
    for n, kind in [(1_000_000, "u32"), (1000, "f64"), (2_000_000, "i32"), (100, "u32"),
                    (500_000, "u64"), (3, "f32"), (1_500_000, "i64")]:
        check_sort(sorter, kind, make_keys(kind, n, "uniform", seed=n))
        check_argsort(sorter, kind, make_keys(kind, n // 2 + 2, "few", seed=n))


def test_deterministic(sorter):
    keys = make_keys("f32", 2_000_000, "few", seed=5)
    a = sorter.argsort_f32(keys)
    b = sorter.argsort_f32(keys)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("dist", ["byte0", "byte1"])
@pytest.mark.parametrize("kind", KINDS)
def test_single_pass_schedules(sorter, kind, dist):
    """Exactly one digit varies: the in-place sort runs one pass and moves the
    result to the caller's buffer through scratch (after the pass for the
    lowest digit, before it otherwise); argsort writes indices directly."""
    n = 300_007
    keys = make_keys(kind, n, dist, seed=17)
    check_sort(sorter, kind, keys)
    passes, mask = sorter.last_pass_info()
    assert passes == 1 and mask == (1 if dist == "byte0" else 2)
    check_argsort(sorter, kind, keys)
    if kind != "f64":                     # sort_pairs_{u32,i32,f32,u64,i64} (lib.rs)
        vals = np.random.Generator(np.random.PCG64(5)).integers(0, 1 << 32, size=n, dtype=np.uint32)
        check_pairs(sorter, kind, keys, vals)
    check_buffer(sorter, kind, keys)


def test_constant_digit_passes_skipped(sorter):
    keys = datagen.low20_u64(1_000_000, high=0x123456789AB)
    check_sort(sorter, "u64", keys)
    passes, mask = sorter.last_pass_info()
    assert passes == 3 and mask == 0b111


def test_encode_sort_async(sorter):
    keys = make_keys("u32", 1_000_003, "uniform", seed=9)
    buf = sorter.alloc_sort_buffer("u32", keys.size)
    buf.copy_from_slice(keys)
    sorter.encode_sort(buf)
    sorter.synchronize()
    assert bits_equal(buf.as_slice(), oracle.sort("u32", keys), "u32")
    buf.free()


def test_slice_staging_ragged_chunks(sorter):
    """Slice calls stage through two 8 MiB pinned host buffers: keys and values
    that span several chunks with a partial last one, one call after another
    (each reuses the buffers while the previous call's copies may be the last
    to have used them), the second call smaller than the first."""
    chunk_u64 = (8 << 20) // 8
    n = 3 * chunk_u64 + 12_345             # keys: 4 chunks; values: 2 chunks
    g = np.random.Generator(np.random.PCG64(131))
    check_pairs(sorter, "u64", datagen.uniform_u64(n, seed=132), g.integers(0, 2**32, n, dtype=np.uint32))
    check_pairs(sorter, "f32", datagen.f32_normal_specials(n - 77_777, seed=133),
                g.integers(0, 2**32, n - 77_777, dtype=np.uint32))
    check_argsort(sorter, "i64", datagen.uniform_i64(2 * chunk_u64 + 1, seed=134))
    check_sort(sorter, "f64", datagen.normal_f64(chunk_u64 + 3, seed=135))
    check_sort(sorter, "u32", datagen.uniform_u32(5, seed=136))


# ---- the fused first pass of keys-only sorts -----------------------------------------

FUSED_CASES = [
    # its regions feed the next pass: every digit varies; only digit 0 (the
    # regions copied back); digits 0 and 1
    (1_000_003, "uniform", 1), (16_777_216, "uniform", 1), (300_007, "byte0", 1), (2_000_000, "lowbits", 1),
    # regions sized by the sampled lowest byte: two values; one value
    (1_000_000, "skew0", 1), (500_000, "byte1", 1),
    # a region overflows (digit 3 crowded into region group 0, which the
    # input-wide sample underrates) or every digit is constant: the standard
    # schedule over the caller's keys
    (2_000_000, "grp0", 2), (100_003, "same", 2),
]


@pytest.mark.parametrize("kind", ["u32", "i32", "f32", "u64", "i64", "f64"])
@pytest.mark.parametrize("n,dist,expect", FUSED_CASES)
def test_fused_first_pass(sorter, kind, n, dist, expect):
    """Keys-only sorts begin with the fused first pass (one read that
    counts the upper digits and scatters by the lowest into regions), here
    forced at every size: exact against the oracle on both of its schedules,
    through the slice and buffer APIs; the histogram read gives the same keys."""
    from forge_sort import (FIRST_HISTOGRAM, FUSED_ALWAYS, FUSED_BY_SIZE, FUSED_NEVER, TEST_FUSED, TEST_TOP16,
                            TOP16_BY_SIZE, TOP16_NEVER)
    keys = make_keys(kind, n, dist, seed=900 + n % 97,
                     tile=sorter.tile_config()[TILE_VARIANT[("sort", BITS[kind] == np.uint64)]])
    sorter.set_test_option(TEST_FUSED, FUSED_ALWAYS)
    sorter.set_test_option(TEST_TOP16, TOP16_NEVER)      # (64-bit keys take it by size from 2^21 keys)
    try:
        check_sort(sorter, kind, keys)
        assert sorter.first_pass() == expect
        passes, mask = sorter.last_pass_info()
        if dist == "same":
            assert (passes, mask) == (0, 0)
        elif dist == "uniform":
            assert (passes, mask) == ((8, 0xFF) if kind.endswith("64") else (4, 0xF))
        check_buffer(sorter, kind, keys)
        assert sorter.first_pass() == expect
        sorter.set_test_option(TEST_FUSED, FUSED_NEVER)
        check_sort(sorter, kind, keys)
        assert sorter.first_pass() == FIRST_HISTOGRAM
        # the same digits run, but a fused pass that used its regions counts
        # as digit 0's pass even where digit 0 is constant
        hp, hm = sorter.last_pass_info()
        assert hm == (mask & ~1 if expect == 1 and dist == "byte1" else mask) and hp == bin(hm).count("1")
    finally:
        sorter.set_test_option(TEST_TOP16, TOP16_BY_SIZE)
        sorter.set_test_option(TEST_FUSED, FUSED_BY_SIZE)


@pytest.mark.parametrize("kind,n,expect", [("u32", 1 << 25, 1), ("f32", 1 << 25, 1), ("u32", (1 << 25) - 1, 0),
                                            ("u32", 1 << 20, 0), ("u32", 44_040_192 - 1, 1), ("u32", 44_040_192, 3),
                                            ("u64", (1 << 21) - 1, 0), ("i64", 1 << 21, 3), ("f64", 1 << 21, 0)])
def test_fused_first_pass_by_size(sorter, kind, n, expect):
    """By default the fused first pass starts at FS_FUSED_MIN_KEYS keys, and
    keys-only integer sorts take the top-16 path from FS_TOP16_MIN_KEYS32
    (u32/i32) or FS_TOP16_MIN_KEYS64 (u64/i64) keys, 64-bit keys below the
    fused range too; float keys never."""
    from forge_sort import TOP16_MIN_KEYS32, TOP16_MIN_KEYS64
    assert (TOP16_MIN_KEYS32, TOP16_MIN_KEYS64) == (44_040_192, 1 << 21)
    keys = make_keys(kind, n, "uniform", seed=950)
    check_buffer(sorter, kind, keys)
    assert sorter.first_pass() == expect


# ---- the top-16 path of keys-only u32/i32 sorts -------------------------------------

TOP16_CASES = [
    # trivial, ragged and mid sizes (segments of the top 8 bits up to 16)
    (2, "uniform", 3), (100, "uniform", 3), (4097, "uniform", 3), (1_000_003, "uniform", 3),
    (16_777_216, "uniform", 3),
    # sorted input: each digit-2 value comes in one short run per digit-3
    # value, so the region groups' shares of it vary and a region may
    # overflow (3 or 4)
    (5_000_000, "sorted", (3, 4)), (3_000_001, "reverse", (3, 4)),
    # constant digits: only the lowest varies, only the low 12 bits vary, a
    # few values; skewed segments (Zipf ranks, two top-byte values) larger
    # than a block holds, sorted a digit at a time by their block
    (300_007, "byte0", 3), (2_000_000, "lowbits", 3), (1_000_000, "few", 3), (2_000_003, "zipf", 3),
    (3_000_000, "top8", 3),
    # a region of the fused pass overflows (byte 2 crowded into region
    # group 0): its second launch re-scatters into exact regions
    (2_000_000, "grp2", 4), (17_000_000, "grp2", 4),
    # every key equal, forced onto the top-16 path (its fused pass counts
    # digit 3 only, so it cannot see the constant digits): one segment of
    # every key, sorted by its block a digit at a time
    (100_003, "same", 3),
]


@pytest.mark.parametrize("kind", ["u32", "i32"])
@pytest.mark.parametrize("n,dist,expect", TOP16_CASES)
def test_top16_path(sorter, kind, n, dist, expect):
    """Keys-only u32/i32 sorts on the top-16 path (fused pass on digit 2,
    stable pass on digit 3 counting the segments, local sort of each
    segment), forced at every size: exact against the oracle through the
    slice and buffer APIs, and beginning the way the case names."""
    from forge_sort import TEST_TOP16, TOP16_ALWAYS, TOP16_BY_SIZE
    keys = make_keys(kind, n, dist, seed=960 + n % 89, tile=sorter.tile_config()["k32"])
    sorter.set_test_option(TEST_TOP16, TOP16_ALWAYS)
    try:
        expect = expect if isinstance(expect, tuple) else (expect,)
        check_sort(sorter, kind, keys)
        assert sorter.first_pass() in expect
        check_buffer(sorter, kind, keys)
        assert sorter.first_pass() in expect
    finally:
        sorter.set_test_option(TEST_TOP16, TOP16_BY_SIZE)


TOP16_CASES_64 = [
    (2, "uniform", 3), (100, "uniform", 3), (4097, "uniform", 3), (1_000_003, "uniform", 3),
    (16_777_216, "uniform", 3), (5_000_000, "sorted", (3, 4)), (3_000_001, "reverse", (3, 4)),
    (300_007, "byte0", 3), (2_000_000, "lowbits", 3), (1_000_000, "few", 3), (2_000_003, "zipf", 3),
    (3_000_000, "top8", 3), (2_000_000, "grp2", 4), (100_003, "same", 3),
    # many equal keys per segment: groups above the comparison limit, each
    # segment sorted by the LSD passes in LDS instead
    (8_000_000, "dup", 3), (300_000, "dup", 3),
]


@pytest.mark.parametrize("kind", ["u64", "i64"])
@pytest.mark.parametrize("n,dist,expect", TOP16_CASES_64)
def test_top16_path_64(sorter, kind, n, dist, expect):
    """Keys-only u64/i64 sorts on the top-16 path (fused pass on byte 6,
    stable pass on byte 7 counting the segments, group sort of each
    segment), forced at every size: exact against the oracle through the
    slice and buffer APIs, and beginning the way the case names."""
    from forge_sort import TEST_TOP16, TOP16_ALWAYS, TOP16_BY_SIZE
    keys = make_keys(kind, n, dist, seed=990 + n % 89, tile=sorter.tile_config()["k64"])
    sorter.set_test_option(TEST_TOP16, TOP16_ALWAYS)
    try:
        expect = expect if isinstance(expect, tuple) else (expect,)
        check_sort(sorter, kind, keys)
        assert sorter.first_pass() in expect
        check_buffer(sorter, kind, keys)
        assert sorter.first_pass() in expect
    finally:
        sorter.set_test_option(TEST_TOP16, TOP16_BY_SIZE)


@pytest.mark.parametrize("dist,expect", [("uniform", (3,)), ("lowbits", (1,)), ("top8", (1,)), ("zipf", (1, 2)),
                                         ("same", (2,))])
def test_top16_sample_chooses(sorter, dist, expect):
    """By size (FS_TOP16_MIN_KEYS32 + 7 u32 keys) the region sample chooses: the top-16
    path for a uniform input; the LSD passes in the same launches when it
    sees oversized segments (keys below 2^12, two top-byte values, Zipf ranks
    below 2^20, whose lowest byte may overflow a region: re-scattered); no
    pass after the fused one when every digit is constant."""
    keys = make_keys("u32", 44_040_192 + 7, dist, seed=975)
    check_buffer(sorter, "u32", keys)
    assert sorter.first_pass() in expect


@pytest.mark.parametrize("kind", ["u64", "i64", "f64"])
@pytest.mark.parametrize("dist", ["uniform", "lowbits", "top8", "same"])
def test_top16_sample_chooses_64(sorter, kind, dist):
    """The same by size for 2^25 + 7 64-bit keys: u64/i64 uniform keys take
    the top-16 path, the others the LSD passes in the same launches (none
    after the fused pass for equal keys); f64 keys always the fused LSD
    passes (float keys do not take the top-16 launch sequence)."""
    keys = make_keys(kind, (1 << 25) + 7, dist, seed=976)
    check_buffer(sorter, kind, keys)
    expect = {"uniform": (3,), "lowbits": (1,), "top8": (1,), "same": (2,)}[dist]
    if kind == "f64":
        expect = (1, 2)
    assert sorter.first_pass() in expect


@pytest.mark.parametrize("bits", [8, 11, 12, 13, 14, 15, 16])
@pytest.mark.parametrize("dist", ["uniform", "few"])
def test_top16_segment_bits(sorter, bits, dist):
    """Every local-sort plan (the segment bits set how many low bits each
    block sorts: 16 bits as 10 + 6, 17-19 as the rest + 8, more as the rest
    + 8 + 8), and segments that are empty, tiny or larger than a block."""
    from forge_sort import TEST_SEG_BITS, TEST_TOP16, TOP16_ALWAYS, TOP16_BY_SIZE
    keys = make_keys("u32", 3_000_017, dist, seed=970 + bits)
    sorter.set_test_option(TEST_TOP16, TOP16_ALWAYS)
    sorter.set_test_option(TEST_SEG_BITS, bits)
    try:
        check_buffer(sorter, "u32", keys)
        assert sorter.first_pass() == 3
    finally:
        sorter.set_test_option(TEST_SEG_BITS, 0)
        sorter.set_test_option(TEST_TOP16, TOP16_BY_SIZE)


def top16_limits(block_keys):
    """The largest input the top-16 path takes on blocks of block_keys
    keys: 2^16 segments of a uniform input within a block, with a five-sigma
    margin."""
    import math
    return (block_keys - 5 * math.isqrt(block_keys)) << 16


def test_top16_size_limit(sorter):
    """The largest input the top-16 path sorts on its 4,608-key local-sort
    blocks (gfx950 build: 256 x 18) and one key more (the wide 9,216-key
    blocks), the largest it sorts on those and one key more (the fused LSD
    passes): ascending, same multiset."""
    limit, wlimit = top16_limits(256 * 18), top16_limits(512 * 18)
    assert (limit, wlimit) == (280_035_328, 572_522_496)
    for n, expect in ((limit, 3), (limit + 1, 3), (wlimit, 3), (wlimit + 1, 1)):
        keys = datagen.uniform_u32(n, seed=980)
        k64 = keys.astype(np.uint64)
        s_sum, s_xor = int(k64.sum()), int(np.bitwise_xor.reduce(keys))
        del k64
        buf = sorter.alloc_sort_buffer("u32", n)
        buf.copy_from_slice(keys)
        del keys
        sorter.sort_buffer(buf)
        assert sorter.first_pass() == expect
        out = buf.as_slice()
        buf.free()
        assert bool(np.all(out[1:] >= out[:-1])), "not ascending"
        assert (int(out.astype(np.uint64).sum()), int(np.bitwise_xor.reduce(out))) == (s_sum, s_xor)
        del out


def test_top16_size_limit_64(sorter):
    """The same for u64 keys: 2,304-key blocks of the 64-bit local sort
    (256 x 9), then the wide 4,608-key blocks, then the fused LSD passes:
    ascending, same multiset."""
    limit, wlimit = top16_limits(256 * 9), top16_limits(512 * 9)
    assert (limit, wlimit) == (135_266_304, 280_035_328)
    g = np.random.Generator(np.random.PCG64(981))
    for n, expect in ((limit, 3), (limit + 1, 3), (wlimit, 3), (wlimit + 1, 1)):
        keys = g.integers(0, 1 << 64, size=n, dtype=np.uint64, endpoint=False)
        s_sum = int(np.bitwise_xor.reduce(keys)), int((keys & np.uint64(0xFFFFFFFF)).sum()), int((keys >> np.uint64(32)).sum())
        buf = sorter.alloc_sort_buffer("u64", n)
        buf.copy_from_slice(keys)
        del keys
        sorter.sort_u64_buffer(buf)
        assert sorter.first_pass() == expect
        out = buf.as_slice()
        buf.free()
        assert bool(np.all(out[1:] >= out[:-1])), "not ascending"
        assert (int(np.bitwise_xor.reduce(out)), int((out & np.uint64(0xFFFFFFFF)).sum()),
                int((out >> np.uint64(32)).sum())) == s_sum
        del out


WIDE_CASES = [(100, "uniform", 3), (4097, "uniform", 3), (1_000_003, "uniform", 3), (3_000_000, "few", 3),
              (2_000_000, "dup", 3), (3_000_000, "top8", 3), (2_000_000, "grp2", 4), (16_777_216, "uniform", 3)]


@pytest.mark.parametrize("kind", ["u32", "i32", "u64", "i64"])
@pytest.mark.parametrize("n,dist,expect", WIDE_CASES)
def test_top16_wide_blocks(sorter, kind, n, dist, expect):
    """The top-16 path with its wide local-sort blocks (512 threads, which
    inputs beyond the other blocks' size limit take), forced at every size:
    exact against the oracle through the slice and buffer APIs; segments
    that are tiny, larger than a block (two top-byte values), full of equal
    keys; a re-scattered region."""
    from forge_sort import TEST_LOCAL_WIDE, TEST_TOP16, TOP16_ALWAYS, TOP16_BY_SIZE
    keys = make_keys(kind, n, dist, seed=995 + n % 83,
                     tile=sorter.tile_config()["k64" if BITS[kind] == np.uint64 else "k32"])
    sorter.set_test_option(TEST_TOP16, TOP16_ALWAYS)
    sorter.set_test_option(TEST_LOCAL_WIDE, 1)
    try:
        check_sort(sorter, kind, keys)
        assert sorter.first_pass() == expect
        check_buffer(sorter, kind, keys)
        assert sorter.first_pass() == expect
    finally:
        sorter.set_test_option(TEST_LOCAL_WIDE, 0)
        sorter.set_test_option(TEST_TOP16, TOP16_BY_SIZE)


def test_fused_first_pass_2_31_keys(sorter):
    """The largest fused sort (n = 2^31, regions of S1 just below 2^32 keys
    in all) and one key more (the histogram read): ascending, same multiset."""
    for n, expect in ((1 << 31, 1), ((1 << 31) + 1, 0)):
        keys = datagen.uniform_u32(n, seed=501)
        k64 = keys.astype(np.uint64)
        s_sum, s_sq, s_xor = int(k64.sum()), int((k64 * k64).sum()), int(np.bitwise_xor.reduce(keys))
        del k64
        buf = sorter.alloc_sort_buffer("u32", n)
        buf.copy_from_slice(keys)
        del keys
        sorter.sort_buffer(buf)
        assert sorter.first_pass() == expect
        out = buf.as_slice()
        buf.free()
        assert bool(np.all(out[1:] >= out[:-1])), "not ascending"
        o64 = out.astype(np.uint64)
        assert (int(o64.sum()), int((o64 * o64).sum()), int(np.bitwise_xor.reduce(out))) == (s_sum, s_sq, s_xor)
        del out, o64


# ---- BASELINE.json configurations at full size ------------------------------------

def test_config0_sort_u32_1m(sorter):
    check_sort(sorter, "u32", datagen.uniform_u32(1 << 20, seed=101))


@pytest.mark.parametrize("n", [16_777_216, 16_000_000, 268_435_456])
def test_config1_sort_buffer_u32(sorter, n):
    check_buffer(sorter, "u32", datagen.uniform_u32(n, seed=102))


def test_config2_sort_f32_specials(sorter):
    keys = datagen.f32_normal_specials(1 << 26, seed=103)
    check_sort(sorter, "f32", keys)


def test_config2_sort_i32(sorter):
    check_sort(sorter, "i32", datagen.uniform_i32(1 << 26, seed=104))


def test_config3_argsort_f32_ties(sorter):
    check_argsort(sorter, "f32", datagen.argsort_f32_ties(1 << 24, seed=105))


def test_config3_pairs_zipf(sorter):
    keys, vals = datagen.zipf_pairs_u32(1 << 26, seed=106)
    check_pairs(sorter, "u32", keys, vals)


@pytest.mark.parametrize("kind", ["u64", "i64", "f64", "low20_zero", "low20_const"])
def test_config4_64bit(sorter, kind):
    n = 134_217_728
    if kind == "u64":
        check_buffer(sorter, "u64", datagen.uniform_u64(n, seed=107))
    elif kind == "i64":
        check_buffer(sorter, "i64", datagen.uniform_i64(n, seed=108))
    elif kind == "f64":
        check_buffer(sorter, "f64", datagen.normal_f64(n, seed=109))
    elif kind == "low20_zero":
        check_buffer(sorter, "u64", datagen.low20_u64(n, high=0, seed=110))
    else:
        check_buffer(sorter, "u64", datagen.low20_u64(n, high=0xABCDEF01234, seed=111))


@pytest.mark.parametrize("kind,n", [("u32", 100_000_003), ("i32", 150_000_001), ("u64", 50_000_017),
                                    ("i64", 3_000_001), ("u64", 200_000_003)])
def test_top16_between_powers_of_two(sorter, kind, n):
    """The top-16 path at sizes that are not powers of two (segment bits
    chosen so that a uniform input's segments fit a block; u64 200M on the
    wide blocks): exact against the oracle."""
    if kind.endswith("32"):
        keys = datagen.uniform_u32(n, seed=990 + n % 13)
        keys = keys.view(np.int32) if kind == "i32" else keys
    else:
        keys = datagen.uniform_u64(n, seed=991 + n % 13)
        keys = keys.view(np.int64) if kind == "i64" else keys
    check_buffer(sorter, kind, keys)
    assert sorter.first_pass() == 3


@pytest.mark.parametrize("kind,n,dist", [
    ("u32", 1 << 28, "below 2^24"), ("i32", 1 << 28, "[-2^23, 2^23)"),
    ("u64", 1 << 27, "below 2^40"), ("u64", 1 << 27, "below 2^48")])
def test_top16_refused_full_size(sorter, kind, n, dist):
    """Narrow keys at the top-16 path's sizes: their top 16 bits take few
    values, the region sample refuses the path, and the LSD passes run in the
    same launch sequence's digit-pass slots (one block per tile; 64-bit keys
    from the fifth slot on, the persistent loop kernel: below 2^48 takes
    slot 4).  Exact against the oracle."""
    from forge_sort import FIRST_FUSED, FIRST_FUSED_OVERFLOW
    g = np.random.Generator(np.random.PCG64(140 + n % 97 + len(dist)))
    if kind == "i32":
        keys = g.integers(-(1 << 23), 1 << 23, size=n, dtype=np.int32)
    else:
        top = {"below 2^24": 1 << 24, "below 2^40": 1 << 40, "below 2^48": 1 << 48}[dist]
        keys = g.integers(0, top, size=n, dtype=np.uint32 if kind == "u32" else np.uint64)
    check_buffer(sorter, kind, keys)
    assert sorter.first_pass() in (FIRST_FUSED, FIRST_FUSED_OVERFLOW)


@pytest.fixture
def force_wide_lookback(sorter):
    """Select the 64-bit look-back tile entries (normally used from n = 2^30
    on) for every sort of the test, through the sorter's testing hook."""
    from forge_sort import TEST_WIDE_LOOKBACK
    sorter.set_test_option(TEST_WIDE_LOOKBACK, 1)
    yield
    sorter.set_test_option(TEST_WIDE_LOOKBACK, 0)


@pytest.mark.parametrize("kind", KINDS)
def test_wide_lookback_entries(sorter, force_wide_lookback, kind):
    n = 1_000_003
    check_sort(sorter, kind, make_keys(kind, n, "uniform", seed=400))
    check_argsort(sorter, kind, make_keys(kind, 70_001, "few", seed=401))
    check_pairs(sorter, kind, make_keys(kind, 100_000, "uniform", seed=402),
                np.arange(100_000, dtype=np.uint32)[::-1].copy())


def test_upsweep_counter_folds_u64(sorter):
    """300M equal u64 keys: each upsweep block counts several chunks, and every
    16-bit counter of the one occupied bin takes its largest per-chunk count
    before each fold.  The histogram must still be exact: all 8 digits are
    found constant, no pass runs, and the keys are unchanged.  Then one key
    differs in its low byte: digit 0 alone must be found varying (one pass)."""
    n = 300_000_000
    c = np.uint64(0x0123456789ABCDEF)
    keys = np.full(n, c, dtype=np.uint64)
    buf = sorter.alloc_sort_buffer("u64", n)
    buf.copy_from_slice(keys)
    sorter.sort_u64_buffer(buf)
    assert sorter.last_pass_info() == (0, 0)
    out = buf.as_slice()
    assert bool(np.all(out == c))
    keys[n // 2] = c ^ np.uint64(0x5A)           # one key differs in its low byte
    buf.copy_from_slice(keys)
    sorter.sort_u64_buffer(buf)
    assert sorter.last_pass_info() == (1, 0b1)
    out = buf.as_slice()
    buf.free()
    # c's low byte is 0xEF; the odd key's is 0xB5, so it sorts first
    assert int(out[0]) == int(c ^ np.uint64(0x5A)) and bool(np.all(out[1:] == c))


def test_more_than_2_30_keys(sorter):
    """n = 2^30 + 12345 u32 keys: inclusive prefixes exceed 30 bits, so the
    64-bit look-back entries are in use.  Checked without the oracle (too slow
    at this size) by properties that fix the result: ascending order and equal
    multisets (sum, xor and sum of squares mod 2^64 of the keys)."""
    n = (1 << 30) + 12345
    keys = datagen.uniform_u32(n, seed=500)
    buf = sorter.alloc_sort_buffer("u32", n)
    buf.copy_from_slice(keys)
    sorter.sort_buffer(buf)
    out = buf.as_slice()
    buf.free()
    assert bool(np.all(out[1:] >= out[:-1])), "not ascending"
    k64, o64 = keys.astype(np.uint64), out.astype(np.uint64)
    assert int(k64.sum()) == int(o64.sum())
    assert int(np.bitwise_xor.reduce(keys)) == int(np.bitwise_xor.reduce(out))
    assert int((k64 * k64).sum()) == int((o64 * o64).sum())


def test_n_within_a_tile_of_2_32(sorter):
    """n = 2^32 - 1, the largest length: the last tile's key indices run past
    2^32 (they are kept in 64 bits).  Keys i & 0xFFFF, so two digits vary;
    value v then occurs (n - 1 - v) // 65536 + 1 times, and the output is
    checked against that closed form: ascending, and every value's first and
    last positions where the counts put them."""
    n = (1 << 32) - 1
    keys = np.arange(n, dtype=np.uint32)
    keys &= np.uint32(0xFFFF)
    buf = sorter.alloc_sort_buffer("u32", n)
    buf.copy_from_slice(keys)
    del keys
    sorter.sort_buffer(buf)
    passes, mask = sorter.last_pass_info()
    assert passes == 2 and mask == 0b11
    out = buf.as_slice()
    buf.free()
    step = 1 << 28
    for s0 in range(0, n, step):
        c = out[s0:min(n, s0 + step + 1)]
        assert bool(np.all(c[1:] >= c[:-1])), f"not ascending near {s0}"
    v = np.arange(1 << 16, dtype=np.int64)
    counts = (n - 1 - v) // (1 << 16) + 1
    first = np.concatenate([[0], np.cumsum(counts)[:-1]])
    assert int(counts.sum()) == n
    assert np.array_equal(np.searchsorted(out, v.astype(np.uint32), side="left"), first)
    assert np.array_equal(out[first + counts - 1].astype(np.int64), v)


@pytest.mark.parametrize("kind", ["u32", "f32", "u64", "i64"])
def test_device_keys_off_16_byte_boundary(sorter, kind):
    """Keys one element past a 16-byte boundary (e.g. a slice of a larger
    device array): the upsweep reads them one at a time."""
    import ctypes
    import forge_sort
    n = 300_007
    keys = make_keys(kind, n, "uniform", seed=600)
    size = keys.itemsize
    buf = sorter.alloc_sort_buffer(kind, n + 1)
    ptr = buf.device_ptr() + size
    L = forge_sort._load()
    sorter._check(L.fs_copy_to_device(sorter._h, ctypes.c_void_p(ptr), keys.ctypes.data, n * size))
    sorter.sort_device(kind, ptr, n)
    out = np.empty_like(keys)
    sorter._check(L.fs_copy_to_host(sorter._h, out.ctypes.data, ctypes.c_void_p(ptr), n * size))
    buf.free()
    exp = oracle.sort(kind, keys)
    assert bits_equal(out, exp, kind), first_diff(out, exp, kind)



# ---- GpuGather (forge-runtime/src/gather.rs) ----------------------------------

@pytest.fixture(scope="module")
def gatherer():
    from forge_sort import GpuGather
    g = GpuGather.new()
    yield g
    g.close()


def gpu_gather(gatherer, src, idx):
    """Device copies of src and idx, gather, copy back (through the library)."""
    import ctypes
    import forge_sort
    L = forge_sort._load()
    is64 = src.dtype == np.uint64
    ps = gatherer.alloc_buffer(max(1, src.nbytes))
    pi = gatherer.alloc_buffer(max(1, idx.nbytes))
    po = gatherer.alloc_buffer(max(1, idx.size * src.itemsize))
    try:
        with_sorter = forge_sort.GpuSorter.new()
        with_sorter._check(L.fs_copy_to_device(with_sorter._h, ctypes.c_void_p(ps), src.ctypes.data, src.nbytes))
        with_sorter._check(L.fs_copy_to_device(with_sorter._h, ctypes.c_void_p(pi), idx.ctypes.data, idx.nbytes))
        (gatherer.gather_u64 if is64 else gatherer.gather_u32)(ps, pi, po, idx.size, src.size)
        out = np.empty(idx.size, dtype=src.dtype)
        with_sorter._check(L.fs_copy_to_host(with_sorter._h, out.ctypes.data, ctypes.c_void_p(po),
                                             idx.size * src.itemsize))
        with_sorter.close()
        return out
    finally:
        for p in (ps, pi, po):
            gatherer.free_buffer(p)


@pytest.mark.parametrize("case", [c for c in load_golden() if c["op"] == "gather"], ids=lambda c: c["name"])
def test_gather_golden(gatherer, case):
    src = np.array(case["values"], dtype=BITS[case["type"]])
    got = gpu_gather(gatherer, src, np.array(case["indices"], dtype=np.uint32))
    assert got.tolist() == case["expected_values"]


@pytest.mark.parametrize("dtype", [np.uint32, np.uint64])
@pytest.mark.parametrize("n", [1, 255, 100_003, 4_000_000])
def test_gather_random(gatherer, dtype, n):
    g = np.random.Generator(np.random.PCG64(n))
    src = g.integers(0, 1 << 63, size=n, dtype=np.uint64).astype(dtype)
    idx = g.integers(0, n, size=n + 17, dtype=np.uint32)
    assert np.array_equal(gpu_gather(gatherer, src, idx), oracle.gather(src, idx))


def test_gather_index_out_of_range(gatherer):
    from forge_sort import GpuExecution
    src = np.arange(10, dtype=np.uint32)
    with pytest.raises(GpuExecution, match="out of range"):
        gpu_gather(gatherer, src, np.array([0, 10, 3], dtype=np.uint32))
    # the gather stays usable afterwards
    assert gpu_gather(gatherer, src, np.array([9, 0], dtype=np.uint32)).tolist() == [9, 0]


def test_sort_then_gather(sorter, gatherer):
    """forge-runtime's sort -> gather pipeline (tests/pipeline_tests.rs:168-205):
    argsort a column, gather a second column through the permutation; the
    result equals the pairs sort of the same data."""
    n = 100_000
    g = np.random.Generator(np.random.PCG64(77))
    keys = g.integers(0, 1000, size=n, dtype=np.uint32)
    other = g.integers(0, 1 << 63, size=n, dtype=np.uint64)
    perm = sorter.argsort_u32(keys)
    got = gpu_gather(gatherer, other, perm)
    assert np.array_equal(got, other[oracle.argsort("u32", keys)])


# ---- hipCUB DeviceRadixSort as an independent cross-check -----------------------

@pytest.fixture(scope="module")
def hipcub():
    """tests/hipcub_xcheck/_build/libhipcub_xcheck.so (built by __graft_entry__.build())."""
    import ctypes
    path = os.path.join(os.path.dirname(__file__), "hipcub_xcheck", "_build", "libhipcub_xcheck.so")
    assert os.path.exists(path), f"{path} not built: run __graft_entry__.build()"
    L = ctypes.CDLL(path)
    vp, u64 = ctypes.c_void_p, ctypes.c_uint64
    fp = ctypes.POINTER(ctypes.c_float)
    L.xc_sort_keys_u32.argtypes = [vp, vp, u64, fp]
    L.xc_sort_keys_u64.argtypes = [vp, vp, u64, fp]
    L.xc_sort_pairs_u32.argtypes = [vp, vp, vp, vp, u64, fp]
    return L


@pytest.mark.parametrize("kind,n", [("u32", 16_777_216), ("u32", 1_000_003), ("u64", 4_000_037)])
def test_hipcub_crosscheck_keys(sorter, hipcub, kind, n):
    """Keys sorted by this library and by hipCUB (ROCm's rocPRIM radix sort) are
    identical, on device buffers."""
    import ctypes
    keys = make_keys(kind, n, "uniform", seed=700 + n)
    a = sorter.alloc_sort_buffer(kind, n)
    b = sorter.alloc_sort_buffer(kind, n)
    a.copy_from_slice(keys)
    ms = ctypes.c_float()
    fn = hipcub.xc_sort_keys_u32 if kind == "u32" else hipcub.xc_sort_keys_u64
    assert fn(ctypes.c_void_p(a.device_ptr()), ctypes.c_void_p(b.device_ptr()), n, ctypes.byref(ms)) == 0
    sorter.sort_device(kind, a.device_ptr(), n)
    a.set_len(n)
    b.set_len(n)
    ours, theirs = a.as_slice(), b.as_slice()
    a.free()
    b.free()
    assert bits_equal(ours, theirs, kind), first_diff(ours, theirs, kind)
    print(f"hipCUB SortKeys {kind} n={n}: {ms.value:.3f} ms")


def test_hipcub_crosscheck_pairs(sorter, hipcub):
    """Stable pairs: hipCUB's SortPairs order equals this library's (ties by
    original position)."""
    import ctypes
    n = 5_000_011
    keys = make_keys("u32", n, "few", seed=710)
    vals = np.arange(n, dtype=np.uint32)
    bufs = [sorter.alloc_sort_buffer("u32", n) for _ in range(4)]
    bufs[0].copy_from_slice(keys)
    bufs[2].copy_from_slice(vals)
    ms = ctypes.c_float()
    assert hipcub.xc_sort_pairs_u32(*[ctypes.c_void_p(b.device_ptr()) for b in (bufs[0], bufs[1], bufs[2], bufs[3])],
                                    n, ctypes.byref(ms)) == 0
    sorter.sort_pairs_device("u32", bufs[0].device_ptr(), bufs[2].device_ptr(), n)
    out = []
    for b in bufs:
        b.set_len(n)
        out.append(b.as_slice())
        b.free()
    assert np.array_equal(out[0], out[1]) and np.array_equal(out[2], out[3])


# ---- caller streams (with_context, encode on a given stream) ---------------------

@pytest.fixture(scope="module")
def hip_stream():
    """A HIP stream of the caller, created through the HIP runtime the library
    itself is linked against."""
    import ctypes
    import forge_sort
    forge_sort._load()                                   # libamdhip64 is loaded with it
    hip = ctypes.CDLL("libamdhip64.so.7")
    st = ctypes.c_void_p()
    assert hip.hipStreamCreate(ctypes.byref(st)) == 0
    yield st.value
    hip.hipStreamSynchronize(st)
    hip.hipStreamDestroy(st)


@pytest.mark.parametrize("op", ["pairs", "sort"])
def test_graph_capture_replays(hip_stream, op):
    """The sort is capturable into a HIP graph: fs_encode on a capturing stream
    records kernel launches only (no memset; the scratch has grown beforehand,
    and the kernels reset the histogram copies, the region cursors, the ticket
    and the look-back entries themselves).  Each replay sorts new data with its
    own device-side schedule (pairs: 4, 4, 2 and 1 passes; keys only: the
    fused first pass's regions, an overflowing region, equal keys, only digit
    0 varying), eager sorts run between the replays, and every replay matches
    the oracle."""
    import ctypes
    from forge_sort import FUSED_ALWAYS, OP_PAIRS, OP_SORT, TEST_FUSED, GpuSorter
    hip = ctypes.CDLL("libamdhip64.so.7")
    st = ctypes.c_void_p(hip_stream)
    s = GpuSorter.with_context(0, hip_stream)
    graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
    pairs = op == "pairs"
    code = OP_PAIRS if pairs else OP_SORT
    s.set_test_option(TEST_FUSED, FUSED_ALWAYS)       # keys only: the fused first pass at this size
    try:
        n, n_other = 1_000_003, 200_001
        g = np.random.Generator(np.random.PCG64(904))
        kb, vb = s.alloc_sort_buffer("u32", n), s.alloc_sort_buffer("u32", n)
        kb.copy_from_slice(make_keys("u32", n, "uniform", seed=900))
        vb.copy_from_slice(g.integers(0, 1 << 32, size=n, dtype=np.uint32))
        s.encode(code, "u32", kb.device_ptr(), vb.device_ptr(), n, stream=hip_stream)
        s.reserve(OP_SORT, "u32", n_other)    # the eager sorts between the replays
        s.synchronize()                       # scratch grown: the captured sort allocates nothing
        assert hip.hipStreamBeginCapture(st, 0) == 0
        s.encode(code, "u32", kb.device_ptr(), vb.device_ptr(), n, stream=hip_stream)
        assert hip.hipStreamEndCapture(st, ctypes.byref(graph)) == 0
        assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, ctypes.c_size_t(0)) == 0
        dists = ["uniform", "few", "lowbits", "byte1"] if pairs else ["uniform", "skew0", "grp0", "same", "byte0",
                                                                       "uniform"]
        for r, dist in enumerate(dists):
            keys = make_keys("u32", n, dist, seed=910 + r, tile=s.tile_config()["k32"])
            vals = g.integers(0, 1 << 32, size=n, dtype=np.uint32)
            kb.copy_from_slice(keys)
            vb.copy_from_slice(vals)
            assert hip.hipGraphLaunch(exe, st) == 0
            assert hip.hipStreamSynchronize(st) == 0
            if pairs:
                ek, ev = oracle.sort_pairs("u32", keys, vals)
                assert np.array_equal(kb.as_slice(), ek) and np.array_equal(vb.as_slice(), ev), f"replay {r} ({dist})"
            else:
                assert np.array_equal(kb.as_slice(), oracle.sort("u32", keys)), f"replay {r} ({dist})"
            other = make_keys("u32", n_other, "uniform", seed=950 + r)   # eager work between replays
            got = other.copy()
            s.sort_u32(got)
            assert np.array_equal(got, oracle.sort("u32", other))
        kb.free()
        vb.free()
    finally:
        if exe.value:
            hip.hipGraphExecDestroy(exe)
        if graph.value:
            hip.hipGraphDestroy(graph)
        s.close()


@pytest.mark.parametrize("wide", [False, True], ids=["blocks", "wide_blocks"])
@pytest.mark.parametrize("kind", ["u32", "u64"])
def test_graph_capture_replays_top16(hip_stream, kind, wide):
    """The top-16 launch sequence captured once and replayed on new data: the
    region sample inside the graph picks, per replay, the top-16 path
    (uniform keys; a region overflow re-scattered; many equal keys, whose
    64-bit segments go to the deferred launch) or the LSD passes in the same
    launches (two top-byte values), or nothing after the fused pass (equal
    keys); eager sorts run between the replays; every replay is exact.  Also
    with the wide local-sort blocks (the sizes beyond the others' limit)."""
    import ctypes
    from forge_sort import TEST_LOCAL_WIDE, TEST_TOP16, TOP16_SAMPLED, OP_SORT, GpuSorter
    hip = ctypes.CDLL("libamdhip64.so.7")
    st = ctypes.c_void_p(hip_stream)
    s = GpuSorter.with_context(0, hip_stream)
    graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
    s.set_test_option(TEST_TOP16, TOP16_SAMPLED)       # the sample chooses at this size
    s.set_test_option(TEST_LOCAL_WIDE, 1 if wide else 0)
    try:
        n, n_other = 1_500_007, 200_001
        tile = s.tile_config()["k64" if kind == "u64" else "k32"]
        kb = s.alloc_sort_buffer(kind, n)
        kb.copy_from_slice(make_keys(kind, n, "uniform", seed=930))
        s.encode(OP_SORT, kind, kb.device_ptr(), None, n, stream=hip_stream)
        s.reserve(OP_SORT, kind, n_other)
        s.synchronize()                                 # scratch grown: the captured sort allocates nothing
        assert hip.hipStreamBeginCapture(st, 0) == 0
        s.encode(OP_SORT, kind, kb.device_ptr(), None, n, stream=hip_stream)
        assert hip.hipStreamEndCapture(st, ctypes.byref(graph)) == 0
        assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, ctypes.c_size_t(0)) == 0
        for r, dist in enumerate(["uniform", "grp2", "top8", "dup", "same", "uniform"]):
            keys = make_keys(kind, n, dist, seed=931 + r, tile=tile)
            kb.copy_from_slice(keys)
            assert hip.hipGraphLaunch(exe, st) == 0
            assert hip.hipStreamSynchronize(st) == 0
            assert np.array_equal(kb.as_slice(), oracle.sort(kind, keys)), f"replay {r} ({dist})"
            other = make_keys(kind, n_other, "uniform", seed=960 + r)   # eager work between replays
            got = other.copy()
            getattr(s, f"sort_{kind}")(got)
            assert np.array_equal(got, oracle.sort(kind, other))
        kb.free()
    finally:
        if exe.value:
            hip.hipGraphExecDestroy(exe)
        if graph.value:
            hip.hipGraphDestroy(graph)
        s.close()


def test_with_context_caller_stream(hip_stream):
    """GpuSorter::with_context on the caller's stream (lib.rs:606-686): every op
    and the async encode run there; results match the oracle."""
    from forge_sort import OP_ARGSORT, OP_PAIRS, GpuSorter
    s = GpuSorter.with_context(0, hip_stream)
    try:
        keys = make_keys("f32", 500_001, "uniform", seed=801)
        got = keys.copy()
        s.sort_f32(got)
        assert bits_equal(got, oracle.sort("f32", keys), "f32")
        k64 = make_keys("i64", 300_007, "few", seed=802)
        assert np.array_equal(s.argsort_i64(k64), oracle.argsort("i64", k64))
        # encode on the caller stream, then wait for it through the sorter
        n = 1_000_003
        keys = make_keys("u32", n, "uniform", seed=803)
        vals = np.arange(n, dtype=np.uint32)
        kb, vb, ib = (s.alloc_sort_buffer("u32", n) for _ in range(3))
        kb.copy_from_slice(keys)
        vb.copy_from_slice(vals)
        s.encode(OP_PAIRS, "u32", kb.device_ptr(), vb.device_ptr(), n, stream=hip_stream)
        s.synchronize()
        ek, ev = oracle.sort_pairs("u32", keys, vals)
        assert np.array_equal(kb.as_slice(), ek) and np.array_equal(vb.as_slice(), ev)
        kb.copy_from_slice(keys)
        s.encode(OP_ARGSORT, "u32", kb.device_ptr(), ib.device_ptr(), n, stream=hip_stream)
        s.synchronize()
        ib.set_len(n)
        assert np.array_equal(ib.as_slice(), oracle.argsort("u32", keys))
        for b in (kb, vb, ib):
            b.free()
    finally:
        s.close()


def test_gather_with_context_caller_stream(hip_stream):
    from forge_sort import GpuGather
    g = GpuGather.with_context(0, hip_stream)
    try:
        src = np.arange(1000, dtype=np.uint64) * 3
        idx = np.random.Generator(np.random.PCG64(5)).integers(0, 1000, size=5000, dtype=np.uint32)
        assert np.array_equal(gpu_gather(g, src, idx), src[idx])
    finally:
        g.close()


# ---- callers of the path (forge-runtime pipelines, gpu-search) --------------------

def test_device_argsort_gather_handoff_one_stream(hip_stream):
    """forge-runtime's filter -> sort -> gather hand-off (buffer.rs:70-92,
    pipeline.rs:98-105, gather.rs:81-119), entirely on the device and on one
    caller stream: the argsort's index buffer leaves its SortBuffer through
    into_raw_parts, is re-owned through from_raw_parts and feeds GpuGather's
    encode directly; the host waits once, at the end.  The gathered column
    must equal the payload in the stable order of the keys."""
    from forge_sort import OP_ARGSORT, GpuGather, GpuSorter, SortBuffer
    s = GpuSorter.with_context(0, hip_stream)
    ga = GpuGather.with_context(0, hip_stream)
    try:
        for n, seed in ((1_000_003, 60), (16_777_216, 61)):
            g = np.random.Generator(np.random.PCG64(seed))
            keys = g.integers(0, 50_000, size=n, dtype=np.uint32)          # many ties
            payload = g.integers(0, 1 << 63, size=n, dtype=np.uint64)
            kb = s.alloc_sort_buffer("u32", n)
            kb.copy_from_slice(keys)
            pb = s.alloc_sort_buffer("u64", n)
            pb.copy_from_slice(payload)
            ib = s.alloc_sort_buffer("u32", n)
            ob = s.alloc_sort_buffer("u64", n)
            s.encode(OP_ARGSORT, "u32", kb.device_ptr(), ib.device_ptr(), n, stream=hip_stream)
            ptr, _, cap = ib.into_raw_parts()            # the index buffer changes owner
            ib.free()                                    # no longer owns it: frees nothing
            idx = SortBuffer.from_raw_parts(s, "u32", ptr, n, cap)
            ga.encode_gather(pb.device_ptr(), idx.device_ptr(), ob.device_ptr(), n, True, n, stream=hip_stream)
            ga.synchronize()                             # the one wait: the stream orders sort then gather
            s.synchronize()
            ob.set_len(n)
            order = oracle.argsort("u32", keys)
            assert np.array_equal(idx.as_slice(), order), f"argsort n={n}"
            assert np.array_equal(ob.as_slice(), payload[order]), f"gathered column n={n}"
            for b in (kb, pb, idx, ob):
                b.free()
    finally:
        ga.close()
        s.close()


def gpu_search_keys(n, seed):
    """gpu-search's composite result keys (content.rs:849-885): (file_index << 32)
    | byte_offset for matches in search order - files of very different match
    counts (Zipf), offsets within each file, emitted by parallel workers in
    interleaved chunks, with repeated (file, offset) pairs."""
    g = np.random.Generator(np.random.PCG64(seed))
    files = np.minimum(g.zipf(1.3, size=n) - 1, 199_999).astype(np.uint64)
    offsets = g.integers(0, 1 << 24, size=n, dtype=np.uint64)
    offsets[g.random(n) < 0.05] = 4096                  # a common offset: repeated (file, offset) pairs
    chunks = g.permutation((n + 4095) // 4096)           # interleaved worker output
    order = np.concatenate([np.arange(c * 4096, min((c + 1) * 4096, n)) for c in chunks])
    return ((files << np.uint64(32)) | offsets)[order].astype(np.uint64), files[order], offsets[order]


@pytest.mark.parametrize("n", [1_048_576, 16_777_216])
def test_gpu_search_composite_key_argsort(sorter, n):
    """The gpu-search caller's u64 argsort: equal to the oracle's stable
    argsort and to the caller's own CPU fallback order (a stable sort by
    file_index, then byte_offset, content.rs:876-881), computed here by numpy's
    stable lexsort of the two columns."""
    keys, files, offsets = gpu_search_keys(n, seed=70 + (n >> 20))
    got = sorter.argsort_u64(keys)
    assert np.array_equal(got, oracle.argsort("u64", keys))
    assert np.array_equal(got, np.lexsort((offsets, files)).astype(np.uint32))
    passes, mask = sorter.last_pass_info()
    assert mask & 0xF0 and passes < 8       # the file index's high bytes are constant: skipped
