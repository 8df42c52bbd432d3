"""Performance guards, after the reference's perf-test suite
(metal-forge-compute/forge-sort/tests/performance.rs:37-207): 16,000,000 keys
per type, one warm-up call, the median of 10 timed calls, a floor in Mkeys/s.

Two sets:
* the reference's own cases and floors, through the same host-slice API
  (copy in, sort, copy out: bound by the host link, not by the kernels);
  inputs from numpy's PCG64 with the reference's seeds (its ChaCha8 stream is
  a Rust crate's and is not available here), the same value ranges;
* the same cases on device-resident buffers (sort_<t>_buffer, argsort and
  pairs on device pointers), the path the kernels set, with floors at about
  half the rates measured on MI355X, so that a regression of the kernels,
  and not of the host link, fails them.
"""
import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

N = 16_000_000
REPS = 10


@pytest.fixture(scope="module")
def sorter():
    from forge_sort import GpuSorter
    s = GpuSorter.new()
    yield s
    s.close()


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def keys_for(kind, seed):
    g = rng(seed)
    if kind in ("u32", "i32", "u64", "i64"):
        bits = np.uint32 if kind.endswith("32") else np.uint64
        b = g.integers(0, 1 << (8 * np.dtype(bits).itemsize), size=N, dtype=bits, endpoint=False)
        return b.view(np.int32 if kind == "i32" else np.int64 if kind == "i64" else bits)
    dt = np.float32 if kind == "f32" else np.float64
    return (g.random(N, dtype=dt) * dt(2000.0) - dt(1000.0)).astype(dt)   # rng.gen::<f>() * 2000 - 1000


def median_mkeys(run, prepare=None):
    """Mkeys/s of the median of REPS timed calls of run() (prepare() before
    each, untimed), after one warm-up call."""
    if prepare:
        prepare()
    run()
    times = []
    for _ in range(REPS):
        if prepare:
            prepare()
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    return N / float(np.median(times)) / 1e6


# (case, seed, floor in Mkeys/s): performance.rs:37-207
SLICE_CASES = [("sort_u32", 42, 2000.0), ("sort_i32", 43, 1900.0), ("sort_f32", 44, 500.0),
               ("argsort_u32", 45, 750.0), ("sort_pairs_f32", 46, 250.0), ("sort_u64", 47, 600.0),
               ("sort_i64", 48, 550.0), ("sort_f64", 49, 100.0)]


@pytest.mark.parametrize("case,seed,floor", SLICE_CASES)
def test_perf_slice(sorter, case, seed, floor):
    """The reference's perf tests and floors, host-slice API (performance.rs:37-207)."""
    kind = case.split("_")[-1]
    keys = keys_for(kind, seed)
    if case.startswith("argsort"):
        mks = median_mkeys(lambda: sorter.argsort_u32(keys))
    elif case.startswith("sort_pairs"):
        vals0 = rng(seed + 1000).integers(0, 1 << 32, size=N, dtype=np.uint32)
        work = {}

        def prep():
            work["k"], work["v"] = keys.copy(), vals0.copy()
        mks = median_mkeys(lambda: sorter.sort_pairs_f32(work["k"], work["v"]), prep)
    else:
        work = {}

        def prep():
            work["k"] = keys.copy()
        mks = median_mkeys(lambda: getattr(sorter, case)(work["k"]), prep)
    print(f"{case} slice 16M: {mks:,.0f} Mkeys/s (floor {floor:,.0f})")
    assert mks >= floor, f"{case}: {mks:,.0f} Mkeys/s < {floor:,.0f}"


# (case, seed, floor in Mkeys/s): device-resident, floors about half the
# rates measured on one MI355X
DEVICE_CASES = [("sort_u32", 42, 35000.0), ("sort_i32", 43, 35000.0), ("sort_f32", 44, 30000.0),
                ("argsort_u32", 45, 25000.0), ("sort_pairs_f32", 46, 20000.0), ("sort_u64", 47, 25000.0),
                ("sort_i64", 48, 25000.0), ("sort_f64", 49, 10000.0)]


@pytest.mark.parametrize("case,seed,floor", DEVICE_CASES)
def test_perf_device(sorter, case, seed, floor):
    """The same cases on device-resident buffers (no host copies timed)."""
    kind = case.split("_")[-1]
    keys = keys_for(kind, seed)
    ksz = keys.dtype.itemsize
    src = sorter.alloc_sort_buffer(kind, N)
    src.copy_from_slice(keys)
    work = sorter.alloc_sort_buffer(kind, N)
    extra = []
    try:
        def copy_keys():
            sorter.copy_device(work.device_ptr(), src.device_ptr(), ksz * N)
            sorter.device_synchronize()
        if case.startswith("argsort"):
            idx = sorter.alloc_sort_buffer("u32", N)
            extra.append(idx)
            mks = median_mkeys(lambda: sorter.argsort_device(kind, work.device_ptr(), N, idx.device_ptr()),
                               copy_keys)
        elif case.startswith("sort_pairs"):
            vsrc = sorter.alloc_sort_buffer("u32", N)
            vsrc.copy_from_slice(rng(seed + 1000).integers(0, 1 << 32, size=N, dtype=np.uint32))
            vals = sorter.alloc_sort_buffer("u32", N)
            extra += [vsrc, vals]

            def copy_both():
                sorter.copy_device(vals.device_ptr(), vsrc.device_ptr(), 4 * N)
                copy_keys()
            mks = median_mkeys(lambda: sorter.sort_pairs_device(kind, work.device_ptr(), vals.device_ptr(), N),
                               copy_both)
        else:
            mks = median_mkeys(lambda: sorter.sort_device(kind, work.device_ptr(), N), copy_keys)
        work.set_len(N)                                  # (filled by device copies, not copy_from_slice)
        out = work.as_slice()
        exp = np.sort(keys)                              # (no NaN in these inputs)
        if not case.startswith("argsort"):
            assert np.array_equal(out, exp), f"{case}: output differs from numpy's sort"
    finally:
        for b in extra:
            b.free()
        work.free()
        src.free()
    print(f"{case} device 16M: {mks:,.0f} Mkeys/s (floor {floor:,.0f})")
    assert mks >= floor, f"{case}: {mks:,.0f} Mkeys/s < {floor:,.0f}"


# (key type, n, floor in Mkeys/s): keys-only sorts on the top-16 path at sizes
# between powers of two, where the segment bits must still keep a uniform
# input's segments within a block, and beyond the 4,608- and 2,304-key
# blocks' size limits (the wide blocks); floors about half the rates
# measured on one MI355X: u32 100M 111,900, 200M 128,300, 400M 134,900;
# u64 50M 66,000, 100M 74,000, 200M 74,800
BETWEEN_CASES = [("u32", 100_000_000, 55000.0), ("u32", 200_000_000, 64000.0), ("u32", 400_000_000, 65000.0),
                 ("u64", 50_000_000, 33000.0), ("u64", 100_000_000, 37000.0), ("u64", 200_000_000, 37000.0)]


@pytest.mark.parametrize("kind,n,floor", BETWEEN_CASES)
def test_perf_device_between_powers_of_two(sorter, kind, n, floor):
    """Device-resident uniform keys at sizes that are not powers of two:
    the median of 10 sorts (a device copy of the input before each, untimed)."""
    dt = np.uint32 if kind == "u32" else np.uint64
    keys = rng(50 + n % 89).integers(0, 1 << (8 * np.dtype(dt).itemsize), size=n, dtype=dt, endpoint=False)
    src = sorter.alloc_sort_buffer(kind, n)
    src.copy_from_slice(keys)
    work = sorter.alloc_sort_buffer(kind, n)
    try:
        def copy_keys():
            sorter.copy_device(work.device_ptr(), src.device_ptr(), keys.itemsize * n)
            sorter.device_synchronize()
        copy_keys()
        sorter.sort_device(kind, work.device_ptr(), n)
        times = []
        for _ in range(REPS):
            copy_keys()
            t0 = time.perf_counter()
            sorter.sort_device(kind, work.device_ptr(), n)
            times.append(time.perf_counter() - t0)
        mks = n / float(np.median(times)) / 1e6
        work.set_len(n)
        out = work.as_slice()
        assert bool(np.all(out[1:] >= out[:-1])), "not ascending"
        assert sorter.first_pass() == 3, "expected the top-16 path"
    finally:
        work.free()
        src.free()
    print(f"sort_{kind} device {n:,}: {mks:,.0f} Mkeys/s (floor {floor:,.0f})")
    assert mks >= floor, f"sort_{kind} {n:,}: {mks:,.0f} Mkeys/s < {floor:,.0f}"


def test_perf_device_many_copies_u64(sorter):
    """u64 keys with many copies of each value (2^27 keys, 2^20 distinct
    values: segments of about 16 values x 128 copies, lumpier than a uniform
    input's): 2.9 ms on one MI355X; the floor catches the deferred launch's
    former 9 ms."""
    n, distinct = 1 << 27, 1 << 20
    g = rng(77)
    values = g.integers(0, 1 << 64, size=distinct, dtype=np.uint64, endpoint=False)
    keys = values[g.integers(0, distinct, size=n)]
    src = sorter.alloc_sort_buffer("u64", n)
    src.copy_from_slice(keys)
    work = sorter.alloc_sort_buffer("u64", n)
    try:
        times = []
        for r in range(REPS + 1):
            sorter.copy_device(work.device_ptr(), src.device_ptr(), 8 * n)
            sorter.device_synchronize()
            t0 = time.perf_counter()
            sorter.sort_device("u64", work.device_ptr(), n)
            if r:
                times.append(time.perf_counter() - t0)
        mks = n / float(np.median(times)) / 1e6
        work.set_len(n)
        assert np.array_equal(work.as_slice(), np.sort(keys))
    finally:
        work.free()
        src.free()
    print(f"sort_u64 many copies {n:,}: {mks:,.0f} Mkeys/s (floor 20,000)")
    assert mks >= 20000.0, f"{mks:,.0f} Mkeys/s < 20,000"
