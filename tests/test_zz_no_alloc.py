"""fs_encode_no_alloc (the entry point that allocates nothing) against
fs_encode, through the C ABI: the same inputs sorted by both must come out
bit-identical, for two calls in a row (the second with a smaller input, so it
finds the first call's contents in the static scratch), for every op and a
32- and a 64-bit key type; a size beyond the scratch is refused."""
import numpy as np
import pytest

import oracle
from forge_sort import datagen

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sorter():
    from forge_sort import GpuSorter
    s = GpuSorter.new()
    yield s
    s.close()


def keys_of(kind, n, seed):
    g = np.random.Generator(np.random.PCG64(seed))
    if kind in ("u32", "f32"):
        b = g.integers(0, 1 << 32, size=n, dtype=np.uint32)
        if kind == "f32":
            return datagen.f32_normal_specials(n, seed)
        return b
    return g.integers(0, 1 << 64, size=n, dtype=np.uint64).view(np.int64 if kind == "i64" else np.uint64)


def run(sorter, op, kind, keys, vals, no_alloc):
    """One sort through fs_encode or fs_encode_no_alloc on device copies;
    returns the host copies of the outputs."""
    from forge_sort import OP_ARGSORT, OP_PAIRS, OP_SORT
    n = keys.size
    kb = sorter.alloc_sort_buffer(kind, n)
    kb.copy_from_slice(keys)
    vb = None
    if op != OP_SORT:
        vb = sorter.alloc_sort_buffer("u32", n)
        if op == OP_PAIRS:
            vb.copy_from_slice(vals)
    enc = sorter.encode_no_alloc if no_alloc else sorter.encode
    enc(op, kind, kb.device_ptr(), vb.device_ptr() if vb is not None else None, n)
    sorter.synchronize()
    out_k = kb.as_slice()
    out_v = None
    if vb is not None:
        vb.set_len(n)
        out_v = vb.as_slice()
        vb.free()
    kb.free()
    return out_k, out_v


@pytest.mark.parametrize("kind", ["u32", "f32", "u64", "i64"])
@pytest.mark.parametrize("opname", ["sort", "argsort", "pairs"])
def test_no_alloc_matches_encode_twice(sorter, kind, opname):
    from forge_sort import NO_ALLOC_MAX_KEYS, OP_ARGSORT, OP_PAIRS, OP_SORT
    op = {"sort": OP_SORT, "argsort": OP_ARGSORT, "pairs": OP_PAIRS}[opname]
    for call, n in enumerate((NO_ALLOC_MAX_KEYS, 300_007)):       # second call smaller
        keys = keys_of(kind, n, seed=500 + call)
        vals = np.arange(n, dtype=np.uint32)[::-1].copy()
        ek, ev = run(sorter, op, kind, keys, vals, no_alloc=False)
        gk, gv = run(sorter, op, kind, keys, vals, no_alloc=True)
        bits = np.uint32 if keys.itemsize == 4 else np.uint64
        assert np.array_equal(gk.view(bits), ek.view(bits)), f"keys differ: {opname} {kind} call {call}"
        if ev is not None:
            assert np.array_equal(gv, ev), f"values differ: {opname} {kind} call {call}"
        if op == OP_SORT and call == 1:                # and both equal the oracle
            assert np.array_equal(gk.view(bits), oracle.sort(kind, keys).view(bits))


def test_no_alloc_refuses_beyond_scratch(sorter):
    from forge_sort import NO_ALLOC_MAX_KEYS, OP_SORT, InvalidArgument
    n = NO_ALLOC_MAX_KEYS + 1
    kb = sorter.alloc_sort_buffer("u32", n)
    try:
        with pytest.raises(InvalidArgument, match="no-allocation scratch"):
            sorter.encode_no_alloc(OP_SORT, "u32", kb.device_ptr(), None, n)
    finally:
        kb.free()
