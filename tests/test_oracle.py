"""Pins the CPU oracle (oracle/forge_sort_oracle.c) before it is trusted as the
checker of the HIP path.

Every oracle function is checked against something that does not share its
formula:
  * the reference's known-answer vectors (tests/golden/golden.json);
  * numpy's sort / stable argsort, with floats ordered by Rust's documented
    total_cmp formula rather than by FloatFlip;
  * brute force over every permutation of small multisets;
  * closed-form transform invariants (round trip, order preservation);
and each planted mistake in the oracle (or_mutation) must make one of these
checks fail.
"""
import itertools
import json
import os

import numpy as np
import pytest

import oracle
from forge_sort import datagen

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden.json")
NP = oracle.NP_DTYPES
BITS = {"u32": np.uint32, "i32": np.uint32, "f32": np.uint32,
        "u64": np.uint64, "i64": np.uint64, "f64": np.uint64}


def load_golden():
    with open(GOLDEN) as f:
        return json.load(f)["cases"]


def as_keys(kind, bits):
    return np.array(bits, dtype=BITS[kind]).view(NP[kind])


def order_key(kind, keys):
    """Independent total order: integers as themselves; floats via Rust's
    total_cmp (bits ^ (((bits >> 31) as u32) >> 1), compared as signed)."""
    if kind in ("u32", "i32", "u64", "i64"):
        return keys
    if kind == "f32":
        s = keys.view(np.int32)
        mask = (s >> 31).view(np.uint32) >> np.uint32(1)
        return (s.view(np.uint32) ^ mask).view(np.int32)
    s = keys.view(np.int64)
    mask = (s >> 63).view(np.uint64) >> np.uint64(1)
    return (s.view(np.uint64) ^ mask).view(np.int64)


def expected_argsort(kind, keys):
    return np.argsort(order_key(kind, keys), kind="stable").astype(np.uint32)


def run_golden_case(c):
    kind = c["type"]
    if c["op"] == "gather":
        src = np.array(c["values"], dtype=BITS[kind])
        got = oracle.gather(src, np.array(c["indices"], dtype=np.uint32))
        return got.tolist() == c["expected_values"]
    keys = as_keys(kind, c["keys"])
    if c["op"] == "sort":
        got = oracle.sort(kind, keys)
        return np.array_equal(got.view(BITS[kind]), np.array(c["expected_keys"], dtype=BITS[kind]))
    if c["op"] == "argsort":
        got = oracle.argsort(kind, keys)
        return np.array_equal(got, np.array(c["expected_indices"], dtype=np.uint32))
    k, v = oracle.sort_pairs(kind, keys, np.array(c["values"], dtype=np.uint32))
    return (np.array_equal(k.view(BITS[kind]), np.array(c["expected_keys"], dtype=BITS[kind]))
            and np.array_equal(v, np.array(c["expected_values"], dtype=np.uint32)))


@pytest.fixture(autouse=True)
def _no_mutation():
    oracle.set_mutation(0)
    yield
    oracle.set_mutation(0)


@pytest.mark.parametrize("case", load_golden(), ids=lambda c: c["name"])
def test_golden_vectors(case):
    assert run_golden_case(case), case["source"]


def random_inputs(kind, n, seed):
    g = np.random.Generator(np.random.PCG64(seed))
    if kind in ("u32", "i32", "f32"):
        bits = g.integers(0, 1 << 32, size=n, dtype=np.uint32)
        if kind == "f32":
            bits[: n // 8] = g.choice(np.array([0, 0x80000000, 0x7F800000, 0xFF800000,
                                                0x7FC00001, 0xFFC00002, 1, 0x80000001],
                                               dtype=np.uint32), n // 8)
        bits[n // 2: n // 2 + n // 8] = bits[0]          # ties
        return bits.view(NP[kind])
    bits = g.integers(0, 1 << 64, size=n, dtype=np.uint64)
    if kind == "f64":
        bits[: n // 8] = g.choice(np.array([0, 1 << 63, 0x7FF0000000000000, 0xFFF0000000000000,
                                            0x7FF8000000000001, 0xFFF8000000000002, 1],
                                           dtype=np.uint64), n // 8)
    bits[n // 2: n // 2 + n // 8] = bits[0]
    return bits.view(NP[kind])


KINDS = ["u32", "i32", "f32", "u64", "i64", "f64"]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n", [2, 257, 4097, 100_003])
def test_against_numpy(kind, n):
    keys = random_inputs(kind, n, seed=n)
    perm = expected_argsort(kind, keys)
    exp_sorted = keys[perm]
    got = oracle.sort(kind, keys)
    assert np.array_equal(got.view(BITS[kind]), exp_sorted.view(BITS[kind]))
    assert np.array_equal(oracle.argsort(kind, keys), perm)
    vals = np.arange(n, dtype=np.uint32)[::-1].copy()
    k, v = oracle.sort_pairs(kind, keys, vals)
    assert np.array_equal(k.view(BITS[kind]), exp_sorted.view(BITS[kind]))
    assert np.array_equal(v, vals[perm])


@pytest.mark.parametrize("kind", ["u32", "i32", "f32", "u64", "i64", "f64"])
def test_brute_force_small_multisets(kind):
    """Every permutation of small multisets: argsort must equal Python's stable
    sorted() under the independent order key."""
    if kind in ("f32", "f64"):
        pool = [-1.0, 0.0, -0.0, 2.5, np.inf, np.nan]
        base = np.array(pool, dtype=NP[kind])
    elif kind in ("i32", "i64"):
        base = np.array([-5, 0, 3, -1, 7, -(2**31)], dtype=NP[kind])
    else:
        base = np.array([0, 1 << 24, 255, 1 << 31, 7, 65536], dtype=NP[kind])
    for combo in [(0, 0, 1, 2), (3, 1, 3, 1, 0), (0, 1, 2, 3, 4, 5), (5, 5, 4, 4, 4, 2)]:
        for perm in set(itertools.permutations(combo)):
            keys = base[list(perm)]
            ok = order_key(kind, keys).tolist()
            expect = sorted(range(len(keys)), key=lambda i: ok[i])
            assert oracle.argsort(kind, keys).tolist() == expect


def test_transform_closed_forms():
    g = np.random.Generator(np.random.PCG64(11))
    b32 = g.integers(0, 1 << 32, size=200_000, dtype=np.uint32)
    b64 = g.integers(0, 1 << 64, size=200_000, dtype=np.uint64)
    # mode 0 is an involution, modes 1 and 2 are inverse bijections
    assert np.array_equal(oracle.transform(oracle.transform(b32, 0), 0), b32)
    assert np.array_equal(oracle.transform(oracle.transform(b32, 1), 2), b32)
    assert np.array_equal(oracle.transform(oracle.transform(b64, 1), 2), b64)
    assert np.array_equal(oracle.transform(oracle.transform(b64, 0), 0), b64)
    # order preservation: FloatFlip(a) < FloatFlip(b)  <=>  total_cmp(a, b) == Less
    a, b = b32[:100_000], b32[100_000:]
    fa, fb = oracle.transform(a, 1), oracle.transform(b, 1)
    ta, tb = order_key("f32", a.view(np.float32)), order_key("f32", b.view(np.float32))
    assert np.array_equal(fa < fb, ta < tb)
    a, b = b64[:100_000], b64[100_000:]
    fa, fb = oracle.transform(a, 1), oracle.transform(b, 1)
    ta, tb = order_key("f64", a.view(np.float64)), order_key("f64", b.view(np.float64))
    assert np.array_equal(fa < fb, ta < tb)
    # sign flip maps signed order to unsigned order
    s = b32.view(np.int32)
    x = oracle.transform(b32, 0)
    assert np.array_equal(x[:-1] < x[1:], s[:-1] < s[1:])


def test_gather_definition():
    """gather = numpy fancy indexing; an index past the source is refused."""
    g = np.random.Generator(np.random.PCG64(3))
    for dt in (np.uint32, np.uint64):
        src = g.integers(0, 1 << 63, size=5000, dtype=np.uint64).astype(dt)
        idx = g.integers(0, 5000, size=20000, dtype=np.uint32)
        assert np.array_equal(oracle.gather(src, idx), src[idx])
        assert oracle.gather(src, np.zeros(0, dtype=np.uint32)).size == 0
        with pytest.raises(IndexError):
            oracle.gather(src, np.array([0, 5000], dtype=np.uint32))


def test_edge_returns():
    assert oracle.sort("u32", np.array([], dtype=np.uint32)).size == 0
    assert oracle.argsort("f32", np.array([3.14], dtype=np.float32)).tolist() == [0]
    with pytest.raises(ValueError, match="length mismatch: keys=3, values=2"):
        oracle.sort_pairs("u32", np.array([1, 2, 3], np.uint32), np.array([10, 20], np.uint32))


def test_config_generators_shape():
    assert datagen.uniform_u32(1000).dtype == np.uint32
    f = datagen.f32_normal_specials(10_000)
    bits = f.view(np.uint32)
    assert np.isnan(f).sum() > 0 and np.isinf(f).sum() > 0
    assert ((bits & 0x7F800000) == 0).sum() > 0                   # zeros / subnormals
    assert len(np.unique(datagen.argsort_f32_ties(100_000))) <= 4096
    k, v = datagen.zipf_pairs_u32(100_000)
    assert k.max() < (1 << 20) and np.array_equal(v, np.arange(100_000, dtype=np.uint32))
    lo = datagen.low20_u64(1000, high=0x123456789AB)
    assert np.all((lo >> np.uint64(20)) == np.uint64(0x123456789AB))


def _all_checks_pass():
    for c in load_golden():
        if not run_golden_case(c):
            return False
    g = np.random.Generator(np.random.PCG64(9))
    for dt in (np.uint32, np.uint64):
        src = g.integers(0, 1 << 32, size=1000, dtype=np.uint64).astype(dt)
        idx = g.integers(0, 1000, size=3000, dtype=np.uint32)
        if not np.array_equal(oracle.gather(src, idx), src[idx]):     # numpy fancy indexing
            return False
    for kind in KINDS:
        keys = random_inputs(kind, 4097, seed=5)
        perm = expected_argsort(kind, keys)
        if not np.array_equal(oracle.argsort(kind, keys), perm):
            return False
        if not np.array_equal(oracle.sort(kind, keys).view(BITS[kind]), keys[perm].view(BITS[kind])):
            return False
    return True


@pytest.mark.parametrize("mutation", [1, 2, 3, 4, 5, 6])
def test_planted_mistakes_are_caught(mutation):
    assert _all_checks_pass()
    oracle.set_mutation(mutation)
    assert not _all_checks_pass(), f"mutation {mutation} slipped through the pinning checks"
