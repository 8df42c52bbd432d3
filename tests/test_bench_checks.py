"""bench.py's output check (host logic): it accepts the oracle's results for
every workload kind and rejects a wrong multiset, a wrong order and an
unstable tie order.  No GPU needed."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import bench  # noqa: E402
import oracle  # noqa: E402

N = 20_000
SMALL = {"u32_256M": N, "f32_64M": N, "i32_64M": N, "argsort_f32_16M": N,
         "pairs_u32_64M": N, "u64_128M": N, "i64_128M": N, "f64_128M": N, "u64_low20_128M": N}


def expected(name, keys, vals):
    op, kind = bench.WORKLOADS[name][:2]
    if op == "sort":
        return oracle.sort(kind, keys), None
    if op == "argsort":
        return keys, oracle.argsort(kind, keys)
    return oracle.sort_pairs(kind, keys, vals)


@pytest.mark.parametrize("name", sorted(SMALL))
def test_accepts_oracle_output(name):
    keys, vals = bench.workload_input(name, SMALL[name])
    ko, vo = expected(name, keys, vals)
    assert bench.check_output(bench.WORKLOADS[name][0], keys, vals, ko, vo)


def test_rejects_changed_key():
    keys, _ = bench.workload_input("u32_256M", N)
    ko = oracle.sort("u32", keys).copy()
    ko[N // 2] += np.uint32(1)                     # still sorted only by luck; multiset differs
    assert not bench.check_output("sort", keys, None, ko, None)


def test_rejects_unsorted():
    keys, _ = bench.workload_input("f64_128M", N)
    ko = oracle.sort("f64", keys).copy()
    ko[[10, 11]] = ko[[11, 10]]
    assert not bench.check_output("sort", keys, None, ko, None)


def test_rejects_unstable_pairs():
    keys, vals = bench.workload_input("pairs_u32_64M", N)
    ko, vo = oracle.sort_pairs("u32", keys, vals)
    vo = vo.copy()
    tie = np.flatnonzero(ko[1:] == ko[:-1])[0]      # Zipf keys: ties abound
    vo[[tie, tie + 1]] = vo[[tie + 1, tie]]
    assert not bench.check_output("pairs", keys, vals, ko, vo)


def test_rejects_unstable_argsort():
    keys, _ = bench.workload_input("argsort_f32_16M", N)
    idx = oracle.argsort("f32", keys).copy()
    o = bench.ordered_bits(keys[idx])
    tie = np.flatnonzero(o[1:] == o[:-1])[0]
    idx[[tie, tie + 1]] = idx[[tie + 1, tie]]
    assert not bench.check_output("argsort", keys, None, keys, idx)


def test_ordered_bits_total_order():
    """-NaN < -inf < -1 < -0.0 < +0.0 < denormal < 1 < inf < +NaN."""
    v = np.array([np.float32(np.nan), -np.inf, -1.0, -0.0, 0.0, 1e-45, 1.0, np.inf], dtype=np.float32)
    b = v.view(np.uint32).copy()
    b[0] |= np.uint32(0x80000000)                  # negative NaN first
    nan_pos = np.array([0x7FC00001], dtype=np.uint32).view(np.float32)
    v = np.concatenate([b.view(np.float32), nan_pos])
    o = bench.ordered_bits(v)
    assert np.all(o[1:] > o[:-1])


def test_rejects_sum_and_xor_preserving_change():
    """{1, 2} -> {0, 3} keeps the sum and the xor of the keys (a multiset test
    by those two would pass it); the exact check must not."""
    keys = np.array([2, 1, 7, 5], dtype=np.uint32)
    wrong = np.array([0, 3, 5, 7], dtype=np.uint32)
    assert int(keys.sum()) == int(wrong.sum()) and np.bitwise_xor.reduce(keys) == np.bitwise_xor.reduce(wrong)
    assert not bench.check_output("sort", keys, None, wrong, None)
    assert bench.check_output("sort", keys, None, np.sort(keys), None)
