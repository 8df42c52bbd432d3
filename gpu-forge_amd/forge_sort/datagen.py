"""Seeded synthetic inputs for the benchmark configurations.

Each generator returns numpy arrays of the exact dtype the sorter takes.  The
distributions follow the workload definitions of the reference's benchmark
(metal-forge-compute/forge-sort/benches/sort_benchmark.rs:20-22 uses uniform
u32 and N(0, 1e3) floats) widened to the skewed cases the sort must survive:

  uniform_u32(n)            uniform over [0, 2^32)
  f32_normal_specials(n)    98% N(0, 1e3); 2% split over -0.0, +0.0, +inf,
                            -inf, subnormals and quiet NaN with payloads
  uniform_i32(n)            uniform over the full i32 range
  argsort_f32_ties(n)       uniform in [-1, 1) quantised to 4096 values
  zipf_pairs_u32(n)         Zipf(s=1.1) over 2^20 ranks, a 10% run of one key,
                            values = original index
  uniform_u64 / uniform_i64 full-range 64-bit
  normal_f64(n)             N(0, 1e6)
  low20_u64(n, const)       high 44 bits fixed, low 20 bits uniform

numpy's PCG64 generator is used throughout, so a (seed, n) pair always gives
the same array.
"""
import numpy as np


def _rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def uniform_u32(n, seed=1):
    return _rng(seed).integers(0, 1 << 32, size=n, dtype=np.uint32)


def uniform_i32(n, seed=2):
    return uniform_u32(n, seed).view(np.int32)


def uniform_u64(n, seed=3):
    return _rng(seed).integers(0, 1 << 64, size=n, dtype=np.uint64, endpoint=False)


def uniform_i64(n, seed=4):
    return uniform_u64(n, seed).view(np.int64)


def f32_normal_specials(n, seed=5):
    """98% N(0, sigma=1e3) rounded to f32; 2% specials at random positions."""
    g = _rng(seed)
    x = (g.standard_normal(n) * 1e3).astype(np.float32)
    bits = x.view(np.uint32)
    n_special = int(n * 0.02)
    pos = g.choice(n, size=n_special, replace=False) if n_special else np.empty(0, np.int64)
    cls = np.arange(n_special) % 6
    sign = g.integers(0, 2, size=n_special, dtype=np.uint32) << 31
    mant = g.integers(1, 1 << 23, size=n_special, dtype=np.uint32)
    payload = g.integers(0, 1 << 22, size=n_special, dtype=np.uint32)
    special = np.select(
        [cls == 0, cls == 1, cls == 2, cls == 3, cls == 4, cls == 5],
        [np.uint32(0x80000000),                  # -0.0
         np.uint32(0x00000000),                  # +0.0
         np.uint32(0x7F800000),                  # +inf
         np.uint32(0xFF800000),                  # -inf
         sign | mant,                            # subnormal, random sign
         sign | np.uint32(0x7FC00000) | payload],  # quiet NaN, random sign and payload
    ).astype(np.uint32)
    bits[pos] = special
    return bits.view(np.float32)


def argsort_f32_ties(n, seed=6):
    """x ~ U[-1, 1), q = floor((x + 1) * 2048) / 2048 - 1: 4096 distinct values."""
    x = _rng(seed).uniform(-1.0, 1.0, size=n)
    q = np.floor((x + 1.0) * 2048.0) / 2048.0 - 1.0
    return q.astype(np.float32)


def zipf_pairs_u32(n, seed=7, s=1.1, ranks=1 << 20):
    """Keys Zipf(s) over ranks 1..2^20 (key = rank - 1) by inverse-CDF lookup;
    a contiguous run of floor(0.1 n) keys is overwritten with one key;
    values are the original indices."""
    g = _rng(seed)
    w = 1.0 / np.power(np.arange(1, ranks + 1, dtype=np.float64), s)
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    u = g.random(n)
    keys = np.searchsorted(cdf, u, side="right").astype(np.uint32)
    keys = np.minimum(keys, ranks - 1).astype(np.uint32)
    run = n // 10
    if run:
        start = int(g.integers(0, n - run + 1))
        keys[start:start + run] = np.uint32(g.integers(0, ranks))
    vals = np.arange(n, dtype=np.uint32)
    return keys, vals


def normal_f64(n, seed=8):
    return _rng(seed).standard_normal(n) * 1e6


def low20_u64(n, high=0, seed=9):
    """High 44 bits = `high` (a constant), low 20 bits uniform."""
    low = _rng(seed).integers(0, 1 << 20, size=n, dtype=np.uint64)
    return (np.uint64(high) << np.uint64(20)) | low
