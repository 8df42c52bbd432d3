"""Writes tests/golden/golden.json: the known-answer vectors of forge-sort's own
test suite (metal-forge-compute/forge-sort/tests/*.rs and src/lib.rs unit tests).

Inputs are transcribed from the reference tests (file:line in each case's
"source").  Expected outputs come from one of two places, recorded per case in
"expected_from":
  * "reference"  -- the test file states the expected output literally;
  * "total_cmp"  -- the test computes it with Rust's sort()/sort_by(total_cmp);
                    here that is Python's stable sorted() with a key that
                    implements Rust's documented total_cmp formula
                    (core::f32::total_cmp: bits ^ (((bits >> 31) as u32) >> 1),
                    compared as signed), which is independent of the
                    FloatFlip transform the oracle and the kernels use.
Argsort/pairs expectations use the stable order (ties by original index).

Run:  python tests/golden/make_golden.py
"""
import json
import os
import struct

HERE = os.path.dirname(os.path.abspath(__file__))
FS = "metal-forge-compute/forge-sort/"


def f32_bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


def f64_bits(x):
    return struct.unpack("<Q", struct.pack("<d", x))[0]


F32_MAX = 0x7F7FFFFF
F32_MIN = 0xFF7FFFFF          # f32::MIN = -MAX
F32_MIN_POS = 0x00800000
F32_EPS = 0x34000000
F32_NAN = 0x7FC00000
F32_INF = 0x7F800000
F32_NINF = 0xFF800000
F64_NAN = 0x7FF8000000000000
F64_INF = 0x7FF0000000000000
F64_NINF = 0xFFF0000000000000
F64_MAX = 0x7FEFFFFFFFFFFFFF
F64_MIN = 0xFFEFFFFFFFFFFFFF
F64_MIN_POS = 0x0010000000000000
F64_EPS = 0x3CB0000000000000


def neg32(b):
    return b ^ 0x80000000


def neg64(b):
    return b ^ 0x8000000000000000


# ---- ordering keys, written from the language definitions -----------------

def total_cmp_key32(bits):
    """Rust f32::total_cmp: left = bits as i32; left ^= (((left >> 31) as u32) >> 1) as i32."""
    s = bits - (1 << 32) if bits & 0x80000000 else bits          # as i32
    mask = ((s >> 31) & 0xFFFFFFFF) >> 1                          # arithmetic >>31, as u32, >>1
    v = (s & 0xFFFFFFFF) ^ mask
    return v - (1 << 32) if v & 0x80000000 else v                 # compare as i32


def total_cmp_key64(bits):
    s = bits - (1 << 64) if bits & (1 << 63) else bits
    mask = ((s >> 63) & 0xFFFFFFFFFFFFFFFF) >> 1
    v = (s & 0xFFFFFFFFFFFFFFFF) ^ mask
    return v - (1 << 64) if v & (1 << 63) else v


def signed(bits, width):
    return bits - (1 << width) if bits >> (width - 1) else bits


def order_key(kind):
    return {
        "u32": lambda b: b, "u64": lambda b: b,
        "i32": lambda b: signed(b, 32), "i64": lambda b: signed(b, 64),
        "f32": total_cmp_key32, "f64": total_cmp_key64,
    }[kind]


def i32(v):
    return v & 0xFFFFFFFF


def i64(v):
    return v & 0xFFFFFFFFFFFFFFFF


# ---- cases -----------------------------------------------------------------

cases = []


def add_sort(name, src, kind, bits, expected=None):
    key = order_key(kind)
    computed = sorted(bits, key=key)
    if expected is not None:
        assert expected == computed, name
    cases.append({"name": name, "source": src, "op": "sort", "type": kind,
                  "keys": bits, "expected_keys": computed,
                  "expected_from": "reference" if expected is not None else "total_cmp"})


def add_argsort(name, src, kind, bits, expected=None):
    key = order_key(kind)
    computed = sorted(range(len(bits)), key=lambda i: key(bits[i]))   # stable
    if expected is not None:
        assert expected == computed, (name, expected, computed)
    cases.append({"name": name, "source": src, "op": "argsort", "type": kind,
                  "keys": bits, "expected_indices": computed,
                  "expected_from": "reference" if expected is not None else "total_cmp"})


def add_pairs(name, src, kind, bits, vals, exp_keys=None, exp_vals=None):
    key = order_key(kind)
    perm = sorted(range(len(bits)), key=lambda i: key(bits[i]))
    ck = [bits[i] for i in perm]
    cv = [vals[i] for i in perm]
    if exp_keys is not None:
        assert exp_keys == ck and exp_vals == cv, name
    cases.append({"name": name, "source": src, "op": "pairs", "type": kind,
                  "keys": bits, "values": vals, "expected_keys": ck, "expected_values": cv,
                  "expected_from": "reference" if exp_keys is not None else "total_cmp"})


# argsort known answers (correctness_argsort.rs)
add_argsort("argsort_u32_basic", FS + "tests/correctness_argsort.rs:8-14", "u32",
            [30, 10, 20], [1, 2, 0])
add_argsort("argsort_u32_stable", FS + "tests/correctness_argsort.rs:43-57", "u32",
            [5, 3, 5, 3, 5], [1, 3, 0, 2, 4])
add_argsort("argsort_i32_basic", FS + "tests/correctness_argsort.rs:79-86", "i32",
            [i32(v) for v in (5, -3, 0, -1, 2)], [1, 3, 2, 4, 0])
add_argsort("argsort_i32_boundaries", FS + "tests/correctness_argsort.rs:88-99", "i32",
            [i32(v) for v in (2**31 - 1, 0, -2**31, -1, 1)], [2, 3, 1, 4, 0])
add_argsort("argsort_f32_basic", FS + "tests/correctness_argsort.rs:101-108", "f32",
            [f32_bits(v) for v in (3.0, -1.0, 0.0, 2.0)], [1, 2, 3, 0])
add_argsort("argsort_f32_nan", FS + "tests/correctness_argsort.rs:110-117", "f32",
            [F32_NAN, f32_bits(1.0), F32_NINF, neg32(F32_NAN), f32_bits(0.0)])
add_argsort("argsort_u32_all_same", FS + "tests/correctness_argsort.rs:135-143", "u32",
            [7] * 100, list(range(100)))
add_argsort("argsort_i64_basic", FS + "tests/correctness_i64.rs:104-116", "i64",
            [i64(v) for v in (30, -10, 20)], [1, 2, 0])
add_argsort("argsort_f64_basic", FS + "tests/correctness_f64.rs:225-232", "f64",
            [f64_bits(v) for v in (3.0, -1.0, 2.0)], [1, 2, 0])
add_argsort("argsort_single_u32", FS + "tests/correctness_argsort.rs:127-133", "u32", [42], [0])
add_argsort("argsort_empty_u32", FS + "tests/correctness_argsort.rs:119-125", "u32", [], [])

# pairs known answers (correctness_sort_pairs.rs, lib.rs unit tests, correctness_i64.rs)
add_pairs("pairs_u32_basic", FS + "tests/correctness_sort_pairs.rs:10-17", "u32",
          [30, 10, 20], [300, 100, 200], [10, 20, 30], [100, 200, 300])
add_pairs("pairs_u32_stable", FS + "tests/correctness_sort_pairs.rs:36-46", "u32",
          [5, 3, 5, 3, 5], [50, 30, 51, 31, 52], [3, 3, 5, 5, 5], [30, 31, 50, 51, 52])
add_pairs("pairs_i32_basic", FS + "tests/correctness_sort_pairs.rs:48-58", "i32",
          [i32(v) for v in (5, -3, 0, -1, 2)], [50, 30, 0, 10, 20],
          [i32(v) for v in (-3, -1, 0, 2, 5)], [30, 10, 0, 20, 50])
add_pairs("pairs_i32_lib_unit", FS + "src/lib.rs:3223-3230", "i32",
          [i32(v) for v in (5, -3, 0, -1, 1)], [50, 30, 0, 10, 10],
          [i32(v) for v in (-3, -1, 0, 1, 5)], [30, 10, 0, 10, 50])
add_pairs("pairs_f32_basic", FS + "tests/correctness_sort_pairs.rs:60-70", "f32",
          [f32_bits(v) for v in (3.0, -1.0, 0.0, 2.0)], [30, 10, 0, 20],
          [f32_bits(v) for v in (-1.0, 0.0, 2.0, 3.0)], [10, 0, 20, 30])
add_pairs("pairs_f32_nan", FS + "tests/correctness_sort_pairs.rs:72-90", "f32",
          [F32_NAN, f32_bits(1.0), F32_NINF, neg32(F32_NAN), f32_bits(0.0)], [99, 11, 22, 88, 0])
add_pairs("pairs_i64_basic", FS + "tests/correctness_i64.rs:118-135", "i64",
          [i64(v) for v in (30, -10, 20, 0)], [100, 200, 300, 400],
          [i64(v) for v in (-10, 0, 20, 30)], [200, 400, 300, 100])
add_pairs("pairs_u32_all_same", FS + "tests/correctness_sort_pairs.rs:162-171", "u32",
          [7] * 100, list(range(100)), [7] * 100, list(range(100)))
add_pairs("pairs_single", FS + "tests/correctness_sort_pairs.rs:152-159", "u32", [42], [99], [42], [99])

# f32 specials (correctness_f32.rs)
add_sort("f32_ieee754_special", FS + "tests/correctness_f32.rs:25-52", "f32", [
    F32_NAN, F32_INF, F32_NINF, F32_MAX, F32_MIN, F32_MIN_POS, neg32(F32_MIN_POS),
    f32_bits(0.0), neg32(0), f32_bits(1.0), f32_bits(-1.0), F32_EPS, neg32(F32_EPS),
    0x7FC00001, 0xFFC00001, 0x00000001, 0x80000001, 0x007FFFFF, 0x807FFFFF])
add_sort("f32_total_cmp_order", FS + "tests/correctness_f32.rs:54-70", "f32", [
    F32_NAN, F32_INF, f32_bits(1.0), f32_bits(0.0), neg32(0), f32_bits(-1.0), F32_NINF,
    neg32(F32_NAN)])
add_sort("f32_neg_zero_first", FS + "tests/correctness_f32.rs:72-84", "f32",
         [0, 0x80000000, 0, 0x80000000, 0, 0x80000000])
add_sort("f32_nan_variants", FS + "tests/correctness_f32.rs:86-98", "f32",
         [0x7FC00000 | i for i in range(1, 11)] + [0xFFC00000 | i for i in range(1, 11)])
add_sort("f32_denormals", FS + "tests/correctness_f32.rs:100-112", "f32",
         list(range(1, 101)) + [0x80000000 | i for i in range(1, 101)]
         + [0, 0x80000000, F32_MIN_POS, neg32(F32_MIN_POS)])

# f64 specials (correctness_f64.rs)
add_sort("f64_total_cmp_order", FS + "tests/correctness_f64.rs:21-39", "f64", [
    F64_NAN, F64_INF, f64_bits(1.0), f64_bits(0.0), neg64(0), f64_bits(-1.0), F64_NINF,
    0xFFF8000000000000])
add_sort("f64_ieee754_special", FS + "tests/correctness_f64.rs:40-67", "f64", [
    F64_NAN, F64_INF, F64_NINF, F64_MAX, F64_MIN, F64_MIN_POS, neg64(F64_MIN_POS),
    0, neg64(0), f64_bits(1.0), f64_bits(-1.0), F64_EPS, neg64(F64_EPS),
    0x7FF8000000000001, 0xFFF8000000000001, 1, 0x8000000000000001,
    0x000FFFFFFFFFFFFF, 0x800FFFFFFFFFFFFF])
add_sort("f64_neg_zero_first", FS + "tests/correctness_f64.rs:70-82", "f64",
         [0, neg64(0), 0, neg64(0), 0, neg64(0)])
add_sort("f64_denormals", FS + "tests/correctness_f64.rs:95-107", "f64",
         list(range(1, 101)) + [neg64(i) for i in range(1, 101)]
         + [0, neg64(0), F64_MIN_POS, neg64(F64_MIN_POS)])
add_sort("f64_buffer_basic", FS + "tests/correctness_f64.rs:156-167", "f64",
         [f64_bits(v) for v in (3.0, -1.0)] + [F64_NAN, 0, neg64(0), F64_INF, F64_NINF])
add_sort("f64_per_byte_isolation", FS + "tests/correctness_f64.rs:234-250", "f64",
         [v << (8 * b) for b in range(8) for v in (0x01, 0x80, 0xFF)])

# integer boundaries (correctness_u64.rs, correctness_i64.rs, correctness_i32.rs)
U64MAX = 2**64 - 1
add_sort("u64_boundaries", FS + "tests/correctness_u64.rs:10-18", "u64",
         [U64MAX, 0, 1, U64MAX - 1], [0, 1, U64MAX - 1, U64MAX])
add_sort("u64_byte_boundaries", FS + "tests/correctness_u64.rs:20-35", "u64",
         [0xFF << (8 * b) for b in range(8)] + [1 << (8 * b) for b in range(8)] + [0, U64MAX])
add_sort("u64_buffer_basic", FS + "tests/correctness_u64.rs:59-68", "u64",
         [100, 3, U64MAX, 0, 42, 1], [0, 1, 3, 42, 100, U64MAX])
add_sort("u64_powers_of_two", FS + "tests/correctness_u64.rs:132-143", "u64",
         [1 << i for i in range(64)] + [0, U64MAX])
add_sort("i64_boundaries", FS + "tests/correctness_i64.rs:7-15", "i64",
         [i64(v) for v in (-2**63, -1, 0, 1, 2**63 - 1)],
         [i64(v) for v in (-2**63, -1, 0, 1, 2**63 - 1)])
add_sort("i64_sign_boundary", FS + "tests/correctness_i64.rs:17-28", "i64",
         [i64(v) for v in list(range(-1000, 1001)) + [-2**63, 2**63 - 1]])
add_sort("i64_buffer_basic", FS + "tests/correctness_i64.rs:66-77", "i64",
         [i64(v) for v in (5, -3, 0, 2**63 - 1, -2**63, 1, -1)])
add_sort("i32_boundaries", FS + "tests/correctness_i32.rs:10-18", "i32",
         [i32(v) for v in (2**31 - 1, 0, -2**31, -1, 1)],
         [i32(v) for v in (-2**31, -1, 0, 1, 2**31 - 1)])
add_sort("i32_buffer_basic", FS + "tests/correctness_i32.rs:90-100", "i32",
         [i32(v) for v in (5, -3, 0, 2**31 - 1, -2**31, 1, -1)])
add_sort("u32_single", FS + "tests/correctness.rs:46-52", "u32", [42], [42])
add_sort("u32_empty", FS + "tests/correctness.rs:38-44", "u32", [], [])

# stability vectors the reference's spec promises (ai/tasks/spec/QA.md)
add_argsort("argsort_spec_stability", FS + "ai/tasks/spec/QA.md:486", "f32",
            [f32_bits(v) for v in (1.0, 2.0, 1.0, 2.0, 1.0)], [0, 2, 4, 1, 3])
add_argsort("argsort_spec_two_reversed", FS + "ai/tasks/spec/QA.md:484", "f32",
            [f32_bits(2.0), f32_bits(1.0)], [1, 0])
add_pairs("pairs_spec_stability_u32", FS + "ai/tasks/spec/QA.md:539", "u32",
          [3, 1, 3, 1, 3], [0, 1, 2, 3, 4], [1, 1, 3, 3, 3], [1, 3, 0, 2, 4])
add_pairs("pairs_spec_stability_f32", FS + "ai/tasks/spec/QA.md:540", "f32",
          [f32_bits(v) for v in (1.0, 2.0, 1.0, 2.0)], [10, 20, 30, 40],
          [f32_bits(v) for v in (1.0, 1.0, 2.0, 2.0)], [10, 30, 20, 40])
add_pairs("pairs_spec_negzero_stability", FS + "ai/tasks/spec/QA.md:542", "f32",
          [0x80000000, 0, 0x80000000, 0], [0, 1, 2, 3],
          [0x80000000, 0x80000000, 0, 0], [0, 2, 1, 3])

# GpuGather known answers (forge-runtime/src/gather.rs tests): output[i] = source[indices[i]]
RT = "metal-forge-compute/forge-runtime/"


def add_gather(name, src, kind, source, indices, expected):
    computed = [source[i] for i in indices]
    assert computed == expected, name
    cases.append({"name": name, "source": src, "op": "gather", "type": kind,
                  "values": source, "indices": indices, "expected_values": computed,
                  "expected_from": "reference"})


add_gather("gather_u32_permutation", RT + "src/gather.rs:213-248", "u32",
           [10, 20, 30, 40], [2, 0, 1, 3], [30, 10, 20, 40])
add_gather("gather_u64_permutation", RT + "src/gather.rs:251-286", "u64",
           [100, 200, 300, 400], [3, 1, 0, 2], [400, 200, 100, 300])
add_gather("gather_u32_identity", RT + "src/gather.rs:289-324", "u32",
           [(i + 1) * 10 for i in range(5)], list(range(5)), [(i + 1) * 10 for i in range(5)])
add_gather("gather_u32_reverse", RT + "src/gather.rs:327-363", "u32",
           [i * 100 for i in range(8)], list(range(7, -1, -1)), [i * 100 for i in range(7, -1, -1)])

if __name__ == "__main__":
    out = os.path.join(HERE, "golden.json")
    with open(out, "w") as f:
        json.dump({"generator": "tests/golden/make_golden.py", "cases": cases}, f, indent=1)
    print(f"wrote {len(cases)} cases to {out}")
