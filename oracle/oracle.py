"""ctypes front end of the CPU oracle (forge_sort_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product package.  The functions
mirror GpuSorter's host entry points (metal-forge-compute/forge-sort/src/lib.rs:
sort_<t> :791/:840/:920/:2238/:2348/:2417, argsort_<t> :1675/:1754/:1838/:2595/
:2669/:2747, sort_pairs_<t> :1923/:2024/:2132/:2826/:2921) on numpy arrays, and
forge-runtime's GpuGather (src/gather.rs:124-143).
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")

KEY_TYPES = {"u32": 0, "i32": 1, "f32": 2, "u64": 3, "i64": 4, "f64": 5}
NP_DTYPES = {"u32": np.uint32, "i32": np.int32, "f32": np.float32,
             "u64": np.uint64, "i64": np.int64, "f64": np.float64}

OK = 0
ERR_LENGTH_MISMATCH = 4

_lib = None


def build():
    """Compile the oracle with gcc (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        vp, u64 = ctypes.c_void_p, ctypes.c_uint64
        L.or_sort.argtypes = [ctypes.c_int, vp, u64]
        L.or_argsort.argtypes = [ctypes.c_int, vp, u64, vp]
        L.or_sort_pairs.argtypes = [ctypes.c_int, vp, u64, vp, u64]
        L.or_transform_32.argtypes = [vp, u64, ctypes.c_uint32]
        L.or_transform_64.argtypes = [vp, u64, ctypes.c_uint32]
        L.or_gather.argtypes = [ctypes.c_int, vp, u64, vp, vp, u64]
        for f in (L.or_sort, L.or_argsort, L.or_sort_pairs, L.or_gather):
            f.restype = ctypes.c_int
        _lib = L
    return _lib


def set_mutation(code):
    """Plant a known mistake in the oracle (meta-tests only); 0 clears it."""
    ctypes.c_int.in_dll(lib(), "or_mutation").value = int(code)


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _check(kind, a):
    a = np.ascontiguousarray(a, dtype=NP_DTYPES[kind])
    return a


def sort(kind, keys):
    """Return a sorted copy of `keys` (same dtype), as GpuSorter::sort_<kind>."""
    k = _check(kind, keys).copy()
    rc = lib().or_sort(KEY_TYPES[kind], _ptr(k), k.size)
    if rc != OK:
        raise RuntimeError(f"oracle sort failed: {rc}")
    return k


def argsort(kind, keys):
    """Stable argsort (ties by original index), as GpuSorter::argsort_<kind>."""
    k = _check(kind, keys)
    out = np.empty(k.size, dtype=np.uint32)
    rc = lib().or_argsort(KEY_TYPES[kind], _ptr(k), k.size, _ptr(out))
    if rc != OK:
        raise RuntimeError(f"oracle argsort failed: {rc}")
    return out


def sort_pairs(kind, keys, values):
    """Stable key/value sort; returns (keys, values) copies, or raises on mismatch."""
    k = _check(kind, keys).copy()
    v = np.ascontiguousarray(values, dtype=np.uint32).copy()
    rc = lib().or_sort_pairs(KEY_TYPES[kind], _ptr(k), k.size, _ptr(v), v.size)
    if rc == ERR_LENGTH_MISMATCH:
        raise ValueError(f"length mismatch: keys={k.size}, values={v.size}")
    if rc != OK:
        raise RuntimeError(f"oracle sort_pairs failed: {rc}")
    return k, v


def transform(bits, mode):
    """Apply sort.metal's transform `mode` (0 xor-sign, 1 FloatFlip, 2 inverse) to raw bits."""
    b = np.ascontiguousarray(bits).copy()
    if b.dtype == np.uint32:
        lib().or_transform_32(_ptr(b), b.size, mode)
    elif b.dtype == np.uint64:
        lib().or_transform_64(_ptr(b), b.size, mode)
    else:
        raise TypeError("transform takes uint32 or uint64 bit patterns")
    return b


def gather(source, indices):
    """GpuGather::gather_u32 / gather_u64: source[indices] for a u32 or u64
    source array; raises IndexError for an index past the source (the product
    reports GpuExecution and writes 0 there)."""
    source = np.ascontiguousarray(source)
    if source.dtype not in (np.uint32, np.uint64):
        raise TypeError("gather source must be u32 or u64")
    indices = np.ascontiguousarray(indices, dtype=np.uint32)
    out = np.zeros(indices.size, dtype=source.dtype)
    st = lib().or_gather(1 if source.dtype == np.uint64 else 0, _ptr(source), source.size,
                         _ptr(indices), _ptr(out), indices.size)
    if st != OK:
        raise IndexError("gather index out of range of the source")
    return out
