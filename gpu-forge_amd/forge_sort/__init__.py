"""forge_sort -- MI355X-native GpuSorter (Python mirror of the Rust API).

Mirrors metal-forge-compute/forge-sort/src/lib.rs over the C ABI in
include/forge_sort.h (libforge_sort.so, which loads the gfx950 code object).
Method names, argument meaning and error behaviour follow the Rust crate:

    sorter = GpuSorter.new()                     # lib.rs:596
    sorter.sort_u32(arr)                         # in place, numpy array (lib.rs:791)
    idx = sorter.argsort_f32(arr)                # np.uint32 permutation (lib.rs:1838)
    sorter.sort_pairs_u32(keys, values)          # both in place (lib.rs:1923)
    buf = sorter.alloc_sort_buffer("u32", cap)   # SortBuffer in HBM (lib.rs:694)
    buf.copy_from_slice(data); sorter.sort_buffer(buf); buf.as_slice()

Errors are SortError subclasses with the reference's Display strings
(lib.rs:94-104).  There is no CPU fallback: if the HIP library is not built,
importing the sorter raises.
"""
import ctypes
import os

import numpy as np

from . import _build

__all__ = [
    "GpuGather",
    "GpuSorter", "SortBuffer", "SortError", "DeviceNotFound", "ShaderCompilation",
    "GpuExecution", "LengthMismatch", "KEY_TYPES", "library_path",
]

KEY_TYPES = {"u32": 0, "i32": 1, "f32": 2, "u64": 3, "i64": 4, "f64": 5}
NP_DTYPES = {"u32": np.uint32, "i32": np.int32, "f32": np.float32,
             "u64": np.uint64, "i64": np.int64, "f64": np.float64}
KEY_SIZE = {"u32": 4, "i32": 4, "f32": 4, "u64": 8, "i64": 8, "f64": 8}   # SortKey::KEY_SIZE
OP_SORT, OP_ARGSORT, OP_PAIRS = 0, 1, 2
NO_ALLOC_MAX_KEYS = 1 << 20          # FS_NO_ALLOC_MAX_KEYS
# fs_test_option and the FS_FAULT_* codes (include/forge_sort.h, csrc/fs_params.h)
TEST_WIDE_LOOKBACK, TEST_UPSWEEP_BLOCKS_PER_CU, TEST_INJECT_FAULT, TEST_FUSED, TEST_TOP16, TEST_SEG_BITS = \
    0, 1, 2, 3, 4, 5
TEST_LOCAL_WIDE = 6
FUSED_BY_SIZE, FUSED_NEVER, FUSED_ALWAYS = 0, 1, 2       # TEST_FUSED values
TOP16_BY_SIZE, TOP16_NEVER, TOP16_ALWAYS, TOP16_SAMPLED = 0, 1, 2, 3   # TEST_TOP16 values
FUSED_MIN_KEYS = 1 << 25                                 # FS_FUSED_MIN_KEYS
TOP16_MIN_KEYS32 = 44_040_192                            # FS_TOP16_MIN_KEYS32
TOP16_MIN_KEYS64 = 1 << 21                               # FS_TOP16_MIN_KEYS64
# fs_sorter_first_pass: how the last sort began
FIRST_HISTOGRAM, FIRST_FUSED, FIRST_FUSED_OVERFLOW, FIRST_TOP16, FIRST_TOP16_RESCATTER = 0, 1, 2, 3, 4
FAULT_NONE, FAULT_BAD_DIGITS, FAULT_BAD_BUFFER, FAULT_EXTRA_BLOCK, FAULT_STALL_TILE, FAULT_SMALL_S1 = 0, 1, 2, 3, 4, 5

FS_OK = 0
FS_ERR_DEVICE_NOT_FOUND = 1
FS_ERR_SHADER_COMPILATION = 2
FS_ERR_GPU_EXECUTION = 3
FS_ERR_LENGTH_MISMATCH = 4
FS_ERR_INVALID_ARGUMENT = 5
FS_ERR_OUT_OF_MEMORY = 6


class SortError(Exception):
    """SortError (lib.rs:94-104)."""


class DeviceNotFound(SortError):
    pass


class ShaderCompilation(SortError):
    pass


class GpuExecution(SortError):
    pass


class LengthMismatch(SortError):
    def __init__(self, keys, values):
        super().__init__(f"length mismatch: keys={keys}, values={values}")
        self.keys = keys
        self.values = values


class InvalidArgument(SortError, ValueError):
    pass


class OutOfMemory(SortError, MemoryError):
    pass


_ERRORS = {
    FS_ERR_DEVICE_NOT_FOUND: DeviceNotFound,
    FS_ERR_SHADER_COMPILATION: ShaderCompilation,
    FS_ERR_GPU_EXECUTION: GpuExecution,
    FS_ERR_INVALID_ARGUMENT: InvalidArgument,
    FS_ERR_OUT_OF_MEMORY: OutOfMemory,
}

_lib = None


def library_path():
    return _build.SO


def _load():
    """Load libforge_sort.so (and through it the gfx950 code object)."""
    global _lib
    if _lib is not None:
        return _lib
    path = _build.SO
    if not os.path.exists(path) or not os.path.exists(_build.HSACO):
        raise ImportError(
            f"forge_sort HIP library not built ({path}); run __graft_entry__.build()")
    L = ctypes.CDLL(path)
    vp, u64, sz, i = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_size_t, ctypes.c_int
    pp = ctypes.POINTER(ctypes.c_void_p)
    u32p = ctypes.POINTER(ctypes.c_uint32)
    sig = {
        "fs_sorter_new": ([i, pp], i),
        "fs_sorter_with_context": ([i, vp, pp], i),
        "fs_sorter_free": ([vp], None),
        "fs_last_error": ([vp], ctypes.c_char_p),
        "fs_status_str": ([i], ctypes.c_char_p),
        "fs_alloc_sort_buffer": ([vp, i, sz, pp], i),
        "fs_free_sort_buffer": ([vp, vp], i),
        "fs_copy_to_device": ([vp, vp, vp, sz], i),
        "fs_copy_to_host": ([vp, vp, vp, sz], i),
        "fs_copy_device": ([vp, vp, vp, sz], i),
        "fs_device_synchronize": ([vp], i),
        "fs_sort": ([vp, i, vp, u64], i),
        "fs_argsort": ([vp, i, vp, u64, vp], i),
        "fs_sort_pairs": ([vp, i, vp, u64, vp, u64], i),
        "fs_sort_buffer": ([vp, i, vp, u64], i),
        "fs_argsort_buffer": ([vp, i, vp, u64, vp], i),
        "fs_sort_pairs_buffer": ([vp, i, vp, vp, u64], i),
        "fs_encode": ([vp, i, i, vp, vp, u64, vp], i),
        "fs_encode_no_alloc": ([vp, i, i, vp, vp, u64, vp], i),
        "fs_reserve": ([vp, i, i, u64], i),
        "fs_allow_scratch_growth": ([vp], i),
        "fs_sorter_set_test_option": ([vp, i, u64], i),
        "fs_sorter_first_pass": ([vp, u32p], i),
        "fs_synchronize": ([vp], i),
        "fs_last_pass_info": ([vp, u32p, u32p], i),
        "fs_set_profiling": ([vp, i], i),
        "fs_profile_count": ([vp], i),
        "fs_profile_reset": ([vp], i),
        "fs_profile_read": ([vp, i, ctypes.POINTER(ctypes.c_char_p),
                             ctypes.POINTER(ctypes.c_float)], i),
        "fs_tile_config": ([vp, u32p], i),
        "fs_set_lookback_stats": ([vp, i], i),
        "fs_read_lookback_stats": ([vp, ctypes.POINTER(ctypes.c_uint64)], i),
        "fs_gather_new": ([i, pp], i),
        "fs_gather_with_context": ([i, vp, pp], i),
        "fs_gather_free": ([vp], None),
        "fs_gather_last_error": ([vp], ctypes.c_char_p),
        "fs_gather_alloc_buffer": ([vp, sz, pp], i),
        "fs_gather_free_buffer": ([vp, vp], i),
        "fs_gather_encode": ([vp, i, vp, u64, vp, vp, u64, vp], i),
        "fs_gather_synchronize": ([vp], i),
        "fs_gather_u32": ([vp, vp, u64, vp, vp, u64], i),
        "fs_gather_u64": ([vp, vp, u64, vp, vp, u64], i),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res
    _lib = L
    return L


def _arr_ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


def _as_keys(kind, data, writable):
    dt = NP_DTYPES[kind]
    if not isinstance(data, np.ndarray) or data.dtype != dt:
        raise TypeError(f"expected a numpy array of {np.dtype(dt).name}")
    if not data.flags.c_contiguous or (writable and not data.flags.writeable):
        raise ValueError("array must be C-contiguous" + (" and writable" if writable else ""))
    return data


class SortBuffer:
    """SortBuffer<T> (lib.rs:160-281): a device allocation of `capacity` keys.

    Unlike Metal's shared storage, HBM is not host-addressable, so
    as_slice()/as_mut_slice() are staging copies: as_slice() returns a host
    copy of the first len() keys, and as_mut_slice() returns a host array of
    `capacity` keys that commit() uploads (copy_from_slice does both).
    """

    def __init__(self, sorter, kind, ptr, capacity, length=0, owned=True):
        self._sorter = sorter
        self.kind = kind
        self._ptr = ptr
        self._capacity = capacity
        self._len = length
        self._owned = owned
        self._mirror = None

    def len(self):
        return self._len

    def __len__(self):
        return self._len

    def is_empty(self):
        return self._len == 0

    def capacity(self):
        return self._capacity

    def device_ptr(self):
        """Device address (the metal_buffer() accessor's role, lib.rs:243)."""
        return self._ptr

    def set_len(self, n):
        if n > self._capacity:
            raise ValueError(f"len {n} exceeds capacity {self._capacity}")
        self._len = n

    def copy_from_slice(self, data):
        data = _as_keys(self.kind, np.ascontiguousarray(data), False)
        if data.size > self._capacity:
            raise ValueError(f"data len {data.size} exceeds capacity {self._capacity}")
        self._sorter._check(_load().fs_copy_to_device(
            self._sorter._h, ctypes.c_void_p(self._ptr), _arr_ptr(data), data.nbytes))
        self._len = data.size

    def copy_to_slice(self, dest):
        n = min(self._len, dest.size)
        if dest.dtype != NP_DTYPES[self.kind] or not dest.flags.c_contiguous:
            raise TypeError("destination must be a contiguous array of the buffer's key type")
        if n:
            self._sorter._check(_load().fs_copy_to_host(
                self._sorter._h, _arr_ptr(dest), ctypes.c_void_p(self._ptr), n * KEY_SIZE[self.kind]))

    def as_slice(self):
        out = np.empty(self._len, dtype=NP_DTYPES[self.kind])
        self.copy_to_slice(out)
        return out

    def as_mut_slice(self):
        if self._mirror is None:
            self._mirror = np.zeros(self._capacity, dtype=NP_DTYPES[self.kind])
        return self._mirror

    def commit(self):
        """Upload the as_mut_slice() mirror (whole capacity); len is unchanged."""
        if self._mirror is not None and self._capacity:
            self._sorter._check(_load().fs_copy_to_device(
                self._sorter._h, ctypes.c_void_p(self._ptr), _arr_ptr(self._mirror),
                self._mirror.nbytes))

    @classmethod
    def from_raw_parts(cls, sorter, kind, device_ptr, length, capacity):
        """from_raw_parts (lib.rs:255-272); takes ownership of device_ptr."""
        if length > capacity:
            raise ValueError(f"len {length} exceeds capacity {capacity}")
        return cls(sorter, kind, device_ptr, capacity, length, owned=True)

    def into_raw_parts(self):
        """into_raw_parts (lib.rs:278-280): (device_ptr, len, capacity); ownership moves out."""
        parts = (self._ptr, self._len, self._capacity)
        self._owned = False
        self._ptr = None
        return parts

    def free(self):
        if self._owned and self._ptr and self._sorter._h:
            _load().fs_free_sort_buffer(self._sorter._h, ctypes.c_void_p(self._ptr))
        self._ptr = None
        self._owned = False

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class GpuSorter:
    """GpuSorter (lib.rs:132-154, impl :594-3017) on one MI355X."""

    def __init__(self, device=0, stream=None, _with_context=False):
        L = _load()
        h = ctypes.c_void_p()
        if _with_context:
            st = L.fs_sorter_with_context(device, ctypes.c_void_p(stream), ctypes.byref(h))
        else:
            st = L.fs_sorter_new(device, ctypes.byref(h))
        if st != FS_OK:
            msg = L.fs_last_error(None).decode() or L.fs_status_str(st).decode()
            raise _ERRORS.get(st, SortError)(msg)
        self._h = h
        self.device = device

    @classmethod
    def new(cls, device=0):
        return cls(device)

    @classmethod
    def with_context(cls, device, stream):
        """with_context (lib.rs:606): share a caller's HIP stream (an int handle,
        e.g. torch.cuda.current_stream().cuda_stream)."""
        return cls(device, stream, _with_context=True)

    def close(self):
        if getattr(self, "_h", None):
            _load().fs_sorter_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, st):
        if st == FS_OK:
            return
        msg = _load().fs_last_error(self._h).decode()
        if st == FS_ERR_LENGTH_MISMATCH:
            raise SortError(msg)
        raise _ERRORS.get(st, SortError)(msg)

    # ---- SortBuffer ---------------------------------------------------------
    def alloc_sort_buffer(self, kind, capacity):
        """alloc_sort_buffer<T>(capacity) (lib.rs:694-702)."""
        p = ctypes.c_void_p()
        self._check(_load().fs_alloc_sort_buffer(self._h, KEY_TYPES[kind], capacity, ctypes.byref(p)))
        return SortBuffer(self, kind, p.value, capacity)

    def _sort_buf(self, buf, kind):
        if buf.kind != kind:
            raise TypeError(f"SortBuffer<{buf.kind}> passed to a {kind} sort")
        self._check(_load().fs_sort_buffer(self._h, KEY_TYPES[kind], ctypes.c_void_p(buf.device_ptr()),
                                           buf.len()))

    def sort_buffer(self, buf):
        """sort_buffer (lib.rs:708): u32 keys, device resident, in place."""
        self._sort_buf(buf, "u32")

    def sort_i32_buffer(self, buf):
        self._sort_buf(buf, "i32")

    def sort_f32_buffer(self, buf):
        self._sort_buf(buf, "f32")

    def sort_u64_buffer(self, buf):
        self._sort_buf(buf, "u64")

    def sort_i64_buffer(self, buf):
        self._sort_buf(buf, "i64")

    def sort_f64_buffer(self, buf):
        self._sort_buf(buf, "f64")

    def encode_sort(self, buf, stream=None):
        """encode_sort (lib.rs:749): enqueue the u32 sort of `buf` on `stream`
        (None = the sorter's stream) without waiting."""
        self.encode(OP_SORT, buf.kind, buf.device_ptr(), None, buf.len(), stream)

    # ---- device pointers (torch tensors' data_ptr() or SortBuffer pointers) --
    def encode(self, op, kind, keys_ptr, values_ptr, n, stream=None):
        self._check(_load().fs_encode(self._h, op, KEY_TYPES[kind], ctypes.c_void_p(keys_ptr),
                                      ctypes.c_void_p(values_ptr or 0), n,
                                      ctypes.c_void_p(stream or 0)))

    def encode_no_alloc(self, op, kind, keys_ptr, values_ptr, n, stream=None):
        """encode() on the code object's static scratch: allocates nothing;
        n <= NO_ALLOC_MAX_KEYS; calls through one sorter must not overlap."""
        self._check(_load().fs_encode_no_alloc(self._h, op, KEY_TYPES[kind], ctypes.c_void_p(keys_ptr),
                                               ctypes.c_void_p(values_ptr or 0), n,
                                               ctypes.c_void_p(stream or 0)))

    def synchronize(self):
        self._check(_load().fs_synchronize(self._h))

    def reserve(self, op, kind, n):
        """Grow the scratch for sorts of up to n keys (e.g. before capturing a
        sort into a HIP graph, after which the scratch may not grow)."""
        self._check(_load().fs_reserve(self._h, op, KEY_TYPES[kind], n))

    def allow_scratch_growth(self):
        """Every graph that captured a sort of this sorter has been destroyed."""
        self._check(_load().fs_allow_scratch_growth(self._h))

    def set_test_option(self, option, value):
        """Testing hooks (TEST_WIDE_LOOKBACK, TEST_UPSWEEP_BLOCKS_PER_CU,
        TEST_INJECT_FAULT, TEST_FUSED, TEST_TOP16, TEST_SEG_BITS): reach layouts the product uses only
        at sizes too large for a test, choose the first pass, or inject a
        device-side fault (emulator builds)."""
        self._check(_load().fs_sorter_set_test_option(self._h, option, value))

    def first_pass(self):
        """How the last sort began: FIRST_HISTOGRAM, FIRST_FUSED (the fused
        first pass, regions used), FIRST_FUSED_OVERFLOW (a region overflowed
        and the keys were re-scattered into exact regions, or every digit is
        constant), FIRST_TOP16 (the top-16
        path) or FIRST_TOP16_RESCATTER (the top-16 path after a region
        overflowed, its keys re-scattered into exact regions)."""
        k = ctypes.c_uint32()
        self._check(_load().fs_sorter_first_pass(self._h, ctypes.byref(k)))
        return k.value

    def device_synchronize(self):
        """Wait for everything on the device (hipDeviceSynchronize)."""
        self._check(_load().fs_device_synchronize(self._h))

    def copy_device(self, dst_ptr, src_ptr, nbytes):
        """Device-to-device copy (e.g. restaging an unsorted input in HBM)."""
        self._check(_load().fs_copy_device(self._h, ctypes.c_void_p(dst_ptr), ctypes.c_void_p(src_ptr), nbytes))

    def sort_device(self, kind, keys_ptr, n):
        self._check(_load().fs_sort_buffer(self._h, KEY_TYPES[kind], ctypes.c_void_p(keys_ptr), n))

    def argsort_device(self, kind, keys_ptr, n, indices_ptr):
        self._check(_load().fs_argsort_buffer(self._h, KEY_TYPES[kind], ctypes.c_void_p(keys_ptr), n,
                                              ctypes.c_void_p(indices_ptr)))

    def sort_pairs_device(self, kind, keys_ptr, values_ptr, n):
        self._check(_load().fs_sort_pairs_buffer(self._h, KEY_TYPES[kind], ctypes.c_void_p(keys_ptr),
                                                 ctypes.c_void_p(values_ptr), n))

    # ---- slice API ------------------------------------------------------------
    def _sort(self, kind, data):
        data = _as_keys(kind, data, True)
        self._check(_load().fs_sort(self._h, KEY_TYPES[kind], _arr_ptr(data), data.size))

    def _argsort(self, kind, data):
        data = _as_keys(kind, np.ascontiguousarray(data), False)
        out = np.empty(data.size, dtype=np.uint32)
        self._check(_load().fs_argsort(self._h, KEY_TYPES[kind], _arr_ptr(data), data.size, _arr_ptr(out)))
        return out

    def _sort_pairs(self, kind, keys, values):
        keys = _as_keys(kind, keys, True)
        if not isinstance(values, np.ndarray) or values.dtype != np.uint32:
            raise TypeError("values must be a numpy uint32 array")
        if keys.size != values.size:
            raise LengthMismatch(keys.size, values.size)       # lib.rs:1928-1934
        if not values.flags.c_contiguous or not values.flags.writeable:
            raise ValueError("values must be C-contiguous and writable")
        self._check(_load().fs_sort_pairs(self._h, KEY_TYPES[kind], _arr_ptr(keys), keys.size,
                                          _arr_ptr(values), values.size))

    def sort_u32(self, data): self._sort("u32", data)            # lib.rs:791
    def sort_i32(self, data): self._sort("i32", data)            # lib.rs:840
    def sort_f32(self, data): self._sort("f32", data)            # lib.rs:920
    def sort_u64(self, data): self._sort("u64", data)            # lib.rs:2238
    def sort_i64(self, data): self._sort("i64", data)            # lib.rs:2348
    def sort_f64(self, data): self._sort("f64", data)            # lib.rs:2417

    def argsort_u32(self, data): return self._argsort("u32", data)   # lib.rs:1675
    def argsort_i32(self, data): return self._argsort("i32", data)   # lib.rs:1754
    def argsort_f32(self, data): return self._argsort("f32", data)   # lib.rs:1838
    def argsort_u64(self, data): return self._argsort("u64", data)   # lib.rs:2595
    def argsort_i64(self, data): return self._argsort("i64", data)   # lib.rs:2669
    def argsort_f64(self, data): return self._argsort("f64", data)   # lib.rs:2747

    def sort_pairs_u32(self, keys, values): self._sort_pairs("u32", keys, values)   # lib.rs:1923
    def sort_pairs_i32(self, keys, values): self._sort_pairs("i32", keys, values)   # lib.rs:2024
    def sort_pairs_f32(self, keys, values): self._sort_pairs("f32", keys, values)   # lib.rs:2132
    def sort_pairs_u64(self, keys, values): self._sort_pairs("u64", keys, values)   # lib.rs:2826
    def sort_pairs_i64(self, keys, values): self._sort_pairs("i64", keys, values)   # lib.rs:2921
    def sort_pairs_f64(self, keys, values): self._sort_pairs("f64", keys, values)   # no reference counterpart

    # ---- introspection --------------------------------------------------------
    def last_pass_info(self):
        """(passes run, bitmask of non-constant digit positions) of the last sort."""
        n, m = ctypes.c_uint32(), ctypes.c_uint32()
        self._check(_load().fs_last_pass_info(self._h, ctypes.byref(n), ctypes.byref(m)))
        return n.value, m.value

    def tile_config(self):
        """Keys per tile of the digit-pass kernels: {u32, u32+values, u64, u64+values}."""
        t = (ctypes.c_uint32 * 4)()
        self._check(_load().fs_tile_config(self._h, t))
        return {"k32": t[0], "k32_v": t[1], "k64": t[2], "k64_v": t[3]}

    def set_lookback_stats(self, enable):
        self._check(_load().fs_set_lookback_stats(self._h, 1 if enable else 0))

    def read_lookback_stats(self):
        """{tiles, rounds, stalls, entries} of the decoupled look-back since the last read."""
        c = (ctypes.c_uint64 * 4)()
        self._check(_load().fs_read_lookback_stats(self._h, c))
        return dict(zip(("tiles", "rounds", "stalls", "entries"), list(c)))

    def set_profiling(self, enable):
        self._check(_load().fs_set_profiling(self._h, 1 if enable else 0))

    def profile_reset(self):
        self._check(_load().fs_profile_reset(self._h))

    def profile(self):
        """[(kernel name, ms)] of every launch since profiling was enabled or reset."""
        L = _load()
        out = []
        for i in range(L.fs_profile_count(self._h)):
            name, ms = ctypes.c_char_p(), ctypes.c_float()
            self._check(L.fs_profile_read(self._h, i, ctypes.byref(name), ctypes.byref(ms)))
            out.append((name.value.decode(), ms.value))
        return out




class GpuGather:
    """GpuGather (forge-runtime/src/gather.rs:26-173): output[i] = source[indices[i]]
    for u32 or u64 elements on device memory.  Pointers are device addresses
    (GpuGather.alloc_buffer, SortBuffer.device_ptr(), a torch tensor's data_ptr()).
    source_len bounds the indices: an index past it yields 0 and raises
    GpuExecution (the reference reads out of bounds)."""

    def __init__(self, device=0, stream=None, _with_context=False):
        L = _load()
        h = ctypes.c_void_p()
        if _with_context:
            st = L.fs_gather_with_context(device, ctypes.c_void_p(stream), ctypes.byref(h))
        else:
            st = L.fs_gather_new(device, ctypes.byref(h))
        if st != FS_OK:
            msg = L.fs_gather_last_error(None).decode() or L.fs_status_str(st).decode()
            raise _ERRORS.get(st, SortError)(msg)
        self._h = h
        self.device = device

    @classmethod
    def new(cls, device=0):
        return cls(device)

    @classmethod
    def with_context(cls, device, stream):
        return cls(device, stream, _with_context=True)

    def close(self):
        if getattr(self, "_h", None):
            _load().fs_gather_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, st):
        if st != FS_OK:
            raise _ERRORS.get(st, SortError)(_load().fs_gather_last_error(self._h).decode())

    def alloc_buffer(self, nbytes):
        """GpuGather::alloc_buffer: device memory; returns its address."""
        p = ctypes.c_void_p()
        self._check(_load().fs_gather_alloc_buffer(self._h, nbytes, ctypes.byref(p)))
        return p.value

    def free_buffer(self, ptr):
        self._check(_load().fs_gather_free_buffer(self._h, ctypes.c_void_p(ptr)))

    def encode_gather(self, source_ptr, indices_ptr, output_ptr, count, is_64bit, source_len, stream=None):
        """encode_gather (gather.rs:81-119): enqueue, no wait."""
        self._check(_load().fs_gather_encode(self._h, 1 if is_64bit else 0, ctypes.c_void_p(source_ptr),
                                             source_len, ctypes.c_void_p(indices_ptr),
                                             ctypes.c_void_p(output_ptr), count, ctypes.c_void_p(stream or 0)))

    def synchronize(self):
        self._check(_load().fs_gather_synchronize(self._h))

    def gather_u32(self, source_ptr, indices_ptr, output_ptr, count, source_len):
        self._check(_load().fs_gather_u32(self._h, ctypes.c_void_p(source_ptr), source_len,
                                          ctypes.c_void_p(indices_ptr), ctypes.c_void_p(output_ptr), count))

    def gather_u64(self, source_ptr, indices_ptr, output_ptr, count, source_len):
        self._check(_load().fs_gather_u64(self._h, ctypes.c_void_p(source_ptr), source_len,
                                          ctypes.c_void_p(indices_ptr), ctypes.c_void_p(output_ptr), count))
