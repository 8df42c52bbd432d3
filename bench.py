#!/usr/bin/env python3
"""Headline benchmark: forge-sort sort_buffer on 268,435,456 uniform u32 keys,
device resident, on one MI355X.

A step is one sort of one freshly-unsorted buffer of n keys already in HBM.
W + K copies of the same seeded input are prepared before timing, so the timed
region holds exactly K back-to-back sorts and no copies.  Per-launch kernel
durations come from HIP events that the library records on the stream the
kernels run on (fs_set_profiling); the dominant kernel is the digit pass
(fs_onesweep_k32), whose algorithmic traffic is one read and one write of
every key per pass: 8 B/key (the 36 B/key whole-sort convention counts 4 such
passes plus one 4 B/key histogram read).

The CPU baseline times the oracle (a scalar C restatement of the reference's
radix sort, oracle/forge_sort_oracle.c) on the same keys on the host, and
reports labelled C++ stand-ins for the reference bench's Rust sort_unstable
and rayon par_sort_unstable (std::sort, __gnu_parallel::sort).

Device memory, copies and synchronisation go through the library itself
(hipMalloc / hipMemcpy / hipDeviceSynchronize behind the C ABI); torch is not
imported, so the library runs on the ROCm HIP runtime it was built against
rather than on the copy bundled with torch (both share one soname, and
whichever loads first would serve both).

Also reported, never as `value`: the slice API (sort_u32 on a 16M-key host
array, host-to-device copy + sort + copy back, so PCIe-bound), as the
reference's bench reports its slice and buffer APIs apart.

Prints one JSON line.  --gpus > 1 is refused: this build measures one GPU.
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "gpu-forge_amd"), os.path.join(ROOT, "oracle")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

METRIC = "Mkeys/s (u32 256M, 1 MI355X) and % of HBM-bandwidth roofline vs host CPU sort"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, 8 TB/s
PASS_BYTES_PER_KEY = 8         # one read + one write of a u32 key per digit pass
SORT_BYTES_PER_KEY = 36        # k + k*2*k for k = 4 (histogram read + 4 passes)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "onesweep_k32_u32_256M_traffic.json")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_baseline(keys, seconds):
    """Oracle ('port', 1 core) on the full input, repeated for ~`seconds`;
    C++ stand-ins once each on the same input."""
    import oracle
    n = keys.size
    runs = []
    t_end = time.perf_counter() + seconds
    while True:
        t0 = time.perf_counter()
        out = oracle.sort("u32", keys)
        runs.append(time.perf_counter() - t0)
        del out
        if time.perf_counter() >= t_end:
            break
    port = n / float(np.median(runs)) / 1e6
    res = {"value": round(port, 1), "unit": "Mkeys/s", "cores": 1, "kind": "port",
           "sample": f"oracle C radix sort (MSD byte 3 + per-bucket LSD bytes 0-2) on the same "
                     f"{n:,} keys, {len(runs)} run(s), median",
           "cpu_model": _cpu_model()}
    try:
        lib = ctypes.CDLL(os.path.join(ROOT, "oracle", "_build", "libcpubase.so"))
        lib.cb_std_sort_u32.argtypes = [ctypes.c_void_p, ctypes.c_uint64]
        lib.cb_parallel_sort_u32.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int]
        threads = min(16, os.cpu_count() or 1)
        a = keys.copy()
        t0 = time.perf_counter()
        lib.cb_std_sort_u32(a.ctypes.data, n)
        t_std = time.perf_counter() - t0
        a = keys.copy()
        t0 = time.perf_counter()
        lib.cb_parallel_sort_u32(a.ctypes.data, n, threads)
        t_par = time.perf_counter() - t0
        del a
        res["stand_ins"] = {
            "std_sort": {"value": round(n / t_std / 1e6, 1), "cores": 1,
                         "stands_in_for": "Rust slice::sort_unstable"},
            "gnu_parallel_sort": {"value": round(n / t_par / 1e6, 1), "cores": threads,
                                  "stands_in_for": "rayon par_sort_unstable"},
        }
    except OSError as e:
        log(f"cpu stand-ins unavailable: {e}")
    return res


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def load_traffic():
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--n", type=int, default=268_435_456)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-slice-api", action="store_true")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the sort is "
              "single-GPU and no multi-GPU path is built", file=sys.stderr)
        sys.exit(2)

    from forge_sort import OP_SORT, DeviceNotFound, GpuSorter, datagen
    try:
        sorter = GpuSorter.new(0)
    except DeviceNotFound:
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)

    n, K, W = args.n, args.steps, args.warmup
    log(f"bench: sort_buffer u32 n={n:,} steps={K} warmup={W}")
    keys = datagen.uniform_u32(n, seed=2024)
    src = sorter.alloc_sort_buffer("u32", n)
    src.copy_from_slice(keys)
    bufs = []
    for _ in range(W + K):
        b = sorter.alloc_sort_buffer("u32", n)
        sorter.copy_device(b.device_ptr(), src.device_ptr(), 4 * n)
        bufs.append(b)
    sorter.device_synchronize()

    for i in range(W):
        sorter.encode(OP_SORT, "u32", bufs[i].device_ptr(), None, n)
    sorter.synchronize()

    sorter.set_profiling(True)
    sorter.profile_reset()
    sorter.device_synchronize()
    t0 = time.perf_counter()
    for i in range(K):
        sorter.encode(OP_SORT, "u32", bufs[W + i].device_ptr(), None, n)
    sorter.synchronize()
    sorter.device_synchronize()
    t1 = time.perf_counter()
    prof = sorter.profile()
    sorter.set_profiling(False)
    log(f"bench: timed {K} sorts in {t1 - t0:.4f} s")

    # sanity: the last output is sorted and holds the same multiset (checksums)
    bufs[-1].set_len(n)
    last = bufs[-1].as_slice()
    ok_sorted = bool(np.all(last[1:] >= last[:-1]))
    ok_sum = int(last.astype(np.uint64).sum()) == int(keys.astype(np.uint64).sum())
    ok_xor = int(np.bitwise_xor.reduce(last)) == int(np.bitwise_xor.reduce(keys))
    del last
    for b in bufs:
        b.free()
    src.free()
    if not (ok_sorted and ok_sum and ok_xor):
        print("bench: output check FAILED", file=sys.stderr)
        sys.exit(3)

    ms_per_step = (t1 - t0) * 1e3 / K
    value = n / (ms_per_step / 1e3) / 1e6

    by_kernel = {}
    for name, ms in prof:
        by_kernel.setdefault(name, []).append(ms)
    passes = by_kernel.get("fs_onesweep_k32", [])
    active = [ms for ms in passes if ms > 0.02]      # constant-digit launches exit at once
    pass_ms = float(np.mean(active)) if active else float("nan")
    achieved = PASS_BYTES_PER_KEY * n / (pass_ms / 1e3) / 1e9
    kernel_sum_ms = sum(ms for _, ms in prof) / K
    traffic = load_traffic()
    roofline = {
        "bound": "hbm", "kernel": "fs_onesweep_k32",
        "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": traffic.get("bytes_per_launch") if traffic else None,
        "bytes_per_launch_algorithmic": PASS_BYTES_PER_KEY * n,
        "avg_launch_ms": round(pass_ms, 4), "launches": len(active),
    }
    kernels = {k: {"avg_ms": round(float(np.mean(v)), 4), "launches": len(v)}
               for k, v in sorted(by_kernel.items())}
    sort_frac = SORT_BYTES_PER_KEY * n / (ms_per_step / 1e3) / (HBM_PEAK_GBS * 1e9)

    # The slice API (sort_u32 on a host array: copy in, sort, copy out), reported
    # on its own as the reference's bench does; PCIe-bound, never `value`.
    slice_api = None
    if not args.no_slice_api:
        ns = 16_777_216
        host = datagen.uniform_u32(ns, seed=7)
        work = host.copy()
        sorter.sort_u32(work)                    # warm-up (grows the staging buffers)
        runs = []
        for _ in range(5):
            work[:] = host
            t0s = time.perf_counter()
            sorter.sort_u32(work)
            runs.append(time.perf_counter() - t0s)
        ok_slice = bool(np.all(work[1:] >= work[:-1]))
        slice_api = {"op": "sort_u32 (host slice: H2D + sort + D2H)", "n": ns,
                     "value": round(ns / float(np.median(runs)) / 1e6, 1), "unit": "Mkeys/s",
                     "ms": round(float(np.median(runs)) * 1e3, 3), "sorted": ok_slice}
        del host, work

    cpu = None
    if not args.no_cpu_baseline:
        log("bench: cpu baseline")
        cpu = cpu_baseline(keys, args.cpu_seconds)

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "Mkeys/s", "n_gpus": 1,
        "steps": K, "warmup": W, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u32",
        "data": "synthetic: uniform u32 over [0, 2^32), numpy PCG64 seed 2024, resident in HBM",
        "config": {"workload": "sort_buffer u32, 268,435,456 keys, device resident (BASELINE.json configs[1])"
                   if n == 268_435_456 else f"sort_buffer u32, {n:,} keys, device resident",
                   "n": n, "key_type": "u32", "op": "sort_buffer"},
        "roofline": roofline,
        "sort_roofline": {"bytes_per_key": SORT_BYTES_PER_KEY, "frac": round(sort_frac, 4),
                          "achieved_GBps": round(sort_frac * HBM_PEAK_GBS, 1)},
        "kernels": kernels, "kernel_ms_per_step": round(kernel_sum_ms, 4),
        "slice_api": slice_api,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
