#!/usr/bin/env python3
"""Headline benchmark: forge-sort sort_buffer on 268,435,456 uniform u32 keys,
device resident, on one MI355X.

A step is one sort of one freshly-unsorted buffer of n keys already in HBM.
W + K copies of the same seeded input are prepared before timing, so the timed
region holds exactly K back-to-back sorts and no copies (and no profiling
events).  Per-launch kernel durations come from K more sorts of the same
input, with HIP events that the library records around every launch on the
stream the kernels run on (fs_set_profiling).  A sort is a fixed sequence of
launches; the roofline is reported for the launch position with the longest
average duration (the dominant kernel): on the headline's top-16 path the
local sort fs_local_k32, whose algorithmic traffic is one read and one write
of every key, 8 B/key (the 36 B/key whole-sort convention counts 4 such
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

--workload picks one of the other BASELINE.json configs (64-bit keys, floats,
argsort, pairs, the 1M and 16M sizes) for the same measurement: its own metric
line with the roofline of its dominant digit-pass kernel, no CPU baseline and
no slice API.  The default (no flag) is the headline line above.  --path lsd
or --path top16 forces the keys-only u32/i32 sort onto one of its two paths
(the LSD digit passes; the top-16 path wherever its sample accepts the input),
for profiling a path at a size where the library would pick the other one.
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
# measured HBM bytes per launch of the headline's dominant kernel (rocprofv3
# FETCH_SIZE / WRITE_SIZE, scaled by a copy kernel's readings)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "{kernel}_u32_256M_traffic.json")


# name -> (op, key type, n, data description, BASELINE.json config)
WORKLOADS = {
    "u32_256M": ("sort", "u32", 268_435_456, "uniform u32 over [0, 2^32), numpy PCG64 seed 2024", "configs[1]"),
    "u32_16M": ("sort", "u32", 16_777_216, "uniform u32 over [0, 2^32), numpy PCG64 seed 2024", "configs[1]"),
    "u32_1M": ("sort", "u32", 1_048_576, "uniform u32 over [0, 2^32), numpy PCG64 seed 2024", "configs[0]"),
    "f32_64M": ("sort", "f32", 67_108_864, "98% N(0, 1e3), 2% -0.0/+0.0/+-inf/subnormals/NaN, seed 5", "configs[2]"),
    "i32_64M": ("sort", "i32", 67_108_864, "uniform over the full i32 range, seed 2", "configs[2]"),
    "argsort_f32_16M": ("argsort", "f32", 16_777_216, "uniform [-1, 1) quantised to 4096 values, seed 6", "configs[3]"),
    "pairs_u32_64M": ("pairs", "u32", 67_108_864, "Zipf(1.1) keys below 2^20 with a 10% run of one key, values = index, seed 7", "configs[3]"),
    "u64_128M": ("sort", "u64", 134_217_728, "uniform u64, seed 3", "configs[4]"),
    "i64_128M": ("sort", "i64", 134_217_728, "uniform i64, seed 4", "configs[4]"),
    "f64_128M": ("sort", "f64", 134_217_728, "N(0, 1e6), seed 8", "configs[4]"),
    "u64_low20_128M": ("sort", "u64", 134_217_728, "high 44 bits 0, low 20 bits uniform, seed 9", "configs[4]"),
}


def workload_input(name, n):
    """Keys (and values for pairs) of a workload, from the seeded generators."""
    from forge_sort import datagen
    kind = WORKLOADS[name][1]
    if name.startswith("u32"):
        return datagen.uniform_u32(n, seed=2024), None
    if name == "f32_64M":
        return datagen.f32_normal_specials(n, 5), None
    if name == "i32_64M":
        return datagen.uniform_i32(n, 2), None
    if name == "argsort_f32_16M":
        return datagen.argsort_f32_ties(n, 6), None
    if name == "pairs_u32_64M":
        return datagen.zipf_pairs_u32(n, 7)
    if name == "u64_128M":
        return datagen.uniform_u64(n, 3), None
    if name == "i64_128M":
        return datagen.uniform_i64(n, 4), None
    if name == "f64_128M":
        return datagen.normal_f64(n, 8), None
    if name == "u64_low20_128M":
        return datagen.low20_u64(n, 0, 9), None
    raise ValueError(kind)


def ordered_bits(a):
    """Keys as unsigned integers in the sort's order: sign flip for signed
    types, FloatFlip (IEEE total order) for floats."""
    w = a.dtype.itemsize * 8
    u = a.view(np.uint32 if w == 32 else np.uint64)
    top = (np.uint32 if w == 32 else np.uint64)(1 << (w - 1))
    if a.dtype.kind == "i":
        return u ^ top
    if a.dtype.kind == "f":
        neg = (u >> (w - 1)).astype(bool)
        return np.where(neg, ~u, u ^ top)
    return u


def check_output(op, keys_in, vals_in, keys_out, vals_out):
    """Bit-for-bit equality with the one correct output, computed by numpy on
    the keys' total-order bits: sorted keys (unique for a multiset), and for
    argsort and pairs the stable order (ties by original index)."""
    o = ordered_bits(keys_in)
    if op == "sort":
        return bool(np.array_equal(ordered_bits(keys_out), np.sort(o)))
    idx = np.argsort(o, kind="stable").astype(np.uint32)
    if op == "argsort":
        return bool(np.array_equal(vals_out, idx))
    return bool(np.array_equal(ordered_bits(keys_out), o[idx]) and np.array_equal(vals_out, vals_in[idx]))


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# The GPU box grants one GPU's share of its host (16 threads, whatever nproc
# shows there); a parallel CPU sort is run on at most that many threads.
BOX_CPU_SHARE = 16


def cpu_baseline(keys, seconds, gpu_out):
    """Oracle ('port', 1 core) on the full input, repeated for ~`seconds`,
    its first output compared bit for bit with the GPU's (`gpu_out`); C++
    stand-ins once each on the same input."""
    import oracle
    n = keys.size
    runs = []
    oracle_match = None
    t_end = time.perf_counter() + seconds
    while True:
        t0 = time.perf_counter()
        out = oracle.sort("u32", keys)
        runs.append(time.perf_counter() - t0)
        if oracle_match is None:
            oracle_match = bool(np.array_equal(out, gpu_out))
        del out
        if time.perf_counter() >= t_end:
            break
    port = n / float(np.median(runs)) / 1e6
    affinity = len(os.sched_getaffinity(0))
    res = {"value": round(port, 1), "unit": "Mkeys/s", "cores": 1, "kind": "port",
           "sample": f"oracle C radix sort (MSD byte 3 + per-bucket LSD bytes 0-2) on the same "
                     f"{n:,} keys, {len(runs)} run(s), median",
           "oracle_match": oracle_match,
           "cpu_model": _cpu_model(), "nproc": os.cpu_count(), "affinity_cpus": affinity}
    try:
        lib = ctypes.CDLL(os.path.join(ROOT, "oracle", "_build", "libcpubase.so"))
        lib.cb_std_sort_u32.argtypes = [ctypes.c_void_p, ctypes.c_uint64]
        lib.cb_parallel_sort_u32.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int]
        threads = max(1, min(BOX_CPU_SHARE, affinity))
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
                                  "stands_in_for": "rayon par_sort_unstable",
                                  "thread_limit": f"min(affinity CPUs {affinity}, the GPU box's per-GPU "
                                                  f"share {BOX_CPU_SHARE}); nproc {os.cpu_count()}"},
        }
    except OSError as e:
        log(f"cpu stand-ins unavailable: {e}")
    return res


def _cpu_model():
    """/proc/cpuinfo's model name, with family/model/stepping (the name alone
    can be as short as "AMD EPYC")."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                k, v = (x.strip() for x in line.split(":", 1))
                if k in ("model name", "cpu family", "model", "stepping") and k not in info:
                    info[k] = v
            if not line.strip() and info:
                break
    except OSError:
        return None
    if not info:
        return None
    return (f"{info.get('model name', '?')} (family {info.get('cpu family', '?')}, "
            f"model {info.get('model', '?')}, stepping {info.get('stepping', '?')})")


def load_traffic(kernel):
    try:
        with open(TRAFFIC_FILE.format(kernel=kernel)) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    return t if t.get("kernel", kernel) == kernel else None


def launch_bytes(name, ksize, vbytes, n):
    """Algorithmic bytes of one launch that does its work: a histogram read
    reads every key; the fused first pass, a digit pass and the local sort
    read and write every key (and value)."""
    if name.startswith("fs_upsweep"):
        return ksize * n
    if name.startswith(("fs_first", "fs_local")):
        return 2 * ksize * n
    if name.startswith("fs_onesweep"):
        return 2 * (ksize + vbytes) * n
    return 0


FIRST_KINDS = ["histogram read", "fused first pass", "fused first pass, region overflow",
               "top-16 path", "top-16 path, region overflow (re-scatter)"]


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="u32_256M")
    ap.add_argument("--n", type=int, default=None, help="override the workload's key count")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-slice-api", action="store_true")
    ap.add_argument("--path", choices=("auto", "lsd", "top16"), default="auto",
                    help="keys-only u32/i32 sorts: the library's choice (auto), the LSD digit passes at any "
                         "size (lsd), or the top-16 path wherever its sample accepts the input (top16)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the sort is "
              "single-GPU and no multi-GPU path is built", file=sys.stderr)
        sys.exit(2)

    from forge_sort import OP_ARGSORT, OP_PAIRS, OP_SORT, DeviceNotFound, GpuSorter, datagen
    try:
        sorter = GpuSorter.new(0)
    except DeviceNotFound:
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)

    if args.path != "auto":
        from forge_sort import TEST_TOP16, TOP16_NEVER, TOP16_SAMPLED
        sorter.set_test_option(TEST_TOP16, TOP16_NEVER if args.path == "lsd" else TOP16_SAMPLED)
    wl = args.workload
    headline = wl == "u32_256M" and args.path == "auto"
    op_name, kind, n_default, data_desc, cfg_ref = WORKLOADS[wl]
    n = args.n or n_default
    K, W = args.steps, args.warmup
    op = {"sort": OP_SORT, "argsort": OP_ARGSORT, "pairs": OP_PAIRS}[op_name]
    log(f"bench: {wl} ({op_name} {kind}) n={n:,} steps={K} warmup={W}")
    keys, vals = workload_input(wl, n)
    ksize = keys.dtype.itemsize
    src = sorter.alloc_sort_buffer(kind, n)
    src.copy_from_slice(keys)
    vsrc = None
    if op == OP_PAIRS:
        vsrc = sorter.alloc_sort_buffer("u32", n)
        vsrc.copy_from_slice(vals)
    bufs, vbufs = [], []
    for _ in range(W + K):
        b = sorter.alloc_sort_buffer(kind, n)
        sorter.copy_device(b.device_ptr(), src.device_ptr(), ksize * n)
        bufs.append(b)
        if op != OP_SORT:
            v = sorter.alloc_sort_buffer("u32", n)
            if op == OP_PAIRS:
                sorter.copy_device(v.device_ptr(), vsrc.device_ptr(), 4 * n)
            vbufs.append(v)
    sorter.device_synchronize()

    def vptr(i):
        return vbufs[i].device_ptr() if vbufs else None

    for i in range(W):
        sorter.encode(op, kind, bufs[i].device_ptr(), vptr(i), n)
    sorter.synchronize()

    # the timed sorts: no profiling events between the launches
    sorter.device_synchronize()
    t0 = time.perf_counter()
    for i in range(K):
        sorter.encode(op, kind, bufs[W + i].device_ptr(), vptr(W + i), n)
    sorter.synchronize()
    sorter.device_synchronize()
    t1 = time.perf_counter()
    first_kind = sorter.first_pass()             # how each sort began (same input every step)
    log(f"bench: timed {K} sorts in {t1 - t0:.4f} s")
    # the last timed output (sorted, same multiset, stable for argsort and
    # pairs), checked below
    bufs[-1].set_len(n)
    keys_out = bufs[-1].as_slice()
    vals_out = None
    if vbufs:
        vbufs[-1].set_len(n)
        vals_out = vbufs[-1].as_slice()
    # K more sorts of the same input, with HIP events around every launch (on
    # the sort's stream): the per-kernel durations
    for i in range(K):
        sorter.copy_device(bufs[W + i].device_ptr(), src.device_ptr(), ksize * n)
        if op == OP_PAIRS:
            sorter.copy_device(vbufs[W + i].device_ptr(), vsrc.device_ptr(), 4 * n)
    sorter.device_synchronize()
    sorter.set_profiling(True)
    sorter.profile_reset()
    for i in range(K):
        sorter.encode(op, kind, bufs[W + i].device_ptr(), vptr(W + i), n)
    sorter.synchronize()
    prof = sorter.profile()
    sorter.set_profiling(False)

    # exact output check: the oracle's sort of the same keys in the cpu_baseline
    # leg of the headline line, numpy's otherwise
    check_with_oracle = headline and not args.no_cpu_baseline
    exact = None if check_with_oracle else check_output(op_name, keys, vals, keys_out, vals_out)
    for b in bufs + vbufs:
        b.free()
    src.free()
    if vsrc is not None:
        vsrc.free()
    if exact is False:
        print("bench: output check FAILED (timed output differs from the exact sort)", file=sys.stderr)
        sys.exit(3)

    ms_per_step = (t1 - t0) * 1e3 / K
    value = n / (ms_per_step / 1e3) / 1e6

    # Launch sequence of one sort (the same for every sort of this input) and
    # the algorithmic bytes per key of the whole sort, B(k,v) = k + 2k(k+v).
    vbytes = 4 if op != OP_SORT else 0
    sort_bytes = ksize + 2 * ksize * (ksize + vbytes)
    L = len(prof) // K
    seq = [{"kernel": prof[j][0], "avg_ms": round(float(np.mean([prof[s * L + j][1] for s in range(K)])), 4)}
           for j in range(L)]
    by_kernel = {}
    for name, ms in prof:
        by_kernel.setdefault(name, []).append(ms)
    kernels = {k: {"avg_ms": round(float(np.mean(v)), 4), "launches": len(v)}
               for k, v in sorted(by_kernel.items())}
    kernel_sum_ms = sum(ms for _, ms in prof) / K
    # the dominant kernel: the launch position with the longest average
    dom = max(range(L), key=lambda j: seq[j]["avg_ms"])
    dom_kernel, dom_ms = seq[dom]["kernel"], seq[dom]["avg_ms"]
    dom_bytes = launch_bytes(dom_kernel, ksize, vbytes, n)
    achieved = dom_bytes / (dom_ms / 1e3) / 1e9
    traffic = load_traffic(dom_kernel) if headline else None
    roofline = {
        "bound": "hbm", "kernel": dom_kernel,
        "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": traffic.get("bytes_per_launch") if traffic else None,
        "bytes_per_launch_algorithmic": dom_bytes,
        "avg_launch_ms": dom_ms, "launch_position": dom,
    }
    for j, e in enumerate(seq):
        b = launch_bytes(e["kernel"], ksize, vbytes, n)
        # (a launch far shorter than its bytes allow had nothing to do: a
        # constant digit's, or the re-scatter launch without an overflow)
        if b and e["avg_ms"] > 0 and b / (e["avg_ms"] / 1e3) / 1e9 <= HBM_PEAK_GBS:
            e["achieved_GBps"] = round(b / (e["avg_ms"] / 1e3) / 1e9, 1)
    first_pass = {"kind": FIRST_KINDS[first_kind] if first_kind < len(FIRST_KINDS) else str(first_kind),
                  "kernel": seq[0]["kernel"] if seq[0]["kernel"].startswith(("fs_first", "fs_upsweep"))
                  else seq[1]["kernel"]}
    sort_frac = sort_bytes * n / (ms_per_step / 1e3) / (HBM_PEAK_GBS * 1e9)

    # The slice API (sort_u32 on a host array: copy in, sort, copy out), reported
    # on its own as the reference's bench does; PCIe-bound, never `value`.
    slice_api = None
    if headline and not args.no_slice_api:
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
    if headline and not args.no_cpu_baseline:
        log("bench: cpu baseline")
        cpu = cpu_baseline(keys, args.cpu_seconds, keys_out)
        if not cpu["oracle_match"]:
            print("bench: timed output differs from the oracle's sort", file=sys.stderr)
            sys.exit(3)
    del keys_out, vals_out

    api = {"sort": "sort_buffer", "argsort": "argsort (device buffers)",
           "pairs": "sort_pairs (device buffers)"}[op_name]
    if headline and n == n_default:
        workload = "sort_buffer u32, 268,435,456 keys, device resident (BASELINE.json configs[1])"
    else:
        workload = f"{api} {kind}, {n:,} keys, device resident (BASELINE.json {cfg_ref})"
        if args.path != "auto":
            workload += f", path forced: {args.path}"
    line = {
        "metric": METRIC if headline else f"Mkeys/s ({wl}, 1 MI355X) and % of HBM-bandwidth roofline",
        "value": round(value, 1), "unit": "Mkeys/s", "n_gpus": 1,
        "steps": K, "warmup": W, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": kind,
        "data": f"synthetic: {data_desc}, resident in HBM",
        "config": {"workload": workload, "n": n, "key_type": kind, "op": api, "path": args.path},
        "roofline": roofline,
        "sort_roofline": {"bytes_per_key": sort_bytes, "frac": round(sort_frac, 4),
                          "achieved_GBps": round(sort_frac * HBM_PEAK_GBS, 1)},
        "oracle_match": cpu["oracle_match"] if cpu else None,
        "exact_match": cpu["oracle_match"] if cpu else exact,
        "first_pass": first_pass,
        "launch_sequence": seq,
        "kernels": kernels, "kernel_ms_per_step": round(kernel_sum_ms, 4),
        "slice_api": slice_api,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
