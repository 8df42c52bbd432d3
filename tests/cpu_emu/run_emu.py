"""Runs the product's C ABI, built for the CPU emulator, against the oracle
(TEST INFRASTRUCTURE ONLY).  Usage: python run_emu.py <small|prod> <case> ...

Executed in a subprocess by tests/test_cpu_emulation.py so that an emulated
device memory fault (the guard pages turn it into SIGSEGV -> exit code 86)
or an emulator deadlock cannot take the test runner down.  The forge_sort
package is pointed at the emulation library only inside this process.
"""
import ctypes
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "gpu-forge_amd"), os.path.join(ROOT, "oracle")]

import numpy as np  # noqa: E402

import oracle  # noqa: E402
import forge_sort  # noqa: E402
from forge_sort import _build  # noqa: E402

BITS = {"u32": np.uint32, "i32": np.uint32, "f32": np.uint32,
        "u64": np.uint64, "i64": np.uint64, "f64": np.uint64}


def use_emulator(flavor):
    lib = os.path.join(HERE, "_build", f"libforge_sort_emu_{flavor}.so")
    _build.SO = lib
    _build.HSACO = lib          # existence check only; the emulator ignores the path
    forge_sort._lib = None


def keys_for(kind, n, dist, seed, tile=None):
    g = np.random.Generator(np.random.PCG64(seed))
    wide = BITS[kind] == np.uint64
    if dist == "uniform":
        b = g.integers(0, 1 << (64 if wide else 32), size=n, dtype=BITS[kind], endpoint=False)
    elif dist == "few":
        b = g.choice(g.integers(0, 1 << (64 if wide else 32), size=5, dtype=BITS[kind], endpoint=False), size=n)
    elif dist == "same":
        b = np.full(n, 7, dtype=BITS[kind])
    elif dist == "low12":
        b = g.integers(0, 1 << 12, size=n, dtype=BITS[kind])
    elif dist == "byte0":
        # one varying digit (the lowest): a single-pass schedule whose pass
        # writes scratch, copied back afterwards
        b = g.integers(0, 256, size=n, dtype=BITS[kind])
    elif dist == "byte1":
        # one varying digit above the lowest: the caller's keys are copied to
        # scratch first and the single pass writes them back
        b = (g.integers(0, 256, size=n, dtype=BITS[kind]) << BITS[kind](8)).astype(BITS[kind])
    elif dist == "skew0":
        # lowest byte 3 or 200, the rest uniform: the fused first pass's
        # sampled region sizes give those two digit values all the room
        b = g.integers(0, 1 << (64 if wide else 32), size=n, dtype=BITS[kind], endpoint=False)
        b = (b & ~BITS[kind](0xFF)) | np.where(g.integers(0, 2, size=n) == 0, 3, 200).astype(BITS[kind])
    elif dist == "grp0":
        # lowest byte 3 in the tiles of the fused pass's region group 0
        # ((tile / 8) % 8 == 0, tiles of `tile` keys), uniform elsewhere: the
        # input-wide sample underrates digit 3 for that group, whose region
        # of it overflows once other groups hold tiles
        b = g.integers(0, 1 << (64 if wide else 32), size=n, dtype=BITS[kind], endpoint=False)
        in0 = (np.arange(n) // tile // 8) % 8 == 0
        b[in0] = (b[in0] & ~BITS[kind](0xFF)) | BITS[kind](3)
    elif dist == "grp2":
        # the byte below the top byte (2, or 6 for 64-bit keys) is 3 in the
        # tiles of region group 0 (as grp0, for the top-16 path's fused pass,
        # which scatters by that byte)
        b = g.integers(0, 1 << (64 if wide else 32), size=n, dtype=BITS[kind], endpoint=False)
        in0 = (np.arange(n) // tile // 8) % 8 == 0
        sh = BITS[kind](48 if wide else 16)
        b[in0] = (b[in0] & ~(BITS[kind](0xFF) << sh)) | (BITS[kind](3) << sh)
    elif dist == "top8":
        # the top byte only two values: segments of the local sort far larger
        # than a block holds
        top = 56 if wide else 24
        b = g.integers(0, 1 << top, size=n, dtype=BITS[kind])
        b |= np.where(g.integers(0, 2, size=n) == 0, 0x10, 0xF0).astype(BITS[kind]) << BITS[kind](top)
    elif dist == "top8grp0":
        # two top-byte values (the top-16 sequence's sample takes the LSD
        # passes) and byte 0 crowded into region group 0 (its region overflows)
        top = 56 if wide else 24
        b = g.integers(0, 1 << top, size=n, dtype=BITS[kind])
        b |= np.where(g.integers(0, 2, size=n) == 0, 0x10, 0xF0).astype(BITS[kind]) << BITS[kind](top)
        in0 = (np.arange(n) // tile // 8) % 8 == 0
        b[in0] = (b[in0] & ~BITS[kind](0xFF)) | BITS[kind](3)
    elif dist == "zipf":
        # a dominant bin: Zipf(1.1) ranks below 2^20 (most keys small, digit 1
        # and 2 mostly zero), as in the pairs benchmark config
        b = np.minimum(g.zipf(1.1, size=n) - 1, (1 << 20) - 1).astype(BITS[kind])
    else:
        raise ValueError(dist)
    return b.view(oracle.NP_DTYPES[kind])


def check_offset(sorter, kind, keys):
    """Sort keys that start one element past a 16-byte boundary (device API):
    the upsweep then reads them one key at a time."""
    import ctypes
    n, size = keys.size, keys.itemsize
    buf = sorter.alloc_sort_buffer(kind, n + 1)
    ptr = buf.device_ptr() + size
    L = forge_sort._load()
    sorter._check(L.fs_copy_to_device(sorter._h, ctypes.c_void_p(ptr), keys.ctypes.data, n * size))
    sorter.sort_device(kind, ptr, n)
    out = np.empty_like(keys)
    sorter._check(L.fs_copy_to_host(sorter._h, out.ctypes.data, ctypes.c_void_p(ptr), n * size))
    buf.free()
    return np.array_equal(out.view(BITS[kind]), oracle.sort(kind, keys).view(BITS[kind]))


def check_gather(kind, n, seed):
    """GpuGather on random indices (u32 or u64 elements by key width)."""
    import ctypes
    g = np.random.Generator(np.random.PCG64(seed))
    src = g.integers(0, 1 << 63, size=n, dtype=np.uint64).astype(BITS[kind])
    idx = g.integers(0, n, size=n + 5, dtype=np.uint32)
    ga = forge_sort.GpuGather.new()
    ps, pi, po = ga.alloc_buffer(src.nbytes), ga.alloc_buffer(idx.nbytes), ga.alloc_buffer(idx.size * src.itemsize)
    L = forge_sort._load()
    s = forge_sort.GpuSorter.new()
    s._check(L.fs_copy_to_device(s._h, ctypes.c_void_p(ps), src.ctypes.data, src.nbytes))
    s._check(L.fs_copy_to_device(s._h, ctypes.c_void_p(pi), idx.ctypes.data, idx.nbytes))
    (ga.gather_u64 if src.dtype == np.uint64 else ga.gather_u32)(ps, pi, po, idx.size, src.size)
    out = np.empty(idx.size, dtype=src.dtype)
    s._check(L.fs_copy_to_host(s._h, out.ctypes.data, ctypes.c_void_p(po), out.nbytes))
    for p in (ps, pi, po):
        ga.free_buffer(p)
    ga.close()
    s.close()
    return np.array_equal(out, oracle.gather(src, idx))


# injected fault -> the message its device-side guard must report
FAULTS = {
    "fault_digits": (forge_sort.FAULT_BAD_DIGITS, "digit count does not match the key width"),
    "fault_buffer": (forge_sort.FAULT_BAD_BUFFER, "device schedule named an unknown buffer"),
    "fault_tile": (forge_sort.FAULT_EXTRA_BLOCK, "digit pass drew a tile id beyond the grid"),
    "fault_stall": (forge_sort.FAULT_STALL_TILE, "look-back wait exceeded its spin bound"),
}


def sorted_ok(sorter, kind, keys):
    got = keys.copy()
    getattr(sorter, f"sort_{kind}")(got)
    return np.array_equal(got.view(BITS[kind]), oracle.sort(kind, keys).view(BITS[kind]))


def check_fault(sorter, op, kind, keys):
    """The injected fault must come back as GpuExecution with its guard's
    message; the next sort without the fault must be exact again."""
    code, message = FAULTS[op]
    sorter.set_test_option(forge_sort.TEST_INJECT_FAULT, code)
    got = keys.copy()
    try:
        getattr(sorter, f"sort_{kind}")(got)
        raised = None
    except forge_sort.GpuExecution as e:
        raised = str(e)
    finally:
        sorter.set_test_option(forge_sort.TEST_INJECT_FAULT, forge_sort.FAULT_NONE)
    if raised is None or message not in raised:
        print(f"  expected GpuExecution '{message}', got {raised!r}", flush=True)
        return False
    return sorted_ok(sorter, kind, keys)


def check_small_s1(sorter, kind, keys):
    """A fused sort whose region sample gets half the S1 budget it was sized
    for: the sample refuses its layout and splits the budget evenly; the
    regions then hold the keys (small inputs, where the per-region margin
    dominates the budget) or overflow into the stable passes.  Exact either
    way, and exact again without the fault."""
    sorter.set_test_option(forge_sort.TEST_INJECT_FAULT, forge_sort.FAULT_SMALL_S1)
    sorter.set_test_option(forge_sort.TEST_FUSED, forge_sort.FUSED_ALWAYS)
    try:
        ok = sorted_ok(sorter, kind, keys)
        first = sorter.first_pass()
    finally:
        sorter.set_test_option(forge_sort.TEST_INJECT_FAULT, forge_sort.FAULT_NONE)
    try:
        ok = ok and sorted_ok(sorter, kind, keys) and sorter.first_pass() == forge_sort.FIRST_FUSED
    finally:
        sorter.set_test_option(forge_sort.TEST_FUSED, FUSED_MODE)
    if first not in (forge_sort.FIRST_FUSED, forge_sort.FIRST_FUSED_OVERFLOW):
        print(f"  first pass {first} with half the budget, expected the fused pass", flush=True)
        ok = False
    print(f"  first pass {first} with half the budget", flush=True)
    return ok


def check_hold(sorter, kind, keys, expect):
    """A digit pass whose XCD queue is held back (EMU_HOLD_QUEUE): held until
    a look-back wait has ended at its spin bound, the sort must report
    GpuExecution ("timeout"); held briefly, far within the bound, it must be
    exact ("exact"); then a sort is exact again."""
    got = keys.copy()
    try:
        getattr(sorter, f"sort_{kind}")(got)
        ok = expect == "exact" and np.array_equal(got.view(BITS[kind]), oracle.sort(kind, keys).view(BITS[kind]))
        print("  held queue: completed", flush=True)
    except forge_sort.GpuExecution as e:
        ok = expect == "timeout" and "look-back wait exceeded its spin bound" in str(e)
        print(f"  held queue: {e}", flush=True)
    return ok and sorted_ok(sorter, kind, keys)


def check_capture(sorter, kind, n, seed):
    """HIP-graph capture rules: a sort enqueued on a capturing stream may not
    grow the scratch (fs_reserve first); after a capture no sort may grow it
    until fs_allow_scratch_growth; sorts that fit keep working."""
    L = forge_sort._load()
    st = L.emu_test_stream_create
    st.restype = ctypes.c_void_p
    stream = st()
    small, big = keys_for(kind, n, "uniform", seed), keys_for(kind, 3 * n, "uniform", seed + 1)
    sorter.reserve(forge_sort.OP_SORT, kind, n)
    buf = sorter.alloc_sort_buffer(kind, 3 * n)
    buf.copy_from_slice(small)
    ok = L.emu_test_begin_capture(ctypes.c_void_p(stream)) == 0
    sorter.encode(forge_sort.OP_SORT, kind, buf.device_ptr(), None, n, stream=stream)   # fits the reserve
    try:
        sorter.encode(forge_sort.OP_SORT, kind, buf.device_ptr(), None, 3 * n, stream=stream)
        ok = False
        print("  growth while capturing was not refused", flush=True)
    except forge_sort.InvalidArgument:
        pass
    ok &= L.emu_test_end_capture(ctypes.c_void_p(stream)) == 0
    sorter.synchronize()
    try:
        sorted_ok(sorter, kind, big)
        ok = False
        print("  growth after a capture was not refused", flush=True)
    except forge_sort.InvalidArgument:
        pass
    ok &= sorted_ok(sorter, kind, keys_for(kind, n // 2, "few", seed + 2))   # fits: still fine
    sorter.allow_scratch_growth()
    ok &= sorted_ok(sorter, kind, big)
    buf.free()
    return ok


def check_no_alloc(sorter, kind, n, dist, seed):
    """fs_encode_no_alloc (static scratch) against fs_encode for every op,
    then the same with a smaller input (which finds the first call's contents
    in the static scratch)."""
    ok = True
    for m in (n, n // 3 + 1):
        keys = keys_for(kind, m, dist, seed + m)
        vals = np.arange(m, dtype=np.uint32)[::-1].copy()
        for op in (forge_sort.OP_SORT, forge_sort.OP_ARGSORT, forge_sort.OP_PAIRS):
            outs = []
            for no_alloc in (False, True):
                kb = sorter.alloc_sort_buffer(kind, m)
                kb.copy_from_slice(keys)
                vb = sorter.alloc_sort_buffer("u32", m)
                if op == forge_sort.OP_PAIRS:
                    vb.copy_from_slice(vals)
                enc = sorter.encode_no_alloc if no_alloc else sorter.encode
                enc(op, kind, kb.device_ptr(), vb.device_ptr(), m)
                sorter.synchronize()
                vb.set_len(m)
                outs.append((kb.as_slice().view(BITS[kind]), vb.as_slice()))
                kb.free()
                vb.free()
            ok &= bool(np.array_equal(outs[0][0], outs[1][0]))
            if op != forge_sort.OP_SORT:
                ok &= bool(np.array_equal(outs[0][1], outs[1][1]))
    return ok


# the fused first pass of keys-only sorts: by size (the default), or
# forced on for every case of a run (EMU_TEST_FUSED=2)
FUSED_MODE = int(os.environ.get("EMU_TEST_FUSED", "0"))
# the top-16 path of keys-only u32/i32 sorts: by size (the default), or
# forced on (EMU_TEST_TOP16=2)
TOP16_MODE = int(os.environ.get("EMU_TEST_TOP16", "0"))
FIRST_PASS = {"fused": forge_sort.FIRST_FUSED, "fusedover": forge_sort.FIRST_FUSED_OVERFLOW,
              "nofused": forge_sort.FIRST_HISTOGRAM, "top16": forge_sort.FIRST_TOP16,
              "top16over": forge_sort.FIRST_TOP16_RESCATTER,
              # the top-16 launch sequence, its sample choosing the LSD passes
              "top16auto_lsd": forge_sort.FIRST_FUSED, "top16auto_lsdover": forge_sort.FIRST_FUSED_OVERFLOW,
              "top16auto": forge_sort.FIRST_TOP16}


def check_first_pass(sorter, op, kind, n, dist, seed):
    """A keys-only sort, exact, that began the way the case names
    (fs_sorter_first_pass), with the fused first pass at every size, or
    ("nofused") never."""
    keys = keys_for(kind, n, dist, seed, tile=sorter.tile_config()["k64" if BITS[kind] == np.uint64 else "k32"])
    # top16w...: the same case on the wide local-sort blocks
    wide = op.startswith("top16w")
    if wide:
        op = "top16" + op[6:]
    top16 = op.startswith("top16")
    sorter.set_test_option(forge_sort.TEST_FUSED,
                           forge_sort.FUSED_NEVER if op == "nofused" else forge_sort.FUSED_ALWAYS)
    sorter.set_test_option(forge_sort.TEST_TOP16, forge_sort.TOP16_SAMPLED if op.startswith("top16auto")
                           else forge_sort.TOP16_ALWAYS if top16 else forge_sort.TOP16_NEVER)
    # top16s<bits>: segments named by that many top bits
    sorter.set_test_option(forge_sort.TEST_SEG_BITS, int(op[6:]) if op.startswith("top16s") else 0)
    sorter.set_test_option(forge_sort.TEST_LOCAL_WIDE, 1 if wide else 0)
    try:
        ok = sorted_ok(sorter, kind, keys)
        first = sorter.first_pass()
        passes, mask = sorter.last_pass_info()
    finally:
        sorter.set_test_option(forge_sort.TEST_FUSED, FUSED_MODE)
        sorter.set_test_option(forge_sort.TEST_TOP16, TOP16_MODE)
        sorter.set_test_option(forge_sort.TEST_SEG_BITS, 0)
        sorter.set_test_option(forge_sort.TEST_LOCAL_WIDE, 0)
    expect = FIRST_PASS["top16" if op.startswith("top16s") else op]
    if top16 and dist == "same" and not op.startswith("top16auto"):
        expect = forge_sort.FIRST_TOP16               # forced onto the top-16 path: one segment of every key
    if first != expect:
        print(f"  first pass {first}, expected {expect}", flush=True)
        ok = False
    if dist == "same" and passes != 0 and expect != forge_sort.FIRST_TOP16:
        print(f"  equal keys ran {passes} passes", flush=True)
        ok = False
    print(f"{'PASS' if ok else 'FAIL'} {op}{' (wide)' if wide else ''} {kind} n={n} {dist} passes={passes} "
          f"mask={mask:#x}", flush=True)
    return ok


def check(sorter, op, kind, n, dist, seed):
    if op in FIRST_PASS or op.startswith(("top16s", "top16w")):
        return check_first_pass(sorter, op, kind, n, dist, seed)
    if op == "noalloc":
        ok = check_no_alloc(sorter, kind, n, dist, seed)
        print(f"{'PASS' if ok else 'FAIL'} {op} {kind} n={n}", flush=True)
        return ok
    if op in FAULTS or op in ("hold_timeout", "hold_exact", "capture", "small_s1"):
        if op == "capture":
            ok = check_capture(sorter, kind, n, seed)
        elif op == "small_s1":
            ok = check_small_s1(sorter, kind, keys_for(kind, n, dist, seed))
        elif op.startswith("hold_"):
            ok = check_hold(sorter, kind, keys_for(kind, n, dist, seed), op[5:])
        else:
            ok = check_fault(sorter, op, kind, keys_for(kind, n, dist, seed))
        print(f"{'PASS' if ok else 'FAIL'} {op} {kind} n={n}", flush=True)
        return ok
    if op == "gather":
        ok = check_gather(kind, n, seed)
        print(f"{'PASS' if ok else 'FAIL'} gather {kind} n={n}", flush=True)
        return ok
    keys = keys_for(kind, n, dist, seed)
    if op == "offset":
        ok = check_offset(sorter, kind, keys)
    elif op == "sort":
        got = keys.copy()
        getattr(sorter, f"sort_{kind}")(got)
        ok = np.array_equal(got.view(BITS[kind]), oracle.sort(kind, keys).view(BITS[kind]))
    elif op == "argsort":
        ok = np.array_equal(getattr(sorter, f"argsort_{kind}")(keys), oracle.argsort(kind, keys))
    else:
        vals = np.arange(n, dtype=np.uint32)[::-1].copy()
        ek, ev = oracle.sort_pairs(kind, keys, vals)
        gk, gv = keys.copy(), vals.copy()
        getattr(sorter, f"sort_pairs_{kind}")(gk, gv)
        ok = np.array_equal(gk.view(BITS[kind]), ek.view(BITS[kind])) and np.array_equal(gv, ev)
    passes, mask = sorter.last_pass_info()
    if dist == "same" and op != "offset" and n > 1:
        ok = ok and passes == 0 and mask == 0     # every digit constant: an exact histogram says so
    print(f"{'PASS' if ok else 'FAIL'} {op} {kind} n={n} {dist} passes={passes} mask={mask:#x}", flush=True)
    return ok


def main():
    flavor = sys.argv[1]
    use_emulator(flavor)
    sorter = forge_sort.GpuSorter.new()
    # layout switches for the cases (testing hooks of the C ABI)
    if os.environ.get("EMU_TEST_WIDE_LOOKBACK") == "1":
        sorter.set_test_option(forge_sort.TEST_WIDE_LOOKBACK, 1)
    if os.environ.get("EMU_TEST_UPSWEEP_PER_CU"):
        sorter.set_test_option(forge_sort.TEST_UPSWEEP_BLOCKS_PER_CU, int(os.environ["EMU_TEST_UPSWEEP_PER_CU"]))
    sorter.set_test_option(forge_sort.TEST_FUSED, FUSED_MODE)
    sorter.set_test_option(forge_sort.TEST_TOP16, TOP16_MODE)
    print("tiles", sorter.tile_config(), flush=True)
    ok = True
    for spec in sys.argv[2:]:
        op, kind, n, dist, seed = spec.split(":")
        ok &= check(sorter, op, kind, int(n), dist, int(seed))
    sorter.close()
    sys.exit(0 if ok else 1)


if __name__ == "__main__":
    main()
