"""The product's kernels and host runtime, compiled for the CPU emulator in
tests/cpu_emu (fibers per GPU thread, guard-paged device allocations), checked
against the oracle.

Each case list runs in a child process (tests/cpu_emu/run_emu.py): an emulated
out-of-bounds device access ends that process with SIGSEGV (exit 86 after the
emulator's report), and a deadlocked emulation is cut off by the timeout,
without taking the test runner down.  Two builds are covered: "small" (tiny
tiles, so a few thousand keys span many tiles, portions of the look-back chain
and the tail paths) "prod" (the tile geometry the gfx950 build uses) and "groups" (tiny tiles
and look-back groups of two tiles, so that look-backs walk whole groups).
"""
import os
import shutil
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
EMU = os.path.join(HERE, "cpu_emu")

pytestmark = pytest.mark.skipif(shutil.which("g++") is None or shutil.which("make") is None,
                                reason="needs g++ and make")


@pytest.fixture(scope="module")
def emulator():
    r = subprocess.run(["make", "-C", EMU, "-j4"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    return EMU


def run_cases(flavor, cases, timeout=300, env=None, parallel=1):
    """Run the cases in `parallel` child processes at once (round-robin
    shares of the list), each with its share of the emulator's worker
    threads; every case must pass."""
    parallel = max(1, min(parallel, len(cases)))
    workers = max(1, (os.cpu_count() or 8) // parallel)
    procs = []
    for j in range(parallel):
        share = cases[j::parallel]
        e = dict(os.environ, **(env or {}))
        if parallel > 1:
            e.setdefault("EMU_WORKERS", str(workers))
        procs.append((share, subprocess.Popen([sys.executable, os.path.join(EMU, "run_emu.py"), flavor, *share],
                                              stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, env=e)))
    lines = []
    for share, p in procs:
        try:
            out, err = p.communicate(timeout=timeout)
        except subprocess.TimeoutExpired:
            for _, q in procs:
                q.kill()
            raise
        got = [ln for ln in out.splitlines() if ln.startswith(("PASS", "FAIL"))]
        assert p.returncode == 0 and len(got) == len(share) and all(ln.startswith("PASS") for ln in got), \
            f"exit {p.returncode}\n{out}\n{err[-4000:]}"
        lines += got
    return lines


SMALL_CASES = [
    # every op x key type, sizes spanning many small tiles
    "sort:u32:5000:uniform:1", "sort:i32:4099:uniform:2", "sort:f32:6001:uniform:3",
    "sort:u64:3000:uniform:4", "sort:i64:2049:uniform:5", "sort:f64:3001:uniform:6",
    "argsort:u32:3000:few:7", "argsort:f32:9000:few:8", "argsort:i64:2500:uniform:9",
    "pairs:u32:8000:uniform:10", "pairs:i32:3333:few:11", "pairs:f64:2500:uniform:12",
    "pairs:u64:1999:few:13",
    # constant digits skipped on the device (2 live passes, 0 live passes)
    "sort:u32:7000:low12:14", "sort:i64:4000:low12:15", "pairs:f32:6000:low12:16",
    "argsort:u32:3000:same:17", "sort:u64:2000:same:18",
    # trivial and ragged lengths (vector path off for odd n)
    "sort:u32:0:uniform:19", "sort:u32:1:uniform:20", "sort:u32:2:uniform:21",
    "sort:u32:63:uniform:22", "sort:u32:65:uniform:23", "pairs:u64:3:uniform:24",
    "argsort:f64:1025:uniform:25",
    # GpuGather
    "gather:u32:5000:uniform:26", "gather:u64:3001:uniform:27",
    # one varying digit: single-pass schedules (copy after / copy before the pass)
    "sort:u32:5000:byte0:31", "sort:i64:3000:byte1:32", "pairs:u32:4000:byte1:33",
    "pairs:f64:2000:byte0:34", "argsort:u32:3000:byte1:35", "sort:f32:4100:byte1:36",
    # dominant bins: histogram atomics of the shared digit added once per wave
    "sort:u32:9000:zipf:28", "pairs:u32:7000:zipf:29", "argsort:u64:3000:zipf:30",
    # several upsweep steps and counter folds per block
    "sort:u64:9000:uniform:37", "sort:u32:9000:same:38", "sort:i64:9000:zipf:39",
    # keys-only 32-bit sorts on the small tiles (below 4096 keys in this
    # build) and at the boundary; a fused first pass forced below it keeps
    # the stable tiles
    "sort:u32:4095:uniform:40", "sort:i32:4096:few:41", "sort:f32:3000:byte1:42", "sort:u32:3001:same:43",
    "fused:u32:3000:uniform:44",
    # argsort / pairs on the small 32-bit tiles, 64-bit sorts on theirs
    # (below 2048 keys in this build) and at that boundary
    "argsort:f32:4095:uniform:45", "pairs:u32:4096:few:46", "sort:i64:2047:few:47", "pairs:f64:2047:uniform:48",
    "argsort:u64:2048:uniform:49",
]

PROD_CASES = [
    "sort:u32:40000:uniform:1", "sort:u32:12289:uniform:2", "argsort:f32:30000:few:3",
    "pairs:u64:20000:uniform:4", "sort:i64:20000:low12:6", "pairs:u32:25000:few:7",
    "sort:f64:9000:uniform:8", "argsort:i32:13000:uniform:9",
    "pairs:u32:30000:zipf:10", "sort:u32:26000:few:11",
    # one key past a tile of the u32 (768 x 23), u64 (768 x 11) and u32+values (768 x 18) variants
    "sort:u32:17665:uniform:12", "sort:u64:8449:uniform:13", "pairs:u32:13825:uniform:14",
]


def test_emulated_small_tiles(emulator):
    run_cases("small", SMALL_CASES, parallel=4)


def test_emulated_production_tiles(emulator):
    run_cases("prod", PROD_CASES)



FUSED_SMALL = [
    # regions used: every digit varies; ragged; tiny; only digit 0 varies (the
    # regions copied back); two digits vary
    "fused:u32:9000:uniform:1", "fused:f32:20000:uniform:2", "fused:u32:1025:uniform:3",
    "fused:i32:2:uniform:4", "fused:i32:5000:byte0:5", "fused:u32:3000:low12:6",
    # skewed lowest byte, lowest byte constant: regions sized by the sample
    "fused:u32:9000:skew0:7", "fused:f32:6000:byte1:8",
    # a region overflows (digit 3 crowded into one region group), or every
    # digit is constant: stable passes over the caller's keys
    "fusedover:u32:30000:grp0:19", "fusedover:f32:30001:grp0:20", "fusedover:u32:50:same:9",
    "fusedover:u32:9000:same:10",
    # the testing hook: the histogram read instead
    "nofused:u32:9000:uniform:11", "nofused:i32:4099:byte0:12",
    # 64-bit keys: seven upper digits counted, regions of 8-byte keys
    "fused:u64:9000:uniform:13", "fused:f64:5001:uniform:14", "fused:i64:3000:byte0:15",
    "fused:u64:6000:skew0:16", "fusedover:u64:20000:grp0:21", "fusedover:f64:40:same:17",
    "nofused:u64:3000:uniform:18",
]


def test_emulated_fused_first_pass(emulator):
    """Keys-only sorts (32- and 64-bit keys) start with the fused first pass: with small
    tiles a tile of the next pass spans dozens of regions, with production
    tiles a region spans several tiles; look-back groups of two tiles follow
    it in the groups build."""
    run_cases("small", FUSED_SMALL, parallel=4)
    run_cases("prod", ["fused:u32:100000:uniform:1", "fused:f32:17665:uniform:2", "fused:u32:40000:byte0:3",
                       "fusedover:u32:450000:grp0:4", "nofused:u32:40000:uniform:5", "fused:u64:30000:uniform:6",
                       "fused:i64:8449:uniform:7", "fused:u32:40000:skew0:8"])
    run_cases("groups", ["fused:u32:70000:uniform:1", "fusedover:i32:30000:grp0:2"], env={"EMU_CUS": "8"})
    # regions larger than tiles: one- and two-region tile descriptors (and
    # more-region tiles where a region holds fewer keys than a tile)
    run_cases("regions", ["fused:u32:60000:uniform:1", "fused:f32:150001:uniform:2", "fused:i32:50000:byte0:3",
                          "fused:u32:40000:low12:4", "fused:u32:60000:skew0:5", "noalloc:u32:60000:uniform:6",
                          "sort:u64:9000:uniform:7", "pairs:u32:9000:uniform:8", "fused:u64:20000:uniform:9",
                          "fused:f64:9000:low12:10"], env={"EMU_TEST_FUSED": "2"})


def test_emulated_lookback_groups(emulator):
    """Look-back groups of two tiles, one tile entry per round trip, eight
    emulated CUs: most look-backs cross several groups, and predecessors are
    often still unpublished."""
    run_cases("groups", ["sort:u32:70000:uniform:2", "sort:i64:9000:uniform:3", "argsort:f32:33333:few:4",
                         "pairs:u64:5000:low12:5", "sort:u32:1025:uniform:6", "pairs:u32:40000:uniform:7"],
              env={"EMU_CUS": "8"})



@pytest.mark.parametrize("flavor", ["small", "groups"])
def test_emulated_wide_lookback_entries(emulator, flavor):
    """The 64-bit look-back tile entries used from n = 2^30 on, forced for
    small inputs (the FS_TEST_WIDE_LOOKBACK testing hook)."""
    run_cases(flavor, ["sort:u32:70000:uniform:2", "sort:i64:9000:uniform:3", "argsort:f32:33333:few:4",
                       "pairs:u64:5000:low12:5", "pairs:u32:40000:uniform:7"],
              env={"EMU_CUS": "8", "EMU_TEST_WIDE_LOOKBACK": "1"})


def test_emulated_upsweep_long_segments(emulator):
    """One upsweep block per emulated CU, one CU: each block counts a long
    segment; all-equal keys must come out with every digit constant (an exact
    histogram, so no pass runs); keys one element past a 16-byte boundary take
    the upsweep's one-key-at-a-time path."""
    cases = ["sort:u32:200000:uniform:1", "sort:u32:150000:same:2", "sort:u64:90000:same:3",
             "sort:i64:70001:uniform:4", "offset:u32:100003:uniform:5", "offset:u64:50001:few:6",
             "offset:f32:3:uniform:7"]
    for flavor in ("small", "prod"):
        run_cases(flavor, cases, env={"EMU_CUS": "1", "EMU_TEST_UPSWEEP_PER_CU": "1"})


def test_emulated_single_dispatch_queue(emulator):
    """Blocks started in plain increasing order from one queue (not dealt over
    XCDs), 72 at a time: a digit-pass tile then may wait on a tile whose block
    starts up to 63 blocks later (8 XCDs x 8 tiles per round), which the
    resident blocks allow."""
    run_cases("small", ["sort:u32:70000:uniform:2", "pairs:u32:40000:uniform:7", "sort:u64:9000:uniform:3"],
              env={"EMU_XCDS": "1", "EMU_WORKERS": "72"})


def test_emulated_device_error_guards(emulator):
    """Each device-side guard, driven by a fault injected in the emulator's
    fault-injection build (never on a GPU), is reported as GpuExecution with
    its own message, and the next sort is exact again: a digit count that does
    not match the key width, a schedule naming an unknown buffer, a digit-pass
    block beyond the tile grid, and a tile that never publishes (its
    successors' look-back waits end at the build's tiny spin bound).  Also the
    region sample's safety net, which raises no error: a region layout larger
    than the S1 budget is replaced by an even split and the sort stays exact."""
    run_cases("faults", ["fault_digits:u32:5000:uniform:1", "fault_digits:u64:3000:uniform:2",
                         "fault_buffer:u32:5000:uniform:3", "fault_buffer:i64:3000:uniform:4",
                         "fault_tile:u32:5000:uniform:5", "fault_tile:f64:3000:uniform:6",
                         "fault_stall:u32:9000:uniform:7", "fault_stall:u64:5000:uniform:8"],
              env={"EMU_CUS": "8"})
    # the same guards behind the fused first pass of keys-only 32-bit sorts
    run_cases("faults", ["fault_digits:u32:5000:uniform:1", "fault_buffer:f32:5000:uniform:3",
                         "fault_tile:u32:5000:uniform:5", "fault_stall:i32:9000:uniform:7"],
              env={"EMU_CUS": "8", "EMU_TEST_FUSED": "2"})
    # the region sample's safety net: a layout that would not fit the S1 the
    # host sized is replaced by an even split (the sort stays exact)
    run_cases("faults", ["small_s1:u32:30000:uniform:9", "small_s1:u64:20000:skew0:10"], env={"EMU_CUS": "8"})


def test_emulated_held_xcd_queue(emulator):
    """One XCD queue of the first digit pass held back (another stream's work
    on that XCD): held until a look-back wait on its tiles has reached the
    spin bound (a build with a bound of 2,048 polls), the sort ends with a
    clean GpuExecution; held for 50 ms, far within the product bound of 2^24
    polls, it completes exactly; either way the next sort is exact."""
    run_cases("faults", ["hold_timeout:u32:40000:uniform:1"], env={"EMU_CUS": "8", "EMU_HOLD_QUEUE": "3:timeout"})
    run_cases("prod", ["hold_exact:u32:200000:uniform:2"], env={"EMU_CUS": "8", "EMU_HOLD_QUEUE": "3:50"})


def test_emulated_no_alloc_entry_point(emulator):
    """fs_encode_no_alloc (static scratch, no allocation) gives fs_encode's
    results for every op, on two calls in a row, the second smaller."""
    run_cases("small", ["noalloc:u32:9000:uniform:1", "noalloc:f64:5000:few:2", "noalloc:i32:4099:zipf:3"])
    run_cases("small", ["noalloc:u32:9000:uniform:4", "noalloc:f32:6000:skew0:5"], env={"EMU_TEST_FUSED": "2"})


def test_emulated_capture_rules(emulator):
    """A sort enqueued on a capturing stream fits the reserved scratch or is
    refused; after a capture, growth is refused until fs_allow_scratch_growth."""
    run_cases("small", ["capture:u32:3000:uniform:1", "capture:f64:2000:uniform:2"])
    run_cases("small", ["capture:u32:3000:uniform:3"], env={"EMU_TEST_FUSED": "2"})


def test_emulated_sanitizers(emulator):
    """The product kernels and host runtime under AddressSanitizer and
    UndefinedBehaviorSanitizer (host build of the emulator, libasan preloaded)."""
    libasan = subprocess.run(["g++", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    if not os.path.isabs(libasan):
        pytest.skip("libasan not found")
    # ASan reports its own faults: the emulator's guard-page handler stays off
    run_cases("san", ["sort:u32:5000:uniform:1", "sort:f32:3001:uniform:3", "argsort:i32:2000:few:7",
                      "pairs:f64:2500:uniform:12", "sort:u32:5000:byte0:31", "sort:u32:9000:zipf:28",
                      "gather:u32:3000:uniform:26", "fused:u32:9000:uniform:40", "fusedover:u32:30000:grp0:41",
                      "fused:u32:5000:byte0:42", "top16:u64:1500:few:47"],
              timeout=600, env={"LD_PRELOAD": libasan, "EMU_NO_SEGV_HANDLER": "1", "EMU_CUS": "4", "EMU_TEST_FUSED": "2",
                                "ASAN_OPTIONS": "detect_leaks=0:detect_stack_use_after_return=0"}, parallel=3)


TOP16_SMALL = [
    # the top-16 launch sequence forced at every size (tiny local-sort blocks
    # of 512 keys in the small build): every plan of the local sort through
    # the segment bits, ragged and tiny inputs, constant digits, segments
    # larger than a block (big-segment path), an overflowing region of the
    # fused pass on digit 2 (re-scattered by its second launch)
    "top16:u32:5000:uniform:1", "top16:i32:20000:uniform:2", "top16:u32:2:uniform:3", "top16:u32:100:uniform:4",
    "top16:u32:1025:uniform:5", "top16:u32:3000:low12:6", "top16:u32:9000:zipf:7", "top16:u32:20000:top8:8",
    "top16:i32:9000:byte0:9", "top16:u32:9000:byte1:10", "top16:u32:3000:few:11", "top16:u32:5000:same:12",
    "top16over:u32:30000:grp2:13", "top16over:i32:40001:grp2:14",
    # (a forced segment count of 2^16 emulates 65,536 blocks: about a minute each)
    "top16s16:u32:9000:uniform:15", "top16s14:u32:5000:few:17",
    "top16s13:i32:20000:uniform:18", "top16s12:u32:20000:uniform:19",
    # the region sample chooses: the top-16 path on a uniform input; the LSD
    # passes in the same launches for oversized segments (two top-byte values,
    # small keys, Zipf ranks), with a region overflow on byte 0, or with every
    # digit constant
    "top16auto:u32:20000:uniform:20", "top16auto_lsd:u32:20000:top8:21", "top16auto_lsd:u32:9000:low12:22",
    "top16auto_lsd:i32:9000:zipf:23", "top16auto_lsdover:u32:30000:top8grp0:24",
    "top16auto_lsdover:u32:20000:same:25",
    # 64-bit keys: the fused pass on byte 6, the stable pass on byte 7, the
    # group sort of each segment; its LSD fallback in LDS (groups of equal
    # keys above the comparison limit), the big-segment path, re-scatter
    "top16:u64:5000:uniform:31", "top16:i64:9000:uniform:32", "top16:u64:2:uniform:33", "top16:i64:100:uniform:34",
    "top16:u64:1500:few:35", "top16:u64:3000:few:36", "top16:u64:5000:same:37", "top16:u64:9000:top8:38",
    "top16:u64:1025:low12:39", "top16:i64:9000:zipf:40", "top16over:u64:30000:grp2:41",
    "top16s12:i64:20000:uniform:43",
    "top16auto:u64:20000:uniform:44", "top16auto_lsd:u64:20000:top8:45", "top16auto_lsdover:i64:30000:top8grp0:46",
    "top16auto_lsd:u64:9000:low12:47",
    # 64-bit segments with many copies of each key: groups of equal keys
    # above the comparison limit ranked by slot (first launch and deferred
    # launch); a large group of different keys in a block-sized segment
    # (the group sort gives way to LSD in LDS in the deferred launch)
    "top16:u64:20000:few:60", "top16:u64:400:low12:61", "top16:i64:500:low12:62",
    # the wide local-sort blocks (FS_LW_BLOCK threads, which sorts beyond the
    # other blocks' size limit take): both key widths, every local plan,
    # equal keys (64-bit LSD fallback in LDS), a re-scattered region
    "top16w:u32:5000:uniform:51", "top16w:u32:3000:few:52", "top16wover:i32:30000:grp2:53",
    "top16ws12:u32:20000:uniform:54", "top16w:u64:3000:uniform:55", "top16w:i64:1500:few:56",
    "top16w:u64:5000:top8:57", "top16wover:u64:30000:grp2:58",
]


def test_emulated_top16_path(emulator):
    """Keys-only u32/i32/u64/i64 sorts on the top-16 launch sequence (region sample,
    fused pass, its re-scatter launch, digit passes, local sort): small
    tiles and blocks; production tiles; look-back groups of two tiles."""
    run_cases("small", TOP16_SMALL, timeout=900, parallel=4)
    run_cases("prod", ["top16:u32:300000:uniform:1", "top16:i32:100000:few:2", "top16over:u32:450000:grp2:3",
                       "top16auto_lsd:u32:200000:top8:4", "top16:u64:200000:uniform:5", "top16:i64:60000:few:6",
                       "top16over:u64:300000:grp2:7", "top16w:u32:300000:uniform:8", "top16w:u64:200000:few:9"],
              timeout=900)
    run_cases("groups", ["top16:u32:70000:uniform:1", "top16over:i32:30000:grp2:2"], env={"EMU_CUS": "8"})


WAVE_SERIAL_CASES = [
    # every kernel family with more than one LDS phase per block: LSD passes
    # (stable, argsort, pairs), the fused first pass, the top-16 path's local
    # sorts with one and two stable passes, the 64-bit group sort and its LDS
    # LSD fallback (many equal keys), the region sample's skewed counting
    "sort:u32:3000:uniform:1", "argsort:f32:2000:few:2", "pairs:u64:1500:uniform:3",
    "fused:u32:4000:uniform:4", "top16:u32:3000:uniform:5", "top16s12:u32:4000:uniform:6",
    "top16:u64:3000:uniform:7", "top16:u64:1500:few:8", "top16auto_lsd:u32:9000:zipf:9",
    "top16w:u32:3000:uniform:10", "top16w:u64:1500:few:11",
    # 64-bit LSD passes in the top-16 sequence's slots, the last three on the
    # persistent loop kernel (a tile loop with a barrier between tiles)
    "top16auto_lsd:u64:20000:top8:12",
    # the deferred launches: group sort giving way to LSD in LDS, and big
    # segments of equal keys
    "top16:u64:400:low12:13", "top16:u64:3000:few:14", "top16:u32:3000:few:15",
]


@pytest.mark.parametrize("order", ["wave", "wave_rev"])
def test_emulated_wave_serial_schedule(emulator, order):
    """The same kernels with one wave of a block at a time, run as far as the
    block barriers let it get ahead (forward and reverse wave order): a
    missing barrier between waves' LDS accesses becomes a wrong result."""
    run_cases("small", WAVE_SERIAL_CASES, timeout=900, env={"EMU_SCHED": order, "EMU_TEST_FUSED": "0"}, parallel=3)
