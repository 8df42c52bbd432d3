"""CPU-side checks of the C-ABI library: it loads, exports every symbol that
include/forge_sort.h declares, and its host-only paths behave (no GPU here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "forge_sort.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fs_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_api():
    names = declared_functions()
    for required in ("fs_sorter_new", "fs_sorter_with_context", "fs_sort", "fs_argsort",
                     "fs_sort_pairs", "fs_sort_buffer", "fs_encode", "fs_alloc_sort_buffer"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from forge_sort import _build
    lib = ctypes.CDLL(_build.SO)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_code_object_is_gfx950():
    from forge_sort import _build
    blob = open(_build.HSACO, "rb").read()
    # hipcc --genco writes a clang offload bundle holding the gfx950 ELF
    assert blob[:4] == b"\x7fELF" or blob.startswith(b"__CLANG_OFFLOAD_BUNDLE__")
    assert b"gfx950" in blob
    for k in (b"fs_upsweep_k32", b"fs_upsweep_k64", b"fs_onesweep_k32", b"fs_onesweep_k64_v", b"fs_iota"):
        assert k in blob


def test_status_strings_match_sort_error_display():
    import forge_sort
    L = forge_sort._load()
    assert L.fs_status_str(4) == b"length mismatch"
    assert L.fs_status_str(3) == b"GPU execution failed"


def test_no_device_is_reported_not_raised_as_crash():
    """Without a GPU (this container), construction fails with DeviceNotFound."""
    from forge_sort import DeviceNotFound, GpuSorter
    try:
        s = GpuSorter.new()
    except DeviceNotFound as e:
        assert str(e) == "no HIP GPU device found"     # SortError::DeviceNotFound's Display
        return
    s.close()
    pytest.skip("a GPU is present")


def test_no_alloc_limits_match_the_scratch_layout(tmp_path):
    """The header's FS_NO_ALLOC_* constants equal the static scratch layout the
    gfx950 build compiles (fs_params.h with its default tile geometry)."""
    import subprocess
    src = tmp_path / "na.c"
    src.write_text(
        '#include "fs_params.h"\n#include "forge_sort.h"\n'
        "_Static_assert(FS_NA_SCRATCH_BYTES == FS_NO_ALLOC_SCRATCH_BYTES, \"scratch bytes\");\n"
        "_Static_assert(FS_NA_MAX_KEYS == FS_NO_ALLOC_MAX_KEYS, \"max keys\");\n"
        "_Static_assert(FS_NA_OFF_S1K % 256 == 0 && FS_NA_OFF_LB0 % 256 == 0, \"aligned\");\n"
        "int main(void) { return 0; }\n")
    r = subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "gpu-forge_amd", "csrc"),
                        "-I", os.path.join(ROOT, "include"), str(src), "-o", str(tmp_path / "na")],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_python_constants_match_the_header():
    """The Python binding's copies of header constants equal the header's."""
    import re
    import forge_sort
    h = open(os.path.join(ROOT, "include", "forge_sort.h")).read()
    val = lambda name: int(re.search(r"#define %s (\d+)u" % name, h).group(1))
    assert forge_sort.FUSED_MIN_KEYS == val("FS_FUSED_MIN_KEYS")
    assert forge_sort.TOP16_MIN_KEYS32 == val("FS_TOP16_MIN_KEYS32")
    assert forge_sort.TOP16_MIN_KEYS64 == val("FS_TOP16_MIN_KEYS64")
    assert forge_sort.NO_ALLOC_MAX_KEYS == val("FS_NO_ALLOC_MAX_KEYS")
    # the test options' numbers (enum fs_test_option)
    opt = lambda name: int(re.search(r"\b%s = (\d+)" % name, h).group(1))
    for name in ("WIDE_LOOKBACK", "UPSWEEP_BLOCKS_PER_CU", "INJECT_FAULT", "FUSED", "TOP16", "SEG_BITS", "LOCAL_WIDE"):
        assert getattr(forge_sort, "TEST_" + name) == opt("FS_TEST_" + name), name
