"""Build of the product: the gfx950 code object and the C-ABI host library.

  radix_kernels.hip --hipcc --genco--> lib/forge_sort_gfx950.hsaco
  forge_sort.cpp    --g++ -lamdhip64--> lib/libforge_sort.so  (loads the .hsaco
                                                               next to itself)
Both land in-tree so that they travel with the repository snapshot.
"""
import os
import re
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(ROOT, "csrc")
LIBDIR = os.path.join(PKG, "lib")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HSACO = os.path.join(LIBDIR, "forge_sort_gfx950.hsaco")
SO = os.path.join(LIBDIR, "libforge_sort.so")

HIPCC_FLAGS = [
    "--genco", "--offload-arch=gfx950", "-O3", "-std=c++17",
    # packed FP32 instructions are kept out of every HIP build
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd):
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def _check_no_spills(report):
    """Every kernel must keep its registers: a build in which the fused pass
    spilled to scratch gave wrong results on the GPU (the same source ran
    exact in the CPU emulator), so a spill fails the build."""
    name, bad = None, []
    for line in report.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and int(m.group(1)) > 0:
            bad.append(f"{name} ({m.group(1)} bytes/lane)")
    if bad:
        raise RuntimeError("kernels spill registers to scratch: " + ", ".join(bad))


def build(verbose=True):
    os.makedirs(LIBDIR, exist_ok=True)
    tmp = HSACO + ".tmp"
    cmd = [os.path.join(ROCM, "bin", "hipcc"), *HIPCC_FLAGS, "-Rpass-analysis=kernel-resource-usage",
           "-I", CSRC, "-o", tmp, os.path.join(CSRC, "radix_kernels.hip")]
    print("+", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stderr)
        raise subprocess.CalledProcessError(r.returncode, cmd)
    _check_no_spills(r.stderr)
    os.replace(tmp, HSACO)
    tmp = SO + ".tmp"
    _run(["g++", "-O2", "-g", "-std=c++17", "-shared", "-fPIC", "-Wall",
          "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROCM, "include"), "-I", CSRC,
          os.path.join(CSRC, "forge_sort.cpp"), "-o", tmp,
          "-L", os.path.join(ROCM, "lib"), "-lamdhip64", "-ldl",
          "-Wl,-rpath," + os.path.join(ROCM, "lib")])
    os.replace(tmp, SO)
    return SO


if __name__ == "__main__":
    build()
    sys.exit(0)
