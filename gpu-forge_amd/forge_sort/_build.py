"""Build of the product: the gfx950 code object and the C-ABI host library.

  radix_kernels.hip --hipcc --genco--> lib/forge_sort_gfx950.hsaco
  forge_sort.cpp    --g++ -lamdhip64--> lib/libforge_sort.so  (loads the .hsaco
                                                               next to itself)
Both land in-tree so that they travel with the repository snapshot.
"""
import os
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


def build(verbose=True):
    os.makedirs(LIBDIR, exist_ok=True)
    tmp = HSACO + ".tmp"
    _run([os.path.join(ROCM, "bin", "hipcc"), *HIPCC_FLAGS,
          "-I", CSRC, "-o", tmp, os.path.join(CSRC, "radix_kernels.hip")])
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
