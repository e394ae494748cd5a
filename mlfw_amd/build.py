"""Build step for the gfx950 library (libq8hip.so) and the Node addon.

`python -m mlfw_amd.build` (or __graft_entry__.build()) compiles every HIP
source under mlfw_amd/csrc with hipcc for gfx950 only, in-tree, so the
built shared object travels with the source tree.  The Node N-API addon
(mlfw_amd/node/q8hip.node) is built with gcc against the Node headers when
they are installed.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libq8hip.so")
NODE_DIR = os.path.join(HERE, "node")
NODE_ADDON = os.path.join(NODE_DIR, "q8hip.node")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# measurement kernels of bench.py, kept out of the product library
CEILING_LIB = os.path.join(HERE, "libq8ceiling.so")
CEILING_SRC = "q8_ceiling.hip"

SOURCES = ["q8_capi.hip", "q8_quant.hip", "q8_gemm.hip", "q8_calib.hip", "q8_conv.hip", "q8_w4.hip",
           "q8_zp.hip", "q8_ewise.hip"]

# IEEE arithmetic everywhere (the kernels reproduce the reference's f64 /
# f32 rounding bit for bit), no packed-FP32 instructions, gfx950 only.
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-fno-gpu-rdc",
    # only the C ABI is exported (q8hip.h marks it visible): the kernels'
    # host stubs and every C++ symbol stay inside the library, so another
    # library with a same-named template instantiation can neither take
    # over nor be taken over by these launches when loaded RTLD_GLOBAL
    "-fvisibility=hidden",
    # and the library's own references (kernel handles included) bind to its
    # own definitions, whatever was loaded before it
    "-Wl,-Bsymbolic",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def build_hip(verbose: bool = False) -> str:
    """Compile every source to an object in parallel (they share no device
    code), then link the shared library."""
    from concurrent.futures import ThreadPoolExecutor

    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    compile_flags = [f for f in HIP_FLAGS if f != "-shared"]

    def compile_one(src):
        obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
        cmd = [HIPCC, *compile_flags, "-I", os.path.join(ROOT, "include"), "-c", "-o", obj,
               os.path.join(CSRC, src)]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        return obj

    workers = min(len(SOURCES), max(1, int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(compile_one, SOURCES))
    tmp = LIB + ".tmp"
    # hiprtc: q8_ewise compiles large elementwise programs at run time
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-Wl,-Bsymbolic", "-o", tmp, *objs,
           "-L/opt/rocm/lib", "-lhiprtc", "-Wl,-rpath,/opt/rocm/lib"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


def build_ceiling(verbose: bool = False) -> str:
    """libq8ceiling.so: the MFMA and streaming-read ceiling kernels bench.py
    reports beside its roofline fractions (no C ABI of the int8 path)."""
    tmp = CEILING_LIB + ".tmp"
    cmd = [HIPCC, *HIP_FLAGS, "-o", tmp, os.path.join(CSRC, CEILING_SRC)]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, CEILING_LIB)
    return CEILING_LIB


def build_node_addon(verbose: bool = False) -> str | None:
    inc = "/usr/include/node"
    src = os.path.join(NODE_DIR, "q8hip_napi.c")
    if not (os.path.isdir(inc) and os.path.exists(src) and shutil.which("gcc")):
        return None
    cmd = ["gcc", "-std=c11", "-O2", "-fPIC", "-shared", "-Wall", "-Wextra",
           "-I", inc, "-I", os.path.join(ROOT, "include"),
           "-o", NODE_ADDON, src,
           "-L", HERE, "-lq8hip", "-Wl,-rpath,$ORIGIN/.."]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    return NODE_ADDON


def build_all(verbose: bool = False) -> None:
    build_hip(verbose)
    build_ceiling(verbose)
    build_node_addon(verbose)


if __name__ == "__main__":
    build_all(verbose="-v" in sys.argv)
