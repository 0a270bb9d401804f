"""Builds libesm_gfx950.so (HIP kernels + C ABI) in-tree for gfx950.

Usage: python esm-cpp_amd/build.py [--jobs N] [--reference-include <esm.cpp>/include]

Each translation unit is compiled with hipcc for --offload-arch=gfx950 and
linked into esm-cpp_amd/lib/libesm_gfx950.so. Packed-fp32 instruction
selection is disabled for device code (-Xclang -target-feature -Xclang
-packed-fp32-ops); hipcc's host pass reports that feature as unknown, which
is harmless.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
OBJDIR = os.path.join(HERE, "_build")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
LIB = os.path.join(LIBDIR, "libesm_gfx950.so")

SOURCES = ["gemm_i8.hip", "attention.hip", "elementwise.hip", "gemm_f32.hip", "x86_exact.hip", "capi.cpp", "gguf.cpp",
           "observer.cpp"]
# Per-file flags: the reference's x86 kernels are restated with every fused
# multiply-add spelled out, so the compiler must form no others.
EXTRA = {"x86_exact.hip": ["-ffp-contract=off"]}

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", f"-I{INCLUDE}",
]


def _compile(src: str) -> str:
    obj = os.path.join(OBJDIR, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *COMMON, *EXTRA.get(src, []), "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


def build(jobs: int = 4) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


BRIDGE_SOURCES = ["gfx950_bridge.cpp", "bridge_capi.cpp"]
BRIDGE_LIB = os.path.join(LIBDIR, "libesm_gfx950_bridge.so")


def build_bridge(reference_include: str) -> str:
    """Builds lib/libesm_gfx950_bridge.so: the reference-side bridge
    (bridge/), compiled with the host compiler against the reference's own
    headers (reference_include = <esm.cpp>/include) and linked to
    libesm_gfx950.so. The reference's src/batch.cpp (BatchView's validating
    constructor, which the forward-level arm takes) is compiled in from the
    reference tree, where it lies, as the library the bridge joins in the
    reference's own build already holds it. Needs build() first."""
    cxx = os.environ.get("CXX", "g++")
    srcs = [os.path.join(HERE, "bridge", f) for f in BRIDGE_SOURCES]
    srcs.append(os.path.join(os.path.dirname(os.path.abspath(reference_include)), "src", "batch.cpp"))
    tmp = BRIDGE_LIB + ".tmp"
    cmd = [cxx, "-std=c++20", "-O2", "-fPIC", "-shared", "-Wall", "-Wextra", f"-I{reference_include}", f"-I{INCLUDE}",
           *srcs, f"-L{LIBDIR}", "-lesm_gfx950", "-Wl,-rpath,$ORIGIN", "-Wl,-rpath-link,/opt/rocm/lib", "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"bridge build failed:\n{res.stderr}")
    os.replace(tmp, BRIDGE_LIB)
    return BRIDGE_LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("--reference-include", default=None,
                    help="also build the reference-side bridge against <esm.cpp>/include")
    args = ap.parse_args()
    print(build(args.jobs))
    if args.reference_include:
        print(build_bridge(args.reference_include))
    sys.exit(0)
