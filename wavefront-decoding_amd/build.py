"""Build recipe for libwfd.so (hand-written HIP kernels for gfx950 behind a C ABI)
and _tick (the native host side of a decode tick, a CPython extension).

Compiles every csrc/*.hip with hipcc for gfx950 into _build/*.o and links
libwfd.so next to this file (in-tree, so it travels with the source tree);
compiles csrc/tick.cpp with the host C++ compiler against the HIP runtime into
_tick<ext suffix> beside it. Run directly
(`python wavefront-decoding_amd/build.py`) or through `__graft_entry__.build()`.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_PATH = os.path.join(PKG_DIR, "libwfd.so")
TICK_SRC = os.path.join(CSRC, "tick.cpp")
TICK_PATH = os.path.join(PKG_DIR, "_tick" + sysconfig.get_config_var("EXT_SUFFIX"))
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    # Packed-FP32 instructions are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(REPO_DIR, "include"),
]


def _hipcc() -> str:
    cand = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(cand):
        raise RuntimeError(f"hipcc not found (looked for {cand})")
    return cand


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src)[:-4] + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
    return obj


def build_tick() -> str:
    """The CPython extension of csrc/tick.cpp (host code only: no kernels)."""
    cxx = os.environ.get("CXX") or shutil.which("g++") or "g++"
    tmp = TICK_PATH + ".tmp"
    cmd = [cxx, "-O2", "-fPIC", "-shared", "-std=c++17", "-Wall", "-D__HIP_PLATFORM_AMD__",
           "-I", sysconfig.get_paths()["include"], "-I", os.path.join(ROCM, "include"), TICK_SRC,
           "-L", os.path.join(ROCM, "lib"), f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}", "-lamdhip64", "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"host compile failed for {TICK_SRC}:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, TICK_PATH)
    return TICK_PATH


def build(verbose: bool = True) -> str:
    """Compile all kernels and link libwfd.so, then the _tick extension;
    returns the library path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        tick = ex.submit(build_tick)
        objs = list(ex.map(_compile, srcs))
        tick.result()
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[wfd build] {len(srcs)} sources -> {LIB_PATH}; {TICK_SRC} -> {TICK_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build()
    sys.exit(0)
