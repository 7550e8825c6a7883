"""Builds libgossmx.so (the HIP kernels and the C ABI) in-tree for gfx950.

`python build.py` builds the product library. `python build.py --sanitize`
builds a test variant into _build/san/libgossmx.so whose host code (the C ABI,
the store's file parsers, the dense path's host side) is instrumented with
AddressSanitizer and UndefinedBehaviorSanitizer; its device code is the
product's. It is loaded by the CPU tests through GOSSMX_LIB with the clang ASan
runtime preloaded (tests/test_sanitize.py)."""
from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libgossmx.so")
SAN_DIR = os.path.join(HERE, "_build", "san")
SAN_LIB = os.path.join(SAN_DIR, "libgossmx.so")
SOURCES = ["gossmx_kernels.hip", "gossmx_api.hip", "gossmx_store.cpp", "gossmx_dense.cpp"]
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

# -ffp-contract=off: the reference's float chains are ordered and unfused.
# -packed-fp32-ops disabled: no v_pk_*_f32 in generated code.
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]
# Host-only sources (.cpp: the store and the dense path's host side) build as plain C++
# with the HIP runtime headers.
HOST_FLAGS = [
    "-x", "c++", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-Wall", "-Wno-unused-function",
]
# The sanitized variant: host code only (each sanitizer flag behind
# -Xarch_host, so that no device code is instrumented), with frame pointers
# for readable reports.
SAN_FLAGS = ["-g", "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
             "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer"]


def asan_runtime() -> str | None:
    """The clang ASan runtime that a host process preloads to load the
    sanitized variant."""
    hits = sorted(glob.glob("/opt/rocm/lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return hits[-1] if hits else None


def _compile(src: str, out_dir: str, extra: list[str]) -> str:
    obj = os.path.join(out_dir, os.path.splitext(src)[0] + ".o")
    flags = HOST_FLAGS if src.endswith(".cpp") else FLAGS
    cmd = [HIPCC, *flags, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed for {src}")
    return obj


def _build(lib: str, out_dir: str, extra: list[str], link_extra: list[str]) -> str:
    os.makedirs(out_dir, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
        objs = list(pool.map(lambda src: _compile(src, out_dir, extra), SOURCES))
    tmp = lib + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *link_extra, "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"link of {lib} failed")
    os.replace(tmp, lib)
    return lib


def build() -> str:
    return _build(LIB, CSRC, [], [])


def build_sanitized() -> str:
    return _build(SAN_LIB, SAN_DIR, SAN_FLAGS, ["-shared-libasan", "-Xarch_host", "-fsanitize=address",
                                                "-Xarch_host", "-fsanitize=undefined"])


if __name__ == "__main__":
    print(build_sanitized() if "--sanitize" in sys.argv else build())
