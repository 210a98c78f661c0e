"""Builds libturboquant_amd.so in-tree with hipcc for gfx950.

Usage: python -m turboquant_amd.build   (or turboquant_amd.build.build()).

Flags: -ffp-contract=off keeps every f32 operation separately rounded (the
reference is Rust, which never contracts a*b+c; fused multiply-adds are
written out explicitly where wanted).  Packed FP32 instructions are disabled
(-packed-fp32-ops).  No fast-math, denormals kept.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OBJ_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libturboquant_amd.so")

ARCH = os.environ.get("TQ_OFFLOAD_ARCH", "gfx950")
COMMON = [
    "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}", f"-I{CSRC}", "-Wall", "-Wno-unused-function",
    # the first 13 kernel-argument dwords arrive in SGPRs at wave launch
    "-mllvm", "-amdgpu-kernarg-preload-count=13",
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _sources():
    return sorted(f for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def _compile(src: str) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    obj = os.path.join(OBJ_DIR, src + ".o")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", *COMMON, "-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd.insert(1, "-x")
        cmd.insert(2, "hip")
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


def build(verbose: bool = True) -> str:
    srcs = _sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    _build_api_test()
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


API_TEST_SRC = os.path.join(ROOT, "tests", "cpp", "api_test.cpp")
API_TEST_BIN = os.path.join(ROOT, "tests", "cpp", "api_test")


def _build_api_test() -> None:
    """The C++ host-API test driver (tests/cpp), linked against the library."""
    if not os.path.exists(API_TEST_SRC):
        return
    cmd = [_hipcc(), "-O2", "-std=c++17", f"-I{INCLUDE}", API_TEST_SRC, f"-L{HERE}", "-lturboquant_amd",
           "-Wl,-rpath,$ORIGIN/../../turboquant_amd", "-o", API_TEST_BIN + ".tmp"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"api_test build failed:\n{res.stderr}")
    os.replace(API_TEST_BIN + ".tmp", API_TEST_BIN)


if __name__ == "__main__":
    build()
    sys.exit(0)
