"""Builds the gfx950 shared library ``orthossm_amd/_lib/libosm.so`` in-tree.

    python -m orthossm_amd.build

Compiles every ``csrc/*.hip`` source with hipcc for gfx950 into one
shared library exporting the C ABI of ``include/osm.h``.  Packed FP32 math
(v_pk_*_f32) is disabled on purpose: the kernels are written in scalar fp32.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB_DIR = os.path.join(PKG_DIR, "_lib")
LIB_PATH = os.path.join(LIB_DIR, "libosm.so")
ARCH = "gfx950"


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the ROCm toolchain is required to build orthossm_amd")


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def common_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
        "-I", INCLUDE, "-I", CSRC,
    ]


def compile_command(out: str) -> list[str]:
    return [hipcc_path(), *common_flags(), "-shared", "-o", out, *sources()]


def device_asm_command(src: str, out: str) -> list[str]:
    """gfx950 assembly of one source (device code only), as the library builds it."""
    return [hipcc_path(), *common_flags(), "--offload-device-only", "-S", "-o", out, src]


def build(verbose: bool = False) -> str:
    """Compiles the library (always, even if one exists) and returns its path."""
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB_PATH + f".tmp{os.getpid()}"
    cmd = compile_command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        if os.path.exists(tmp):
            os.remove(tmp)
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-8000:]}")
    os.replace(tmp, LIB_PATH)
    build_c_smoke(verbose)
    return LIB_PATH


C_SMOKE_SRC = os.path.join(ROOT, "tests", "c_abi", "osm_c_smoke.cpp")
C_SMOKE_BIN = os.path.join(ROOT, "tests", "c_abi", "osm_c_smoke")


def build_c_smoke(verbose: bool = False) -> str:
    """Compiles the C-ABI test program (host code only, linked against the
    library with an rpath to it), used by tests/test_gpu_c_abi.py."""
    cmd = [hipcc_path(), *common_flags(), "-o", C_SMOKE_BIN, C_SMOKE_SRC, "-L", LIB_DIR, "-losm",
           "-Wl,-rpath,$ORIGIN/../../orthossm_amd/_lib"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on the C-ABI test program ({res.returncode}):\n{res.stderr[-4000:]}")
    return C_SMOKE_BIN


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
