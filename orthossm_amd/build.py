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
    """One-step build of the whole library (kept for reference and tooling;
    build() compiles the sources in parallel and links them)."""
    return [hipcc_path(), *common_flags(), "-shared", "-o", out, *sources()]


OBJ_DIR = os.path.join(PKG_DIR, "_build")


def object_command(src: str, obj: str) -> list[str]:
    return [hipcc_path(), *common_flags(), "-c", "-o", obj, src]


def link_command(objs: list[str], out: str) -> list[str]:
    return [hipcc_path(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", out, *objs]


def device_asm_command(src: str, out: str) -> list[str]:
    """gfx950 assembly of one source (device code only), as the library builds it."""
    return [hipcc_path(), *common_flags(), "--offload-device-only", "-S", "-o", out, src]


def build(verbose: bool = False) -> str:
    """Compiles the library (always, even if one exists) and returns its path."""
    os.makedirs(LIB_DIR, exist_ok=True)
    os.makedirs(OBJ_DIR, exist_ok=True)
    tag = os.getpid()
    objs, procs = [], []
    # One hipcc per source, all at once (each kernel file is its own
    # translation unit), then one link.
    for src in sources():
        obj = os.path.join(OBJ_DIR, os.path.basename(src)[:-4] + f".{tag}.o")
        cmd = object_command(src, obj)
        if verbose:
            print(" ".join(cmd), flush=True)
        objs.append(obj)
        procs.append(subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True))
    errors = []
    for src, pr in zip(sources(), procs):
        _, err = pr.communicate()
        if pr.returncode != 0:
            errors.append(f"{os.path.basename(src)}: hipcc failed ({pr.returncode}):\n{err[-8000:]}")
    tmp = LIB_PATH + f".tmp{tag}"
    try:
        if errors:
            raise RuntimeError("\n".join(errors))
        cmd = link_command(objs, tmp)
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link failed ({res.returncode}):\n{res.stderr[-8000:]}")
        os.replace(tmp, LIB_PATH)
    finally:
        for f in objs + [tmp]:
            if os.path.exists(f):
                os.remove(f)
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
