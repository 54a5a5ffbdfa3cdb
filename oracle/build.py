"""Builds oracle/_build/libosm_oracle.so from oracle/cheby_ema_c.c (the C
restatement of the float64 oracle; test infrastructure only).

    python -m oracle.build

gcc, -O2, OpenMP; no -ffast-math (IEEE semantics: NaN, Inf, no reassociation).
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "cheby_ema_c.c")
LIB = os.path.join(HERE, "_build", "libosm_oracle.so")


def build(verbose: bool = False) -> str:
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    tmp = LIB + f".tmp{os.getpid()}"
    cmd = ["gcc", "-O2", "-std=c11", "-fopenmp", "-fPIC", "-shared", "-o", tmp, SRC, "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        if os.path.exists(tmp):
            os.remove(tmp)
        raise RuntimeError(f"gcc failed on the C oracle ({res.returncode}):\n{res.stderr[-4000:]}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
