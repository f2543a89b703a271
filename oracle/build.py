"""Build recipe for the C oracle (TEST INFRASTRUCTURE ONLY).

Compiles oracle/qattn_oracle.c with gcc into oracle/_build/libqattn_oracle.so.
The reference (saifmb0/QAttention) is Python + Triton with no C/C++ sources,
so there is nothing to build into oracle/_ref; the restatement here is the
only compiled checker.
"""
from __future__ import annotations

import os
import subprocess

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
BUILD_DIR = os.path.join(ORACLE_DIR, "_build")
SRC = os.path.join(ORACLE_DIR, "qattn_oracle.c")
LIB = os.path.join(BUILD_DIR, "libqattn_oracle.so")


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    tmp = LIB + ".tmp"
    cmd = ["gcc", "-O2", "-fPIC", "-shared", "-std=c11", "-fopenmp", "-Wall", "-Wextra",
           "-o", tmp, SRC, "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


def needs_build() -> bool:
    return (not os.path.exists(LIB)) or os.path.getmtime(LIB) < os.path.getmtime(SRC)


if __name__ == "__main__":
    print(build(verbose=True))
