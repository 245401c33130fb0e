"""Compile the plain-C oracle (oracle/co_alibi_ref.c) -- TEST INFRASTRUCTURE ONLY.

Writes oracle/_build/co_alibi_ref.o (linked into the C-ABI check program of tests/capi)
and oracle/_build/libco_alibi_ref.so (loaded by tests/test_oracle_c.py).  There is no
build of the reference itself: it is Python and Triton, nothing under /root/reference
compiles with gcc on its own.
"""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "_build")
SRC = os.path.join(HERE, "co_alibi_ref.c")
OBJ = os.path.join(OUT, "co_alibi_ref.o")
LIB = os.path.join(OUT, "libco_alibi_ref.so")


def build(verbose: bool = False) -> None:
    os.makedirs(OUT, exist_ok=True)
    for cmd in (["gcc", "-O2", "-std=c99", "-fPIC", "-Wall", "-Werror", "-c", SRC, "-o", OBJ],
                ["gcc", "-shared", OBJ, "-o", LIB, "-lm"]):
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)


if __name__ == "__main__":
    build(verbose=True)
