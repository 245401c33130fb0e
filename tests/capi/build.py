"""Build tests/capi/capi_check, the torch-free C-ABI check program (host code only).

It links the C oracle object (oracle/build.py) and co_alibi_attn/_lib/libco_alibi.so, found
at run time through an rpath relative to the binary, so it runs from any copy of the tree.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
SRC = os.path.join(HERE, "capi_check.cpp")
BIN = os.path.join(HERE, "capi_check")


def build(verbose: bool = False) -> None:
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    from co_alibi_attn._build import LIB_DIR, _hipcc
    from oracle import build as oracle_build

    oracle_build.build(verbose)
    # Host code only: ROCm's clang++ (for _Float16 on the host) with the HIP runtime headers,
    # no device pass.
    rocm = os.environ.get("ROCM_PATH") or os.path.dirname(os.path.dirname(os.path.realpath(_hipcc())))
    cmd = [os.path.join(rocm, "llvm", "bin", "clang++"), "-O2", "-std=c++17", "-Wall", "-Werror",
           "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(rocm, "include"), SRC, oracle_build.OBJ,
           "-L", LIB_DIR, "-lco_alibi", "-L", os.path.join(rocm, "lib"), "-lamdhip64",
           "-Wl,-rpath,$ORIGIN/../../co_alibi_attn/_lib:" + os.path.join(rocm, "lib"), "-lm", "-o", BIN]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


if __name__ == "__main__":
    build(verbose=True)
