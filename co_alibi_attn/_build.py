"""Build the gfx950 HIP library and its torch operators.

Each ``csrc/*.hip`` file is compiled to an object with hipcc (in parallel), then
linked into ``co_alibi_attn/_lib/libco_alibi.so``, which exports the C ABI declared
in ``include/co_alibi.h``.  ``csrc/torch_ops.cpp`` (host code only) is then compiled
against torch's headers and libraries into ``co_alibi_attn/_lib/libco_alibi_torch.so``,
the PyTorch-ROCm operators ``co_alibi::*`` over that C ABI.  Run
``python -m co_alibi_attn._build``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
OBJ_DIR = os.path.join(PKG_DIR, "_build")
LIB_DIR = os.path.join(PKG_DIR, "_lib")
LIB_PATH = os.path.join(LIB_DIR, "libco_alibi.so")
TORCH_LIB_PATH = os.path.join(LIB_DIR, "libco_alibi_torch.so")
ARCH = "gfx950"
SOURCES = ("coalibi_fwd.hip", "coalibi_bwd.hip", "coalibi_decode.hip", "coalibi_probe.hip", "coalibi_capi.hip")

# Packed fp32 VALU forms are disabled for all device code (the compiler would
# otherwise form v_pk_{add,mul,fma}_f32 from scalar float code).
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in res.stdout.splitlines() if "packed-fp32-ops" not in line
    )
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")


def _torch_ops_cmd(out: str) -> list[str]:
    """g++ command of the torch operator library (host code: torch headers, HIP runtime headers)."""
    import torch.utils.cpp_extension as ce

    cxx = os.environ.get("CXX") or shutil.which("g++") or "g++"
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    abi = int(__import__("torch")._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}"]
    cmd += [f"-I{p}" for p in ce.include_paths()] + [f"-I{os.path.join(rocm, 'include')}"]
    cmd += [os.path.join(CSRC, "torch_ops.cpp"), "-o", out]
    cmd += [f"-L{p}" for p in ce.library_paths()]
    cmd += ["-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_hip", "-ltorch", f"-L{LIB_DIR}", "-lco_alibi",
            "-Wl,-rpath,$ORIGIN"]
    return cmd


def build(verbose: bool = False) -> str:
    """Compile every source and link the library, then the torch operators; returns the library's path."""
    hipcc = _hipcc()
    os.makedirs(OBJ_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    objs = []
    cmds = []
    for src in SOURCES:
        obj = os.path.join(OBJ_DIR, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([hipcc, *COMMON_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        for cmd, _ in zip(cmds, ex.map(_run, cmds)):
            if verbose:
                print(" ".join(cmd), flush=True)
    tmp = LIB_PATH + ".tmp"
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    _run(link)
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(" ".join(link), flush=True)
        print(f"built {LIB_PATH}", flush=True)
    tmp = TORCH_LIB_PATH + ".tmp"
    cmd = _torch_ops_cmd(tmp)
    _run(cmd)
    os.replace(tmp, TORCH_LIB_PATH)
    if verbose:
        print(" ".join(cmd), flush=True)
        print(f"built {TORCH_LIB_PATH}", flush=True)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
