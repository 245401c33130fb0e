"""Writes the golden fixtures in this directory (run: python tests/golden/make_golden.py).

The reference ships no golden vectors (its checks are unseeded, warn-only
scripts: model.py:100-159, co_alibi_attn/benchmark_fwd_pass.py:66-84), so these
fixtures are produced by this repository's CPU oracle (oracle/co_alibi_ref.py,
itself pinned by tests/test_oracle.py) evaluated in float64 on inputs that are
exactly representable in the case's dtype.  Each .npz holds the inputs
(q, k, v, do in the case dtype, stored as float32), the effective slopes, the
scalar settings and the expected o, lse, dq, dk, dv (float32 rounding of the
float64 results).
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import co_alibi_ref as ref  # noqa: E402

CASES = {
    # B=1, Hq=Hkv=2, S=128, D=64, fp32, causal, N(0,1), seed 0.
    "cpu_config_fp32": dict(B=1, Hq=2, Hkv=2, Sq=128, Skv=128, D=64, dtype=torch.float32, causal=True, scale=1.0),
    # grouped heads, sequence length not a multiple of any tile, fp16 inputs
    "gqa_tail_fp16": dict(B=2, Hq=4, Hkv=2, Sq=77, Skv=77, D=64, dtype=torch.float16, causal=True, scale=0.5),
    # non-causal, Sq != Skv, D=128, bf16 inputs
    "noncausal_rect_bf16": dict(B=1, Hq=2, Hkv=2, Sq=40, Skv=96, D=128, dtype=torch.bfloat16, causal=False, scale=0.5),
    # causal with more queries than keys (top-left alignment), fp32
    "causal_tall_fp32": dict(B=1, Hq=3, Hkv=1, Sq=70, Skv=33, D=64, dtype=torch.float32, causal=True, scale=1.0),
}


def make_case(name, B, Hq, Hkv, Sq, Skv, D, dtype, causal, scale, seed=0, bias_max=8.0):
    gen = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, Hq, Sq, D, generator=gen) * scale).to(dtype)
    k = (torch.randn(B, Hkv, Skv, D, generator=gen) * scale).to(dtype)
    v = (torch.randn(B, Hkv, Skv, D, generator=gen) * scale).to(dtype)
    do = torch.randn(B, Hq, Sq, D, generator=gen).to(dtype)
    lam = ref.slopes(Hq, bias_max, dtype=dtype)
    sm_scale = 1.0 / D ** 0.5
    f64 = [t.double() for t in (q, k, v, do)]
    o, lse = ref.forward(f64[0], f64[1], f64[2], lam.double(), causal=causal, scale=sm_scale)
    dq, dk, dv = ref.backward(f64[3], f64[0], f64[1], f64[2], lam.double(), causal=causal, scale=sm_scale)
    arrays = {n: t.float().numpy() for n, t in dict(q=q, k=k, v=v, do=do, o=o, lse=lse, dq=dq, dk=dk, dv=dv).items()}
    arrays["slopes"] = lam.float().numpy()
    arrays["settings"] = np.array([float(causal), sm_scale, bias_max], dtype=np.float64)
    arrays["dtype"] = np.array(str(dtype).split(".")[-1])
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **arrays)


if __name__ == "__main__":
    for name, cfg in CASES.items():
        make_case(name, **cfg)
        print("wrote", name)
