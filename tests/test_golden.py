"""The committed golden fixtures (tests/golden/*.npz) against the CPU oracle.

The fixtures were written by tests/golden/make_golden.py from the float64
oracle; this keeps the oracle from drifting.  The GPU comparison of the HIP
kernels with the same fixtures lives in tests/test_gpu_parity.py.
"""
import glob
import os

import numpy as np
import pytest
import torch

from oracle import co_alibi_ref as ref

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


def load_golden(path):
    z = np.load(path, allow_pickle=False)
    t = {n: torch.from_numpy(z[n]) for n in ("q", "k", "v", "do", "o", "lse", "dq", "dk", "dv", "slopes")}
    causal, sm_scale, bias_max = (float(x) for x in z["settings"])
    return t, bool(causal), sm_scale, bias_max, str(z["dtype"])


def test_fixtures_present():
    assert len(GOLDEN) >= 4


@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: os.path.basename(p)[:-4])
def test_oracle_reproduces_golden(path):
    t, causal, sm_scale, _, _ = load_golden(path)
    f64 = {n: t[n].double() for n in t}
    o, lse = ref.forward(f64["q"], f64["k"], f64["v"], f64["slopes"], causal=causal, scale=sm_scale)
    dq, dk, dv = ref.backward(f64["do"], f64["q"], f64["k"], f64["v"], f64["slopes"], causal=causal, scale=sm_scale)
    for name, got in dict(o=o, lse=lse, dq=dq, dk=dk, dv=dv).items():
        torch.testing.assert_close(got.float(), t[name], rtol=0, atol=1e-5, msg=name)
