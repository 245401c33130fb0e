"""Pins the plain-C oracle (oracle/co_alibi_ref.c) against the Python oracle.

The Python oracle is itself pinned (tests/test_oracle.py: closed forms, brute force,
finite differences); the two restatements share no code, so agreement to fp64 rounding
on random tiny shapes pins the C one.  It must also reproduce the committed golden
fixtures (tests/golden/*.npz).  The C oracle is what the torch-free C-ABI check
program (tests/capi/capi_check.cpp) compares the library against.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import build as oracle_build
from oracle import co_alibi_ref as ref

_DP = ctypes.POINTER(ctypes.c_double)


@pytest.fixture(scope="module")
def lib():
    oracle_build.build()
    so = ctypes.CDLL(oracle_build.LIB)
    ints = [ctypes.c_int] * 7
    so.co_alibi_ref_forward.argtypes = ints + [ctypes.c_double] + [_DP] * 6
    so.co_alibi_ref_forward.restype = None
    so.co_alibi_ref_backward.argtypes = ints + [ctypes.c_double] + [_DP] * 8
    so.co_alibi_ref_backward.restype = None
    return so


def _ptr(a: np.ndarray):
    assert a.dtype == np.float64 and a.flags.c_contiguous
    return a.ctypes.data_as(_DP)


CASES = [
    # B, Hq, Hkv, Sq, Skv, D, causal
    (1, 1, 1, 1, 1, 4, True),
    (1, 2, 2, 7, 7, 8, True),
    (2, 4, 2, 9, 9, 16, True),
    (1, 6, 3, 5, 12, 8, True),     # causal with more keys than queries (top-left mask)
    (1, 3, 1, 12, 5, 8, True),     # causal with more queries than keys
    (2, 2, 1, 6, 11, 8, False),
    (1, 4, 4, 1, 17, 32, False),   # a decode step
]


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Skv,D,causal", CASES)
def test_c_oracle_matches_python_oracle(lib, B, Hq, Hkv, Sq, Skv, D, causal):
    g = torch.Generator().manual_seed(B * 1000 + Hq * 100 + Sq * 10 + Skv)
    q = torch.randn(B, Hq, Sq, D, generator=g, dtype=torch.float64)
    k = torch.randn(B, Hkv, Skv, D, generator=g, dtype=torch.float64)
    v = torch.randn(B, Hkv, Skv, D, generator=g, dtype=torch.float64)
    do = torch.randn(B, Hq, Sq, D, generator=g, dtype=torch.float64)
    lam = ref.slopes(Hq, 8.0, torch.float64)
    scale = 1.0 / D ** 0.5
    o_w, lse_w = ref.forward(q, k, v, lam, causal, scale)
    dq_w, dk_w, dv_w = ref.backward(do, q, k, v, lam, causal, scale)

    qn, kn, vn, don, ln = (t.numpy().copy() for t in (q, k, v, do, lam))
    o, lse = np.zeros_like(qn), np.zeros((B, Hq, Sq))
    dq, dk, dv = np.zeros_like(qn), np.zeros_like(kn), np.zeros_like(vn)
    dims = (B, Hq, Hkv, Sq, Skv, D, int(causal))
    lib.co_alibi_ref_forward(*dims, scale, _ptr(ln), _ptr(qn), _ptr(kn), _ptr(vn), _ptr(o), _ptr(lse))
    lib.co_alibi_ref_backward(*dims, scale, _ptr(ln), _ptr(qn), _ptr(kn), _ptr(vn), _ptr(don), _ptr(dq), _ptr(dk),
                              _ptr(dv))
    for got, want in ((o, o_w), (lse, lse_w), (dq, dq_w), (dk, dk_w), (dv, dv_w)):
        np.testing.assert_allclose(got, want.numpy(), rtol=1e-10, atol=1e-12)


def test_c_oracle_planted_mistake_is_caught(lib):
    """A plausible slip (dropping the slope term from the backward's dP) must not pass the
    comparison above: the check is sensitive to the penalty's gradient."""
    g = torch.Generator().manual_seed(7)
    B, Hq, Hkv, S, D = 1, 2, 1, 8, 8
    q, k, v, do = (torch.randn(B, h, S, D, generator=g, dtype=torch.float64) for h in (Hq, Hkv, Hkv, Hq))
    lam = ref.slopes(Hq, 8.0, torch.float64)
    dq_w, _, _ = ref.backward(do, q, k, v, lam, True, 0.35)
    dq_no_slope, _, _ = ref.backward(do, q, k, v, torch.zeros_like(lam), True, 0.35)
    qn, kn, vn, don, ln = (t.numpy().copy() for t in (q, k, v, do, lam))
    dq, dk, dv = np.zeros_like(qn), np.zeros_like(kn), np.zeros_like(vn)
    lib.co_alibi_ref_backward(B, Hq, Hkv, S, S, D, 1, 0.35, _ptr(ln), _ptr(qn), _ptr(kn), _ptr(vn), _ptr(don),
                              _ptr(dq), _ptr(dk), _ptr(dv))
    np.testing.assert_allclose(dq, dq_w.numpy(), rtol=1e-10, atol=1e-12)
    assert np.abs(dq - dq_no_slope.numpy()).max() > 1e-3



def test_c_oracle_reproduces_golden(lib):
    """The C oracle against the committed golden fixtures (written from the float64 Python oracle)."""
    from tests.test_golden import GOLDEN, load_golden

    assert GOLDEN
    for path in GOLDEN:
        t, causal, sm_scale, _, _ = load_golden(path)
        B, Hq, Sq, D = t["q"].shape
        Hkv, Skv = t["k"].shape[1], t["k"].shape[2]
        qn, kn, vn, don, ln = (t[n].double().numpy().copy() for n in ("q", "k", "v", "do", "slopes"))
        o, lse = np.zeros_like(qn), np.zeros((B, Hq, Sq))
        dq, dk, dv = np.zeros_like(qn), np.zeros_like(kn), np.zeros_like(vn)
        dims = (B, Hq, Hkv, Sq, Skv, D, int(causal))
        lib.co_alibi_ref_forward(*dims, sm_scale, _ptr(ln), _ptr(qn), _ptr(kn), _ptr(vn), _ptr(o), _ptr(lse))
        lib.co_alibi_ref_backward(*dims, sm_scale, _ptr(ln), _ptr(qn), _ptr(kn), _ptr(vn), _ptr(don), _ptr(dq),
                                  _ptr(dk), _ptr(dv))
        for name, got in dict(o=o, lse=lse, dq=dq, dk=dk, dv=dv).items():
            np.testing.assert_allclose(got, t[name].double().numpy(), rtol=0, atol=1e-5, err_msg=f"{path}: {name}")
