"""co_alibi_decode_noalloc (the decode entry point that allocates nothing) against co_alibi_decode.

Both run the same split and merge kernels with the same split count; only the place of the
split-K partials differs (the library's per-GPU scratch instead of a caller workspace), so the
outputs must agree bit for bit.  The no-allocation entry point is called twice in a row, the
second time on a smaller decode, to check that the scratch kept from the first call does not
leak into the second.  Both are also checked against the CPU oracle (max-abs 1e-4 in fp32,
2e-2 in fp16 / bf16).  Needs an MI355X.
"""
import math

import pytest
import torch

from co_alibi_attn import _native
from co_alibi_attn.co_alibi_attn import _get_coalibi_slopes
from oracle import co_alibi_ref as ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = {torch.float32: 1e-4, torch.float16: 2e-2, torch.bfloat16: 2e-2}


def _inputs(B, Hq, Hkv, L, cap, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, Hq, 1, D, generator=g) * 0.5).to(dtype)
    k = (torch.randn(B, Hkv, cap, D, generator=g) * 0.5).to(dtype)
    v = (torch.randn(B, Hkv, cap, D, generator=g) * 0.5).to(dtype)
    k[:, :, L:] = 100.0  # rows past the filled length must not leak in
    v[:, :, L:] = -1000.0
    return q, k, v


def _run(noalloc, q, k, v, L, lens=None):
    """One decode through the C ABI; returns (o, lse) on the device."""
    lib = _native.lib()
    B, Hq, _, D = q.shape
    Hkv, cap = k.shape[1], k.shape[2]
    lam = (2.0 * _get_coalibi_slopes(Hq)).to(q.dtype).float().to(DEV)
    o = torch.empty_like(q)
    lse = torch.empty(B, Hq, 1, device=DEV, dtype=torch.float32)
    code = _native.DTYPE_CODES[q.dtype]
    lens_p = 0 if lens is None else lens.data_ptr()
    st = torch.cuda.current_stream().cuda_stream
    scale = 1.0 / math.sqrt(D)
    if noalloc:
        rc = lib.co_alibi_decode_noalloc(code, q.data_ptr(), k.data_ptr(), v.data_ptr(), lam.data_ptr(), lens_p,
                                         o.data_ptr(), lse.data_ptr(), B, Hq, Hkv, L, cap, D, scale, st)
    else:
        ws_bytes = lib.co_alibi_decode_workspace_bytes(B, Hq, L, D)
        ws = torch.empty(ws_bytes, device=DEV, dtype=torch.uint8)
        rc = lib.co_alibi_decode(code, q.data_ptr(), k.data_ptr(), v.data_ptr(), lam.data_ptr(), lens_p,
                                 o.data_ptr(), lse.data_ptr(), ws.data_ptr(), ws_bytes, B, Hq, Hkv, L, cap, D,
                                 scale, st)
    _native.check(rc)
    torch.cuda.synchronize()
    return o, lse


def _oracle(q, k, v, n):
    lam = ref.slopes(q.shape[1], 8.0, dtype=q.dtype).float()
    return ref.forward(q.float(), k[:, :, :n].float(), v[:, :, :n].float(), lam, causal=False,
                       scale=1.0 / math.sqrt(q.shape[-1]))


# Two calls in a row, the second smaller: (B, Hq, Hkv, L, cap, D) per call.
SEQUENCES = [
    ((2, 32, 8, 8192, 8192, 128), (1, 8, 2, 700, 1024, 128)),
    ((4, 16, 4, 3000, 4096, 64), (1, 4, 4, 129, 129, 64)),
    ((1, 32, 1, 20000, 20000, 256), (1, 2, 1, 1, 1, 256)),
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("calls", SEQUENCES, ids=lambda c: "then".join("B{}H{}_{}L{}D{}".format(*s[:4], s[5]) for s in c))
def test_noalloc_decode_matches_decode(calls, dtype):
    if dtype == torch.float32 and any(s[5] == 256 for s in calls):
        pytest.skip("head_dim 256 needs fp16 or bf16")
    for i, (B, Hq, Hkv, L, cap, D) in enumerate(calls):
        print(f"call {i}: B{B} Hq{Hq} Hkv{Hkv} L{L} cap{cap} D{D} {dtype}", flush=True)
        q, k, v = _inputs(B, Hq, Hkv, L, cap, D, dtype, seed=L + i)
        qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
        o_na, lse_na = _run(True, qd, kd, vd, L)
        o_ws, lse_ws = _run(False, qd, kd, vd, L)
        assert torch.equal(o_na, o_ws), f"call {i}: O differs from co_alibi_decode"
        assert torch.equal(lse_na, lse_ws), f"call {i}: LSE differs from co_alibi_decode"
        ro, rlse = _oracle(q, k, v, L)
        err_o = (o_na.float().cpu() - ro).abs().max().item()
        err_l = (lse_na.cpu() - rlse).abs().max().item()
        print(f"  vs oracle: o {err_o:.2e}, lse {err_l:.2e} (tol {TOL[dtype]:g})", flush=True)
        assert err_o <= TOL[dtype] and err_l <= TOL[dtype]


def test_noalloc_decode_per_sequence_lengths():
    """Per-sequence lengths (0 included) twice in a row, the second batch smaller."""
    for i, lens in enumerate(([5000, 0, 1, 2049], [300, 17])):
        B, Hq, Hkv, cap, D = len(lens), 8, 2, 5000, 128
        q, k, v = _inputs(B, Hq, Hkv, cap, cap, D, torch.bfloat16, seed=7 + i)
        for b, n in enumerate(lens):
            k[b, :, n:] = 100.0
            v[b, :, n:] = -1000.0
        seq = torch.tensor(lens, dtype=torch.int32, device=DEV)
        qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
        o_na, lse_na = _run(True, qd, kd, vd, max(lens), seq)
        o_ws, lse_ws = _run(False, qd, kd, vd, max(lens), seq)
        assert torch.equal(o_na, o_ws) and torch.equal(lse_na, lse_ws), f"call {i}"
        for b, n in enumerate(lens):
            if n == 0:
                assert torch.all(o_na[b] == 0) and torch.isneginf(lse_na[b]).all()
                continue
            ro, _ = _oracle(q[b:b + 1], k[b:b + 1], v[b:b + 1], n)
            assert (o_na[b:b + 1].float().cpu() - ro).abs().max().item() <= 2e-2


def test_noalloc_decode_rejects_partials_beyond_scratch():
    """A batch whose split-K partials exceed the library scratch is refused with EINVAL, before any launch.
    The tensor pointers are NULL: the size check comes first, and were it ever moved after the
    pointer checks, the call would still stop there (q is NULL) rather than launch."""
    lib = _native.lib()
    B, Hq, Hkv, L, D = 2048, 32, 32, 128, 256  # one split per head: 65536 x (4 + 256) fp32 > 32 MiB
    assert B * Hq * (4 + D) * 4 > _native.DECODE_SCRATCH_BYTES
    rc = lib.co_alibi_decode_noalloc(1, None, None, None, None, None, None, None, B, Hq, Hkv, L, L, D, 0.1, None)
    assert rc == 1
    assert "above the library scratch" in lib.co_alibi_last_error().decode()
