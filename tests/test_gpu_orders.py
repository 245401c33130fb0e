"""Work orders of the tail skip (coalibi_kernels.h).  The forward's key-norm launch writes, into
the saved statistics, the order in which the forward and backward pass 1 take their 128-row
blocks and, with one query head per key head, the order of pass 2's 64-key blocks (the index
order else); the inference forward writes the row order into its workspace.  Each order must be
a permutation of its grid's items, so that every block is processed exactly once, and it must
equal the stable descending sort of the predicted costs, restated here in numpy.  The
statistics' header flags which tables the backward may follow.  With the tail skip switched
off no table is written or flagged and every kstart is 0.  The kernels' results do not depend
on the order (the parity tests cover them).  Needs an MI355X.
"""
import math

import numpy as np
import pytest
import torch

from co_alibi_attn import _native
from co_alibi_attn.co_alibi_attn import _get_coalibi_slopes

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
BUCKETS = 256
SKIP_LOG2 = {torch.float16: 26.0, torch.bfloat16: 32.0, torch.float32: 64.0}


def window(dtype):
    """Keys a row keeps left of its diagonal per unit slope: (T + 8) / (0.5 log2 e), in fp32."""
    return np.float32(SKIP_LOG2[dtype] + 8.0) / (np.float32(0.5) * np.float32(1.4426950408889634))


def capped(extent, lam, win):
    """min(extent, win / lam) in fp32, or extent where the slope does not skip (<= 0)."""
    pos = lam > 0
    w = np.where(pos, win / np.where(pos, lam, np.float32(1)), np.float32(np.inf)).astype(np.float32)
    return np.minimum(extent.astype(np.float32), w)


def buckets_of(work, extent_max):
    """Cost classes of ceil(extent_max / BUCKETS) keys or rows each, in fp32."""
    unit = np.float32(-(-extent_max // BUCKETS))
    return np.minimum((work / unit).astype(np.int64), BUCKETS - 1)


def stable_desc(b):
    return np.lexsort((np.arange(len(b)), -b)).astype(np.int32)


def row_order(slopes, B, Hq, Sq, Skv, causal, dtype):
    heads, nqb = B * Hq, -(-Sq // 128)
    i = np.arange(nqb * heads)
    rank, bh = i // heads, i % heads
    qb = nqb - 1 - rank
    keys = np.minimum((qb + 1) * 128, Skv) if causal else np.full_like(qb, Skv)
    return stable_desc(buckets_of(capped(keys, slopes[bh % Hq], window(dtype)), Skv))


def key_order(slopes, B, H, Sq, Skv, causal, dtype):
    """One query head per key head: key blocks by the rows that see them, capped by the window."""
    heads, nkb = B * H, -(-Skv // 64)
    i = np.arange(nkb * heads)
    kb, bh = i // heads, i % heads
    rows = np.maximum(Sq - kb * 64, 0) if causal else np.full_like(kb, Sq)
    return stable_desc(buckets_of(capped(rows, slopes[bh % H], window(dtype)), Sq))


def run_fwd(B, Hq, Hkv, Sq, Skv, D, dtype, causal, slopes, skip=True):
    lib = _native.lib()
    g = torch.Generator().manual_seed(1)
    q, k, v = ((torch.randn(B, h, s, D, generator=g) * 0.5).to(dtype).to(DEV)
               for h, s in ((Hq, Sq), (Hkv, Skv), (Hkv, Skv)))
    lam = torch.tensor(slopes, dtype=torch.float32, device=DEV)
    o = torch.empty_like(q)
    lse = torch.empty(B, Hq, Sq, device=DEV)
    stats = torch.full((lib.co_alibi_stats_numel(B, Hq, Sq, Skv),), -1.0, device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    ws_bytes = lib.co_alibi_fwd_inference_workspace_bytes(B, Hq, Sq, Skv)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=DEV)
    o_inf = torch.empty_like(q)
    with _native.tail_skip(skip):
        _native.check(lib.co_alibi_fwd(_native.DTYPE_CODES[dtype], q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                       lam.data_ptr(), o.data_ptr(), lse.data_ptr(), stats.data_ptr(), B, Hq, Hkv,
                                       Sq, Skv, D, int(causal), 1.0 / math.sqrt(D), st))
        _native.check(lib.co_alibi_fwd_inference(_native.DTYPE_CODES[dtype], q.data_ptr(), k.data_ptr(),
                                                 v.data_ptr(), lam.data_ptr(), o_inf.data_ptr(), ws.data_ptr(),
                                                 ws_bytes, B, Hq, Hkv, Sq, Skv, D, int(causal), 1.0 / math.sqrt(D),
                                                 st))
    torch.cuda.synchronize()
    return stats.cpu(), ws.cpu(), o.cpu(), o_inf.cpu()


CASES = [
    # (B, Hq, Hkv, Sq, Skv, D, dtype, causal, slopes: "alibi" or a list per query head)
    (1, 4, 4, 1000, 1000, 64, torch.float16, True, "alibi"),
    (2, 8, 2, 300, 700, 128, torch.bfloat16, True, "alibi"),
    (1, 3, 3, 513, 257, 64, torch.float32, False, [0.5, 0.0, -0.25]),
    (2, 5, 5, 257, 900, 32, torch.bfloat16, True, [1e-4, 0.03, 0.3, 1.5, 4.0]),
    (4, 16, 16, 4096, 4096, 128, torch.float16, True, "alibi"),  # the headline grid
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}H{c[1]}/{c[2]}S{c[3]}x{c[4]}D{c[5]}"
                         f"{'c' if c[7] else 'n'}-{str(c[6])[6:]}")
def test_orders_are_sorted_permutations(case):
    B, Hq, Hkv, Sq, Skv, D, dtype, causal, sl = case
    if sl == "alibi":
        slopes = (2.0 * _get_coalibi_slopes(Hq, 8.0)).to(dtype).float().numpy()
    else:
        slopes = np.array(sl, dtype=np.float32)
    stats, ws, o, o_inf = run_fwd(B, Hq, Hkv, Sq, Skv, D, dtype, causal, slopes.tolist())
    bh, nqb, nkc, nkb = B * Hq, -(-Sq // 128), -(-Skv // 256), -(-Skv // 64)
    ints = stats.view(torch.int32).numpy()
    # header: the row table and, with one query head per key head, the key table are flagged, and
    # so is the tail skip
    assert ints[0] == 1 | (2 if Hq == Hkv else 0) | 4 and not ints[1:4].any()
    tail = 4 + bh * (nqb + nkc)
    rows = ints[tail: tail + bh * nqb]
    assert np.array_equal(np.sort(rows), np.arange(bh * nqb)), "row order is not a permutation"
    assert np.array_equal(rows, row_order(slopes, B, Hq, Sq, Skv, causal, dtype))
    region = ints[tail + bh * nqb: tail + bh * nqb + bh * nkb]
    keys, rest = region[:B * Hkv * nkb], region[B * Hkv * nkb:]
    assert np.array_equal(np.sort(keys), np.arange(B * Hkv * nkb)), "key order is not a permutation"
    if Hq == Hkv:
        assert np.array_equal(keys, key_order(slopes, B, Hq, Sq, Skv, causal, dtype))
    else:  # unused with grouped heads: the index order
        assert np.array_equal(keys, np.arange(B * Hkv * nkb))
    assert not rest.any(), "the key table's unused room is not zero"
    # The inference forward: the same row order after its key-norm floats, and the same output.
    inf_rows = ws.view(torch.int32).numpy()[B * Hq * nkc: B * Hq * nkc + bh * nqb]
    assert np.array_equal(inf_rows, rows)
    assert torch.equal(o, o_inf)


@pytest.mark.parametrize("case", CASES[:2], ids=["mha", "gqa"])
def test_no_tables_without_the_tail_skip(case):
    """With the tail skip switched off the forward flags no work order (the backward then uses
    its fixed orders), records kstart = 0 for every row block, and gives the same O as the
    inference forward under the same setting."""
    B, Hq, Hkv, Sq, Skv, D, dtype, causal, _ = case
    slopes = (2.0 * _get_coalibi_slopes(Hq, 8.0)).to(dtype).float().numpy()
    stats, _, o, o_inf = run_fwd(B, Hq, Hkv, Sq, Skv, D, dtype, causal, slopes.tolist(), skip=False)
    ints = stats.view(torch.int32).numpy()
    nqb = -(-Sq // 128)
    assert not ints[:4].any()
    assert not ints[4: 4 + B * Hq * nqb].any()
    assert torch.equal(o, o_inf)
