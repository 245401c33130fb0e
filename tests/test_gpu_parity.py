"""HIP kernels vs the CPU oracle (the parity gate).  Needs an MI355X.

Bar: max-abs <= 1e-4 in the fp32 validation mode,
<= 2e-2 for O, dQ, dK, dV with fp16/bf16 inputs, against the oracle run in
fp32 on the same (dtype-rounded) inputs with the same dtype-rounded slopes.

The bar is applied as written, with no allowance, to every fp32 output, and to every
16-bit output whose largest reference value is at most REF_SCALE[dtype].  Past that
magnitude no kernel can meet an absolute bar in a 16-bit output type: its own rounding
is up to half an ulp of the value, |x| 2^-8 in bf16 (2e-2 at |x| = 5.1) and |x| 2^-11
in fp16 (at |x| = 41).  Such outputs (grouped-query dK/dV, non-causal sums, reaching
10-160 in the random sweeps) get the bar scaled by max|ref| / REF_SCALE[dtype].
REF_SCALE is where that rounding takes 39 % of the bar, in both types (2 in bf16, 16
in fp16), so both keep the same room for the computation's own error.  The worst error
as a share of its bar is printed per dtype at the end of the module.
Every GPU call goes through the C ABI (directly, or via the drop-in API and the
torch operators over it).
"""
import ctypes
import math

import pytest
import torch

from co_alibi_attn import _native, co_alibi_attention, co_alibi_decode
from co_alibi_attn.co_alibi_attn import CoALIBIAttention, _get_coalibi_slopes
from co_alibi_attn.workloads import WORKLOADS, make_inputs
from oracle import co_alibi_ref as ref
from tests.test_golden import GOLDEN, load_golden

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = {torch.float32: 1e-4, torch.float16: 2e-2, torch.bfloat16: 2e-2}


def hip_fwd_bwd(q, k, v, do, causal=True, sm_scale=None, bias_max=8.0):
    """Drop-in API forward + backward on the GPU; returns CPU fp32 (o, dq, dk, dv)."""
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    o = co_alibi_attention(qd, kd, vd, causal=causal, sm_scale=sm_scale, bias_max=bias_max)
    o.backward(do.to(DEV))
    torch.cuda.synchronize()
    return tuple(t.detach().float().cpu() for t in (o, qd.grad, kd.grad, vd.grad))


def oracle_fwd_bwd(q, k, v, do, causal=True, sm_scale=None, bias_max=8.0, heads=None):
    lam = ref.slopes(q.shape[1], bias_max, dtype=q.dtype).float()
    qf, kf, vf, dof = (t.float() for t in (q, k, v, do))
    scale = 1.0 / math.sqrt(q.shape[-1]) if sm_scale is None else sm_scale
    o, lse = ref.forward(qf, kf, vf, lam, causal=causal, scale=scale, heads=heads)
    dq, dk, dv = ref.backward(dof, qf, kf, vf, lam, causal=causal, scale=scale, heads=heads)
    return o, lse, dq, dk, dv


def rand_inputs(B, Hq, Hkv, Sq, Skv, D, dtype, seed=0, scale=0.5):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, Hq, Sq, D, generator=g) * scale).to(dtype)
    k = (torch.randn(B, Hkv, Skv, D, generator=g) * scale).to(dtype)
    v = (torch.randn(B, Hkv, Skv, D, generator=g) * scale).to(dtype)
    do = torch.randn(B, Hq, Sq, D, generator=g).to(dtype)
    return q, k, v, do


# Largest reference magnitude at which the absolute bar applies unchanged (see the module docstring):
# fp32 outputs carry no output rounding of that size, so their bar is never scaled.
REF_SCALE = {torch.float32: math.inf, torch.float16: 16.0, torch.bfloat16: 2.0}
WORST = {}  # dtype name -> (worst error / bar, label)


def assert_parity(got, want, tol, label, dtype=torch.float32):
    """max-abs <= tol for outputs up to REF_SCALE[dtype] in magnitude, tol * max|ref| / REF_SCALE beyond
    (16-bit types only)."""
    for name, g, w in zip(("o", "dq", "dk", "dv"), got, want):
        assert torch.isfinite(g).all(), f"{label}: {name} has non-finite values"
        w = w.float()
        err = (g - w).abs().max().item()
        ref_max = w.abs().max().item()
        bar = tol * max(1.0, ref_max / REF_SCALE[dtype])
        key = str(dtype).split(".")[-1]
        if err / bar > WORST.get(key, (0.0, ""))[0]:
            WORST[key] = (err / bar, f"{label} {name}")
        print(f"  {label} {name}: max-abs {err:.3e}, |ref| max {ref_max:.2f}, bar {bar:.3g} "
              f"({err / bar:.0%} of it)", flush=True)
        assert err <= bar, f"{label}: {name} max-abs {err:.3e} > {bar:.3g}"


@pytest.fixture(scope="module", autouse=True)
def _report_worst_ratio():
    yield
    for key, (ratio, label) in sorted(WORST.items()):
        print(f"worst error / bar, {key}: {ratio:.1%} ({label})", flush=True)


def hip_fwd_raw(q, k, v, slopes, causal, sm_scale):
    """co_alibi_fwd through the C ABI; returns (o, lse, stats) on the device."""
    lib = _native.lib()
    B, Hq, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    o = torch.empty_like(q)
    lse = torch.empty(B, Hq, Sq, device=DEV, dtype=torch.float32)
    stats = torch.empty(lib.co_alibi_stats_numel(B, Hq, Sq, Skv), device=DEV, dtype=torch.float32)
    _native.check(lib.co_alibi_fwd(_native.DTYPE_CODES[q.dtype], q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                   slopes.data_ptr(), o.data_ptr(), lse.data_ptr(), stats.data_ptr(), B, Hq, Hkv,
                                   Sq, Skv, D, int(causal), sm_scale, torch.cuda.current_stream().cuda_stream))
    return o, lse, stats


# --------------------------------------------------------------------------- small shapes

def bwd_workspace_bytes(lib, path, dtype, B, Hq, Hkv, Sq, Skv, D, causal):
    """Workspace size that selects a backward path: "recompute" (pass 2 recomputes s and dS
    from cb) or "store" (pass 1 keeps them in the score store)."""
    if path == "recompute":
        return lib.co_alibi_bwd_workspace_bytes(B, Hq, Sq, Skv)
    n = lib.co_alibi_bwd_score_store_workspace_bytes(_native.DTYPE_CODES[dtype], B, Hq, Hkv, Sq, Skv, D, int(causal))
    assert n > 0, "no score-store path for this dtype / head dim"
    return n


PATHS = ["recompute", "store"]


def test_cpu_config_fp32_validation_mode():
    """BASELINE configs[0] in the fp32 validation mode: max-abs <= 1e-4."""
    w = WORKLOADS["cpu"]
    q, k, v, do = make_inputs(w, seed=0)
    got = hip_fwd_bwd(q, k, v, do, causal=True)
    o, lse, dq, dk, dv = oracle_fwd_bwd(q, k, v, do, causal=True)
    assert_parity(got, (o, dq, dk, dv), 1e-4, "cpu-config fp32")


CASES = [
    # (B, Hq, Hkv, Sq, Skv, D, causal)
    (1, 2, 2, 128, 128, 64, True),
    (1, 2, 2, 256, 256, 128, True),
    (2, 4, 2, 200, 200, 64, True),      # tails, grouped heads
    (1, 4, 1, 97, 97, 128, True),       # odd length, 4 query heads per key head
    (1, 2, 2, 1, 1, 64, True),          # single query / key
    (1, 2, 2, 1, 50, 128, True),        # Sq = 1 with many keys (only key 0 visible)
    (1, 2, 2, 130, 77, 64, True),       # more queries than keys (top-left causal)
    (1, 2, 2, 50, 300, 128, True),      # more keys than queries
    (1, 2, 2, 100, 100, 64, False),     # non-causal
    (1, 4, 2, 70, 190, 128, False),     # non-causal, rectangular, grouped
    (1, 2, 2, 300, 300, 64, True),      # several key tiles, partial last tile
    (1, 4, 2, 150, 150, 32, True),      # head dim 32, grouped heads
    (1, 2, 2, 90, 200, 32, False),      # head dim 32, non-causal, rectangular
    (2, 4, 2, 260, 260, 16, True),      # head dim 16 (a 32-wide head dim with zero padding), grouped
    (1, 3, 3, 70, 190, 16, False),      # head dim 16, non-causal, rectangular, tails
    (1, 8, 1, 129, 129, 16, True),      # head dim 16, 8 query heads per key head
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}H{}/{}S{}x{}D{}{}".format(*c[:6], "c" if c[6] else "n"))
def test_small_shapes(case, dtype):
    B, Hq, Hkv, Sq, Skv, D, causal = case
    print(f"case {case} {dtype}", flush=True)
    q, k, v, do = rand_inputs(B, Hq, Hkv, Sq, Skv, D, dtype, seed=1)
    got = hip_fwd_bwd(q, k, v, do, causal=causal)
    o, lse, dq, dk, dv = oracle_fwd_bwd(q, k, v, do, causal=causal)
    assert_parity(got, (o, dq, dk, dv), TOL[dtype], f"{case}", dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["fp16", "fp32"])
def test_lse_and_penalty_statistics(dtype):
    """LSE (natural log, m + log(l + 1e-9)); the row sigmoid sums R the forward saves (hi + lo);
    and what backward pass 1 rebuilds from them while it walks each row's keys left to right,
    read from the recompute path's workspace: zb[J][i] = sum of sigma_ik over k >= 32J and
    cb[J][i] = sum of dA_ik over k < 32J, against the oracle's per-pair terms.  Also the saved
    statistics' O(B*Hq*S) size and kstart = 0 (the slopes here are too flat to skip anything)."""
    lib = _native.lib()
    B, Hq, Hkv, S, D = 1, 2, 2, 150, 64
    q, k, v, do = rand_inputs(B, Hq, Hkv, S, S, D, dtype, seed=2)
    lam = ref.slopes(Hq, dtype=dtype).float()
    scale = 1.0 / math.sqrt(D)
    qd, kd, vd, dod, lamd = (t.to(DEV) for t in (q, k, v, do, lam))
    o, lse, stats = hip_fwd_raw(qd, kd, vd, lamd, True, scale)
    ws_bytes = lib.co_alibi_bwd_workspace_bytes(B, Hq, S, S)
    ws = torch.zeros(ws_bytes, device=DEV, dtype=torch.uint8)
    dq = torch.empty_like(qd)
    _native.check(lib.co_alibi_bwd_dq(_native.DTYPE_CODES[dtype], dod.data_ptr(), qd.data_ptr(), kd.data_ptr(),
                                      vd.data_ptr(), o.data_ptr(), lse.data_ptr(), stats.data_ptr(),
                                      lamd.data_ptr(), dq.data_ptr(), ws.data_ptr(), ws_bytes, B, Hq, Hkv, S, S, D,
                                      1, scale, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    _, lse_ref = ref.forward(q.float(), k.float(), v.float(), lam, causal=True, scale=scale)
    tol = 1e-4 if dtype == torch.float32 else 5e-3
    assert (lse.cpu() - lse_ref).abs().max().item() <= tol
    nqb, nkc, nkb = (S + 127) // 128, (S + 255) // 256, (S + 63) // 64
    assert stats.numel() == 4 + B * Hq * (2 * nqb + nkc + nkb + 2 * S)
    st = stats.cpu()
    assert not st[4:4 + B * Hq * nqb].view(torch.int32).any(), "kstart of flat slopes is 0"
    r0 = 4 + B * Hq * (2 * nqb + nkc + nkb)
    rsum = (st[r0:r0 + B * Hq * S].double() + st[r0 + B * Hq * S:r0 + 2 * B * Hq * S].double()).view(B * Hq, S)
    nzb = (S + 31) // 32
    rows_bytes = (B * Hq * S * 4 + 255) // 256 * 256
    blk_bytes = (B * Hq * nzb * S * 4 + 255) // 256 * 256
    wsf = ws.cpu()
    zb = wsf[rows_bytes:rows_bytes + B * Hq * nzb * S * 4].view(torch.float32).view(B * Hq, nzb, S)
    cb = wsf[rows_bytes + blk_bytes:rows_bytes + blk_bytes + B * Hq * nzb * S * 4].view(torch.float32)
    cb = cb.view(B * Hq, nzb, S)
    for h in range(Hq):
        _, sig, da, _ = ref._rows_terms(q[0, h].float(), do[0, h].float(), k[0, h].float(), v[0, h].float(), lam[h],
                                        True, scale, 0)
        assert (rsum[h] - sig.double().sum(-1)).abs().max().item() <= 1e-5 * S
        suffix = torch.cumsum(sig.flip(-1), -1).flip(-1)  # [i, j] = sum_{k >= j} sigma_ik
        prefix = torch.cumsum(da, -1) - da                # [i, j] = sum_{k < j} dA_ik
        for J in range(nzb):
            rows = torch.arange(32 * J, S)  # rows whose 32-row block processes key block J
            err_z = (zb[h, J, rows] - suffix[rows, 32 * J]).abs().max().item()
            err_c = (cb[h, J, rows] - prefix[rows, 32 * J]).abs().max().item()
            assert err_z <= 1e-4 * max(1.0, S / 32), f"zb head {h} block {J}: {err_z}"
            assert err_c <= (1e-5 if dtype == torch.float32 else 2e-3), f"cb head {h} block {J}: {err_c}"


@pytest.mark.parametrize("path", PATHS)
def test_split_backward_equals_full(path):
    """co_alibi_bwd_dq then co_alibi_bwd_dkdv == co_alibi_bwd, bit for bit, on either path."""
    lib = _native.lib()
    B, Hq, Hkv, S, D = 1, 4, 2, 190, 128
    dtype = torch.float16
    q, k, v, do = (t.to(DEV) for t in rand_inputs(B, Hq, Hkv, S, S, D, dtype, seed=3))
    lam = ref.slopes(Hq, dtype=dtype).float().to(DEV)
    scale = 1.0 / math.sqrt(D)
    o, lse, stats = hip_fwd_raw(q, k, v, lam, True, scale)
    ws_bytes = bwd_workspace_bytes(lib, path, dtype, B, Hq, Hkv, S, S, D, True)
    st = torch.cuda.current_stream().cuda_stream
    outs = []
    for split in (False, True):
        ws = torch.empty(ws_bytes, device=DEV, dtype=torch.uint8)
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        common = (B, Hq, Hkv, S, S, D, 1, scale, st)
        if split:
            _native.check(lib.co_alibi_bwd_dq(1, do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                              lse.data_ptr(), stats.data_ptr(), lam.data_ptr(), dq.data_ptr(),
                                              ws.data_ptr(), ws_bytes, *common))
            _native.check(lib.co_alibi_bwd_dkdv(1, do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                                lse.data_ptr(), stats.data_ptr(), lam.data_ptr(), dk.data_ptr(),
                                                dv.data_ptr(), ws.data_ptr(), ws_bytes, *common))
        else:
            _native.check(lib.co_alibi_bwd(1, do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                           lse.data_ptr(), stats.data_ptr(), lam.data_ptr(), dq.data_ptr(),
                                           dk.data_ptr(),
                                           dv.data_ptr(), ws.data_ptr(), ws_bytes, *common))
        torch.cuda.synchronize()
        outs.append((dq.cpu(), dk.cpu(), dv.cpu()))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_repeat_call_deterministic():
    q, k, v, do = rand_inputs(1, 4, 2, 333, 333, 128, torch.bfloat16, seed=4)
    r1 = hip_fwd_bwd(q, k, v, do)
    r2 = hip_fwd_bwd(q, k, v, do)
    for a, b in zip(r1, r2):
        assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=["fp16", "bf16", "fp32"])
def test_inference_forward_equals_training_forward(dtype):
    """Without gradients the forward writes no LSE / statistics and returns bit-identical O (drop-in API
    under no_grad, with inputs that need no grad: co_alibi_fwd_inference, whose tail skip takes
    the same decisions as the training forward's).  co_alibi_fwd with NULL statistics skips
    nothing: equal in fp16 (every skipped weight rounds to zero in P), within 1e-6 otherwise."""
    lib = _native.lib()
    for B, Hq, Hkv, Sq, Skv, D, causal in [(1, 4, 2, 200, 200, 64, True), (1, 2, 2, 70, 190, 128, False),
                                           (1, 4, 2, 1200, 1200, 64, True)]:  # the last one skips
        q, k, v, _ = rand_inputs(B, Hq, Hkv, Sq, Skv, D, dtype, seed=9)
        qd, kd, vd = (t.to(DEV) for t in (q, k, v))
        o_train = co_alibi_attention(qd.clone().requires_grad_(), kd, vd, causal=causal)
        assert o_train.grad_fn is not None
        with torch.no_grad():
            o_nograd = co_alibi_attention(qd.clone().requires_grad_(), kd, vd, causal=causal)
        o_plain = co_alibi_attention(qd, kd, vd, causal=causal)
        assert o_nograd.grad_fn is None and o_plain.grad_fn is None
        assert torch.equal(o_train.detach(), o_nograd) and torch.equal(o_nograd, o_plain)
        lam = ref.slopes(Hq, 8.0, dtype=dtype).float().to(DEV)  # the drop-in's slopes, kept alive
        st = torch.cuda.current_stream().cuda_stream
        o_abi, o_inf = torch.empty_like(qd), torch.empty_like(qd)
        _native.check(lib.co_alibi_fwd(_native.DTYPE_CODES[dtype], qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                                       lam.data_ptr(), o_abi.data_ptr(), 0, 0, B, Hq, Hkv, Sq, Skv, D,
                                       int(causal), 1.0 / math.sqrt(D), st))
        ws_bytes = lib.co_alibi_fwd_inference_workspace_bytes(B, Hq, Sq, Skv)
        ws = torch.empty(ws_bytes, device=DEV, dtype=torch.uint8)
        _native.check(lib.co_alibi_fwd_inference(_native.DTYPE_CODES[dtype], qd.data_ptr(), kd.data_ptr(),
                                                 vd.data_ptr(), lam.data_ptr(), o_inf.data_ptr(), ws.data_ptr(),
                                                 ws_bytes, B, Hq, Hkv, Sq, Skv, D, int(causal),
                                                 1.0 / math.sqrt(D), st))
        torch.cuda.synchronize()
        assert torch.equal(o_inf, o_plain)
        if dtype == torch.float16:
            assert torch.equal(o_abi, o_plain)
        else:
            assert (o_abi.float() - o_plain.float()).abs().max().item() <= 1e-6


@pytest.mark.parametrize("path", PATHS)
@pytest.mark.parametrize("causal", [True, False], ids=["causal", "noncausal"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=["fp16", "bf16", "fp32"])
def test_tail_skip(dtype, causal, path):
    """Slopes large enough that the forward stops early (keys whose weight is below 2^-26 (fp16),
    2^-32 (bf16) or 2^-64 (fp32) of their row's total are left out, and the backward passes
    leave out the same keys):
    - the first processed key per 128-row block (in the statistics) is a multiple of 64, positive for
      the steep heads, zero for the flat one, and no later than the block's diagonal tile;
    - O equals the forward without statistics, which skips nothing (bit for bit in fp16,
      where each skipped weight rounds to zero; within 1e-6 in bf16 and fp32);
    - forward and backward match the oracle, which computes every key, under the parity bar."""
    lib = _native.lib()
    B, Hq, Hkv, S, D = 1, 4, 2, 1000, 64
    q, k, v, do = rand_inputs(B, Hq, Hkv, S, S, D, dtype, seed=21)
    # Steep slopes concentrate each row's weight on a few keys: causal, dV_k is close to a few dO
    # rows; non-causal, every row weighs the last keys, so their dV sums all 1000 rows.  dO is
    # scaled so that |dV| stays within the range where the bar applies unscaled (in fp32 the
    # arithmetic's own rounding, the oracle's included, reaches 1e-4 at |dV| ~ 30 with slope 4).
    do = (do.float() * (0.5 if causal else 0.05)).to(dtype)
    lam = torch.tensor([4.0, 1.0, 0.25, 1e-3]).to(dtype).float()
    scale = 1.0 / math.sqrt(D)
    if path == "store" and dtype == torch.float32:
        pytest.skip("the score store is a 16-bit path")
    print(f"tail skip {dtype} causal={causal} {path}", flush=True)
    qd, kd, vd, dod, lamd = (t.to(DEV) for t in (q, k, v, do, lam))
    o, lse, stats = hip_fwd_raw(qd, kd, vd, lamd, causal, scale)
    st = torch.cuda.current_stream().cuda_stream
    o_plain = torch.empty_like(qd)
    _native.check(lib.co_alibi_fwd(_native.DTYPE_CODES[dtype], qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                                   lamd.data_ptr(), o_plain.data_ptr(), 0, 0, B, Hq, Hkv, S, S, D, int(causal),
                                   scale, st))
    ws_bytes = bwd_workspace_bytes(lib, path, dtype, B, Hq, Hkv, S, S, D, causal)
    ws = torch.empty(ws_bytes, device=DEV, dtype=torch.uint8)
    dq, dk, dv = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
    _native.check(lib.co_alibi_bwd(_native.DTYPE_CODES[dtype], dod.data_ptr(), qd.data_ptr(), kd.data_ptr(),
                                   vd.data_ptr(), o.data_ptr(), lse.data_ptr(), stats.data_ptr(), lamd.data_ptr(),
                                   dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws_bytes, B, Hq, Hkv,
                                   S, S, D, int(causal), scale, st))
    torch.cuda.synchronize()
    nqb = (S + 127) // 128
    kstart = stats[4:4 + B * Hq * nqb].view(torch.int32).view(Hq, nqb).cpu()
    print(f"  first processed key per 128-row block:\n{kstart}", flush=True)
    assert (kstart % 64 == 0).all() and (kstart >= 0).all()
    last_tile = torch.tensor([(min(qb * 128 + 127, S - 1) if causal else S - 1) // 64 * 64 for qb in range(nqb)])
    assert (kstart <= last_tile).all()
    assert (kstart[0] > 0).sum() >= nqb - 2 and (kstart[3] == 0).all()
    if dtype == torch.float16:
        assert torch.equal(o, o_plain)
    else:
        assert (o.float() - o_plain.float()).abs().max().item() <= 1e-6
    ro, _ = ref.forward(q.float(), k.float(), v.float(), lam, causal=causal, scale=scale)
    rdq, rdk, rdv = ref.backward(do.float(), q.float(), k.float(), v.float(), lam, causal=causal, scale=scale)
    assert_parity(tuple(t.float().cpu() for t in (o, dq, dk, dv)), (ro, rdq, rdk, rdv), TOL[dtype],
                  f"tail skip causal={causal} {path}", dtype)


def _fwd_bwd_raw(qd, kd, vd, dod, lamd, causal, scale, path, skip):
    """co_alibi_fwd then co_alibi_bwd through the C ABI under the given tail-skip setting; returns
    (o, dq, dk, dv, kstart) on the CPU."""
    lib = _native.lib()
    B, Hq, Sq, D = qd.shape
    Hkv, Skv = kd.shape[1], kd.shape[2]
    dtype = qd.dtype
    with _native.tail_skip(skip):
        o, lse, stats = hip_fwd_raw(qd, kd, vd, lamd, causal, scale)
    ws_bytes = bwd_workspace_bytes(lib, path, dtype, B, Hq, Hkv, Sq, Skv, D, causal)
    ws = torch.empty(ws_bytes, device=DEV, dtype=torch.uint8)
    dq, dk, dv = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
    _native.check(lib.co_alibi_bwd(_native.DTYPE_CODES[dtype], dod.data_ptr(), qd.data_ptr(), kd.data_ptr(),
                                   vd.data_ptr(), o.data_ptr(), lse.data_ptr(), stats.data_ptr(), lamd.data_ptr(),
                                   dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws_bytes, B, Hq, Hkv,
                                   Sq, Skv, D, int(causal), scale, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    nqb = (Sq + 127) // 128
    kstart = stats[4:4 + B * Hq * nqb].view(torch.int32).view(B * Hq, nqb).cpu()
    return tuple(t.float().cpu() for t in (o, dq, dk, dv)) + (kstart,)


@pytest.mark.parametrize("path", PATHS)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=["fp16", "bf16", "fp32"])
def test_tail_skip_backward_matches_full_work(dtype, path):
    """The backward with the tail skip against the same backward with the skip switched off (every
    key processed, kstart = 0), on slopes steep enough to skip most keys.  A skipped pair has
    s < 2^-T (T = 26, 32, 64 for fp16, bf16, fp32), so its dA = s (dS - D) and its share of the
    prefix C are below 2^-T of the row's scale, and the gradients' fp32 accumulators differ by
    far less than one rounding step of the output type.  The bound: one unit in the last place
    of the output type at the output's largest magnitude (16-bit), or 1e-6 of it (fp32)."""
    if path == "store" and dtype == torch.float32:
        pytest.skip("the score store is a 16-bit path")
    B, Hq, Hkv, S, D = 1, 4, 2, 1000, 64
    q, k, v, do = rand_inputs(B, Hq, Hkv, S, S, D, dtype, seed=21)
    do = (do.float() * 0.5).to(dtype)
    lam = torch.tensor([4.0, 1.0, 0.25, 1e-3]).to(dtype).float()
    scale = 1.0 / math.sqrt(D)
    print(f"skipped vs full-work backward {dtype} {path}", flush=True)
    qd, kd, vd, dod, lamd = (t.to(DEV) for t in (q, k, v, do, lam))
    got = _fwd_bwd_raw(qd, kd, vd, dod, lamd, True, scale, path, skip=True)
    full = _fwd_bwd_raw(qd, kd, vd, dod, lamd, True, scale, path, skip=False)
    assert (got[4][0] > 0).sum() >= 6 and not full[4].any(), "the steep head skips; the full run skips nothing"
    mant = {torch.float16: 10, torch.bfloat16: 7}
    for name, a, b in zip(("o", "dq", "dk", "dv"), got[:4], full[:4]):
        top = max(b.abs().max().item(), 1e-30)
        bound = 2.0 ** (math.floor(math.log2(top)) - mant[dtype]) if dtype in mant else 1e-6 * top
        err = (a - b).abs().max().item()
        print(f"  {name}: skipped vs full work {err:.3e} (bound {bound:.3e})", flush=True)
        assert err <= bound, f"{name}: {err} > {bound}"


@pytest.mark.parametrize("path", PATHS)
@pytest.mark.parametrize("causal", [True, False], ids=["causal", "noncausal"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_tail_skip_grouped_rectangular(dtype, causal, path):
    """The tail skip with grouped query heads of mixed steepness (the key head's pass-2 work list
    mixes heads whose skipped ranges differ), Sq != Skv (top-left causal), two batches and
    D = 128: forward and backward against the oracle."""
    lib = _native.lib()
    B, Hq, Hkv, Sq, Skv, D = 2, 6, 3, 700, 1100, 128
    q, k, v, do = rand_inputs(B, Hq, Hkv, Sq, Skv, D, dtype, seed=23)
    do = (do.float() * 0.5).to(dtype)
    lam = torch.tensor([3.0, 0.02, 1.0, 0.5, 0.002, 2.0]).to(dtype).float()
    scale = 1.0 / math.sqrt(D)
    print(f"tail skip grouped {dtype} causal={causal} {path}", flush=True)
    qd, kd, vd, dod, lamd = (t.to(DEV) for t in (q, k, v, do, lam))
    o, lse, stats = hip_fwd_raw(qd, kd, vd, lamd, causal, scale)
    st = torch.cuda.current_stream().cuda_stream
    ws_bytes = bwd_workspace_bytes(lib, path, dtype, B, Hq, Hkv, Sq, Skv, D, causal)
    ws = torch.empty(ws_bytes, device=DEV, dtype=torch.uint8)
    dq, dk, dv = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
    _native.check(lib.co_alibi_bwd(_native.DTYPE_CODES[dtype], dod.data_ptr(), qd.data_ptr(), kd.data_ptr(),
                                   vd.data_ptr(), o.data_ptr(), lse.data_ptr(), stats.data_ptr(), lamd.data_ptr(),
                                   dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws_bytes, B, Hq, Hkv,
                                   Sq, Skv, D, int(causal), scale, st))
    torch.cuda.synchronize()
    nqb = (Sq + 127) // 128
    kstart = stats[4:4 + B * Hq * nqb].view(torch.int32).view(B, Hq, nqb).cpu()
    assert (kstart[:, 0].max() > 0) and (kstart[:, 4] == 0).all()  # the steep head skips, the flattest does not
    ro, _ = ref.forward(q.float(), k.float(), v.float(), lam, causal=causal, scale=scale)
    rdq, rdk, rdv = ref.backward(do.float(), q.float(), k.float(), v.float(), lam, causal=causal, scale=scale)
    assert_parity(tuple(t.float().cpu() for t in (o, dq, dk, dv)), (ro, rdq, rdk, rdv), TOL[dtype],
                  f"tail skip grouped causal={causal} {path}", dtype)


STORE_CASES = [  # B, Hq, Hkv, Sq, Skv, D, causal
    (1, 2, 2, 64, 64, 64, True),
    (2, 4, 2, 190, 190, 128, True),
    (1, 4, 1, 150, 150, 64, False),
    (1, 2, 2, 100, 300, 128, True),   # Skv > Sq: key blocks past the last row block have no records
    (1, 2, 1, 300, 100, 64, True),    # Sq > Skv
    (2, 2, 2, 33, 97, 128, False),
    (1, 8, 2, 520, 520, 128, True),   # several work items per key block, group of 4
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("case", STORE_CASES, ids=lambda c: "B{}H{}/{}S{}x{}D{}{}".format(*c[:6], "c" if c[6] else "n"))
def test_score_store_matches_recompute(case, dtype):
    """The score-store backward against the recompute backward (same forward statistics) and
    the oracle: dq is bit-identical (pass 1 computes it the same way on both paths), dk and dv
    agree within the rounding of the recomputed scores, and both meet the bar."""
    lib = _native.lib()
    B, Hq, Hkv, Sq, Skv, D, causal = case
    q, k, v, do = rand_inputs(B, Hq, Hkv, Sq, Skv, D, dtype, seed=31)
    lam = ref.slopes(Hq, dtype=dtype).float()
    scale = 1.0 / math.sqrt(D)
    print(f"score store {case} {dtype}", flush=True)
    qd, kd, vd, dod, lamd = (t.to(DEV) for t in (q, k, v, do, lam))
    o, lse, stats = hip_fwd_raw(qd, kd, vd, lamd, causal, scale)
    st = torch.cuda.current_stream().cuda_stream
    outs = {}
    for path in PATHS:
        ws_bytes = bwd_workspace_bytes(lib, path, dtype, B, Hq, Hkv, Sq, Skv, D, causal)
        ws = torch.empty(ws_bytes, device=DEV, dtype=torch.uint8)
        dq, dk, dv = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
        _native.check(lib.co_alibi_bwd(_native.DTYPE_CODES[dtype], dod.data_ptr(), qd.data_ptr(), kd.data_ptr(),
                                       vd.data_ptr(), o.data_ptr(), lse.data_ptr(), stats.data_ptr(), lamd.data_ptr(),
                                       dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws_bytes, B, Hq,
                                       Hkv, Sq, Skv, D, int(causal), scale, st))
        torch.cuda.synchronize()
        outs[path] = tuple(t.float().cpu() for t in (dq, dk, dv))
    assert torch.equal(outs["store"][0], outs["recompute"][0])
    for a, b, name in zip(outs["store"][1:], outs["recompute"][1:], ("dk", "dv")):
        # the same bar as against the oracle: a flipped output rounding is one ulp of |b|
        err = (a - b).abs().max().item()
        bar = TOL[dtype] * max(1.0, b.abs().max().item() / REF_SCALE[dtype])
        print(f"  store vs recompute {name}: {err:.3e} (bar {bar:.3g})", flush=True)
        assert err <= bar, name
    ro, _ = ref.forward(q.float(), k.float(), v.float(), lam, causal=causal, scale=scale)
    rdq, rdk, rdv = ref.backward(do.float(), q.float(), k.float(), v.float(), lam, causal=causal, scale=scale)
    for path in PATHS:
        assert_parity((o.float().cpu(),) + outs[path], (ro, rdq, rdk, rdv), TOL[dtype], f"{path} {case}", dtype)


def test_sm_scale_and_bias_max_arguments():
    q, k, v, do = rand_inputs(1, 3, 3, 120, 120, 64, torch.float32, seed=5)
    got = hip_fwd_bwd(q, k, v, do, causal=True, sm_scale=0.3, bias_max=4.0)
    o, _, dq, dk, dv = oracle_fwd_bwd(q, k, v, do, causal=True, sm_scale=0.3, bias_max=4.0)
    assert_parity(got, (o, dq, dk, dv), 1e-4, "sm_scale=0.3 bias_max=4 H=3")


# Head dim 256.  In fp32 the kernels hold more than the register file and spill to scratch,
# and backward pass 2 reads the transposed Q and dO operands element by element.
CASES_D256 = [
    (1, 2, 2, 200, 200, 256, True),     # two query blocks, partial last key tile
    (1, 4, 2, 70, 150, 256, False),     # non-causal, rectangular, grouped
    (2, 4, 1, 700, 700, 256, True),     # several row and key blocks, four query heads per kv head
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("case", CASES_D256, ids=lambda c: "B{}H{}/{}S{}x{}D{}{}".format(*c[:6], "c" if c[6] else "n"))
def test_head_dim_256(case, dtype):
    B, Hq, Hkv, Sq, Skv, D, causal = case
    print(f"case {case} {dtype}", flush=True)
    q, k, v, do = rand_inputs(B, Hq, Hkv, Sq, Skv, D, dtype, seed=2)
    got = hip_fwd_bwd(q, k, v, do, causal=causal)
    o, lse, dq, dk, dv = oracle_fwd_bwd(q, k, v, do, causal=causal)
    assert_parity(got, (o, dq, dk, dv), TOL[dtype], f"{case}", dtype)


def test_unsupported_inputs_raise():
    q = torch.randn(1, 2, 8, 96, device=DEV, dtype=torch.float16)
    with pytest.raises(ValueError, match="head_dim"):
        co_alibi_attention(q, q, q)
    q = torch.randn(1, 2, 1, 256, device=DEV, dtype=torch.float32)
    with pytest.raises(ValueError, match="decode at head_dim 256"):
        co_alibi_decode(q, q, q)
    q = torch.randn(1, 2, 8, 64, device=DEV, dtype=torch.float64)
    with pytest.raises(TypeError):
        co_alibi_attention(q, q, q)


# --------------------------------------------------------------------------- golden fixtures

@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: p.rsplit("/", 1)[-1][:-4])
def test_golden_fixtures(path):
    t, causal, sm_scale, bias_max, dtype_name = load_golden(path)
    dtype = getattr(torch, dtype_name)
    q, k, v, do = (t[n].to(dtype) for n in ("q", "k", "v", "do"))
    got = hip_fwd_bwd(q, k, v, do, causal=causal, sm_scale=sm_scale, bias_max=bias_max)
    assert_parity(got, (t["o"], t["dq"], t["dk"], t["dv"]), TOL[dtype], path.rsplit("/", 1)[-1], dtype)


@pytest.mark.parametrize("causal", [True, False], ids=["causal", "noncausal"])
@pytest.mark.parametrize("shape", [(0, 4, 2, 64, 64), (2, 4, 2, 0, 64), (2, 4, 2, 64, 0)], ids=["B0", "Sq0", "Skv0"])
def test_empty_inputs(shape, causal):
    """No launch: an empty batch or no query rows give empty outputs; rows that see no key give
    O = 0 and LSE = -inf (the reference's l = 0 with its 1e-9 term); every gradient is zero."""
    B, Hq, Hkv, Sq, Skv = shape
    D = 64
    q = torch.randn(B, Hq, Sq, D, device=DEV, dtype=torch.float16, requires_grad=True)
    k = torch.randn(B, Hkv, Skv, D, device=DEV, dtype=torch.float16, requires_grad=True)
    v = torch.randn(B, Hkv, Skv, D, device=DEV, dtype=torch.float16, requires_grad=True)
    o = co_alibi_attention(q, k, v, causal=causal)
    assert o.shape == (B, Hq, Sq, D) and o.dtype == torch.float16
    assert torch.all(o == 0)
    o.backward(torch.randn_like(o))
    for t in (q, k, v):
        assert t.grad is not None and t.grad.shape == t.shape and torch.all(t.grad == 0)
    slopes = (2.0 * _get_coalibi_slopes(Hq)).to(DEV, torch.float16)
    _, lse, _ = torch.ops.co_alibi.fwd(q.detach(), k.detach(), v.detach(), slopes, causal, 0.125, True)
    assert lse.shape == (B, Hq, Sq) and torch.all(torch.isneginf(lse))


# --------------------------------------------------------------------------- full-size configs

FULL = ("headline", "gqa", "long")


@pytest.mark.parametrize("name", FULL)
def test_full_size_config(name):
    """BASELINE configs[1..3] at full size: every (batch, query head) of O and dQ and every
    (batch, key head) of dK and dV against the chunked CPU oracle, with the bar of assert_parity,
    both with the tail skip (the default) and with it switched off (every key processed, as the
    reference's kernels do; the mode the full-work measurements run in)."""
    w = WORKLOADS[name]
    print(f"config {name}: B{w.batch} Hq{w.heads_q} Hkv{w.heads_kv} S{w.seq} D{w.head_dim} {w.dtype}", flush=True)
    q, k, v, do = make_inputs(w, seed=0)
    runs = {}
    for skip in (True, False):
        with _native.tail_skip(skip):
            runs[skip] = hip_fwd_bwd(q, k, v, do, causal=w.causal, bias_max=w.bias_max)
    # Size-independent identity: sum over keys of dV = sum over rows of dO (weights sum to 1).
    g = w.heads_q // w.heads_kv
    do_sum = do.double().view(w.batch, w.heads_kv, g, w.seq, w.head_dim).sum((2, 3))
    for skip, got in runs.items():
        dv_sum = got[3].double().sum(2)                                     # (B, Hkv, D)
        rel = ((dv_sum - do_sum).abs().max() / do_sum.abs().max()).item()
        print(f"  tail skip {skip}: sum_j dV_j vs sum_i dO_i: rel {rel:.2e}", flush=True)
        assert rel < 1e-2
    ro, _, rdq, rdk, rdv = oracle_fwd_bwd(q, k, v, do, causal=w.causal, bias_max=w.bias_max)
    for skip, got in runs.items():
        label = f"{name} (all heads, tail skip {'on' if skip else 'off'})"
        # Per-head maxima, so a failure names its head.
        for n_, a_, b_ in zip(("o", "dq", "dk", "dv"), got, (ro, rdq, rdk, rdv)):
            per_head = (a_ - b_).abs().amax(dim=(2, 3))
            b0, h0 = divmod(int(per_head.argmax()), per_head.shape[1])
            print(f"  {label} {n_}: worst head (b{b0}, h{h0}) max-abs {per_head.max().item():.3e} over "
                  f"{per_head.numel()} heads", flush=True)
        assert_parity(got, (ro, rdq, rdk, rdv), TOL[w.dtype], label, w.dtype)


@pytest.mark.parametrize("name", FULL)
def test_full_size_invariances(name):
    """Identities of the math at the BASELINE sizes, over every head (the oracle above samples a few):
    - the backward is linear in dO: doubling dO doubles dQ, dK and dV (x2 is exact; the 16-bit
      kernels round dP to the input type, so values in the subnormal range may move by an ulp);
    - the softmax weights sum to 1 and D_i = dO_i.O_i absorbs the shift of dS_ij = dO_i.v_j, so a
      constant added to V adds it to O and leaves dQ and dK unchanged, and dV bit for bit (nothing
      dV reads depends on V)."""
    w = WORKLOADS[name]
    ulp = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}[w.dtype]
    print(f"invariances {name}: B{w.batch} Hq{w.heads_q} Hkv{w.heads_kv} S{w.seq} D{w.head_dim} {w.dtype}", flush=True)
    q, k, v, do = make_inputs(w, seed=1)
    run = lambda q_, k_, v_, do_: hip_fwd_bwd(q_, k_, v_, do_, causal=w.causal, bias_max=w.bias_max)  # noqa: E731
    o, dq, dk, dv = run(q, k, v, do)
    _, dq2, dk2, dv2 = run(q, k, v, (do.float() * 2).to(w.dtype))
    for n_, a, b in (("dq", dq2, dq), ("dk", dk2, dk), ("dv", dv2, dv)):
        excess = ((a - 2 * b).abs() - 2 * ulp * (2 * b).abs()).max().item()
        print(f"  2 dO -> {n_}: largest error beyond 2 ulp {excess:.2e}", flush=True)
        assert excess <= 1e-5, f"{n_} is not linear in dO"
    c = 0.25
    v_shift = (v.float() + c).to(w.dtype)
    o3, dq3, dk3, dv3 = run(q, k, v_shift, do)
    # v_shift - v is c up to the rounding of v + c (half an ulp of |v| + c), O up to its own rounding
    shift = (o3 - o - c).abs().max().item()
    print(f"  v + {c} -> o + {c}: max-abs {shift:.2e}", flush=True)
    assert shift <= 8 * ulp
    assert torch.equal(dv3, dv), "dV must not depend on V"
    for n_, a, b in (("dq", dq3, dq), ("dk", dk3, dk)):
        err = (a - b).abs().max().item()
        print(f"  v + {c} -> {n_} unchanged: max-abs {err:.2e}", flush=True)
        assert err <= TOL[w.dtype]


# --------------------------------------------------------------------------- long sequences

LONG_ROWS = [
    # (S, D, dtype): two query heads on one key head (slopes 0.125 and 2^-7), past the BASELINE
    # configs' 16384.  At 49152 the backward takes the score store (9.7 GB of records); at 2^17
    # the records (69 GB) would pass the store's 16 GiB limit and it takes the recompute path
    # (8.6 GB of zb / cb); fp32 runs its own kernels.
    (49152, 64, torch.float16),
    (131072, 64, torch.bfloat16),
    (32768, 128, torch.float32),
]


@pytest.mark.parametrize("S,D,dtype", LONG_ROWS, ids=lambda x: str(x).split(".")[-1])
def test_long_sequence_rows(S, D, dtype):
    """Sequence lengths past the BASELINE configs, with the tail skip on and off.  The oracle
    evaluates what it can afford at these lengths: O and dQ of three 64-row bands (the first, one
    in the middle, the last: each row needs only its own keys), and dK / dV of the last 64 keys,
    which only the last 64 rows see (causal).  Besides the bar of assert_parity, every output is
    within 5 % of its largest reference magnitude (rows that average many keys have small
    outputs).  Over the whole sequence, sum_j dV_j = sum_i dO_i (the weights of a row sum to 1)."""
    Hq = 2
    print(f"long sequence: B1 Hq{Hq} Hkv1 S{S} D{D} {dtype}", flush=True)
    q, k, v, do = rand_inputs(1, Hq, 1, S, S, D, dtype, seed=S + D)
    runs = {}
    for skip in (True, False):
        with _native.tail_skip(skip):
            runs[skip] = hip_fwd_bwd(q, k, v, do)
    do_sum = do.double().sum((1, 2))
    for skip, got in runs.items():
        rel = ((got[3].double().sum((1, 2)) - do_sum).abs().max() / do_sum.abs().max()).item()
        print(f"  tail skip {skip}: sum_j dV_j vs sum_i dO_i: rel {rel:.2e}", flush=True)
        assert rel < 1e-2
    lam = ref.slopes(Hq, 8.0, dtype=dtype).float()
    scale = 1.0 / math.sqrt(D)
    kf, vf = k[0, 0].float(), v[0, 0].float()
    bands = [(0, 64), (S // 2 - 32, S // 2 + 32), (S - 64, S)]
    rows = torch.cat([torch.arange(r0, r1) for r0, r1 in bands])
    want_o, want_dq = [], []
    want_dk = torch.zeros(64, D)
    want_dv = torch.zeros(64, D)
    for h in range(Hq):
        qf, dof = q[0, h].float(), do[0, h].float()
        for r0, r1 in bands:
            ob, *_ = ref._rows_forward(qf[r0:r1], kf[:r1], vf[:r1], lam[h], True, scale, r0)
            dqb, dkb, dvb = ref._rows_backward(qf[r0:r1], dof[r0:r1], kf[:r1], vf[:r1], lam[h], True, scale, r0)
            want_o.append(ob)
            want_dq.append(dqb)
        # The last band's contributions to the last 64 keys are their whole dK / dV from head h.
        want_dk += dkb[S - 64:]
        want_dv += dvb[S - 64:]
    want = (torch.cat(want_o), torch.cat(want_dq), want_dk, want_dv)
    for skip, (o, dq, dk, dv) in runs.items():
        got = (o[0][:, rows].reshape(-1, D), dq[0][:, rows].reshape(-1, D), dk[0, 0, S - 64:], dv[0, 0, S - 64:])
        label = f"S{S} D{D} (tail skip {'on' if skip else 'off'})"
        assert_parity(got, want, TOL[dtype], label, dtype)
        for n_, g_, w_ in zip(("o", "dq", "dk", "dv"), got, want):
            rel = ((g_ - w_).abs().max() / w_.abs().max()).item()
            print(f"  {label} {n_}: max-abs / max|ref| {rel:.2e}", flush=True)
            assert rel <= 0.05, f"{label}: {n_} off by {rel:.1%} of its magnitude"


# --------------------------------------------------------------------------- seeded random shapes

def _random_cases(n=18, seed=2024):
    """Seeded shapes across the edge space: lengths not multiple of any tile, Sq != Skv, GQA 1..8."""
    g = torch.Generator().manual_seed(seed)
    pick = lambda seq: seq[int(torch.randint(len(seq), (1,), generator=g))]  # noqa: E731
    cases = []
    for i in range(n):
        D = pick([32, 64, 128])
        Hkv = pick([1, 2, 3])
        grp = pick([1, 2, 4, 8])
        Sq = int(torch.randint(1, 400, (1,), generator=g))
        Skv = Sq if i % 3 else int(torch.randint(1, 400, (1,), generator=g))
        causal = bool(i % 4 != 3)
        dtype = pick([torch.float16, torch.bfloat16, torch.float32])
        B = pick([1, 2])
        cases.append((B, Hkv * grp, Hkv, Sq, Skv, D, causal, dtype))
    return cases


@pytest.mark.parametrize("case", _random_cases(),
                         ids=lambda c: "B{}H{}/{}S{}x{}D{}{}-{}".format(*c[:6], "c" if c[6] else "n", str(c[7])[6:]))
def test_random_shapes(case):
    B, Hq, Hkv, Sq, Skv, D, causal, dtype = case
    print(f"case {case}", flush=True)
    q, k, v, do = rand_inputs(B, Hq, Hkv, Sq, Skv, D, dtype, seed=Sq * 7 + Skv)
    got = hip_fwd_bwd(q, k, v, do, causal=causal)
    o, lse, dq, dk, dv = oracle_fwd_bwd(q, k, v, do, causal=causal)
    assert_parity(got, (o, dq, dk, dv), TOL[dtype], f"{case}", dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_non_contiguous_inputs(dtype):
    """Views in a model's (B, S, H, D) layout, transposed to (B, H, S, D), and sliced views give
    the same O and gradients, bit for bit, as contiguous copies of the same values (the
    wrapper makes them contiguous, as co_alibi_attn.py:137-148 does)."""
    B, Hq, Hkv, S, D = 2, 8, 2, 200, 64
    g = torch.Generator().manual_seed(17)
    qb = (torch.randn(B, S, Hq, D, generator=g) * 0.5).to(dtype).to(DEV)
    kb = (torch.randn(B, S + 3, Hkv, D, generator=g) * 0.5).to(dtype).to(DEV)
    vb = (torch.randn(B, S, Hkv, 2 * D, generator=g) * 0.5).to(dtype).to(DEV)
    do = torch.randn(B, Hq, S, D, generator=g).to(dtype).to(DEV)
    views = [qb.transpose(1, 2), kb[:, 3:].transpose(1, 2), vb[..., D:].transpose(1, 2)]
    assert not any(t.is_contiguous() for t in views)
    leaves = [t.detach().requires_grad_() for t in views]
    dense = [t.detach().contiguous().requires_grad_() for t in views]
    o1 = co_alibi_attention(*leaves)
    o1.backward(do)
    o2 = co_alibi_attention(*dense)
    o2.backward(do)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    for a, b in zip(leaves, dense):
        assert torch.equal(a.grad, b.grad)


def test_partial_gradients():
    """Only some inputs require grad: those get the same gradients as in the full backward,
    the others get none (autograd semantics of co_alibi_attn.py:72-135)."""
    q, k, v, do = (t.to(DEV) for t in rand_inputs(1, 4, 2, 150, 150, 64, torch.float16, seed=5))
    full = [t.clone().requires_grad_() for t in (q, k, v)]
    co_alibi_attention(*full).backward(do)
    for mask in ((True, False, False), (False, True, False), (False, False, True), (False, True, True)):
        ins = [t.clone().requires_grad_(m) for t, m in zip((q, k, v), mask)]
        co_alibi_attention(*ins).backward(do)
        torch.cuda.synchronize()
        for t, f, m in zip(ins, full, mask):
            if m:
                assert torch.equal(t.grad, f.grad), f"mask {mask}"
            else:
                assert t.grad is None, f"mask {mask}"


def _wide_cases():
    """A wider seeded sweep: COALIBI_WIDE_CASES cases (8 by default) from seed
    COALIBI_WIDE_SEED.  Head dims up to 256, lengths up to 2100, up to 5 kv heads with up
    to 8 query heads each, batch up to 3."""
    import os

    n = int(os.environ.get("COALIBI_WIDE_CASES", "8"))
    g = torch.Generator().manual_seed(int(os.environ.get("COALIBI_WIDE_SEED", "4242")))
    pick = lambda seq: seq[int(torch.randint(len(seq), (1,), generator=g))]  # noqa: E731
    cases = []
    for i in range(n):
        D = pick([32, 64, 128, 256])
        dtype = pick([torch.float16, torch.bfloat16, torch.float32])
        Hkv = pick([1, 2, 3, 5])
        grp = pick([1, 2, 3, 4, 8])
        Sq = int(torch.randint(1, 2100, (1,), generator=g))
        Skv = Sq if i % 3 else int(torch.randint(1, 2100, (1,), generator=g))
        causal = bool(i % 4 != 3)
        B = pick([1, 2, 3])
        cases.append((B, Hkv * grp, Hkv, Sq, Skv, D, causal, dtype, i))
    return cases


@pytest.mark.parametrize("case", _wide_cases(),
                         ids=lambda c: "{}-B{}H{}/{}S{}x{}D{}{}-{}".format(c[8], *c[:6], "c" if c[6] else "n",
                                                                        str(c[7])[6:]))
def test_random_shapes_wide(case):
    B, Hq, Hkv, Sq, Skv, D, causal, dtype, i = case
    print(f"case {case}", flush=True)
    q, k, v, do = rand_inputs(B, Hq, Hkv, Sq, Skv, D, dtype, seed=Sq * 13 + Skv + i)
    got = hip_fwd_bwd(q, k, v, do, causal=causal)
    o, lse, dq, dk, dv = oracle_fwd_bwd(q, k, v, do, causal=causal)
    assert_parity(got, (o, dq, dk, dv), TOL[dtype], f"{case}", dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["fp16", "fp32"])
@pytest.mark.parametrize("kv_form", ["expanded", "grouped", "mha"])
def test_autograd_function_apply(kv_form, dtype):
    """The reference's autograd function, CoALIBIAttention.apply(q, k, v, slopes, causal, sm_scale)
    (co_alibi_attn.py:24-135), forward and backward on the GPU against the oracle.

    expanded: K / V of 2 key heads repeated to the 8 query heads with repeat_interleave inside
      autograd, exactly as the reference's wrapper passes them (co_alibi_attn.py:143-147); the
      gradients of the unexpanded K / V are the group sums autograd forms through the repeat;
    grouped: the same K / V passed with their 2 heads (the native grouped-query form);
    mha: 8 key heads of their own.
    """
    B, Hq, S, D = 2, 8, 200, 64
    Hkv = 8 if kv_form == "mha" else 2
    print(f"apply {kv_form} {dtype}", flush=True)
    q, k, v, do = rand_inputs(B, Hq, Hkv, S, S, D, dtype, seed=11)
    slopes = (2.0 * _get_coalibi_slopes(Hq, 8.0)).to(DEV, dtype)  # co_alibi_attn.py:147
    sm_scale = 1.0 / math.sqrt(D)
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    if kv_form == "expanded":
        g = Hq // Hkv
        ka, va = kd.repeat_interleave(g, dim=1), vd.repeat_interleave(g, dim=1)
    else:
        ka, va = kd, vd
    o = CoALIBIAttention.apply(qd, ka, va, slopes, True, sm_scale)
    assert o.shape == (B, Hq, S, D) and o.dtype == dtype and o.grad_fn is not None
    o.backward(do.to(DEV))
    torch.cuda.synchronize()
    got = tuple(t.detach().float().cpu() for t in (o, qd.grad, kd.grad, vd.grad))
    ro, _, rdq, rdk, rdv = oracle_fwd_bwd(q, k, v, do, causal=True)
    assert_parity(got, (ro, rdq, rdk, rdv), TOL[dtype], f"apply {kv_form}", dtype)
    # The drop-in entry point (native grouped heads, no expansion) gives the same values.
    ref_api = hip_fwd_bwd(q, k, v, do, causal=True)
    tol = 0.0 if kv_form != "expanded" else TOL[dtype]
    for name, a, b in zip(("o", "dq", "dk", "dv"), got, ref_api):
        assert (a - b).abs().max().item() <= tol, f"apply {kv_form}: {name} differs from co_alibi_attention"
