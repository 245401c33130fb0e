"""Pins the CPU oracle (oracle/co_alibi_ref.py) to mathematics it must satisfy.

None of these checks retypes the oracle's formula: each compares against a
closed form, an independent library routine, an explicit-loop formulation, or
finite differences.  The last group plants plausible mistakes into the oracle
(on the CPU) and asserts that the checks catch every one of them.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from co_alibi_attn.co_alibi_attn import _get_coalibi_slopes
from oracle import brute
from oracle import co_alibi_ref as ref

D64 = torch.float64


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=D64) * scale


# --------------------------------------------------------------------------- slopes

def _closed_form_slopes(n_heads, bias_max):
    n = 2 ** int(math.floor(math.log2(n_heads)))
    out = []
    for h in range(n_heads):
        if h < n:
            out.append(2.0 * 2.0 ** (-bias_max * (h + 1) / n))
        else:
            t = h - n
            out.append(2.0 * 2.0 ** (-(bias_max / 2.0) * (2 * t + 1) / n))
    return torch.tensor(out, dtype=D64)


@pytest.mark.parametrize("n_heads", [1, 2, 3, 5, 8, 12, 16, 32, 48, 64])
@pytest.mark.parametrize("bias_max", [8.0, 4.0])
def test_slopes_closed_form(n_heads, bias_max):
    got = ref.slopes(n_heads, bias_max).to(D64)
    torch.testing.assert_close(got, _closed_form_slopes(n_heads, bias_max), rtol=2e-6, atol=0)
    # the product's helper (x2, as the drop-in applies it) is the same tensor
    assert torch.equal(2.0 * _get_coalibi_slopes(n_heads, bias_max), ref.slopes(n_heads, bias_max))


def test_slopes_table():
    # Effective slopes listed for the benchmark head counts (exact in fp16 for powers of two).
    assert ref.slopes(2).tolist() == [0.125, 0.0078125]
    assert ref.slopes(8, dtype=torch.float16).tolist() == [2.0 ** -h for h in range(8)]
    h16 = ref.slopes(16, dtype=torch.float16).to(D64)
    torch.testing.assert_close(h16, torch.tensor([2.0 ** (0.5 - h / 2) for h in range(16)], dtype=D64),
                               rtol=5e-4, atol=0)
    h12 = ref.slopes(12, dtype=torch.float32).to(D64)
    want = [2.0 ** -h for h in range(8)] + [2.0 ** 0.5, 2.0 ** -0.5, 2.0 ** -1.5, 2.0 ** -2.5]
    torch.testing.assert_close(h12, torch.tensor(want, dtype=D64), rtol=2e-6, atol=0)


# --------------------------------------------------------------------------- forward pins
# Each check takes a forward callable fwd(q, k, v, lam, causal) -> (o, lse) and returns an error.

def check_q_zero_alibi(fwd):
    """q = 0: sigma = 1/2, z_ij = (#visible keys >= j)/2, so the weights are geometric (ALiBi, slope/2)."""
    err = 0.0
    for causal in (True, False):
        B, H, S, D = 1, 3, 23, 8
        q = torch.zeros(B, H, S, D, dtype=D64)
        k = _rand((B, H, S, D), 1)
        v = _rand((B, H, S, D), 2)
        lam = torch.tensor([0.9, 0.25, 0.03], dtype=D64)
        o, lse = fwd(q, k, v, lam, causal)
        for h in range(H):
            for i in range(S):
                last = i if causal else S - 1
                js = torch.arange(0, last + 1, dtype=D64)
                a = -lam[h] * (last - js + 1) / 2.0           # z_ij = (last - j + 1) / 2
                w = torch.exp(a - a.max())
                want_o = (w[:, None] * v[0, h, : last + 1]).sum(0) / (w.sum() + 1e-9)
                want_lse = a.max() + torch.log(w.sum() + 1e-9)
                err = max(err, (o[0, h, i] - want_o).abs().max().item(), abs(lse[0, h, i].item() - want_lse.item()))
    return err


def check_zero_slope_sdpa(fwd):
    """slope = 0: plain softmax attention (torch scaled_dot_product_attention, math path)."""
    err = 0.0
    for causal in (True, False):
        B, H, S, D = 2, 2, 19, 16
        q, k, v = _rand((B, H, S, D), 3), _rand((B, H, S, D), 4), _rand((B, H, S, D), 5)
        o, _ = fwd(q, k, v, torch.zeros(H, dtype=D64), causal)
        want = F.scaled_dot_product_attention(q, k, v, is_causal=causal, scale=1.0 / math.sqrt(D))
        err = max(err, (o - want).abs().max().item())
    return err


def check_single_query(fwd):
    """Sq = 1, causal: only key 0 is visible, O = v_0 (up to the 1e-9 in the normaliser)."""
    q, k, v = _rand((1, 2, 1, 8), 6), _rand((1, 2, 9, 8), 7), _rand((1, 2, 9, 8), 8)
    o, lse = fwd(q, k, v, torch.tensor([0.7, 0.1], dtype=D64), True)
    p0 = (q[0, :, 0] * k[0, :, 0]).sum(-1) / math.sqrt(8)
    a0 = p0 - torch.tensor([0.7, 0.1], dtype=D64) * torch.sigmoid(p0)
    return max((o[0, :, 0] - v[0, :, 0]).abs().max().item(), (lse[0, :, 0] - a0).abs().max().item())


def check_constant_v(fwd):
    """Rows of O are convex combinations: constant v gives O = v (weights sum to 1 - O(1e-9))."""
    q, k = _rand((1, 2, 17, 8), 9), _rand((1, 2, 17, 8), 10)
    v = torch.ones(1, 2, 17, 8, dtype=D64) * torch.arange(8, dtype=D64)
    o, _ = fwd(q, k, v, torch.tensor([0.5, 0.05], dtype=D64), True)
    return (o - v).abs().max().item()


def check_brute_force(fwd):
    """Explicit triple-loop formulation (oracle/brute.py), incl. grouped heads and non-causal."""
    err = 0.0
    for (B, Hq, Hkv, S, D, causal) in [(1, 2, 2, 6, 4, True), (2, 4, 2, 5, 3, True), (1, 2, 1, 7, 4, False)]:
        q, k, v = _rand((B, Hq, S, D), 11), _rand((B, Hkv, S, D), 12), _rand((B, Hkv, S, D), 13)
        lam = torch.linspace(0.05, 1.3, Hq, dtype=D64)
        o, lse = fwd(q, k, v, lam, causal)
        bo, bl = brute.forward(q.tolist(), k.tolist(), v.tolist(), lam.tolist(), causal)
        err = max(err, (o - torch.tensor(bo, dtype=D64)).abs().max().item(),
                  (lse - torch.tensor(bl, dtype=D64)).abs().max().item())
    return err


FORWARD_CHECKS = [check_q_zero_alibi, check_zero_slope_sdpa, check_single_query, check_constant_v,
                  check_brute_force]


def _oracle_fwd(q, k, v, lam, causal):
    return ref.forward(q, k, v, lam, causal=causal, row_chunk=7)


# Tolerances: fp64 rounding, except where the reference's "+1e-9" in the softmax
# normaliser (model.py:36) separates the oracle from a library routine or an
# exact identity by a relative 1e-9.
PIN_TOL = {check_q_zero_alibi: 1e-12, check_zero_slope_sdpa: 1e-8, check_single_query: 1e-8,
           check_constant_v: 1e-8, check_brute_force: 1e-12}


@pytest.mark.parametrize("check", FORWARD_CHECKS, ids=lambda c: c.__name__)
def test_forward_pins(check):
    assert check(_oracle_fwd) < PIN_TOL[check]


def test_row_chunking_is_exact():
    q, k, v = _rand((1, 2, 40, 8), 14), _rand((1, 2, 40, 8), 15), _rand((1, 2, 40, 8), 16)
    lam = torch.tensor([0.4, 0.02], dtype=D64)
    o1, l1 = ref.forward(q, k, v, lam, row_chunk=40)
    o2, l2 = ref.forward(q, k, v, lam, row_chunk=3)
    # BLAS may block differently per chunk size: equal up to fp64 rounding.
    torch.testing.assert_close(o1, o2, rtol=0, atol=1e-13)
    torch.testing.assert_close(l1, l2, rtol=0, atol=1e-13)


def test_forward_autograd_form_matches():
    q, k, v = _rand((2, 4, 21, 8), 17), _rand((2, 2, 21, 8), 18), _rand((2, 2, 21, 8), 19)
    lam = torch.linspace(0.1, 1.0, 4, dtype=D64)
    for causal in (True, False):
        o, _ = ref.forward(q, k, v, lam, causal=causal)
        torch.testing.assert_close(ref.forward_autograd(q, k, v, lam, causal=causal), o, rtol=0, atol=1e-12)


# --------------------------------------------------------------------------- backward pins

class _OracleFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, lam, causal):
        ctx.save_for_backward(q, k, v, lam)
        ctx.causal = causal
        return ref.forward(q, k, v, lam, causal=causal, row_chunk=5)[0]

    @staticmethod
    def backward(ctx, do):
        q, k, v, lam = ctx.saved_tensors
        dq, dk, dv = ref.backward(do, q, k, v, lam, causal=ctx.causal, row_chunk=5)
        return dq, dk, dv, None, None


def check_gradcheck():
    """Explicit backward == finite differences of the forward (fp64)."""
    ok = True
    for (B, Hq, Hkv, S, D, causal) in [(1, 2, 2, 6, 4, True), (1, 4, 2, 5, 3, True), (1, 2, 1, 6, 4, False)]:
        q = _rand((B, Hq, S, D), 20).requires_grad_()
        k = _rand((B, Hkv, S, D), 21).requires_grad_()
        v = _rand((B, Hkv, S, D), 22).requires_grad_()
        lam = torch.linspace(0.2, 1.4, Hq, dtype=D64)
        ok &= torch.autograd.gradcheck(lambda a, b, c: _OracleFn.apply(a, b, c, lam, causal), (q, k, v),
                                       eps=1e-6, atol=1e-7, rtol=1e-5, raise_exception=False)
    return ok


def check_backward_vs_autograd():
    q = _rand((1, 4, 48, 16), 23).requires_grad_()
    k = _rand((1, 2, 48, 16), 24).requires_grad_()
    v = _rand((1, 2, 48, 16), 25).requires_grad_()
    do = _rand((1, 4, 48, 16), 26)
    lam = torch.linspace(0.05, 1.2, 4, dtype=D64)
    ref.forward_autograd(q, k, v, lam).backward(do)
    dq, dk, dv = ref.backward(do, q.detach(), k.detach(), v.detach(), lam, row_chunk=13)
    return max((dq - q.grad).abs().max().item(), (dk - k.grad).abs().max().item(),
               (dv - v.grad).abs().max().item())


def test_backward_gradcheck():
    assert check_gradcheck()


def test_backward_matches_autograd():
    # model.py:64's explicit backward treats s as an exact softmax; the forward's
    # "+1e-9" normaliser makes the true gradient differ by a relative ~1e-9.
    assert check_backward_vs_autograd() < 1e-8


def test_grouped_heads_equal_expanded():
    B, Hq, Hkv, S, D = 2, 6, 2, 15, 8
    q, k, v, do = _rand((B, Hq, S, D), 27), _rand((B, Hkv, S, D), 28), _rand((B, Hkv, S, D), 29), _rand((B, Hq, S, D), 30)
    lam = torch.linspace(0.1, 0.9, Hq, dtype=D64)
    g = Hq // Hkv
    ke, ve = k.repeat_interleave(g, dim=1), v.repeat_interleave(g, dim=1)
    o1, l1 = ref.forward(q, k, v, lam)
    o2, l2 = ref.forward(q, ke, ve, lam)
    torch.testing.assert_close(o1, o2, rtol=0, atol=1e-13)
    torch.testing.assert_close(l1, l2, rtol=0, atol=1e-13)
    dq1, dk1, dv1 = ref.backward(do, q, k, v, lam)
    dq2, dk2, dv2 = ref.backward(do, q, ke, ve, lam)
    torch.testing.assert_close(dq1, dq2, rtol=0, atol=1e-13)
    torch.testing.assert_close(dk1, dk2.view(B, Hkv, g, S, D).sum(2), rtol=0, atol=1e-12)
    torch.testing.assert_close(dv1, dv2.view(B, Hkv, g, S, D).sum(2), rtol=0, atol=1e-12)


def test_prefix_c_equals_negative_suffix():
    """sum_j dA_ij = D_i (1 - sum_j s_ij) ~ 0, the identity the suffix-form backward relies on."""
    q, k, v, do = (_rand((1, 1, 30, 8), s) for s in (31, 32, 33, 34))
    _, _, s, sig, mask = ref._rows_forward(q[0, 0], k[0, 0], v[0, 0], 0.6, True, 1 / math.sqrt(8), 0)
    ds = do[0, 0] @ v[0, 0].T
    da = (s * (ds - (ds * s).sum(-1, keepdim=True))).masked_fill(mask, 0)
    assert da.sum(-1).abs().max().item() < 1e-8  # = D_i * 1e-9 / (l_i + 1e-9)


# --------------------------------------------------------------------------- planted mistakes

def _mutant_forward(kind):
    """A copy of the oracle's row forward with one plausible mistake planted."""
    def rows_forward(qr, k, v, lam, causal, scale, row0):
        nq, nk = qr.shape[0], k.shape[0]
        neg = -torch.finfo(qr.dtype).max
        if kind == "mask_off_by_one":
            mask = ref._mask(nq, nk, row0 + 1, causal)
        else:
            mask = ref._mask(nq, nk, row0, causal)
        p = (qr @ k.T) * scale
        pm = p.masked_fill(mask, neg)
        sig = torch.sigmoid(pm).masked_fill(mask, 0.0)
        if kind == "prefix_instead_of_suffix":
            z = torch.cumsum(sig, dim=-1)
        elif kind == "exclusive_suffix":
            z = torch.cumsum(sig.flip(-1), -1).flip(-1) - sig
        else:
            z = torch.cumsum(sig.flip(-1), -1).flip(-1)
        lam_eff = {"slope_sign": -lam, "no_slope": 0.0 * lam, "half_slope": 0.5 * lam}.get(kind, lam)
        a = (pm - lam_eff * z).masked_fill(mask, neg)
        m = a.max(-1, keepdim=True).values
        e = torch.exp(a - m).masked_fill(mask, 0.0)
        den = e.sum(-1, keepdim=True) + 1e-9
        s = (e / den).masked_fill(mask, 0.0)
        o = s @ (k if kind == "keys_as_values" else v)
        return o, m.squeeze(-1) + torch.log(den.squeeze(-1)), s, sig, mask
    return rows_forward


def _mutant_backward(kind):
    def rows_backward(qr, dor, k, v, lam, causal, scale, row0):
        _, _, s, sig, mask = ref._rows_forward(qr, k, v, lam, causal, scale, row0)
        dv = s.T @ dor
        ds = dor @ v.T
        dsum = (ds * s).sum(-1, keepdim=True)
        da = (s * (ds - dsum)).masked_fill(mask, 0.0)
        sp = sig * (1.0 - sig) if kind != "sigma_instead_of_derivative" else sig
        c = torch.cumsum(da, -1) if kind != "suffix_c" else torch.cumsum(da.flip(-1), -1).flip(-1)
        if kind == "exclusive_c":
            c = c - da
        lam_eff = -lam if kind == "penalty_grad_sign" else (0.0 * lam if kind == "no_penalty_grad" else lam)
        dp = (da - lam_eff * sp * c).masked_fill(mask, 0.0)
        return (dp @ k) * scale, (dp.T @ qr) * scale, dv
    return rows_backward


@pytest.mark.parametrize("kind", ["mask_off_by_one", "prefix_instead_of_suffix", "exclusive_suffix",
                                  "slope_sign", "no_slope", "half_slope", "keys_as_values"])
def test_forward_checks_catch_planted_mistake(kind, monkeypatch):
    monkeypatch.setattr(ref, "_rows_forward", _mutant_forward(kind))
    errors = [check(_oracle_fwd) for check in FORWARD_CHECKS]
    assert max(errors) > 1e-6, f"planted mistake {kind!r} went unnoticed: {errors}"


@pytest.mark.parametrize("kind", ["sigma_instead_of_derivative", "suffix_c", "exclusive_c",
                                  "penalty_grad_sign", "no_penalty_grad"])
def test_backward_checks_catch_planted_mistake(kind, monkeypatch):
    monkeypatch.setattr(ref, "_rows_backward", _mutant_backward(kind))
    assert not check_gradcheck() or check_backward_vs_autograd() > 1e-6, f"planted mistake {kind!r} went unnoticed"
