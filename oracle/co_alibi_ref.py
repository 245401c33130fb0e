"""CPU oracle for Co-ALiBi attention -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
use this module, and only as the checker / the timed CPU path.  The product
(``co_alibi_attn``) never imports it and has no CPU fallback.

It restates the reference's PyTorch algorithm (model.py:13-76) with the
per-head penalty slope that the reference's kernels and validation scripts
apply (co_alibi_attn/co_alibi_attn.py:147, benchmark_fwd_pass.py:34-35,50,
benchmark_bwd_pass.py:89-91), plus the reference kernels' non-causal mode
(co_alibi_attn/co_alibi_fwd_kernel.py:80-90: only keys >= Skv are masked) and
grouped-query heads (co_alibi_attn.py:143-146: repeat K/V per query head, sum
the K/V gradients over each group).  Rows are processed in chunks per
(batch, head) so the full-size configs fit in memory.

Pinning (tests/test_oracle.py): every function below is checked against
closed forms or independent formulations, never against a retyped copy of
itself:
  * slopes            -- the closed form 2^(-bias_max(h+1)/n) and odd-power branch
  * forward           -- q = 0 (exact ALiBi with slope/2, geometric weights),
                         slope = 0 (torch scaled_dot_product_attention),
                         Sq = 1 (O = v_0), constant v, row-stochastic weights,
                         brute-force triple loop (oracle/brute.py) on tiny shapes
  * backward          -- finite differences of the forward (torch gradcheck,
                         fp64) and autograd of the forward
  * grouped heads     -- equality with the expanded-head computation
There are no golden vectors in the reference (its checks are unseeded and
warn-only, model.py:100-159), so those checks are the pin.
"""
from __future__ import annotations

import math

import torch



def slopes(n_heads: int, bias_max: float = 8.0, dtype: torch.dtype | None = None) -> torch.Tensor:
    """Effective per-head penalty slope: 2 x the ALiBi slope, optionally rounded to ``dtype``.

    co_alibi_attn.py:11-22 (slope table) and :147 (x2, cast to q.dtype).  Uses
    the same torch.pow(float, int64 tensor) evaluation so the fp32 values match.
    """
    n = 2 ** int(math.floor(math.log2(n_heads)))
    base = torch.pow(2.0 ** (-bias_max / n), torch.arange(1, 1 + n))
    if n < n_heads:
        extra = torch.pow(2.0 ** (-(bias_max / 2) / n), torch.arange(1, 1 + 2 * (n_heads - n), 2))
        base = torch.cat([base, extra])
    lam = 2.0 * base.abs()
    if dtype is not None:
        lam = lam.to(dtype)
    return lam


def _mask(nq: int, nk: int, row0: int, causal: bool, device=None) -> torch.Tensor:
    """True where key j is NOT visible from query row0+i (model.py:18: triu(diagonal=1))."""
    i = torch.arange(row0, row0 + nq, device=device).unsqueeze(1)
    j = torch.arange(nk, device=device).unsqueeze(0)
    if causal:
        return j > i
    return torch.zeros(nq, nk, dtype=torch.bool, device=device)


def _rows_forward(qr, k, v, lam, causal, scale, row0):
    """Forward for a block of query rows of one head (model.py:15-40 with slope)."""
    nq, nk = qr.shape[0], k.shape[0]
    neg = -torch.finfo(qr.dtype).max
    mask = _mask(nq, nk, row0, causal, qr.device)
    p = (qr @ k.transpose(0, 1)) * scale                                  # model.py:15
    p_masked = p.masked_fill(mask, neg)                                   # model.py:21
    sig = torch.sigmoid(p_masked).masked_fill(mask, 0.0)                  # model.py:23
    z = torch.cumsum(sig.flip(dims=[-1]), dim=-1).flip(dims=[-1])         # model.py:24
    a = (p_masked - lam * z).masked_fill(mask, neg)                       # model.py:26-27 (+ slope)
    m = a.max(dim=-1, keepdim=True).values                                # model.py:29
    e = torch.exp(a - m).masked_fill(mask, 0.0)                           # model.py:32-33
    denom = e.sum(dim=-1, keepdim=True) + 1e-9                            # model.py:35-36
    s = (e / denom).masked_fill(mask, 0.0)                                # model.py:38-39
    o = s @ v                                                             # model.py:40
    lse = m.squeeze(-1) + torch.log(denom.squeeze(-1))                    # co_alibi_fwd_kernel.py:120
    return o, lse, s, sig, mask


def _rows_terms(qr, dor, k, v, lam, causal, scale, row0):
    """Per-pair terms of the backward for a block of query rows: (s, sigma, dA, mask) with
    dA = s (dS - sum_j dS s) (model.py:38-39, 23, 62-66)."""
    _, _, s, sig, mask = _rows_forward(qr, k, v, lam, causal, scale, row0)
    ds = dor @ v.transpose(0, 1)                                          # model.py:62
    dsum = (ds * s).sum(dim=-1, keepdim=True)                             # model.py:64
    da = (s * (ds - dsum)).masked_fill(mask, 0.0)                         # model.py:65-66
    return s, sig, da, mask


def _rows_backward(qr, dor, k, v, lam, causal, scale, row0):
    """Backward for a block of query rows (model.py:57-76 with slope as benchmark_bwd_pass.py:89-91).

    Returns (dq rows, dk contribution, dv contribution)."""
    s, sig, da, mask = _rows_terms(qr, dor, k, v, lam, causal, scale, row0)
    dv = s.transpose(0, 1) @ dor                                          # model.py:61
    sig_prime = sig * (1.0 - sig)                                         # model.py:68
    c = torch.cumsum(da, dim=-1)                                          # model.py:69
    dp = (da - lam * sig_prime * c).masked_fill(mask, 0.0)                # model.py:71-73 (+ slope)
    dq = (dp @ k) * scale                                                 # model.py:75
    dk = (dp.transpose(0, 1) @ qr) * scale                                # model.py:76
    return dq, dk, dv


def _check(q, k, v, lam):
    B, Hq, Sq, D = q.shape
    assert k.shape[0] == B and k.shape[3] == D and v.shape == k.shape
    Hkv = k.shape[1]
    assert Hq % Hkv == 0
    lam = torch.as_tensor(lam, dtype=q.dtype).reshape(-1)
    assert lam.numel() == Hq
    return Hkv, Hq // Hkv, lam


def forward(q, k, v, lam, causal=True, scale=None, row_chunk=512, heads=None):
    """O (B,Hq,Sq,D) and LSE (B,Hq,Sq) in q's dtype.

    ``lam``: Hq slopes (already rounded as the caller wants).  ``heads``: optional
    list of (b, h) pairs to evaluate (others are left at zero) for sampled checks.
    """
    Hkv, g, lam = _check(q, k, v, lam)
    B, Hq, Sq, D = q.shape
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    o = torch.zeros_like(q)
    lse = torch.zeros(B, Hq, Sq, dtype=q.dtype)
    pairs = heads if heads is not None else [(b, h) for b in range(B) for h in range(Hq)]
    for b, h in pairs:
        kk, vv = k[b, h // g], v[b, h // g]
        for r0 in range(0, Sq, row_chunk):
            r1 = min(Sq, r0 + row_chunk)
            ob, lb, *_ = _rows_forward(q[b, h, r0:r1], kk, vv, lam[h], causal, scale, r0)
            o[b, h, r0:r1] = ob
            lse[b, h, r0:r1] = lb
    return o, lse


def backward(do, q, k, v, lam, causal=True, scale=None, row_chunk=512, heads=None):
    """(dq, dk, dv); dk/dv have k's head count (summed over each query-head group)."""
    Hkv, g, lam = _check(q, k, v, lam)
    B, Hq, Sq, D = q.shape
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    dq = torch.zeros_like(q)
    dk = torch.zeros_like(k)
    dv = torch.zeros_like(v)
    pairs = heads if heads is not None else [(b, h) for b in range(B) for h in range(Hq)]
    for b, h in pairs:
        kk, vv = k[b, h // g], v[b, h // g]
        for r0 in range(0, Sq, row_chunk):
            r1 = min(Sq, r0 + row_chunk)
            dqb, dkb, dvb = _rows_backward(q[b, h, r0:r1], do[b, h, r0:r1], kk, vv, lam[h], causal, scale, r0)
            dq[b, h, r0:r1] = dqb
            dk[b, h // g] += dkb
            dv[b, h // g] += dvb
    return dq, dk, dv


def forward_autograd(q, k, v, lam, causal=True, scale=None):
    """Differentiable dense forward (same math as ``forward``) for autograd / gradcheck."""
    Hkv, g, lam = _check(q, k, v, lam)
    B, Hq, Sq, D = q.shape
    Skv = k.shape[2]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    if g > 1:
        k = k.repeat_interleave(g, dim=1)
        v = v.repeat_interleave(g, dim=1)
    neg = -torch.finfo(q.dtype).max
    mask = _mask(Sq, Skv, 0, causal)
    p = torch.einsum("bhid,bhjd->bhij", q, k) * scale
    p_masked = p.masked_fill(mask, neg)
    sig = torch.sigmoid(p_masked).masked_fill(mask, 0.0)
    z = torch.cumsum(sig.flip(dims=[-1]), dim=-1).flip(dims=[-1])
    a = (p_masked - lam.view(1, Hq, 1, 1) * z).masked_fill(mask, neg)
    m = a.max(dim=-1, keepdim=True).values
    e = torch.exp(a - m).masked_fill(mask, 0.0)
    s = e / (e.sum(dim=-1, keepdim=True) + 1e-9)
    return torch.einsum("bhij,bhjd->bhid", s, v)
