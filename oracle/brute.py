"""Brute-force Co-ALiBi forward by explicit loops -- TEST INFRASTRUCTURE ONLY.

An independent formulation of the forward for tiny shapes (pure Python floats,
double precision): every penalty term is the explicit sum
z_ij = sum_{k=j}^{last visible} sigmoid(p_ik) instead of a flipped cumsum, and
the softmax is written out term by term.  Used only by tests/test_oracle.py to
pin oracle/co_alibi_ref.py (reference semantics: model.py:13-40 with the
per-head slope of co_alibi_attn.py:147).
"""
from __future__ import annotations

import math


def forward(q, k, v, lam, causal=True, scale=None):
    """q: [B][Hq][Sq][D], k/v: [B][Hkv][Skv][D] nested lists; lam: Hq floats.

    Returns (o [B][Hq][Sq][D], lse [B][Hq][Sq]) as nested lists.
    """
    B, Hq, Sq, D = len(q), len(q[0]), len(q[0][0]), len(q[0][0][0])
    Hkv, Skv = len(k[0]), len(k[0][0])
    g = Hq // Hkv
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    out, lses = [], []
    for b in range(B):
        ob, lb = [], []
        for h in range(Hq):
            kh, vh = k[b][h // g], v[b][h // g]
            oh, lh = [], []
            for i in range(Sq):
                vis = [j for j in range(Skv) if (not causal) or j <= i]
                p = {j: scale * sum(q[b][h][i][d] * kh[j][d] for d in range(D)) for j in vis}
                sig = {j: 1.0 / (1.0 + math.exp(-p[j])) for j in vis}
                a = {}
                for j in vis:
                    z = 0.0
                    for kk in vis:
                        if kk >= j:
                            z += sig[kk]
                    a[j] = p[j] - lam[h] * z
                m = max(a.values())
                w = {j: math.exp(a[j] - m) for j in vis}
                denom = sum(w.values()) + 1e-9
                oh.append([sum(w[j] * vh[j][d] for j in vis) / denom for d in range(D)])
                lh.append(m + math.log(denom))
            ob.append(oh)
            lb.append(lh)
        out.append(ob)
        lses.append(lb)
    return out, lses
