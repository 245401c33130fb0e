"""Decode step (co_alibi_decode) vs the CPU oracle and vs the native forward.  Needs an MI355X.

A decode step is the reference forward with causal=False and Sq = 1 over the
cache's first seq_len rows (co_alibi_attn.py:137-148; its top-left causal mask
would show an Sq = 1 query only key 0).  Bar: max-abs <= 1e-4 (fp32) or 2e-2
(fp16 / bf16) on O, the same on the natural-log LSE, against the oracle in fp32
on the same dtype-rounded inputs and slopes.
"""
import math

import pytest
import torch

from co_alibi_attn import co_alibi_attention, co_alibi_decode
from oracle import co_alibi_ref as ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = {torch.float32: 1e-4, torch.float16: 2e-2, torch.bfloat16: 2e-2}
DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def cache_inputs(B, Hq, Hkv, L, cap, D, dtype, seed=0, scale=0.5):
    """q (B,Hq,1,D) and caches (B,Hkv,cap,D); rows >= L hold large garbage that must not leak in."""
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, Hq, 1, D, generator=g) * scale).to(dtype)
    k = (torch.randn(B, Hkv, cap, D, generator=g) * scale).to(dtype)
    v = (torch.randn(B, Hkv, cap, D, generator=g) * scale).to(dtype)
    k[:, :, L:] = 100.0
    v[:, :, L:] = -1000.0
    return q, k, v


def oracle_decode(q, k, v, L, sm_scale=None, bias_max=8.0):
    lam = ref.slopes(q.shape[1], bias_max, dtype=q.dtype).float()
    scale = 1.0 / math.sqrt(q.shape[-1]) if sm_scale is None else sm_scale
    o, lse = ref.forward(q.float(), k[:, :, :L].float(), v[:, :, :L].float(), lam, causal=False, scale=scale)
    return o, lse


def check(label, got, want, tol):
    assert torch.isfinite(got).all(), f"{label}: non-finite values"
    err = (got.float().cpu() - want.float()).abs().max().item()
    print(f"  {label}: max-abs {err:.3e} (tol {tol:g})", flush=True)
    assert err <= tol, f"{label}: max-abs {err:.3e} > {tol:g}"


# (B, Hq, Hkv, seq_len, capacity, D)
CASES = [
    (1, 4, 4, 1, 1, 64),            # one key: O = v_0
    (2, 8, 2, 300, 512, 128),       # group of 4, capacity > seq_len, last 128-key chunk 44 keys
    (1, 6, 2, 1000, 1000, 32),      # group of 3 (not a power of two)
    (1, 32, 1, 700, 768, 64),       # group of 32 (every MFMA column)
    (2, 16, 16, 257, 300, 128),     # no grouping, one key past a chunk
    (1, 32, 8, 4113, 4113, 128),    # Llama-style 4:1 grouping, ragged tail
    (2, 8, 2, 700, 1024, 16),       # head dim 16 (the operator pads the heads to 32)
]
# Head dim 256 (fp16 / bf16 only).
CASES_D256 = [
    (2, 8, 2, 1300, 1536, 256),
]


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16), ids=("float16", "bfloat16"))
@pytest.mark.parametrize("case", CASES_D256, ids=lambda c: "B{}_Hq{}_Hkv{}_L{}_cap{}_D{}".format(*c))
def test_decode_head_dim_256(case, dtype):
    B, Hq, Hkv, L, cap, D = case
    q, k, v = cache_inputs(B, Hq, Hkv, L, cap, D, dtype, seed=L)
    o, lse = co_alibi_decode(q.to(DEV), k.to(DEV), v.to(DEV), seq_len=L, return_lse=True)
    torch.cuda.synchronize()
    ro, rlse = oracle_decode(q, k, v, L)
    check("o", o, ro, TOL[dtype])
    check("lse", lse, rlse, TOL[dtype])


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}_Hq{}_Hkv{}_L{}_cap{}_D{}".format(*c))
def test_decode_matches_oracle(case, dtype):
    B, Hq, Hkv, L, cap, D = case
    q, k, v = cache_inputs(B, Hq, Hkv, L, cap, D, dtype, seed=L)
    print(f"decode {case} {dtype}", flush=True)
    o, lse = co_alibi_decode(q.to(DEV), k.to(DEV), v.to(DEV), seq_len=L, return_lse=True)
    torch.cuda.synchronize()
    ro, rlse = oracle_decode(q, k, v, L)
    check("o", o, ro, TOL[dtype])
    check("lse", lse, rlse, TOL[dtype])
    if L == 1:  # a single visible key: the softmax weight is exactly 1
        check("o == v_0", o, v[:, :, :1].float().repeat_interleave(Hq // Hkv, dim=1), TOL[dtype])


def test_decode_long_cache_merges_many_chunks():
    """70000 keys = 547 chunks of 128 in 183 splits of 3 chunks (on 256 CUs): every split walks several
    chunks, carrying sigma across them, and the last one is partial."""
    B, Hq, Hkv, L, D = 1, 8, 2, 70000, 128
    q, k, v = cache_inputs(B, Hq, Hkv, L, L, D, torch.float16, seed=7)
    o, lse = co_alibi_decode(q.to(DEV), k.to(DEV), v.to(DEV), return_lse=True)
    torch.cuda.synchronize()
    ro, rlse = oracle_decode(q, k, v, L)
    check("o", o, ro, TOL[torch.float16])
    check("lse", lse, rlse, TOL[torch.float16])


def test_decode_maximum_length():
    """seq_len = 2^21, the largest accepted: 16384 chunks in 512 splits (on 256 CUs), so the merge's
    suffix scan of the split sigma totals crosses its 256-split step."""
    B, Hq, Hkv, L, D = 1, 2, 1, 1 << 21, 64
    q, k, v = cache_inputs(B, Hq, Hkv, L, L, D, torch.bfloat16, seed=11)
    o, lse = co_alibi_decode(q.to(DEV), k.to(DEV), v.to(DEV), return_lse=True)
    torch.cuda.synchronize()
    ro, rlse = oracle_decode(q, k, v, L)
    check("o", o, ro, TOL[torch.bfloat16])
    check("lse", lse, rlse, TOL[torch.bfloat16])


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_decode_equals_forward_non_causal(dtype):
    """Same inputs through co_alibi_attention(causal=False) with Sq = 1 (the native forward kernel)."""
    B, Hq, Hkv, L, D = 2, 12, 4, 1500, 64
    q, k, v = cache_inputs(B, Hq, Hkv, L, L, D, dtype, seed=3)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    with torch.no_grad():
        want = co_alibi_attention(qd, kd, vd, causal=False)
    got = co_alibi_decode(qd, kd, vd)
    torch.cuda.synchronize()
    check("decode vs forward", got, want.cpu(), TOL[dtype])


def test_decode_after_prefill_is_the_last_causal_row():
    """The last row of a causal prefill over L positions sees all L keys: it is the decode step."""
    B, Hq, Hkv, L, D = 1, 16, 8, 777, 128
    g = torch.Generator().manual_seed(5)
    q = (torch.randn(B, Hq, L, D, generator=g) * 0.5).half().to(DEV)
    k = (torch.randn(B, Hkv, L, D, generator=g) * 0.5).half().to(DEV)
    v = (torch.randn(B, Hkv, L, D, generator=g) * 0.5).half().to(DEV)
    with torch.no_grad():
        prefill = co_alibi_attention(q, k, v, causal=True)
    step = co_alibi_decode(q[:, :, -1:], k, v)
    torch.cuda.synchronize()
    check("decode vs last prefill row", step, prefill[:, :, -1:].cpu(), TOL[torch.float16])


def test_decode_is_deterministic_and_lse_optional():
    B, Hq, Hkv, L, D = 1, 8, 2, 5000, 128
    q, k, v = (t.to(DEV) for t in cache_inputs(B, Hq, Hkv, L, L, D, torch.float16, seed=9))
    a, lse = co_alibi_decode(q, k, v, return_lse=True)
    b = co_alibi_decode(q, k, v)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert lse.shape == (B, Hq, 1) and lse.dtype == torch.float32


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_decode_per_sequence_lengths(dtype):
    """A serving batch: each sequence against its own filled prefix of the cache (lengths 1 .. capacity, and 0)."""
    B, Hq, Hkv, cap, D = 5, 16, 4, 1500, 128
    lens = [700, 1, 1500, 0, 257]
    q, k, v = cache_inputs(B, Hq, Hkv, cap, cap, D, dtype, seed=21)
    for b, n in enumerate(lens):  # rows past each sequence's length hold garbage that must not leak in
        k[b, :, n:] = 100.0
        v[b, :, n:] = -1000.0
    seq = torch.tensor(lens, dtype=torch.int32, device=DEV)
    o, lse = co_alibi_decode(q.to(DEV), k.to(DEV), v.to(DEV), seq_len=seq, return_lse=True)
    torch.cuda.synchronize()
    for b, n in enumerate(lens):
        if n == 0:
            assert torch.equal(o[b].float().cpu(), torch.zeros(Hq, 1, D)), "empty sequence: O must be 0"
            assert torch.isneginf(lse[b]).all(), "empty sequence: LSE must be -inf"
            continue
        ro, rlse = oracle_decode(q[b:b + 1], k[b:b + 1], v[b:b + 1], n)
        check(f"o[{b}] (len {n})", o[b:b + 1], ro, TOL[dtype])
        check(f"lse[{b}] (len {n})", lse[b:b + 1], rlse, TOL[dtype])


def test_decode_lengths_are_clamped_to_the_bound():
    """Per-sequence lengths past max_seq_len count as max_seq_len (the kernel clamps device data)."""
    B, Hq, Hkv, cap, D = 2, 8, 2, 2048, 64
    q, k, v = (t.to(DEV) for t in cache_inputs(B, Hq, Hkv, cap, cap, D, torch.float16, seed=4))
    seq = torch.tensor([5000, 1000], dtype=torch.int32, device=DEV)
    got = co_alibi_decode(q, k, v, seq_len=seq, max_seq_len=1000)
    want = co_alibi_decode(q, k, v, seq_len=1000)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def _random_decode_cases(n=10, seed=99):
    """Seeded serving batches: 1-4 sequences of random lengths (0 included) over caches of
    random capacity, 1-8 kv heads with 1-8 query heads each, every head dim and dtype."""
    g = torch.Generator().manual_seed(seed)
    pick = lambda seq: seq[int(torch.randint(len(seq), (1,), generator=g))]  # noqa: E731
    cases = []
    for i in range(n):
        D = pick([32, 64, 128, 256])
        dtype = pick([torch.float16, torch.bfloat16] + ([torch.float32] if D != 256 else []))
        Hkv = pick([1, 2, 3, 8])
        grp = pick([1, 2, 4, 5, 8])
        B = pick([1, 2, 3, 4])
        cap = int(torch.randint(1, 5000, (1,), generator=g))
        lens = [int(torch.randint(0, cap + 1, (1,), generator=g)) for _ in range(B)]
        cases.append((B, Hkv * grp, Hkv, cap, D, dtype, tuple(lens), i))
    return cases


@pytest.mark.parametrize("case", _random_decode_cases(),
                         ids=lambda c: "{}-B{}_Hq{}_Hkv{}_cap{}_D{}-{}".format(c[7], *c[:5], str(c[5])[6:]))
def test_decode_random_batches(case):
    B, Hq, Hkv, cap, D, dtype, lens, i = case
    print(f"case {case}", flush=True)
    q, k, v = cache_inputs(B, Hq, Hkv, cap, cap, D, dtype, seed=100 + i)
    for b, n in enumerate(lens):
        k[b, :, n:] = 100.0
        v[b, :, n:] = -1000.0
    seq = torch.tensor(lens, dtype=torch.int32, device=DEV)
    o, lse = co_alibi_decode(q.to(DEV), k.to(DEV), v.to(DEV), seq_len=seq, return_lse=True)
    torch.cuda.synchronize()
    for b, n in enumerate(lens):
        if n == 0:
            assert torch.equal(o[b].float().cpu(), torch.zeros(Hq, 1, D)), "empty sequence: O must be 0"
            assert torch.isneginf(lse[b]).all(), "empty sequence: LSE must be -inf"
            continue
        ro, rlse = oracle_decode(q[b:b + 1], k[b:b + 1], v[b:b + 1], n)
        check(f"o[{b}] (len {n})", o[b:b + 1], ro, TOL[dtype])
        check(f"lse[{b}] (len {n})", lse[b:b + 1], rlse, TOL[dtype])
