"""Synthetic workloads of the benchmark configurations.

Each config is one of the five in BASELINE.json ``configs`` (the four attention
ones here; the GPT training step is not part of the attention hot path).
Inputs are drawn on the CPU from ``torch.Generator().manual_seed(seed)`` in
the order q, k, v, dO (the reference seeds with 0: benchmark_flops.py:28,
benchmark_fwd_pass.py:70), scaled, cast to the run dtype, and only then moved
to the device, so a CPU checker sees exactly the values the kernels see.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class Workload:
    name: str
    batch: int
    heads_q: int
    heads_kv: int
    seq: int
    head_dim: int
    dtype: torch.dtype
    causal: bool = True
    bias_max: float = 8.0
    qk_scale: float = 1.0      # q, k ~ qk_scale * N(0, 1)
    v_uniform: bool = False    # v ~ U(-1, 1) instead of v_scale * N(0, 1)
    v_scale: float = 1.0


WORKLOADS = {
    # CPU reference case, fp32 validation mode.
    "cpu": Workload("cpu", 1, 2, 2, 128, 64, torch.float32),
    # headline op.
    "headline": Workload("headline", 4, 16, 16, 4096, 128, torch.float16, qk_scale=0.5, v_scale=0.5),
    # grouped-query long context.
    "gqa": Workload("gqa", 1, 32, 8, 8192, 128, torch.bfloat16, qk_scale=0.5, v_scale=0.5),
    # small head dim, very long sequence.
    "long": Workload("long", 1, 8, 8, 16384, 64, torch.float16, qk_scale=0.3, v_uniform=True),
}


def make_inputs(w: Workload, seed: int = 0, device: str | torch.device = "cpu", seq: int | None = None,
                batch: int | None = None):
    """(q, k, v, dO) of workload ``w`` (optionally with a smaller seq / batch), in w.dtype."""
    S = w.seq if seq is None else seq
    B = w.batch if batch is None else batch
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(B, w.heads_q, S, w.head_dim, generator=gen) * w.qk_scale
    k = torch.randn(B, w.heads_kv, S, w.head_dim, generator=gen) * w.qk_scale
    if w.v_uniform:
        v = torch.rand(B, w.heads_kv, S, w.head_dim, generator=gen) * 2.0 - 1.0
    else:
        v = torch.randn(B, w.heads_kv, S, w.head_dim, generator=gen) * w.v_scale
    do = torch.randn(B, w.heads_q, S, w.head_dim, generator=gen)
    return tuple(t.to(w.dtype).to(device) for t in (q, k, v, do))


@dataclass(frozen=True)
class DecodeWorkload:
    """One decode step: a query per (batch, query head) against caches of ``seq_kv`` filled rows."""

    name: str
    batch: int
    heads_q: int
    heads_kv: int
    seq_kv: int
    head_dim: int
    dtype: torch.dtype
    bias_max: float = 8.0
    scale: float = 0.5  # q, k, v ~ scale * N(0, 1)

    def cache_bytes(self) -> int:
        """Bytes of the K and V rows one step reads."""
        return 2 * self.batch * self.heads_kv * self.seq_kv * self.head_dim * torch.finfo(self.dtype).bits // 8


DECODE_WORKLOADS = {
    # The next token after a prefill of BASELINE configs[2] (grouped-query, 8192 positions).
    "decode_gqa": DecodeWorkload("decode_gqa", 1, 32, 8, 8192, 128, torch.bfloat16),
    # The same model serving 16 sequences at once.
    "decode_serving": DecodeWorkload("decode_serving", 16, 32, 8, 8192, 128, torch.bfloat16),
    # One long-context sequence.
    "decode_long": DecodeWorkload("decode_long", 1, 32, 8, 131072, 128, torch.bfloat16),
}


def make_decode_inputs(w: DecodeWorkload, seed: int = 0, device: str | torch.device = "cpu"):
    """(q (B,Hq,1,D), k_cache, v_cache (B,Hkv,seq_kv,D)) of decode workload ``w``, in w.dtype."""
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(w.batch, w.heads_q, 1, w.head_dim, generator=gen) * w.scale
    k = torch.randn(w.batch, w.heads_kv, w.seq_kv, w.head_dim, generator=gen) * w.scale
    v = torch.randn(w.batch, w.heads_kv, w.seq_kv, w.head_dim, generator=gen) * w.scale
    return tuple(t.to(w.dtype).to(device) for t in (q, k, v))
