"""PyTorch operators over the native library: ``co_alibi::fwd``, ``co_alibi::bwd``, ``co_alibi::bwd_dq``,
``co_alibi::decode``.

The operators are defined in C++ (``csrc/torch_ops.cpp``, built into
``_lib/libco_alibi_torch.so`` and loaded here): each one is one C-ABI launch
(include/co_alibi.h) on the caller's current HIP stream under a device guard, with its
outputs allocated through torch's caching allocator.  ``co_alibi::fwd`` carries its
backward as a C++ autograd kernel (``co_alibi::bwd``, or ``co_alibi::bwd_dq`` alone when
only q needs a gradient).  This module registers their shape functions, so that:
- ``torch.compile`` sees a single opaque node per launch and FakeTensor / meta tracing
  gives the output shapes and dtypes without running anything;
- nothing in them allocates outside torch's caching allocator or synchronises, so they
  can be captured in a CUDA (HIP) graph.

They replace the reference's two Triton launches with their buffer set-up:
``_co_alibi_fwd_kernel[grid](...)`` with the O / LSE / RowSigTotal allocations
(co_alibi_attn/co_alibi_attn.py:35-57) and ``_co_alibi_bwd_kernel[grid](...)`` with its
dK / dV partial buffers and their reduction (:83-133).  ``co_alibi::decode`` has no
counterpart in the reference (its forward with Sq = 1 over a cache).

Operands are (B, H, S, D) tensors as in include/co_alibi.h; the operators make them
contiguous and 16-byte aligned (a copy only when they are not).  Argument checking with
the reference's error types happens in the public functions of co_alibi_attn.py.
"""
import os

import torch
from torch import Tensor

from . import _native

__all__ = ["fwd", "bwd", "bwd_dq", "backward_for", "decode", "stats_numel", "TORCH_LIB_PATH"]

TORCH_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libco_alibi_torch.so")


def _load() -> str | None:
    """Load the C++ operators (once); returns why they are unavailable, or None.  There is
    no Python fallback: without them every operator raises (so the package still imports,
    as the build itself needs)."""
    if hasattr(torch.ops.co_alibi, "fwd"):
        return None
    if not os.path.exists(TORCH_LIB_PATH):
        return (f"co_alibi_attn: torch operator library {TORCH_LIB_PATH} is not built; "
                "run `python -m co_alibi_attn._build`")
    try:
        _native.lib()  # the C-ABI library the operators call, with its ABI version check
    except RuntimeError as e:
        return str(e)
    torch.ops.load_library(TORCH_LIB_PATH)
    return None


_MISSING = _load()


def require() -> None:
    """Raise the reason the operators are unavailable, if they are."""
    if _MISSING is not None:
        raise RuntimeError(_MISSING)


def _unavailable(*args, **kwargs):
    require()


if _MISSING is None:
    fwd = torch.ops.co_alibi.fwd
    bwd = torch.ops.co_alibi.bwd
    bwd_dq = torch.ops.co_alibi.bwd_dq
    decode = torch.ops.co_alibi.decode
else:
    fwd = bwd = bwd_dq = decode = _unavailable


def stats_numel(batch: int, heads_q: int, seq_q: int, seq_kv: int) -> int:
    """4-byte words of the forward's saved statistics besides LSE (the value co_alibi_stats_numel
    of the C ABI returns), O(B*Hq*S): a 4-word header, then B*Hq * (ceil(Sq/128)  first processed
    key per 128-row block, + ceil(Skv/256)  key-norm chunk maxima, + ceil(Sq/128) and
    ceil(Skv/64)  work orders of the row and key blocks, + 2*Sq  each row's sigmoid sum as a
    compensated hi / lo pair)."""
    return 4 + batch * heads_q * (2 * ((seq_q + 127) // 128) + (seq_kv + 255) // 256 + (seq_kv + 63) // 64
                                  + 2 * seq_q)


def _empty_stats(q: Tensor) -> Tensor:
    return q.new_empty((0,), dtype=torch.float32)


def backward_for(needs_input_grad, do, q, k, v, o, lse, stats, slopes, causal, sm_scale):
    """(dq, dk, dv) for the inputs whose flag in ``needs_input_grad`` (q, k, v first) is set,
    None for the others -- the rule of co_alibi::fwd's C++ autograd kernel, for Python autograd
    functions over the same operators.  dK needs backward pass 1's per-row statistics, so pass 1
    runs whenever any gradient is wanted; pass 2 runs only when dK or dV is."""
    need_q, need_k, need_v = needs_input_grad[:3]
    if not (need_k or need_v):
        return (bwd_dq(do, q, k, v, o, lse, stats, slopes, causal, sm_scale) if need_q else None), None, None
    dq, dk, dv = bwd(do, q, k, v, o, lse, stats, slopes, causal, sm_scale)
    return dq if need_q else None, dk if need_k else None, dv if need_v else None


# ------------------------------------------------------------------ shape functions


def _register_fakes() -> None:
    """Shape functions of the four operators (FakeTensor / meta tracing, torch.compile)."""

    @torch.library.register_fake("co_alibi::fwd")
    def _fwd_fake(q, k, v, slopes, causal, sm_scale, with_stats):
        """o (B, Hq, Sq, D) in q.dtype; with_stats: lse (B, Hq, Sq) in fp32 and the statistics
        (stats_numel(...),) as 4-byte words, else both empty.  With the tail skip off the key
        norms and work orders in the statistics are left unwritten (their header says so)."""
        batch, heads_q, seq_q, _ = q.shape
        o = torch.empty_like(q, memory_format=torch.contiguous_format)
        if not with_stats:
            return o, _empty_stats(q), _empty_stats(q)
        lse = q.new_empty((batch, heads_q, seq_q), dtype=torch.float32)
        stats = q.new_empty((stats_numel(batch, heads_q, seq_q, k.shape[2]),), dtype=torch.float32)
        return o, lse, stats

    @torch.library.register_fake("co_alibi::bwd")
    def _bwd_fake(do, q, k, v, o, lse, stats, slopes, causal, sm_scale):
        """(dq, dk, dv) in the input dtype; dk / dv have k's head count (summed over each group)."""
        cf = torch.contiguous_format
        return (torch.empty_like(q, memory_format=cf), torch.empty_like(k, memory_format=cf),
                torch.empty_like(v, memory_format=cf))

    @torch.library.register_fake("co_alibi::bwd_dq")
    def _bwd_dq_fake(do, q, k, v, o, lse, stats, slopes, causal, sm_scale):
        """dq alone (backward pass 1), bit-identical to co_alibi::bwd's dq."""
        return torch.empty_like(q, memory_format=torch.contiguous_format)

    @torch.library.register_fake("co_alibi::decode")
    def _decode_fake(q, k_cache, v_cache, slopes, seq_lens, max_seq_len, sm_scale, with_lse):
        """o (B, Hq, 1, D) in q.dtype and, with with_lse, the natural-log LSE (B, Hq, 1) in fp32."""
        batch, heads_q, _, _ = q.shape
        o = torch.empty_like(q, memory_format=torch.contiguous_format)
        lse = q.new_empty((batch, heads_q, 1), dtype=torch.float32) if with_lse else _empty_stats(q)
        return o, lse


if _MISSING is None:
    _register_fakes()
