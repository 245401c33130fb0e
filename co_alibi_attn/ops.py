"""PyTorch operators over the native library: ``co_alibi::fwd``, ``co_alibi::bwd``, ``co_alibi::bwd_dq``,
``co_alibi::decode``.

Each operator is one ``torch.library.custom_op`` around one C-ABI launch
(include/co_alibi.h), so that:
- ``torch.compile`` sees a single opaque node per launch instead of a graph break at
  the ctypes call;
- the fake implementations give output shapes and dtypes without running anything
  (FakeTensor / meta tracing, ahead-of-time autograd);
- ``co_alibi::fwd`` carries its backward (``co_alibi::bwd``) through
  ``torch.library.register_autograd``;
- nothing in them allocates outside torch's caching allocator or synchronises, so
  they can be captured in a CUDA (HIP) graph.

They replace the reference's two Triton launches with their buffer set-up:
``_co_alibi_fwd_kernel[grid](...)`` with the O / LSE / RowSigTotal allocations
(co_alibi_attn/co_alibi_attn.py:35-57) and ``_co_alibi_bwd_kernel[grid](...)`` with its
dK / dV partial buffers and their reduction (:83-133).  ``co_alibi::decode`` has no
counterpart in the reference (its forward with Sq = 1 over a cache).

Operands are (B, H, S, D) tensors as in include/co_alibi.h; they are made contiguous
and 16-byte aligned here (a copy only when they are not).  Argument checking with the
reference's error types happens in the public functions of co_alibi_attn.py.
"""
from typing import Optional, Tuple

import torch
from torch import Tensor

from . import _native

__all__ = ["fwd", "bwd", "bwd_dq", "backward_for", "decode", "zb_numel"]


def zb_numel(batch: int, heads_q: int, seq_q: int, seq_kv: int) -> int:
    """fp32 elements of the forward's penalty statistics: B*Hq * ceil(Skv/32) * Sq
    (the value co_alibi_zb_numel of the C ABI returns)."""
    return batch * heads_q * ((seq_kv + 31) // 32) * seq_q


def _aligned(t: Tensor) -> Tensor:
    """Contiguous tensor whose data pointer is 16-byte aligned (what the kernels load)."""
    t = t.contiguous()
    if t.data_ptr() % 16 != 0:
        t = t.clone()
    return t


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _empty_stats(q: Tensor) -> Tensor:
    return q.new_empty((0,), dtype=torch.float32)


# ---------------------------------------------------------------------------- forward


@torch.library.custom_op("co_alibi::fwd", mutates_args=(), device_types="cuda")
def fwd(q: Tensor, k: Tensor, v: Tensor, slopes: Tensor, causal: bool, sm_scale: float,
        with_stats: bool) -> Tuple[Tensor, Tensor, Tensor]:
    """Forward: returns (o, lse, zb).  o is (B, Hq, Sq, D) in q.dtype; lse (B, Hq, Sq) is the
    natural-log log-sum-exp and zb the penalty statistics co_alibi::bwd reads, both fp32.
    Causal: zb entries of 32-key blocks that lie wholly past a row's diagonal are left
    unwritten, as no reader needs them.  With ``with_stats`` false (inference) lse and zb
    are empty and the kernel writes neither."""
    batch, heads_q, seq_q, head_dim = q.shape
    heads_kv, seq_kv = k.shape[1], k.shape[2]
    if q.numel() == 0 or seq_kv == 0:
        # Nothing to launch.  Rows that see no key get what the reference's l = 0 gives:
        # O = 0 / (0 + 1e-9) = 0 and LSE = -inf + log(1e-9) = -inf (co_alibi_fwd_kernel.py:115,120).
        o = torch.zeros(q.shape, device=q.device, dtype=q.dtype)
        if not with_stats:
            return o, _empty_stats(q), _empty_stats(q)
        lse = torch.full((batch, heads_q, seq_q), float("-inf"), device=q.device, dtype=torch.float32)
        return o, lse, q.new_empty((zb_numel(batch, heads_q, seq_q, seq_kv),), dtype=torch.float32)
    q, k, v = _aligned(q), _aligned(k), _aligned(v)
    slopes32 = slopes.detach().to(device=q.device, dtype=torch.float32).contiguous()
    o = torch.empty_like(q)
    if with_stats:
        lse = torch.empty((batch, heads_q, seq_q), device=q.device, dtype=torch.float32)
        zb = torch.empty(zb_numel(batch, heads_q, seq_q, seq_kv), device=q.device, dtype=torch.float32)
    else:
        lse, zb = _empty_stats(q), _empty_stats(q)
    lib = _native.lib()
    with torch.cuda.device(q.device):
        _native.check(
            lib.co_alibi_fwd(
                _native.DTYPE_CODES[q.dtype], q.data_ptr(), k.data_ptr(), v.data_ptr(), slopes32.data_ptr(),
                o.data_ptr(), lse.data_ptr() if with_stats else 0, zb.data_ptr() if with_stats else 0,
                batch, heads_q, heads_kv, seq_q, seq_kv, head_dim, 1 if causal else 0, float(sm_scale),
                _stream(q.device),
            )
        )
    return o, lse, zb


@fwd.register_fake
def _fwd_fake(q, k, v, slopes, causal, sm_scale, with_stats):
    batch, heads_q, seq_q, _ = q.shape
    o = torch.empty_like(q, memory_format=torch.contiguous_format)
    if not with_stats:
        return o, _empty_stats(q), _empty_stats(q)
    lse = q.new_empty((batch, heads_q, seq_q), dtype=torch.float32)
    zb = q.new_empty((zb_numel(batch, heads_q, seq_q, k.shape[2]),), dtype=torch.float32)
    return o, lse, zb


def _fwd_setup_context(ctx, inputs, output):
    q, k, v, slopes, causal, sm_scale, with_stats = inputs
    o, lse, zb = output
    ctx.save_for_backward(q, k, v, o, lse, zb, slopes)
    ctx.causal, ctx.sm_scale, ctx.with_stats = causal, sm_scale, with_stats
    ctx.mark_non_differentiable(lse, zb)


def backward_for(needs_input_grad, do, q, k, v, o, lse, zb, slopes, causal, sm_scale):
    """(dq, dk, dv) for the inputs whose flag in ``needs_input_grad`` (q, k, v first) is set,
    None for the others.  dK needs backward pass 1's per-row statistics, so pass 1 runs
    whenever any gradient is wanted; pass 2 runs only when dK or dV is."""
    need_q, need_k, need_v = needs_input_grad[:3]
    if not (need_k or need_v):
        return (bwd_dq(do, q, k, v, o, lse, zb, slopes, causal, sm_scale) if need_q else None), None, None
    dq, dk, dv = bwd(do, q, k, v, o, lse, zb, slopes, causal, sm_scale)
    return dq if need_q else None, dk if need_k else None, dv if need_v else None


def _fwd_backward(ctx, do, _dlse, _dzb):
    if not ctx.with_stats:
        raise RuntimeError("co_alibi::fwd ran with with_stats=False (inference) and has no backward")
    q, k, v, o, lse, zb, slopes = ctx.saved_tensors
    dq, dk, dv = backward_for(ctx.needs_input_grad, do, q, k, v, o, lse, zb, slopes, ctx.causal, ctx.sm_scale)
    return dq, dk, dv, None, None, None, None


torch.library.register_autograd("co_alibi::fwd", _fwd_backward, setup_context=_fwd_setup_context)


# --------------------------------------------------------------------------- backward


@torch.library.custom_op("co_alibi::bwd", mutates_args=(), device_types="cuda")
def bwd(do: Tensor, q: Tensor, k: Tensor, v: Tensor, o: Tensor, lse: Tensor, zb: Tensor, slopes: Tensor,
        causal: bool, sm_scale: float) -> Tuple[Tensor, Tensor, Tensor]:
    """Backward: given dO and the forward's q, k, v, o, lse, zb, returns (dq, dk, dv) in the
    input dtype; for Hkv < Hq dk / dv are summed over each group's query heads."""
    batch, heads_q, seq_q, head_dim = q.shape
    heads_kv, seq_kv = k.shape[1], k.shape[2]
    if q.numel() == 0 or k.numel() == 0:  # no (query, key) pair: every gradient is zero
        return tuple(torch.zeros(t.shape, device=t.device, dtype=t.dtype) for t in (q, k, v))
    q, k, v, o = _aligned(q), _aligned(k), _aligned(v), _aligned(o)
    do = _aligned(do.to(q.dtype))
    lse, zb = lse.contiguous(), zb.contiguous()
    slopes32 = slopes.detach().to(device=q.device, dtype=torch.float32).contiguous()
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    lib = _native.lib()
    ws_bytes = lib.co_alibi_bwd_workspace_bytes(batch, heads_q, seq_q, seq_kv)
    workspace = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8)
    with torch.cuda.device(q.device):
        _native.check(
            lib.co_alibi_bwd(
                _native.DTYPE_CODES[q.dtype], do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                o.data_ptr(), lse.data_ptr(), zb.data_ptr(), slopes32.data_ptr(), dq.data_ptr(), dk.data_ptr(),
                dv.data_ptr(), workspace.data_ptr(), ws_bytes, batch, heads_q, heads_kv, seq_q, seq_kv,
                head_dim, 1 if causal else 0, float(sm_scale), _stream(q.device),
            )
        )
    return dq, dk, dv


@bwd.register_fake
def _bwd_fake(do, q, k, v, o, lse, zb, slopes, causal, sm_scale):
    cf = torch.contiguous_format
    return (torch.empty_like(q, memory_format=cf), torch.empty_like(k, memory_format=cf),
            torch.empty_like(v, memory_format=cf))


@torch.library.custom_op("co_alibi::bwd_dq", mutates_args=(), device_types="cuda")
def bwd_dq(do: Tensor, q: Tensor, k: Tensor, v: Tensor, o: Tensor, lse: Tensor, zb: Tensor, slopes: Tensor,
           causal: bool, sm_scale: float) -> Tensor:
    """dQ alone (backward pass 1, the C ABI's co_alibi_bwd_dq), for callers whose k and v need no
    gradient: the same dq as co_alibi::bwd, bit for bit, without the key-major pass 2."""
    batch, heads_q, seq_q, head_dim = q.shape
    heads_kv, seq_kv = k.shape[1], k.shape[2]
    if q.numel() == 0 or k.numel() == 0:
        return torch.zeros(q.shape, device=q.device, dtype=q.dtype)
    q, k, v, o = _aligned(q), _aligned(k), _aligned(v), _aligned(o)
    do = _aligned(do.to(q.dtype))
    lse, zb = lse.contiguous(), zb.contiguous()
    slopes32 = slopes.detach().to(device=q.device, dtype=torch.float32).contiguous()
    dq = torch.empty_like(q)
    lib = _native.lib()
    ws_bytes = lib.co_alibi_bwd_workspace_bytes(batch, heads_q, seq_q, seq_kv)
    workspace = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8)
    with torch.cuda.device(q.device):
        _native.check(
            lib.co_alibi_bwd_dq(
                _native.DTYPE_CODES[q.dtype], do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                o.data_ptr(), lse.data_ptr(), zb.data_ptr(), slopes32.data_ptr(), dq.data_ptr(),
                workspace.data_ptr(), ws_bytes, batch, heads_q, heads_kv, seq_q, seq_kv, head_dim,
                1 if causal else 0, float(sm_scale), _stream(q.device),
            )
        )
    return dq


@bwd_dq.register_fake
def _bwd_dq_fake(do, q, k, v, o, lse, zb, slopes, causal, sm_scale):
    return torch.empty_like(q, memory_format=torch.contiguous_format)


# ----------------------------------------------------------------------------- decode


@torch.library.custom_op("co_alibi::decode", mutates_args=(), device_types="cuda")
def decode(q: Tensor, k_cache: Tensor, v_cache: Tensor, slopes: Tensor, seq_lens: Optional[Tensor],
           max_seq_len: int, sm_scale: float, with_lse: bool) -> Tuple[Tensor, Tensor]:
    """Decode step: q (B, Hq, 1, D) against caches (B, Hkv, capacity, D) whose first
    ``max_seq_len`` rows (or seq_lens[b] rows, int32, clamped to [0, max_seq_len]) are
    filled.  Returns (o, lse): o (B, Hq, 1, D) in q.dtype and, with ``with_lse``, the
    natural-log LSE (B, Hq, 1) in fp32 (else an empty tensor)."""
    batch, heads_q, _, head_dim = q.shape
    heads_kv, capacity = k_cache.shape[1], k_cache.shape[2]
    if q.numel() == 0:  # an empty batch
        o = torch.empty(q.shape, device=q.device, dtype=q.dtype)
        lse = torch.empty((batch, heads_q, 1), device=q.device, dtype=torch.float32) if with_lse else _empty_stats(q)
        return o, lse
    q, k_cache, v_cache = _aligned(q), _aligned(k_cache), _aligned(v_cache)
    lens = None if seq_lens is None else seq_lens.to(device=q.device, dtype=torch.int32).contiguous()
    slopes32 = slopes.detach().to(device=q.device, dtype=torch.float32).contiguous()
    o = torch.empty_like(q)
    lse = (torch.empty((batch, heads_q, 1), device=q.device, dtype=torch.float32) if with_lse
           else _empty_stats(q))
    lib = _native.lib()
    ws_bytes = lib.co_alibi_decode_workspace_bytes(batch, heads_q, max_seq_len, head_dim)
    workspace = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8)
    with torch.cuda.device(q.device):
        _native.check(
            lib.co_alibi_decode(
                _native.DTYPE_CODES[q.dtype], q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                slopes32.data_ptr(), 0 if lens is None else lens.data_ptr(), o.data_ptr(),
                lse.data_ptr() if with_lse else 0, workspace.data_ptr(), ws_bytes, batch, heads_q, heads_kv,
                max_seq_len, capacity, head_dim, float(sm_scale), _stream(q.device),
            )
        )
    return o, lse


@decode.register_fake
def _decode_fake(q, k_cache, v_cache, slopes, seq_lens, max_seq_len, sm_scale, with_lse):
    batch, heads_q, _, _ = q.shape
    o = torch.empty_like(q, memory_format=torch.contiguous_format)
    lse = q.new_empty((batch, heads_q, 1), dtype=torch.float32) if with_lse else _empty_stats(q)
    return o, lse
