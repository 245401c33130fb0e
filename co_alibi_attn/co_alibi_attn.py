"""Drop-in Co-ALiBi attention for MI355X.

Same public surface as the reference module co_alibi_attn/co_alibi_attn.py:
``co_alibi_attention(q, k, v, causal=True, sm_scale=None, bias_max=8.0)``
(reference :137-148), the autograd function ``CoALIBIAttention`` (:24-135) and
the slope helper ``_get_coalibi_slopes`` (:11-22), plus ``co_alibi_decode``, a
split-K decode step over a key / value cache that the reference lacks.  The work runs in the
hand-written gfx950 kernels of ``libco_alibi.so`` (C ABI in include/co_alibi.h), reached
through the torch operators ``co_alibi::fwd``, ``co_alibi::bwd`` and ``co_alibi::decode``
(co_alibi_attn/ops.py); grouped-query attention is handled inside the kernels instead of
by ``repeat_interleave``.
"""
from __future__ import annotations

import torch

from . import _native, ops

__all__ = ["co_alibi_attention", "co_alibi_decode", "CoALIBIAttention", "_get_coalibi_slopes"]


def _get_coalibi_slopes(n_heads: int, bias_max: float = 8.0) -> torch.Tensor:
    """ALiBi slopes with a configurable ``bias_max`` (reference co_alibi_attn.py:11-22).

    With n the largest power of two <= n_heads, head h < n gets
    2^(-bias_max*(h+1)/n); the remaining heads t = 0.. take the odd powers
    2^(-(bias_max/2)*(2t+1)/n).  Computed with torch.pow on a float base and an
    integer exponent tensor, so the values (default float dtype) are the
    reference's bit for bit.
    """
    n = 1 << (int(n_heads).bit_length() - 1)
    slopes = torch.pow(2.0 ** (-bias_max / n), torch.arange(1, n + 1))
    extra = n_heads - n
    if extra > 0:
        odd_powers = torch.arange(1, 2 * extra, 2)
        slopes = torch.cat([slopes, torch.pow(2.0 ** (-(bias_max / 2) / n), odd_powers)])
    return slopes.abs()


_DEVICE_SLOPES: dict = {}


def _device_slopes(n_heads: int, bias_max: float, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    """The penalty slopes 2 * _get_coalibi_slopes(n_heads, bias_max) rounded to ``dtype`` (reference
    co_alibi_attn.py:147), held in fp32 on ``device`` -- the form the kernels read, so no call
    converts them -- and kept per (n_heads, bias_max, dtype, device): a copy from pageable host
    memory synchronises the stream, which would drain the GPU's queue at every call and make a
    graph capture fail.  Under torch.compile the values are computed in the traced graph instead."""
    if torch.compiler.is_compiling():
        return (2.0 * _get_coalibi_slopes(n_heads, bias_max)).to(dtype).to(device, dtype=torch.float32)
    key = (int(n_heads), float(bias_max), dtype, torch.device(device))
    slopes = _DEVICE_SLOPES.get(key)
    if slopes is None:
        slopes = (2.0 * _get_coalibi_slopes(n_heads, bias_max)).to(dtype).to(device, dtype=torch.float32)
        if type(slopes) is torch.Tensor:  # not a FakeTensor made under a tracing mode
            _DEVICE_SLOPES[key] = slopes
    return slopes


def _check_head_dim(head_dim: int, dtype: torch.dtype, decode: bool = False) -> None:
    if head_dim not in _native.SUPPORTED_HEAD_DIMS:
        raise ValueError(f"head_dim must be one of {_native.SUPPORTED_HEAD_DIMS}, got {head_dim}")
    if decode and head_dim == 256 and dtype == torch.float32:
        raise ValueError("decode at head_dim 256 needs float16 or bfloat16 inputs")


def _check_inputs(q, k, v, slopes) -> None:
    """The reference's checks (co_alibi_attn.py:30-33, AssertionError) plus the kernels'
    dtype (TypeError) and head-dim (ValueError) limits."""
    batch_size, num_heads, _, head_dim = q.shape
    num_kv_heads, seq_len_kv = k.shape[1], k.shape[2]
    assert num_kv_heads >= 1 and num_heads % num_kv_heads == 0
    assert k.shape == (batch_size, num_kv_heads, seq_len_kv, head_dim)
    assert v.shape == (batch_size, num_kv_heads, seq_len_kv, head_dim)
    assert q.is_cuda and k.is_cuda and v.is_cuda, "Inputs must be CUDA tensors"
    assert slopes.shape == (num_heads,), f"Slopes shape {slopes.shape} doesn't match num_heads {num_heads}"
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in _native.DTYPE_CODES:
        raise TypeError(f"q, k, v must share one dtype of float32/float16/bfloat16, got {q.dtype}, {k.dtype}, {v.dtype}")
    _check_head_dim(head_dim, q.dtype)


class CoALIBIAttention(torch.autograd.Function):
    """Autograd function over the native forward / backward (reference co_alibi_attn.py:24-135).

    ``apply(q, k, v, slopes, causal, sm_scale)``: q is (B, Hq, Sq, D); k and v
    are (B, Hkv, Skv, D) with Hq a multiple of Hkv (Hkv == Hq is the
    reference's only form); slopes holds Hq penalty slopes.  The launches are the
    operators ``co_alibi::fwd`` and ``co_alibi::bwd`` (co_alibi_attn/ops.py), which
    ``co_alibi_attention`` calls directly.
    """

    @staticmethod
    def forward(ctx, q, k, v, slopes, causal, sm_scale):
        _check_inputs(q, k, v, slopes)
        o, lse, stats = ops.fwd(q, k, v, slopes, bool(causal), float(sm_scale), True)
        ctx.save_for_backward(q, k, v, o, lse, stats, slopes)
        ctx.sm_scale = float(sm_scale)
        ctx.causal = bool(causal)
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse, stats, slopes = ctx.saved_tensors
        dq, dk, dv = ops.backward_for(ctx.needs_input_grad, do, q, k, v, o, lse, stats, slopes, ctx.causal,
                                      ctx.sm_scale)
        return dq, dk, dv, None, None, None


def co_alibi_attention(q, k, v, causal=True, sm_scale=None, bias_max=8.0):
    """Co-ALiBi attention (reference co_alibi_attn.py:137-148).

    q: (B, Hq, Sq, D); k, v: (B, Hkv, Skv, D) with Hq a multiple of Hkv; query
    head h uses key/value head h // (Hq // Hkv).  Returns (B, Hq, Sq, D) in
    q.dtype.  ``sm_scale`` defaults to D**-0.5; the per-head slope is twice the
    ALiBi slope of ``_get_coalibi_slopes(Hq, bias_max)``, rounded to q.dtype.
    The launch is the operator ``co_alibi::fwd``, differentiable through
    ``co_alibi::bwd``.  When no gradient can flow (grad mode off, or no input
    requires grad) the forward neither allocates nor writes the statistics only the
    backward reads.
    """
    if sm_scale is None:
        sm_scale = 1.0 / (q.shape[-1] ** 0.5)
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    num_q_heads = q.shape[1]
    slopes = _device_slopes(num_q_heads, bias_max, q.dtype, q.device)
    _check_inputs(q, k, v, slopes)
    needs_grad = torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad)
    return ops.fwd(q, k, v, slopes, bool(causal), float(sm_scale), needs_grad)[0]


def co_alibi_decode(q, k_cache, v_cache, seq_len=None, sm_scale=None, bias_max=8.0, return_lse=False,
                    max_seq_len=None):
    """One decode step: the newest query of every head against a key / value cache.

    q: (B, Hq, 1, D); k_cache, v_cache: (B, Hkv, capacity, D) with the first
    ``seq_len`` rows of every head filled.  ``seq_len`` is an int (every sequence; default:
    capacity) or an integer tensor of B per-sequence lengths on q's device (a serving
    batch); then ``max_seq_len`` (default: capacity) bounds them and sizes the launch, and
    lengths outside [0, max_seq_len] are clamped by the kernel.  All filled rows are
    visible to the query, so the result for sequence b equals
    ``co_alibi_attention(q[b:b+1], k_cache[b:b+1, :, :n_b], v_cache[b:b+1, :, :n_b],
    causal=False, sm_scale, bias_max)`` (reference co_alibi_attn.py:137-148; its top-left
    causal mask would let an Sq = 1 query see only the first key).  A sequence of length 0
    gets O = 0 and LSE = -inf.  Inference only: no autograd record.  Returns o
    (B, Hq, 1, D) in q.dtype, and with ``return_lse`` also the natural-log LSE (B, Hq, 1)
    in fp32.
    """
    if q.dim() != 4 or q.shape[2] != 1:
        raise ValueError(f"q must be (B, Hq, 1, D), got {tuple(q.shape)}")
    batch_size, num_heads, _, head_dim = q.shape
    num_kv_heads, capacity = k_cache.shape[1], k_cache.shape[2]
    assert k_cache.shape == (batch_size, num_kv_heads, capacity, head_dim)
    assert v_cache.shape == k_cache.shape
    assert num_kv_heads >= 1 and num_heads % num_kv_heads == 0
    assert q.is_cuda and k_cache.is_cuda and v_cache.is_cuda, "Inputs must be CUDA tensors"
    lens = None
    if isinstance(seq_len, torch.Tensor):
        if seq_len.shape != (batch_size,) or seq_len.dtype not in (torch.int32, torch.int64):
            raise ValueError(f"per-sequence lengths must be an integer tensor of shape ({batch_size},)")
        lens = seq_len.to(device=q.device, dtype=torch.int32).contiguous()
        bound = capacity if max_seq_len is None else int(max_seq_len)
        if not 1 <= bound <= capacity:
            raise ValueError(f"max_seq_len must be in [1, {capacity}], got {bound}")
    else:
        bound = capacity if seq_len is None else int(seq_len)
        if not 1 <= bound <= capacity:
            raise ValueError(f"seq_len must be in [1, {capacity}], got {bound}")
    if not (q.dtype == k_cache.dtype == v_cache.dtype) or q.dtype not in _native.DTYPE_CODES:
        raise TypeError(
            f"q and the caches must share one dtype of float32/float16/bfloat16, got "
            f"{q.dtype}, {k_cache.dtype}, {v_cache.dtype}"
        )
    _check_head_dim(head_dim, q.dtype, decode=True)
    if sm_scale is None:
        sm_scale = 1.0 / (head_dim ** 0.5)

    slopes = _device_slopes(num_heads, bias_max, q.dtype, q.device)
    o, lse = ops.decode(q.detach(), k_cache.detach(), v_cache.detach(), slopes, lens, bound, float(sm_scale),
                        bool(return_lse))
    return (o, lse) if return_lse else o
