"""The torch operators co_alibi::fwd / bwd / decode without a GPU: schemas, fake (meta)
shapes, the autograd wiring of co_alibi::fwd, and tracing of the public functions under
FakeTensorMode.  Their numerics run through the same launches as the GPU parity tests."""
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import co_alibi_attn
from co_alibi_attn import _native, ops


def meta(*shape, dtype=torch.float16, grad=False):
    return torch.empty(*shape, device="meta", dtype=dtype, requires_grad=grad)


def test_operators_are_registered_with_their_schemas():
    fwd = str(torch.ops.co_alibi.fwd.default._schema)
    bwd = str(torch.ops.co_alibi.bwd.default._schema)
    dec = str(torch.ops.co_alibi.decode.default._schema)
    bwd_dq = str(torch.ops.co_alibi.bwd_dq.default._schema)
    assert bwd_dq == ("co_alibi::bwd_dq(Tensor do, Tensor q, Tensor k, Tensor v, Tensor o, Tensor lse, Tensor stats, "
                      "Tensor slopes, bool causal, float sm_scale) -> Tensor")
    assert fwd == ("co_alibi::fwd(Tensor q, Tensor k, Tensor v, Tensor slopes, bool causal, float sm_scale, "
                   "bool with_stats) -> (Tensor, Tensor, Tensor)")
    assert bwd == ("co_alibi::bwd(Tensor do, Tensor q, Tensor k, Tensor v, Tensor o, Tensor lse, Tensor stats, "
                   "Tensor slopes, bool causal, float sm_scale) -> (Tensor, Tensor, Tensor)")
    assert dec == ("co_alibi::decode(Tensor q, Tensor k_cache, Tensor v_cache, Tensor slopes, Tensor? seq_lens, "
                   "SymInt max_seq_len, float sm_scale, bool with_lse) -> (Tensor, Tensor)")


@pytest.mark.parametrize("shape", [(1, 2, 128, 128, 64), (2, 8, 100, 105, 32), (1, 32, 7, 300, 128)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_fwd_fake_shapes(shape, dtype):
    B, Hq, Sq, Skv, D = shape
    Hkv = max(1, Hq // 4)
    q, k, v = meta(B, Hq, Sq, D, dtype=dtype), meta(B, Hkv, Skv, D, dtype=dtype), meta(B, Hkv, Skv, D, dtype=dtype)
    o, lse, stats = torch.ops.co_alibi.fwd(q, k, v, meta(Hq, dtype=dtype), True, 0.1, True)
    assert o.shape == q.shape and o.dtype == dtype and o.is_contiguous()
    assert lse.shape == (B, Hq, Sq) and lse.dtype == torch.float32
    assert stats.shape == (ops.stats_numel(B, Hq, Sq, Skv),) and stats.dtype == torch.float32
    o, lse, stats = torch.ops.co_alibi.fwd(q, k, v, meta(Hq, dtype=dtype), False, 0.1, False)
    assert o.shape == q.shape and lse.numel() == 0 and stats.numel() == 0


def test_stats_numel_matches_the_library():
    lib = _native.lib()
    for args in [(1, 1, 1, 1), (4, 16, 4096, 4096), (1, 32, 8192, 8192), (2, 3, 100, 33), (1, 2, 5, 64)]:
        assert ops.stats_numel(*args) == lib.co_alibi_stats_numel(*args)


def test_fwd_autograd_reaches_bwd():
    """Backward of co_alibi::fwd is co_alibi::bwd: gradients of the input shapes and dtypes,
    for grouped heads; lse and stats carry no gradient."""
    B, Hq, Hkv, Sq, Skv, D = 2, 8, 2, 64, 96, 64
    q, k, v = meta(B, Hq, Sq, D, grad=True), meta(B, Hkv, Skv, D, grad=True), meta(B, Hkv, Skv, D, grad=True)
    o, lse, stats = torch.ops.co_alibi.fwd(q, k, v, meta(Hq), True, 0.125, True)
    assert o.requires_grad and not lse.requires_grad and not stats.requires_grad
    o.float().sum().backward()
    for t in (q, k, v):
        assert t.grad.shape == t.shape and t.grad.dtype == t.dtype


@pytest.mark.parametrize("mask", [(True, False, False), (False, True, False), (False, False, True), (True, True, False)])
def test_partial_gradients_reach_the_right_operator(mask):
    """Only the inputs that require grad get one; dQ alone runs co_alibi::bwd_dq (pass 1 only),
    any key / value gradient runs co_alibi::bwd (the C++ autograd kernel of co_alibi::fwd)."""
    from torch.utils._python_dispatch import TorchDispatchMode

    class Record(TorchDispatchMode):
        def __init__(self):
            super().__init__()
            self.ops = []

        def __torch_dispatch__(self, func, types, args=(), kwargs=None):
            if func.namespace == "co_alibi":
                self.ops.append(func.__name__.split(".")[0])
            return func(*args, **(kwargs or {}))

    B, Hq, Hkv, S, D = 1, 4, 2, 64, 64
    q, k, v = (meta(B, h, S, D, grad=m) for h, m in zip((Hq, Hkv, Hkv), mask))
    o, _, _ = torch.ops.co_alibi.fwd(q, k, v, meta(Hq), True, 0.125, True)
    with Record() as rec:
        o.float().sum().backward()
    assert rec.ops == (["bwd_dq"] if mask == (True, False, False) else ["bwd"])
    for t, m in zip((q, k, v), mask):
        assert (t.grad is not None) == m


def test_inference_forward_has_no_backward():
    q = meta(1, 2, 32, 64, grad=True)
    o, _, _ = torch.ops.co_alibi.fwd(q, meta(1, 2, 32, 64), meta(1, 2, 32, 64), meta(2), True, 0.125, False)
    with pytest.raises(RuntimeError, match="with_stats=False"):
        o.float().sum().backward()


def test_bwd_and_decode_fake_shapes():
    q, k = meta(2, 8, 50, 128, dtype=torch.bfloat16), meta(2, 2, 70, 128, dtype=torch.bfloat16)
    dq, dk, dv = torch.ops.co_alibi.bwd(q, q, k, k, q, meta(2, 8, 50, dtype=torch.float32),
                                        meta(ops.stats_numel(2, 8, 50, 70), dtype=torch.float32),
                                        meta(8, dtype=torch.bfloat16), True, 0.1)
    assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == k.shape and dq.dtype == torch.bfloat16
    qd, cache = meta(3, 16, 1, 64), meta(3, 4, 1000, 64)
    o, lse = torch.ops.co_alibi.decode(qd, cache, cache, meta(16), None, 700, 0.125, True)
    assert o.shape == qd.shape and lse.shape == (3, 16, 1) and lse.dtype == torch.float32
    o, lse = torch.ops.co_alibi.decode(qd, cache, cache, meta(16), meta(3, dtype=torch.int32), 700, 0.125, False)
    assert o.shape == qd.shape and lse.numel() == 0


def test_public_functions_trace_under_fake_tensors():
    """co_alibi_attention and co_alibi_decode run their checks and reach the operators'
    fake implementations with CUDA fake tensors (shape propagation as torch.compile does it)."""
    with FakeTensorMode(allow_non_fake_inputs=True):
        q = torch.empty(2, 12, 40, 64, device="cuda", dtype=torch.bfloat16)
        kv = torch.empty(2, 4, 40, 64, device="cuda", dtype=torch.bfloat16)
        o = co_alibi_attn.co_alibi_attention(q, kv, kv)
        assert o.shape == q.shape and o.dtype == torch.bfloat16 and o.device.type == "cuda"
        o, lse = co_alibi_attn.co_alibi_decode(q[:, :, :1], kv, kv, seq_len=30, return_lse=True)
        assert o.shape == (2, 12, 1, 64) and lse.shape == (2, 12, 1)
        with pytest.raises(AssertionError):  # 12 query heads cannot share 5 key heads
            co_alibi_attn.co_alibi_attention(q, kv[:, :1].expand(2, 5, 40, 64), kv[:, :1].expand(2, 5, 40, 64))


def test_slopes_are_kept_per_device_and_never_fake():
    """The device slopes are built once per (heads, bias_max, dtype, device), equal the
    reference formula rounded to the dtype (held in fp32, the kernels' form), and a FakeTensor
    made while tracing is not kept."""
    from co_alibi_attn.co_alibi_attn import _DEVICE_SLOPES, _device_slopes, _get_coalibi_slopes
    a = _device_slopes(12, 8.0, torch.bfloat16, torch.device("cpu"))
    assert a is _device_slopes(12, 8.0, torch.bfloat16, torch.device("cpu"))
    assert a.dtype == torch.float32
    assert torch.equal(a, (2.0 * _get_coalibi_slopes(12, 8.0)).to(torch.bfloat16).float())
    with FakeTensorMode(allow_non_fake_inputs=True):
        _device_slopes(6, 4.0, torch.float16, torch.device("cuda", 0))
    assert (6, 4.0, torch.float16, torch.device("cuda", 0)) not in _DEVICE_SLOPES
