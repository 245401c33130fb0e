"""Host-side behaviour that needs no GPU: the C ABI library, argument checks, the drop-in surface."""
import ctypes
import os
import re

import pytest
import torch

import co_alibi_attn
from co_alibi_attn import _native
from co_alibi_attn.co_alibi_attn import CoALIBIAttention, _get_coalibi_slopes

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "co_alibi.h")


def _declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:size_t|int|const char\*)\s+(co_alibi_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    declared = _declared_functions()
    assert declared, "no declarations parsed from include/co_alibi.h"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in co_alibi.h but not exported"
    assert sorted(_native.EXPORTS) == declared
    assert lib.co_alibi_abi_version() == _native.ABI_VERSION == 6


def test_sizes():
    lib = _native.lib()
    # stats: a 4-word header, then B*Hq * (ceil(Sq/128) kstart + ceil(Skv/256) key-norm chunks +
    # ceil(Sq/128) row order + ceil(Skv/64) key order + 2*Sq row sigmoid sums): O(B*Hq*S), no
    # per-block penalty sums
    assert lib.co_alibi_stats_numel(4, 16, 4096, 4096) == 4 + 4 * 16 * (32 + 16 + 32 + 64 + 2 * 4096)
    assert lib.co_alibi_stats_numel(1, 2, 5, 33) == 4 + 1 * 2 * (1 + 1 + 1 + 1 + 10)
    assert lib.co_alibi_stats_numel(1, 8, 65536, 65536) == 4 + 8 * (512 + 256 + 512 + 1024 + 2 * 65536)
    assert lib.co_alibi_stats_numel(0, 2, 5, 33) == 0
    # the recompute path's workspace: dO.O per row, then zb and cb (each 256-byte rounded)
    rows = 4 * 16 * 4096
    assert lib.co_alibi_bwd_workspace_bytes(4, 16, 4096, 4096) == rows * 4 + 2 * 4 * 16 * 128 * 4096 * 4
    assert lib.co_alibi_bwd_workspace_bytes(1, 1, 3, 3) == 256 + 2 * 256


def test_tail_skip_setting():
    """The library's tail-skip setting: on by default, returned by each set call, restored by the
    context manager (no GPU call is involved)."""
    lib = _native.lib()
    assert lib.co_alibi_tail_skip() == 1
    assert lib.co_alibi_set_tail_skip(0) == 1
    assert lib.co_alibi_tail_skip() == 0
    assert lib.co_alibi_set_tail_skip(5) == 0  # any non-zero value turns it on
    assert lib.co_alibi_tail_skip() == 1
    with _native.tail_skip(False):
        assert lib.co_alibi_tail_skip() == 0
        with _native.tail_skip(True):
            assert lib.co_alibi_tail_skip() == 1
        assert lib.co_alibi_tail_skip() == 0
    assert lib.co_alibi_tail_skip() == 1


def test_score_store_sizes():
    """The score store: 4 KB per (32-key block, 32-row block) that can hold a visible pair,
    after the per-row dO.O floats; only fp16 / bf16 at head dims 64 and 128 have it."""
    lib = _native.lib()
    f16, bf16, f32 = 1, 2, 0
    rows = 4 * 16 * 4096
    tri = 128 * 129 // 2  # causal: blocks (jb, qb) with qb >= jb of 128 x 128
    assert lib.co_alibi_bwd_score_store_workspace_bytes(f16, 4, 16, 16, 4096, 4096, 128, 1) == rows * 4 + 64 * tri * 4096
    assert lib.co_alibi_bwd_score_store_workspace_bytes(bf16, 4, 16, 4, 4096, 4096, 64, 0) == rows * 4 + 64 * 128 * 128 * 4096
    # rectangular causal (top-left): Skv > Sq leaves key blocks past the last row block out
    assert lib.co_alibi_bwd_score_store_workspace_bytes(f16, 1, 1, 1, 64, 1000, 64, 1) == 256 + 3 * 4096
    # Sq > Skv: every key block, rows from its own block down
    assert lib.co_alibi_bwd_score_store_workspace_bytes(f16, 1, 1, 1, 100, 40, 64, 1) == 512 + (4 + 3) * 4096
    for dtype, d in ((f32, 128), (f16, 32), (f16, 256), (bf16, 16)):
        assert lib.co_alibi_bwd_score_store_workspace_bytes(dtype, 1, 2, 2, 64, 64, d, 1) == 0
    assert lib.co_alibi_bwd_score_store_workspace_bytes(f16, 0, 2, 2, 64, 64, 64, 1) == 0
    # pass 2 keeps a processed bit per 128-row block of each grouped head: at most 256 heads
    # per key head x 8192 rows (or fewer heads x more rows)
    assert lib.co_alibi_bwd_score_store_workspace_bytes(f16, 1, 256, 1, 8192, 64, 64, 1) > 0
    assert lib.co_alibi_bwd_score_store_workspace_bytes(f16, 1, 256, 1, 8193, 64, 64, 1) == 0
    assert lib.co_alibi_bwd_score_store_workspace_bytes(f16, 1, 32, 1, 65536, 64, 64, 1) > 0
    assert lib.co_alibi_bwd_score_store_workspace_bytes(f16, 1, 32, 1, 65537, 64, 64, 1) == 0


def _fwd(lib, **over):
    args = dict(dtype=1, q=16, k=16, v=16, slopes=16, o=16, lse=16, stats=16, B=1, Hq=2, Hkv=2, Sq=8, Skv=8,
                D=64, causal=1, scale=0.125)
    args.update(over)
    return lib.co_alibi_fwd(args["dtype"], args["q"], args["k"], args["v"], args["slopes"], args["o"],
                            args["lse"], args["stats"], args["B"], args["Hq"], args["Hkv"], args["Sq"],
                            args["Skv"], args["D"], args["causal"], args["scale"], None)


@pytest.mark.parametrize("over,code,msg", [
    (dict(q=None), 1, "q is NULL"),
    (dict(k=24), 1, "k is not 16-byte aligned"),
    (dict(lse=2), 1, "lse is not 4-byte aligned"),
    (dict(D=96), 2, "head_dim must be 16, 32, 64, 128 or 256"),
    (dict(D=8), 2, "head_dim must be 16, 32, 64, 128 or 256"),
    (dict(dtype=7), 2, "dtype must be"),
    (dict(Hq=3, Hkv=2), 1, "multiple of heads_kv"),
    (dict(Sq=0), 1, ">= 1"),
    (dict(scale=float("nan")), 1, "sm_scale must be finite"),
])
def test_fwd_argument_errors(over, code, msg):
    lib = _native.lib()
    assert _fwd(lib, **over) == code
    assert msg in lib.co_alibi_last_error().decode()


def test_fwd_inference_workspace():
    """co_alibi_fwd_inference: its scratch is the key-norm chunk maxima (B*Hq*ceil(Skv/256) floats)
    and the row-block work order (B*Hq*ceil(Sq/128) ints), 256-byte rounded, and a smaller or
    misaligned workspace is rejected before any launch."""
    lib = _native.lib()
    assert lib.co_alibi_fwd_inference_workspace_bytes(4, 16, 4096, 4096) == 4 * 16 * (16 + 32) * 4
    assert lib.co_alibi_fwd_inference_workspace_bytes(1, 3, 300, 300) == 256
    assert lib.co_alibi_fwd_inference_workspace_bytes(1, 3, 70000, 300) == 3 * (547 + 2) * 4 // 256 * 256 + 256
    assert lib.co_alibi_fwd_inference_workspace_bytes(0, 3, 300, 300) == 0
    assert lib.co_alibi_fwd_inference_workspace_bytes(1, 3, 0, 300) == 0
    P = 256
    rc = lib.co_alibi_fwd_inference(1, P, P, P, P, P, P, 0, 1, 2, 2, 8, 8, 64, 1, 0.125, None)
    assert rc == 1 and "workspace of 0 bytes, need 256" in lib.co_alibi_last_error().decode()
    rc = lib.co_alibi_fwd_inference(1, P, P, P, P, P, 16, 1 << 20, 1, 2, 2, 8, 8, 64, 1, 0.125, None)
    assert rc == 1 and "workspace" in lib.co_alibi_last_error().decode()
    rc = lib.co_alibi_fwd_inference(1, P, P, P, P, P, P, 1 << 20, 1, 2, 2, 8, 8, 48, 1, 0.125, None)
    assert rc == 2 and "head_dim" in lib.co_alibi_last_error().decode()


def test_bwd_argument_errors():
    lib = _native.lib()
    P = 256
    rc = lib.co_alibi_bwd(1, P, P, P, P, P, P, P, P, P, P, P, P, 0, 1, 2, 2, 8, 8, 64, 1, 0.125, None)
    assert rc == 1 and "workspace of 0 bytes" in lib.co_alibi_last_error().decode()
    rc = lib.co_alibi_bwd_dkdv(1, P, P, P, P, P, P, P, None, P, P, 1 << 20, 1, 2, 2, 8, 8, 64, 1, 0.125, None)
    assert rc == 1 and "dk is NULL" in lib.co_alibi_last_error().decode()
    # pass 1 does not need dk / dv
    rc = lib.co_alibi_bwd_dq(1, P, P, P, P, P, P, P, P, None, P, 1 << 20, 1, 2, 2, 8, 8, 64, 1, 0.125, None)
    assert rc == 1 and "dq is NULL" in lib.co_alibi_last_error().decode()


def test_public_surface_matches_reference():
    # the reference package exports exactly co_alibi_attention; the decode step is an addition
    assert co_alibi_attn.__all__ == ["co_alibi_attention", "co_alibi_decode"]
    import inspect
    sig = inspect.signature(co_alibi_attn.co_alibi_attention)
    assert list(sig.parameters) == ["q", "k", "v", "causal", "sm_scale", "bias_max"]
    assert sig.parameters["causal"].default is True
    assert sig.parameters["sm_scale"].default is None
    assert sig.parameters["bias_max"].default == 8.0


def test_cpu_tensors_rejected_like_reference():
    q = torch.randn(1, 2, 8, 64)
    with pytest.raises(AssertionError, match="CUDA"):
        co_alibi_attn.co_alibi_attention(q, q, q)


def test_shape_asserts():
    q = torch.randn(1, 4, 8, 64)
    k = torch.randn(1, 3, 8, 64)  # 4 query heads cannot share 3 key heads
    with pytest.raises(AssertionError):
        co_alibi_attn.co_alibi_attention(q, k, k)
    with pytest.raises(AssertionError):
        CoALIBIAttention.apply(q, q, q, torch.ones(3), True, 0.1)  # slope count


def test_slopes_dtype_rounding():
    s16 = (2.0 * _get_coalibi_slopes(16)).to(torch.float16)
    # 2^(0.5 - h/2): odd h are exact powers of two, even h round in fp16
    assert s16[1].item() == 1.0 and s16[15].item() == 2.0 ** -7
    assert abs(s16[0].item() - 2 ** 0.5) < 2 ** 0.5 * 2 ** -11


def test_decode_sizes():
    lib = _native.lib()
    # min(ceil(L / 128), 1024) splits; per (b, h, split): max, sum, sigma total (each array
    # 256-byte padded) + D floats
    parts = 2 * 32 * 128  # B=2, Hq=32, 16384 keys
    assert lib.co_alibi_decode_workspace_bytes(2, 32, 16384, 128) == 3 * parts * 4 + parts * 128 * 4
    assert lib.co_alibi_decode_workspace_bytes(1, 1, 257, 64) == 3 * 256 + 3 * 64 * 4
    parts = 1024  # 2^21 keys: 16384 chunks, at most 1024 splits
    assert lib.co_alibi_decode_workspace_bytes(1, 1, 1 << 21, 64) == 3 * parts * 4 + parts * 64 * 4
    assert lib.co_alibi_decode_workspace_bytes(1, 1, 0, 64) == 0


def _decode(lib, **over):
    args = dict(dtype=1, q=256, k=256, v=256, slopes=256, lens=None, o=256, lse=None, ws=256, ws_bytes=1 << 20, B=1, Hq=8,
                Hkv=2, L=300, cap=512, D=128, scale=0.125)
    args.update(over)
    return lib.co_alibi_decode(args["dtype"], args["q"], args["k"], args["v"], args["slopes"], args["lens"],
                               args["o"], args["lse"], args["ws"], args["ws_bytes"], args["B"], args["Hq"],
                               args["Hkv"], args["L"], args["cap"], args["D"], args["scale"], None)


@pytest.mark.parametrize("over,code,msg", [
    (dict(k=None), 1, "k_cache is NULL"),
    (dict(lens=2), 1, "seq_lens is not 4-byte aligned"),
    (dict(v=8), 1, "v_cache is not 16-byte aligned"),
    (dict(ws=16), 1, "workspace is not 256-byte aligned"),
    (dict(ws_bytes=1000), 1, "workspace of 1000 bytes"),
    (dict(cap=299), 1, "kv_capacity is below seq_kv"),
    (dict(L=(1 << 21) + 1, cap=1 << 22), 1, "seq_kv above 2097152"),
    (dict(Hq=66, Hkv=1), 2, "at most 32 query heads per kv head"),
    (dict(Hq=6, Hkv=4), 1, "multiple of heads_kv"),
    (dict(D=80), 2, "head_dim must be 16, 32, 64, 128 or 256"),
    (dict(D=16), 2, "head_dim 16 has no decode kernel"),
    (dict(D=256, dtype=0), 2, "decode at head_dim 256 needs fp16 or bf16"),
    (dict(L=0), 1, ">= 1"),
    (dict(scale=float("inf")), 1, "sm_scale must be finite"),
])
def test_decode_argument_errors(over, code, msg):
    lib = _native.lib()
    assert _decode(lib, **over) == code
    assert msg in lib.co_alibi_last_error().decode()


def test_decode_python_checks():
    q = torch.randn(1, 4, 2, 64)
    kc = torch.randn(1, 2, 16, 64)
    with pytest.raises(ValueError, match=r"\(B, Hq, 1, D\)"):
        co_alibi_attn.co_alibi_decode(q, kc, kc)
    with pytest.raises(AssertionError, match="CUDA"):
        co_alibi_attn.co_alibi_decode(q[:, :, :1], kc, kc)
    with pytest.raises(AssertionError):
        co_alibi_attn.co_alibi_decode(q[:, :, :1], kc, kc[:, :, :8])
