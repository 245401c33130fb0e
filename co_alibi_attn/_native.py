"""ctypes binding of the C ABI in ``include/co_alibi.h``.

The library is loaded after ``torch`` so that it shares torch's HIP runtime
(both carry the soname ``libamdhip64.so.7``; the already-loaded one is reused).
There is no fallback: if the library is missing, every call raises.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must be imported before the HIP library is loaded)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libco_alibi.so")

DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
SUPPORTED_HEAD_DIMS = (16, 32, 64, 128, 256)

ABI_VERSION = 6

# Size of the library-held split-K scratch of co_alibi_decode_noalloc (CO_ALIBI_DECODE_SCRATCH_BYTES).
DECODE_SCRATCH_BYTES = 32 << 20

# Symbols declared in include/co_alibi.h.
EXPORTS = (
    "co_alibi_stats_numel",
    "co_alibi_set_tail_skip",
    "co_alibi_tail_skip",
    "co_alibi_bwd_workspace_bytes",
    "co_alibi_bwd_score_store_workspace_bytes",
    "co_alibi_fwd",
    "co_alibi_fwd_inference_workspace_bytes",
    "co_alibi_fwd_inference",
    "co_alibi_bwd",
    "co_alibi_bwd_dq",
    "co_alibi_bwd_dkdv",
    "co_alibi_decode_workspace_bytes",
    "co_alibi_decode",
    "co_alibi_decode_noalloc",
    "co_alibi_probe_mfma",
    "co_alibi_last_error",
    "co_alibi_abi_version",
)

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_Z = ctypes.c_size_t

_SIGNATURES = {
    "co_alibi_stats_numel": (_Z, [_I, _I, _I, _I]),
    "co_alibi_set_tail_skip": (_I, [_I]),
    "co_alibi_tail_skip": (_I, []),
    "co_alibi_bwd_workspace_bytes": (_Z, [_I, _I, _I, _I]),
    "co_alibi_bwd_score_store_workspace_bytes": (_Z, [_I, _I, _I, _I, _I, _I, _I, _I]),
    "co_alibi_fwd": (_I, [_I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _P]),
    "co_alibi_fwd_inference_workspace_bytes": (_Z, [_I, _I, _I, _I]),
    "co_alibi_fwd_inference": (_I, [_I, _P, _P, _P, _P, _P, _P, _Z, _I, _I, _I, _I, _I, _I, _I, _F, _P]),
    "co_alibi_bwd": (
        _I,
        [_I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _Z, _I, _I, _I, _I, _I, _I, _I, _F, _P],
    ),
    "co_alibi_bwd_dq": (
        _I,
        [_I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _Z, _I, _I, _I, _I, _I, _I, _I, _F, _P],
    ),
    "co_alibi_bwd_dkdv": (
        _I,
        [_I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _Z, _I, _I, _I, _I, _I, _I, _I, _F, _P],
    ),
    "co_alibi_decode_workspace_bytes": (_Z, [_I, _I, _I, _I]),
    "co_alibi_decode": (_I, [_I, _P, _P, _P, _P, _P, _P, _P, _P, _Z, _I, _I, _I, _I, _I, _I, _F, _P]),
    "co_alibi_decode_noalloc": (_I, [_I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P]),
    "co_alibi_probe_mfma": (_I, [_P, _P, _I, _I, _P]),
    "co_alibi_last_error": (ctypes.c_char_p, []),
    "co_alibi_abi_version": (_I, []),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Load (once) and return the native library, or raise if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"co_alibi_attn: native library {LIB_PATH} is not built; "
                "run `python -m co_alibi_attn._build`"
            )
        handle = ctypes.CDLL(LIB_PATH)
        # The version first: a library of another ABI may lack some of the symbols below.
        handle.co_alibi_abi_version.restype = ctypes.c_int
        handle.co_alibi_abi_version.argtypes = []
        if handle.co_alibi_abi_version() != ABI_VERSION:
            raise RuntimeError("co_alibi_attn: native library ABI version mismatch; "
                               "run `python -m co_alibi_attn._build`")
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


class tail_skip:
    """Context manager over the library's tail-skip setting (co_alibi_set_tail_skip): within
    ``with tail_skip(False):`` every forward processes every key, as the reference does; the
    previous setting comes back on exit."""

    def __init__(self, enabled: bool):
        self.enabled = bool(enabled)
        self.prev = None

    def __enter__(self):
        self.prev = lib().co_alibi_set_tail_skip(int(self.enabled))
        return self

    def __exit__(self, *exc):
        lib().co_alibi_set_tail_skip(self.prev)
        return False


def check(rc: int) -> None:
    """Raise RuntimeError with the library's message for a non-zero status."""
    if rc != 0:
        msg = lib().co_alibi_last_error().decode("utf-8", "replace")
        raise RuntimeError(f"co_alibi_attn: {msg} (status {rc})")
