"""Loader for libskv.so, the C ABI over the gfx950 HIP kernels (include/skv.h).

torch is imported first on purpose: torch ships its own libamdhip64.so.7,
and loading it before libskv.so makes the library bind to that same HIP
runtime, so torch's streams and device pointers are valid on both sides.

There is no fallback: if the library is missing the import of any op fails
with a RuntimeError that says how to build it.
"""
from __future__ import annotations

import ctypes
import os
import re

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_ROOT, "libskv.so")
HEADER_PATH = os.path.join(os.path.dirname(PKG_ROOT), "include", "skv.h")

F32, BF16 = 0, 1
SKV_E_INVALID, SKV_E_UNSUPPORTED, SKV_E_WORKSPACE, SKV_E_HIP = -22, -95, -28, -5

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_Z = ctypes.c_size_t

# name -> (restype, argtypes); every function declared in include/skv.h
_SIGNATURES = {
    "skv_last_error": (ctypes.c_char_p, []),
    "skv_version": (_I, []),
    "skv_append": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "skv_append_paged": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "skv_append_chunk": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "skv_advance": (_I, [_P, _P, _I, _I, _I, _P]),
    "skv_decode_plan": (_I, [_I, _I, _I, _I, _I, _I, ctypes.c_longlong, _I, ctypes.POINTER(_I),
                                 ctypes.POINTER(_I)]),
    "skv_decode_workspace_bytes": (_Z, [_I, _I, _I, _I]),
    "skv_prefill_plan": (_I, [_I, _I, _I, _I, _I, ctypes.POINTER(_I)]),
    "skv_prefill_workspace_bytes": (_Z, [_I, _I, _I, _I, _I]),
    "skv_prefill_attn": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I, _P, _Z,
                              _I, _I, _I, _P]),
    "skv_append_prefill_attn": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I,
                                     _F, _I, _P, _Z, _I, _I, _I, _I, _P]),
    "skv_embed": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "skv_layernorm": (_I, [_P, _P, _P, _P, _I, _I, _F, _P]),
    "skv_linear": (_I, [_P, _P, _P, _P, _P, _P, _P, _F, _I, _I, _I, _I, _I, _P, _Z, _P]),
    "skv_linear_workspace_bytes": (_Z, [_I, _I, _I]),
    "skv_linear_fold_ln": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _P]),
    "skv_linear_folded": (_I, [_P, _P, _P, _P, _P, _P, _F, _I, _I, _I, _I, _I, _P]),
    "skv_linear_packed_bytes": (_Z, [_I, _I]),
    "skv_linear_pack": (_I, [_P, _P, _I, _I, _P]),
    "skv_linear_packed": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P]),
    "skv_linear_packed_cand_bytes": (_Z, [_I]),
    "skv_append_decode_attn_direct": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I,
                                           _I, _I, _I, _I, _P, _Z, _P]),
    "skv_decode_direct_workspace_bytes": (_Z, [_I, _I, _I, _I]),
    "skv_linear_cand": (_I, [_P, _P, _P, _P, _I, _I, _I, _P, _P, _Z, _P]),
    "skv_linear_cand_bytes": (_Z, [_I, _I, _I]),
    "skv_next_embed": (_I, [_P, _P, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _P, _P, _I, _I, _I,
                            _P, _P, _I, _P, _P]),
    "skv_argmax_workspace_bytes": (_Z, [_I, _I]),
    "skv_argmax": (_I, [_P, _P, _I, _I, _P, _Z, _P]),
    "skv_sample": (_I, [_P, _P, _P, _P, _I, _P, _I, _I, _F, _I, _F, _F, _F, _I,
                        ctypes.c_ulonglong, _P, _Z, _P]),
    "skv_sample_workspace_bytes": (_Z, [_I, _I]),
    "skv_flash_fwd": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P]),
    "skv_flash_bwd_workspace_bytes": (_Z, [_I, _I, _I]),
    "skv_flash_bwd_fast_workspace_bytes": (_Z, [_I, _I, _I, _I]),
    "skv_flash_bwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P, _Z,
                           _P]),
    "skv_bpe_train": (_I, [_P, _Z, _I, _P, _I, ctypes.POINTER(_I)]),
    "skv_bpe_encode": (_I, [_P, _Z, _P, _I, _P, ctypes.POINTER(_Z)]),
    "skv_next_tokens": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _P, _P, _I, _P, _P]),
    "skv_gather_rows": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "skv_decode_attn": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _I, _P, _Z,
                             _I, _I, _I, _P]),
    "skv_append_decode_attn": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _I,
                                    _P, _Z, _I, _I, _I, _I, _P]),
    "skv_append_decode_attn_paged": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I,
                                          _I, _F, _I, _I, _P, _Z, _I, _I, _I, _I, _P]),
    "skv_decode_attn_paged": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I,
                                   _I, _P, _Z, _I, _I, _I, _P]),
    "skv_decode_attn_noalloc": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _I, _I, _I,
                                     _I, _P]),
}

_lib = None


class SkvError(RuntimeError):
    """A HIP-side failure reported by libskv (SKV_E_HIP)."""


def header_functions() -> list[str]:
    """Names of the functions include/skv.h declares."""
    with open(HEADER_PATH) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\**\s+\**(skv_[a-z0-9_]+)\s*\(",
                      text, flags=re.M)


def lib():
    """The loaded library; raises RuntimeError if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libskv.so not found at {LIB_PATH}; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` from the repo root")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    """Map a libskv status to the reference's exception types."""
    if rc == 0:
        return
    msg = lib().skv_last_error().decode(errors="replace") or what
    if rc in (SKV_E_INVALID, SKV_E_UNSUPPORTED, SKV_E_WORKSPACE):
        raise ValueError(msg)
    raise SkvError(f"{msg} (status {rc})")


_DTYPE_CODES = {torch.float32: F32, torch.bfloat16: BF16}


def dtype_code(dt: torch.dtype) -> int:
    code = _DTYPE_CODES.get(dt)
    if code is None:
        raise ValueError(f"unsupported dtype {dt} (float32 or bfloat16)")
    return code


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device | None = None) -> int:
    """hipStream_t of torch's current stream on `device`. The raw query
    (what torch's generated code calls) skips building a Stream object:
    0.3 instead of 2 us of host time per launch."""
    idx = device if isinstance(device, int) else getattr(device, "index", None)
    if _RAW_STREAM is not None and idx is not None and torch.cuda.is_initialized():
        return _RAW_STREAM(idx)
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor) -> int:
    return t.data_ptr()
