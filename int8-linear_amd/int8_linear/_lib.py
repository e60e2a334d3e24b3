"""Loader of the gfx950 C-ABI library (libint8_linear_amd.so, declared in
include/int8_linear_amd.h) and the mapping of its status codes to Python exceptions.

There is no CPU or Python fallback: if the library is missing, every entry point raises.
torch is imported first so that the library binds to the HIP runtime torch already loaded
(one runtime per process, so torch's streams and device pointers are valid here).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("libint8_linear_amd.so")

OK, UNSUPPORTED, INVALID_ARG, HIP_ERROR = 0, 1, 2, 3
DTYPE_NONE, BF16, F16, F32, I32 = 0, 1, 2, 3, 4
DTYPE_CODE = {torch.bfloat16: BF16, torch.float16: F16, torch.float32: F32, torch.int32: I32}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32


class CConfig(ctypes.Structure):
    """struct i8l_config (include/int8_linear_amd.h)."""
    _fields_ = [("bm", _I32), ("bn", _I32), ("bk", _I32), ("warps", _I32), ("stages", _I32),
                ("group_m", _I32)]


EXPORTS = ("i8l_w8a8_mm", "i8l_w8a8_mm_supported", "i8l_default_config",
           "i8l_add_rmsnorm_quant", "i8l_silu_mul_quant", "i8l_quant_per_token",
           "i8l_w8a8_mm_dynq", "i8l_w8a8_mm_dynq_supported",
           "i8l_silu_mul_quant_mm", "i8l_silu_mul_quant_mm_supported", "i8l_w8a8_mm_ws",
           "i8l_w8a8_mm_workspace_bytes", "i8l_w8a8_mm_noalloc", "i8l_init",
           "i8l_add_rmsnorm_quant_mm", "i8l_add_rmsnorm_quant_mm_supported",
           "i8l_w8a8_mm_silu_mul", "i8l_w8a8_mm_silu_mul_supported", "i8l_last_error",
           "i8l_version")

_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library with its argument types declared (loaded once)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python int8-linear_amd/build_lib.py` "
            "(there is no fallback path)")
    L = ctypes.CDLL(str(LIB_PATH))
    L.i8l_w8a8_mm.argtypes = [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _P, _I64, _P, _I32,
                              _P, _I64, _I32, _I64, _I64, _I64, ctypes.POINTER(CConfig), _P]
    L.i8l_w8a8_mm_supported.argtypes = [_I64, _I64, _I64, ctypes.POINTER(CConfig)]
    L.i8l_default_config.argtypes = [_I64, _I64, _I64, ctypes.POINTER(CConfig)]
    L.i8l_add_rmsnorm_quant.argtypes = [_P, _P, _P, ctypes.c_float, _P, _P, _P, _I64, _I64, _I32,
                                        _I32, _I32, _P]
    L.i8l_silu_mul_quant.argtypes = [_P, _P, _P, _I64, _I64, _I32, _I32, _I32, _P]
    L.i8l_quant_per_token.argtypes = [_P, _I64, _P, _P, _I64, _I64, _I32, _I32, _P]
    L.i8l_w8a8_mm_dynq.argtypes = [_P, _I64, _I32, _I32, _P, _I64, _I64, _P, _I64, _P, _I32,
                                   _P, _I64, _I32, _P, _I64, _I64, _I64,
                                   ctypes.POINTER(CConfig), _P]
    L.i8l_w8a8_mm_dynq_supported.argtypes = [_I64, _I64, _I64, ctypes.POINTER(CConfig)]
    L.i8l_silu_mul_quant_mm.argtypes = [_P, _I64, _I32, _I32, _I32, _P, _I64, _I64, _P, _I64,
                                        _P, _I32, _P, _I64, _I32, _P, _I64, _I64, _I64,
                                        ctypes.POINTER(CConfig), _P]
    L.i8l_silu_mul_quant_mm_supported.argtypes = [_I64, _I64, _I64, ctypes.POINTER(CConfig)]
    L.i8l_w8a8_mm_ws.argtypes = L.i8l_w8a8_mm.argtypes[:-2] + [_P, _I64] + \
        L.i8l_w8a8_mm.argtypes[-2:]
    L.i8l_w8a8_mm_workspace_bytes.argtypes = [_I64, _I64, _I64, ctypes.POINTER(CConfig)]
    L.i8l_w8a8_mm_noalloc.argtypes = L.i8l_w8a8_mm.argtypes
    L.i8l_init.argtypes = [_I32]
    L.i8l_add_rmsnorm_quant_mm.argtypes = [_P, _P, _P, ctypes.c_float, _I32, _I32, _I32, _P, _P,
                                           _I64, _I64, _P, _I64, _P, _I32, _P, _I64, _I32, _P,
                                           _I64, _I64, _I64, ctypes.POINTER(CConfig), _P]
    L.i8l_add_rmsnorm_quant_mm_supported.argtypes = [_I64, _I64, _I64, ctypes.POINTER(CConfig)]
    L.i8l_w8a8_mm_silu_mul.argtypes = [_P, _I64, _P, _I64, _I64, _P, _I64, _P, _I64, _P, _I32,
                                       _P, _I64, _I32, _I64, _I64, _I64,
                                       ctypes.POINTER(CConfig), _P]
    L.i8l_w8a8_mm_silu_mul_supported.argtypes = [_I64, _I64, _I64, ctypes.POINTER(CConfig)]
    for name in EXPORTS[:-2]:
        getattr(L, name).restype = ctypes.c_int
    L.i8l_w8a8_mm_workspace_bytes.restype = _I64
    L.i8l_last_error.restype = ctypes.c_char_p
    L.i8l_version.restype = ctypes.c_char_p
    _lib = L
    return L


FAST_NAME = "_i8l_fast"
_fast_mod = None
_fast_checked = False


def fast():
    """The C++ eager binding over this library (csrc/i8l_torch.cpp), or None when it is not
    built, in which case every call goes through ctypes.  It launches the same kernels
    through the same entry points; a binding that is built but does not import raises."""
    global _fast_mod, _fast_checked
    if not _fast_checked:
        lib()
        if any(LIB_PATH.parent.glob(FAST_NAME + ".*.so")):
            import importlib
            _fast_mod = importlib.import_module("int8_linear." + FAST_NAME)
        _fast_checked = True
    return _fast_mod


def last_error() -> str:
    return lib().i8l_last_error().decode(errors="replace")


def check(status: int, not_supported: type[Exception]) -> None:
    """Raise the reference's exception for a non-zero status."""
    if status == OK:
        return
    msg = last_error()
    if status == UNSUPPORTED:
        raise not_supported(msg)
    if status == INVALID_ARG:
        raise ValueError(msg)
    raise RuntimeError(f"int8_linear_amd: {msg}")


def stream_of(t: torch.Tensor) -> int:
    """The caller's current HIP stream on t's device (what the launch is queued on)."""
    return torch.cuda.current_stream(t.device).cuda_stream
