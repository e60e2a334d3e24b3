"""numpy front end of the CPU oracle (oracle/_build/liboracle.so) -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module,
and only as the checker.  Every function restates a step of the reference's arithmetic
(AshrithaG/int8-linear); the C source names the file:line each one follows, and
tests/test_oracle.py pins each against mathematics independent of the restatement.

Activations, bias and 16-bit outputs travel as their raw bit patterns (numpy uint16).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

SO = Path(__file__).resolve().parent / "_build" / "liboracle.so"
BF16, F16, F32, I32 = 1, 2, 3, 4
NONE = 0

_lib = None
_P = ctypes.c_void_p
_I = ctypes.c_int64
_C = ctypes.c_int


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not SO.exists():
            raise RuntimeError(f"{SO} is not built: run python oracle/build_oracle.py")
        L = ctypes.CDLL(str(SO))
        L.or_gemm_i32.argtypes = [_P, _I, _I, _P, _I, _I, _P, _I, _I, _I]
        L.or_epilogue.argtypes = [_P, _I, _I, _P, _I, _P, _I, _P, _C, _P, _C]
        L.or_quantize_row.argtypes = [_P, _I, _C, _P, _P]
        L.or_add_rmsnorm_quant.argtypes = [_P, _P, _P, ctypes.c_float, _P, _P, _P, _I, _I, _C,
                                           _C, _C]
        L.or_silu_mul_quant.argtypes = [_P, _P, _P, _I, _I, _C, _C, _C]
        L.or_quant_per_token.argtypes = [_P, _P, _P, _I, _I, _C, _C]
        L.or_quant_rows_div.argtypes = [_P, _C, _P, _P, _I, _I]
        for name in ("or_expf_n", "or_rsqrtf_n", "or_f32_to_bf16_n", "or_f32_to_f16_n",
                     "or_f16_to_f32_n"):
            getattr(L, name).argtypes = [_P, _P, _I]
        for name in ("or_gemm_i32", "or_epilogue", "or_quantize_row", "or_add_rmsnorm_quant",
                     "or_silu_mul_quant", "or_quant_per_token", "or_quant_rows_div"):
            getattr(L, name).restype = None
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ------------------------------------------------------------------------ conversions
def f32_to_bf16(x) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().or_f32_to_bf16_n(_p(x), _p(y), x.size)
    return y


def bf16_to_f32(h) -> np.ndarray:
    return (_c(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_f16(x) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().or_f32_to_f16_n(_p(x), _p(y), x.size)
    return y


def f16_to_f32(h) -> np.ndarray:
    h = _c(h, np.uint16)
    y = np.empty(h.shape, np.float32)
    lib().or_f16_to_f32_n(_p(h), _p(y), h.size)
    return y


def act_to_f32(h, dt: int) -> np.ndarray:
    return bf16_to_f32(h) if dt == BF16 else f16_to_f32(h)


def expf(x) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().or_expf_n(_p(x), _p(y), x.size)
    return y


def rsqrtf(x) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().or_rsqrtf_n(_p(x), _p(y), x.size)
    return y


# ------------------------------------------------------------------------ GEMM
def gemm_i32(a: np.ndarray, b_nk: np.ndarray) -> np.ndarray:
    """Exact int32 A[M,K] @ W[N,K]^T."""
    a, b = _c(a, np.int8), _c(b_nk, np.int8)
    M, K = a.shape
    N = b.shape[0]
    acc = np.empty((M, N), np.int32)
    lib().or_gemm_i32(_p(a), K, 1, _p(b), 1, K, _p(acc), M, N, K)
    return acc


def gemm_i32_strided(a_buf: np.ndarray, sam: int, sak: int, b_buf: np.ndarray, sbk: int,
                     sbn: int, M: int, N: int, K: int) -> np.ndarray:
    """Exact product with arbitrary element strides into flat int8 buffers."""
    a_buf, b_buf = _c(a_buf, np.int8), _c(b_buf, np.int8)
    acc = np.empty((M, N), np.int32)
    lib().or_gemm_i32(_p(a_buf), sam, sak, _p(b_buf), sbk, sbn, _p(acc), M, N, K)
    return acc


def epilogue(acc: np.ndarray, sa: np.ndarray, sb: np.ndarray, bias: np.ndarray | None,
             bias_dt: int, out_dt: int) -> np.ndarray:
    """Scaled output: uint16 bit patterns for BF16/F16, float32 for F32, int32 for I32."""
    acc = _c(acc, np.int32)
    M, N = acc.shape
    sa, sb = _c(sa, np.float32).reshape(-1), _c(sb, np.float32).reshape(-1)
    if bias is not None:
        bias = _c(bias, np.float32 if bias_dt == F32 else np.uint16).reshape(-1)
    else:
        bias_dt = NONE
    out = np.empty((M, N), {BF16: np.uint16, F16: np.uint16, F32: np.float32,
                            I32: np.int32}[out_dt])
    lib().or_epilogue(_p(acc), M, N, _p(sa), sa.size, _p(sb), sb.size, _p(bias), bias_dt,
                      _p(out), out_dt)
    return out


def w8a8_mm(a: np.ndarray, b_nk: np.ndarray, sa, sb, bias=None, bias_dt: int = NONE,
            out_dt: int = BF16) -> np.ndarray:
    """The reference's CPU path of one linear: exact int32 product, then the epilogue."""
    return epilogue(gemm_i32(a, b_nk), sa, sb, bias, bias_dt, out_dt)


# ------------------------------------------------------------------------ quantizers
def quantize_row(y, precise_div: bool = True) -> tuple[np.ndarray, np.float32]:
    y = _c(y, np.float32).reshape(-1)
    q = np.empty(y.size, np.int8)
    s = np.empty(1, np.float32)
    lib().or_quantize_row(_p(y), y.size, int(precise_div), _p(q), _p(s))
    return q, s[0]


def add_rmsnorm_quant(x: np.ndarray, residual: np.ndarray | None, weight: np.ndarray,
                      eps: float, act_dt: int = BF16, w_dt: int = BF16,
                      precise_div: bool = True):
    """(q int8 [M,H], scale float32 [M,1], residual_out uint16 [M,H] or None)."""
    x = _c(x, np.uint16)
    M, H = x.shape
    r = None if residual is None else _c(residual, np.uint16)
    w = _c(weight, np.uint16)
    q = np.empty((M, H), np.int8)
    s = np.empty((M, 1), np.float32)
    rout = None if r is None else np.empty((M, H), np.uint16)
    lib().or_add_rmsnorm_quant(_p(x), _p(r), _p(w), ctypes.c_float(eps), _p(q), _p(s), _p(rout),
                               M, H, act_dt, w_dt, int(precise_div))
    return q, s, rout


def silu_mul_quant(gate_up: np.ndarray, act_dt: int = BF16, round_silu: bool = False,
                   precise_div: bool = True):
    gu = _c(gate_up, np.uint16)
    M, I2 = gu.shape
    I = I2 // 2
    q = np.empty((M, I), np.int8)
    s = np.empty((M, 1), np.float32)
    lib().or_silu_mul_quant(_p(gu), _p(q), _p(s), M, I, act_dt, int(round_silu),
                            int(precise_div))
    return q, s


def quant_per_token(x: np.ndarray, act_dt: int = BF16, precise_div: bool = True):
    x = _c(x, np.uint16)
    M, H = x.shape
    q = np.empty((M, H), np.int8)
    s = np.empty((M, 1), np.float32)
    lib().or_quant_per_token(_p(x), _p(q), _p(s), M, H, act_dt, int(precise_div))
    return q, s


def quant_rows_div(x: np.ndarray, dt: int = BF16):
    """bench/bench_linear.py:146-150: (q int8 [R,C] in [-127,127], scale float32 [R,1])."""
    x = _c(x, np.uint16)
    R, C = x.shape
    q = np.empty((R, C), np.int8)
    s = np.empty((R, 1), np.float32)
    lib().or_quant_rows_div(_p(x), dt, _p(q), _p(s), R, C)
    return q, s
