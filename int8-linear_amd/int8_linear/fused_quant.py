"""The activation quantizer fused into the kernel before it, as MI355X HIP kernels.

A W8A8 layer quantizes its input per token right before the matmul.  These kernels fold
that quantizer into the op that produces the input, one workgroup per token row:

    add_rmsnorm_quant(x, residual, w, eps) -> (x_q, scale, residual_out)
    rmsnorm_quant(x, w, eps)               -> (x_q, scale)
    silu_mul_quant(gate_up)                -> (x_q, scale)
    quant_per_token(x)                     -> (x_q, scale)
    quant_mm(x, b_q, scale_b)              -> w8a8_mm(*quant_per_token(x), b_q, ...)
    silu_mul_quant_mm(gate_up, b_q, ...)   -> w8a8_mm(*silu_mul_quant(gate_up), b_q, ...)

Same Python surface and arithmetic as the reference's int8_linear/fused_quant.py
(AshrithaG/int8-linear, 41-124): residual add and norm in fp32, the normalized value rounded
to the weight dtype, times the weight, rounded to the activation dtype; SiLU optionally
rounded before the multiply; then

    scale = absmax / 127,   x_q = round_half_even(x * (127 / absmax)), saturated

The sum of squares is a fixed pairwise tree in double, rsqrt is the correctly rounded
double result rounded to float, and exp is a fixed Cody-Waite/Taylor routine, so the CPU
oracle reproduces every code and scale bit for bit.  PRECISE_DIV=True selects IEEE
division (the reference default); False multiplies by the IEEE reciprocal instead.

Each is also a torch custom op, so torch.compile treats it as one opaque kernel.
"""

from __future__ import annotations

import torch

from int8_linear import _lib
from int8_linear.kernel import NotSupported, same_device

_ACT = {torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


def _fast(name: str, *args):
    """The call through the C++ binding, or None (not built, or not the plain case: the
    Python path below then handles it, with its own checks and errors)."""
    f = _lib.fast()
    if f is None:
        return None
    try:
        return getattr(f, name)(*args)
    except (TypeError, AttributeError):
        return None


def _act_code(t: torch.Tensor, what: str) -> int:
    code = _ACT.get(t.dtype)
    if code is None:
        raise NotSupported(f"{what} must be bfloat16 or float16, got {t.dtype}")
    if not t.is_cuda:
        raise NotSupported(f"{what} must be on a HIP device")
    return code


def add_rmsnorm_quant(x: torch.Tensor, residual: torch.Tensor | None, weight: torch.Tensor,
                      eps: float, precise_div: bool = True):
    """(x_q int8 [M, K], scale fp32 [M, 1], residual_out [M, K] or None)."""
    r = _fast("add_rmsnorm_quant", x, residual, weight, eps, precise_div)
    if r is not None:
        return r
    assert x.is_contiguous() and x.dim() == 2
    M, K = x.shape
    act = _act_code(x, "x")
    wcode = _act_code(weight, "weight")
    if weight.numel() != K:
        raise ValueError(f"weight has {weight.numel()} values for rows of {K}")
    weight = weight.contiguous()
    same_device(x.device, weight=weight, residual=residual)
    if residual is not None:
        assert residual.is_contiguous() and residual.shape == x.shape
        if residual.dtype != x.dtype:
            raise NotSupported("residual must have x's dtype")
    q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    s = torch.empty((M, 1), dtype=torch.float32, device=x.device)
    rout = torch.empty_like(x) if residual is not None else None
    if M:
        status = _lib.lib().i8l_add_rmsnorm_quant(
            x.data_ptr(), residual.data_ptr() if residual is not None else None,
            weight.data_ptr(), float(eps), q.data_ptr(), s.data_ptr(),
            rout.data_ptr() if rout is not None else None, M, K, act, wcode,
            int(bool(precise_div)), _lib.stream_of(x))
        _lib.check(status, NotSupported)
    return q, s, rout


def silu_mul_quant(gate_up: torch.Tensor, precise_div: bool = True, round_silu: bool = False):
    """silu(gate) * up, quantized: (x_q int8 [M, I], scale fp32 [M, 1])."""
    r = _fast("silu_mul_quant", gate_up, precise_div, round_silu)
    if r is not None:
        return r
    assert gate_up.is_contiguous() and gate_up.dim() == 2
    M, I2 = gate_up.shape
    I = I2 // 2
    act = _act_code(gate_up, "gate_up")
    q = torch.empty((M, I), dtype=torch.int8, device=gate_up.device)
    s = torch.empty((M, 1), dtype=torch.float32, device=gate_up.device)
    if M and I:
        status = _lib.lib().i8l_silu_mul_quant(
            gate_up.data_ptr(), q.data_ptr(), s.data_ptr(), M, I, act, int(bool(round_silu)),
            int(bool(precise_div)), _lib.stream_of(gate_up))
        _lib.check(status, NotSupported)
    return q, s


def quant_per_token(x: torch.Tensor, precise_div: bool = True):
    """Per-token int8 quantization of a bf16/fp16 [M, K] tensor: (x_q, scale fp32 [M, 1]).

    The quantizer of the two fused kernels on its own, with vLLM scaled_int8_quant's
    convention; it quantizes the o_proj input, which has no kernel before it to fuse into.
    x may be a column slice of a wider tensor (unit column stride, any row stride), such
    as the q columns of a qkv output: it is read in place, with no copy.
    """
    r = _fast("quant_per_token", x, precise_div)
    if r is not None:
        return r
    assert x.dim() == 2 and (x.stride(1) == 1 or x.shape[1] <= 1)
    M, K = x.shape
    act = _act_code(x, "x")
    q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    s = torch.empty((M, 1), dtype=torch.float32, device=x.device)
    if M and K:
        ldx = x.stride(0) if M > 1 else K
        status = _lib.lib().i8l_quant_per_token(x.data_ptr(), ldx, q.data_ptr(), s.data_ptr(), M,
                                                K, act, int(bool(precise_div)), _lib.stream_of(x))
        _lib.check(status, NotSupported)
    return q, s


# Largest M that quant_mm takes.  Every column tile quantizes the token rows itself, so the
# fused launch pays off only for few tokens: measured on MI355X (graph replay, cold weights),
# one launch vs quant_per_token + w8a8_mm is 3.73 vs 4.77 us at M = 1 and 4.01 vs 5.44 at
# M = 8 for K = N = 2048 (o_proj), 4.97 vs 6.84 at M = 1 and 7.40 vs 7.79 at M = 8 for
# K = 6144, N = 2048 (down_proj, whose 12-wave tile takes at most 8 rows).  The K = 2048 tile
# takes 16-row blocks, but past 8 tokens the fold gains little or loses (5.40 vs 5.54 us at
# M = 16, 7.03 vs 5.61 at 24, 7.92 vs 5.74 at 32).
QUANT_MM_MAX_M = 8


def _mm_operands(x, b_q, scale_b, bias, out_dtype, what):
    """Checks shared by the folded-quantizer matmuls: returns (N, scale_b flat, bias or None,
    bias dtype code, output dtype code), or raises the reference's exception."""
    if b_q.dtype != torch.int8 or not b_q.is_cuda:
        raise NotSupported(f"{what}: b_q must be an int8 HIP tensor")
    same_device(x.device, b_q=b_q, scale_b=scale_b, bias=bias)
    N = b_q.shape[1]
    sb = scale_b.reshape(-1).contiguous()
    if sb.dtype != torch.float32:
        raise NotSupported(f"float32 scale_b only, got {sb.dtype}")
    if sb.numel() not in (1, N):
        raise ValueError(f"scale_b has {sb.numel()} values for N={N}")
    if bias is not None:
        if tuple(bias.shape) != (N,):
            raise ValueError(f"bias must have shape ({N},), got {tuple(bias.shape)}")
        bias = bias.contiguous()
        bias_code = _lib.DTYPE_CODE.get(bias.dtype)
        if bias_code not in (_lib.BF16, _lib.F16, _lib.F32):
            raise NotSupported(f"bias dtype {bias.dtype} is not supported")
    else:
        bias_code = _lib.DTYPE_NONE
    out_code = _lib.DTYPE_CODE.get(out_dtype)
    if out_code not in (_lib.BF16, _lib.F16, _lib.F32):
        raise NotSupported(f"output dtype {out_dtype} is not supported")
    return N, sb, bias, bias_code, out_code


def quant_mm(x: torch.Tensor, b_q: torch.Tensor, scale_b: torch.Tensor,
             out_dtype: torch.dtype = torch.bfloat16, bias: torch.Tensor | None = None,
             precise_div: bool = True, *, config=None, return_scale: bool = False):
    """quant_per_token(x) followed by w8a8_mm, as one kernel, for up to QUANT_MM_MAX_M tokens.

    Bit for bit w8a8_mm(*quant_per_token(x, precise_div), b_q, ..., scale_b, out_dtype,
    bias): the same quantizer arithmetic runs inside the GEMM (reference fused_quant.py:41-53
    and kernel.py:202-257 in one launch).  x is bf16/fp16 [M, K], contiguous or a column
    slice with unit column stride; b_q the K-contiguous [K, N] view of an [N, K] weight.
    Raises NotSupported for more tokens, for a K that no single-step tile takes, or for
    layouts the fused kernel does not read (the caller then makes the two calls).
    """
    from int8_linear.kernel import Config, _cconfig
    if x.dim() != 2 or b_q.dim() != 2 or x.shape[1] != b_q.shape[0]:
        raise ValueError(f"cannot multiply {tuple(x.shape)} by {tuple(b_q.shape)}")
    act = _act_code(x, "x")
    M, K = x.shape
    if M > QUANT_MM_MAX_M:
        raise NotSupported(f"quant_mm takes up to {QUANT_MM_MAX_M} tokens, got {M}")
    if x.stride(1) != 1 and K > 1:
        raise NotSupported("x needs a unit column stride")
    N, sb, bias, bias_code, out_code = _mm_operands(x, b_q, scale_b, bias, out_dtype, "quant_mm")
    out = torch.empty((M, N), dtype=out_dtype, device=x.device)
    s = torch.empty((M, 1), dtype=torch.float32, device=x.device) if return_scale else None
    ldx = x.stride(0) if M > 1 else K
    cfg = _cconfig(config) if isinstance(config, Config) else None
    status = _lib.lib().i8l_w8a8_mm_dynq(
        x.data_ptr(), ldx, act, int(bool(precise_div)), b_q.data_ptr(), b_q.stride(0),
        b_q.stride(1), sb.data_ptr(), sb.numel(),
        bias.data_ptr() if bias is not None else None, bias_code, out.data_ptr(),
        out.stride(0), out_code, s.data_ptr() if s is not None else None, M, N, K, cfg,
        _lib.stream_of(x))
    _lib.check(status, NotSupported)
    return (out, s) if return_scale else out


def quant_mm_supported(m: int, n: int, k: int, config=None) -> bool:
    """Whether quant_mm takes (M, N, K) (under `config`, default the library's choice)."""
    from int8_linear.kernel import Config, _cconfig
    if m > QUANT_MM_MAX_M:
        return False
    cfg = _cconfig(config) if isinstance(config, Config) else None
    return _lib.lib().i8l_w8a8_mm_dynq_supported(m, n, k, cfg) == _lib.OK


# Largest M that silu_mul_quant_mm takes.  Every column tile reads and computes the
# SiLU-and-mul of its token rows (2K values a row), so the folded launch pays off only for
# very few tokens: measured in the 28-layer Qwen3-1.7B stand-in on MI355X (graph replay, the
# norm folded too), 19.28 against 21.56 us a layer at M = 1 and 20.95 against 23.06 at M = 2,
# where the SiLU epilogue of gate_up does better still (20.34); earlier builds of the fold
# lost at 4 and 8 tokens (32.15 against 29.36, 40.02 against 31.08; the kernel itself takes
# up to 8 rows).
SILU_MM_MAX_M = 2


def silu_mul_quant_mm(gate_up: torch.Tensor, b_q: torch.Tensor, scale_b: torch.Tensor,
                      out_dtype: torch.dtype = torch.bfloat16, bias: torch.Tensor | None = None,
                      precise_div: bool = True, round_silu: bool = False, *, config=None,
                      return_scale: bool = False):
    """silu_mul_quant(gate_up) followed by w8a8_mm, as one kernel, for up to SILU_MM_MAX_M
    tokens: the MLP's down projection fed straight from gate_up_proj's output.

    Bit for bit w8a8_mm(*silu_mul_quant(gate_up, precise_div, round_silu), b_q, ..., scale_b,
    out_dtype, bias) (reference fused_quant.py:76-88 and kernel.py:202-257 in one launch).
    gate_up is bf16/fp16 [M, 2K] with unit column stride, the gate values first; b_q the
    K-contiguous [K, N] view of the down weight.  Raises NotSupported for more tokens, a K no
    built tile takes, or layouts the fused kernel does not read (make the two calls then).
    """
    from int8_linear.kernel import Config, _cconfig
    if gate_up.dim() != 2 or b_q.dim() != 2 or gate_up.shape[1] != 2 * b_q.shape[0]:
        raise ValueError(f"gate_up {tuple(gate_up.shape)} does not feed b_q {tuple(b_q.shape)}")
    act = _act_code(gate_up, "gate_up")
    M, K = gate_up.shape[0], b_q.shape[0]
    if M > SILU_MM_MAX_M:
        raise NotSupported(f"silu_mul_quant_mm takes up to {SILU_MM_MAX_M} tokens, got {M}")
    if gate_up.stride(1) != 1:
        raise NotSupported("gate_up needs a unit column stride")
    N, sb, bias, bias_code, out_code = _mm_operands(gate_up, b_q, scale_b, bias, out_dtype,
                                                    "silu_mul_quant_mm")
    out = torch.empty((M, N), dtype=out_dtype, device=gate_up.device)
    s = torch.empty((M, 1), dtype=torch.float32, device=gate_up.device) if return_scale else None
    ldgu = gate_up.stride(0) if M > 1 else 2 * K
    cfg = _cconfig(config) if isinstance(config, Config) else None
    status = _lib.lib().i8l_silu_mul_quant_mm(
        gate_up.data_ptr(), ldgu, act, int(bool(round_silu)), int(bool(precise_div)),
        b_q.data_ptr(), b_q.stride(0), b_q.stride(1), sb.data_ptr(), sb.numel(),
        bias.data_ptr() if bias is not None else None, bias_code, out.data_ptr(),
        out.stride(0), out_code, s.data_ptr() if s is not None else None, M, N, K, cfg,
        _lib.stream_of(gate_up))
    _lib.check(status, NotSupported)
    return (out, s) if return_scale else out


def silu_mul_quant_mm_supported(m: int, n: int, k: int, config=None) -> bool:
    """Whether silu_mul_quant_mm takes M tokens of gate_up [M, 2K] into an [N, K] weight."""
    from int8_linear.kernel import Config, _cconfig
    if m > SILU_MM_MAX_M:
        return False
    cfg = _cconfig(config) if isinstance(config, Config) else None
    return _lib.lib().i8l_silu_mul_quant_mm_supported(m, n, k, cfg) == _lib.OK


# Largest M that add_rmsnorm_quant_mm takes (the kernel's limit): every workgroup normalizes
# and quantizes the token rows itself, while its first weight tile is in flight.
NORM_MM_MAX_M = 8
# Largest M for which the decoder stand-in folds the norm into its projections.  Every
# workgroup repeats the row work, so the fold pays only for few tokens: measured on MI355X
# (HIP graph, cold weights, K = 2048), the folded launch takes 3.64 / 4.17 / 4.83 / 4.89 /
# 6.55 us at N = 4096 and 1 / 2 / 3 / 4 / 8 tokens, against 5.98 / 6.13 / 6.38 / 6.37 / 6.39
# for add_rmsnorm_quant + w8a8_mm, and 5.96 / 6.16 / 7.19 / 7.51 / 9.21 at N = 12288 against
# 8.59 / 8.85 / 8.84 / 9.00 / 9.09; in the 28-layer stand-in (SiLU epilogue on) the folds win
# up to 5 tokens (26.89 us a layer folded at 5 against 27.32 unfolded) and lose from 6 (27.46
# against 27.18 at 6, 29.22 against 28.44 at 8).
NORM_MM_FOLD_M = 5


def add_rmsnorm_quant_mm(x: torch.Tensor, residual: torch.Tensor | None, weight: torch.Tensor,
                         eps: float, b_q: torch.Tensor, scale_b: torch.Tensor,
                         out_dtype: torch.dtype = torch.bfloat16,
                         bias: torch.Tensor | None = None, precise_div: bool = True, *,
                         config=None, return_scale: bool = False, silu_mul: bool = False,
                         round_silu: bool = False):
    """add_rmsnorm_quant(x, residual, weight, eps) followed by w8a8_mm, as one kernel, for up
    to NORM_MM_MAX_M tokens: (out [M, N], residual_out [M, K] or None), and the per-token
    scales [M, 1] last with return_scale.

    Bit for bit the two calls (reference fused_quant.py:56-73, 95-110 then kernel.py:202-257
    in one launch): out = w8a8_mm(q, b_q, s, scale_b, out_dtype, bias) with (q, s,
    residual_out) = add_rmsnorm_quant(x, residual, weight, eps, precise_div).  x and residual
    are contiguous bf16/fp16 [M, K], weight [K] of x's dtype, b_q the K-contiguous [K, N]
    view of an [N, K] weight.  With silu_mul, b_q is a gate_up weight and out is
    y = silu(gate) * up [M, N/2] as w8a8_mm_silu_mul gives it (bf16, a residual, no bias).
    Raises NotSupported for more tokens, a K no built tile takes, or layouts the fused kernel
    does not read (the caller then makes the two calls).
    """
    from int8_linear.kernel import Config, _cconfig
    if x.dim() != 2 or b_q.dim() != 2 or x.shape[1] != b_q.shape[0]:
        raise ValueError(f"cannot multiply {tuple(x.shape)} by {tuple(b_q.shape)}")
    act = _act_code(x, "x")
    M, K = x.shape
    if M > NORM_MM_MAX_M:
        raise NotSupported(f"add_rmsnorm_quant_mm takes up to {NORM_MM_MAX_M} tokens, got {M}")
    if weight.numel() != K:
        raise ValueError(f"weight has {weight.numel()} values for rows of {K}")
    if weight.dtype != x.dtype:
        raise NotSupported("the fused kernel takes a norm weight of x's dtype")
    if not x.is_contiguous():
        raise NotSupported("x must be contiguous")
    weight = weight.contiguous()
    same_device(x.device, weight=weight, residual=residual)
    if residual is not None:
        if residual.shape != x.shape or residual.dtype != x.dtype or not residual.is_contiguous():
            raise NotSupported("residual must be a contiguous tensor of x's shape and dtype")
    N, sb, bias, bias_code, out_code = _mm_operands(x, b_q, scale_b, bias, out_dtype,
                                                    "add_rmsnorm_quant_mm")
    out = torch.empty((M, N // 2 if silu_mul else N), dtype=out_dtype, device=x.device)
    rout = torch.empty_like(x) if residual is not None else None
    s = torch.empty((M, 1), dtype=torch.float32, device=x.device) if return_scale else None
    cfg = _cconfig(config) if isinstance(config, Config) else None
    epi = (2 if round_silu else 1) if silu_mul else 0
    status = _lib.lib().i8l_add_rmsnorm_quant_mm(
        x.data_ptr(), residual.data_ptr() if residual is not None else None, weight.data_ptr(),
        float(eps), act, int(bool(precise_div)), epi,
        rout.data_ptr() if rout is not None else None,
        b_q.data_ptr(), b_q.stride(0), b_q.stride(1), sb.data_ptr(), sb.numel(),
        bias.data_ptr() if bias is not None else None, bias_code, out.data_ptr(),
        out.stride(0), out_code, s.data_ptr() if s is not None else None, M, N, K, cfg,
        _lib.stream_of(x))
    _lib.check(status, NotSupported)
    return (out, rout, s) if return_scale else (out, rout)


def add_rmsnorm_quant_mm_supported(m: int, n: int, k: int, config=None) -> bool:
    """Whether add_rmsnorm_quant_mm takes M tokens of hidden size K into an [N, K] weight."""
    from int8_linear.kernel import Config, _cconfig
    if m > NORM_MM_MAX_M:
        return False
    cfg = _cconfig(config) if isinstance(config, Config) else None
    return _lib.lib().i8l_add_rmsnorm_quant_mm_supported(m, n, k, cfg) == _lib.OK


# Token counts for which the decoder stand-in computes the SiLU-and-mul in gate_up_proj's
# epilogue and folds the quantizer into down_proj (the kernel takes up to 16 tokens).
# Measured in the 28-layer stand-in on MI355X (graph replay), us a layer with / without:
# with the norm folded too, 19.57 / 19.28 at 1 token (where silu_mul_quant_mm folds the whole
# SiLU chain into down_proj instead), 20.34 / 20.95 at 2, 23.03 / 25.06 at 3, 23.88 / 25.58 at
# 4; with the norm unfolded, 27.55 / 27.93 at 5, 28.19 / 28.04 at 6, 28.51 / 28.49 at 7 and
# 28.94 / 29.12 at 8 (at 6-7 within the run-to-run spread).
SILU_EPI_MIN_M = 2
SILU_EPI_MAX_M = 8


def w8a8_mm_silu_mul(a_q: torch.Tensor, b_q: torch.Tensor, scale_a: torch.Tensor,
                     scale_b: torch.Tensor, round_silu: bool = False,
                     bias: torch.Tensor | None = None, *, config=None) -> torch.Tensor:
    """The gate_up projection with the SiLU-and-mul in its epilogue, for few tokens (up to
    16): y = silu(g) * u, [M, N/2] bf16, where g | u = w8a8_mm(a_q, b_q, scale_a, scale_b,
    bf16, bias) split at N/2.

    y is bit for bit the values silu_mul_quant(g | u, round_silu=round_silu) quantizes
    (reference fused_quant.py:76-88), so quant_per_token(y), or quant_mm(y, ...) into the
    down projection, gives its codes and scales; each value is computed once, by the
    workgroup whose tile holds that gate and up column.  b_q is the K-contiguous [K, N] view
    of the [N, K] gate_up weight (gate rows first), scale_b per channel [N], bias None or
    bf16 [N].  Raises NotSupported for more tokens or what the kernel does not take.
    """
    from int8_linear.kernel import Config, _cconfig
    if a_q.dtype != torch.int8 or b_q.dtype != torch.int8:
        raise NotSupported(f"int8 operands only, got {a_q.dtype} and {b_q.dtype}")
    if a_q.dim() != 2 or b_q.dim() != 2 or a_q.shape[1] != b_q.shape[0]:
        raise ValueError(f"cannot multiply {tuple(a_q.shape)} by {tuple(b_q.shape)}")
    if not (a_q.is_cuda and a_q.stride(1) == 1):
        raise NotSupported("a_q must be a K-contiguous HIP tensor")
    M, K = a_q.shape
    N, sb, bias, bias_code, _ = _mm_operands(a_q, b_q, scale_b, bias, torch.bfloat16,
                                             "w8a8_mm_silu_mul")
    sa = scale_a.reshape(-1).contiguous()
    if sa.dtype != torch.float32:
        raise NotSupported(f"float32 scale_a only, got {sa.dtype}")
    same_device(a_q.device, scale_a=sa)
    out = torch.empty((M, N // 2), dtype=torch.bfloat16, device=a_q.device)
    cfg = _cconfig(config) if isinstance(config, Config) else None
    status = _lib.lib().i8l_w8a8_mm_silu_mul(
        a_q.data_ptr(), a_q.stride(0) if M > 1 else K, b_q.data_ptr(), b_q.stride(0),
        b_q.stride(1), sa.data_ptr(), sa.numel(), sb.data_ptr(), sb.numel(),
        bias.data_ptr() if bias is not None else None, bias_code, out.data_ptr(),
        out.stride(0), int(bool(round_silu)), M, N, K, cfg, _lib.stream_of(a_q))
    _lib.check(status, NotSupported)
    return out


def w8a8_mm_silu_mul_supported(m: int, n: int, k: int, config=None) -> bool:
    """Whether w8a8_mm_silu_mul takes M tokens into an [N, K] gate_up weight."""
    from int8_linear.kernel import Config, _cconfig
    cfg = _cconfig(config) if isinstance(config, Config) else None
    return _lib.lib().i8l_w8a8_mm_silu_mul_supported(m, n, k, cfg) == _lib.OK


# Numerics the custom ops use (reference fused_quant.py:127-129 defaults);
# vllm_fuse_patch.use_measured_numerics switches them to the served configuration.
PRECISE_DIV = True
ROUND_SILU = False


@torch.library.custom_op("int8_linear::rmsnorm_quant", mutates_args=())
def rmsnorm_quant_op(x: torch.Tensor, weight: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    q, s, _ = add_rmsnorm_quant(x.contiguous(), None, weight, eps, PRECISE_DIV)
    return q, s


@rmsnorm_quant_op.register_fake
def _(x, weight, eps):
    return (x.new_empty(x.shape, dtype=torch.int8),
            x.new_empty((x.shape[0], 1), dtype=torch.float32))


@torch.library.custom_op("int8_linear::add_rmsnorm_quant", mutates_args=())
def add_rmsnorm_quant_op(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                         eps: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return add_rmsnorm_quant(x.contiguous(), residual.contiguous(), weight, eps, PRECISE_DIV)


@add_rmsnorm_quant_op.register_fake
def _(x, residual, weight, eps):
    return (x.new_empty(x.shape, dtype=torch.int8),
            x.new_empty((x.shape[0], 1), dtype=torch.float32),
            torch.empty_like(x))


@torch.library.custom_op("int8_linear::silu_mul_quant", mutates_args=())
def silu_mul_quant_op(gate_up: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    return silu_mul_quant(gate_up.contiguous(), PRECISE_DIV, ROUND_SILU)


@silu_mul_quant_op.register_fake
def _(gate_up):
    return (gate_up.new_empty((gate_up.shape[0], gate_up.shape[1] // 2), dtype=torch.int8),
            gate_up.new_empty((gate_up.shape[0], 1), dtype=torch.float32))


@torch.library.custom_op("int8_linear::quant_per_token", mutates_args=())
def quant_per_token_op(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    return quant_per_token(x.contiguous(), PRECISE_DIV)


@quant_per_token_op.register_fake
def _(x):
    return (x.new_empty(x.shape, dtype=torch.int8),
            x.new_empty((x.shape[0], 1), dtype=torch.float32))
