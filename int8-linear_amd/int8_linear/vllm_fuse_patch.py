"""Feed vLLM's int8 linears from the fused quantizers instead of from their own quantizer.

A W8A8 linear in vLLM quantizes its bf16 input per token, then multiplies.  In Qwen3 every
such input except o_proj's is the output of an RMSNorm or of SiLU-and-mul, so the quantizer
can run inside that kernel (int8_linear.fused_quant) and the linear can take int8 codes
directly.  Two things have to change in vLLM for that, and `patch_vllm` makes both in the
calling process (its engine must run in-process, VLLM_ENABLE_V1_MULTIPROCESSING=0):

* the producers: Qwen3's decoder layer and the Qwen2/3 MLP hand their linears a `PreQuant`
  (codes, per-token scales, output dtype) made by add_rmsnorm_quant / silu_mul_quant;
* the consumers: the int8 kernel classes' `apply_weights` send a `PreQuant` to the matmul
  with its scales, and anything else to their own method as before.

Each consumer route remembers the method it replaced (`_ROUTES`), so patching twice changes
nothing and `unpatch_vllm` puts every method back.  `PREQUANT_CALLS` counts matmuls fed a
`PreQuant`: a model in which the routing never fired shows zero.

Contract followed: AshrithaG/int8-linear int8_linear/vllm_fuse_patch.py:33-103 (names,
counter, the symmetric-dynamic-only rule, the numerics record of results/fuse_numerics.json).
"""

from __future__ import annotations

import json
from pathlib import Path
from typing import Callable, NamedTuple

import torch

from int8_linear import fused_quant
from int8_linear.fused_quant import add_rmsnorm_quant_op, rmsnorm_quant_op, silu_mul_quant_op

PREQUANT_CALLS = 0

# This package's copy of the numerics record; its choice (IEEE division, SiLU rounded to bf16
# before the multiply) is the one that reproduces vLLM's unfused silu_and_mul +
# scaled_int8_quant bit for bit.
NUMERICS_PATH = Path(__file__).with_name("fuse_numerics.json")


class PreQuant(NamedTuple):
    """Per-token int8 codes of a linear's input, their fp32 scales [M, 1], and the dtype the
    linear's output should have (the dtype of the activation they were made from)."""
    data: torch.Tensor
    scale: torch.Tensor
    dtype: torch.dtype


# class -> its apply_weights before routing (the function found on the class itself)
_ROUTES: dict[type, Callable] = {}
# (owner class, attribute) -> the original forward replaced by a producer
_PRODUCERS: dict[tuple[type, str], Callable] = {}


def _scheme_operands(kernel, layer):
    """(w_q, w_s) of a symmetric dynamic per-token layer; other schemes are refused."""
    w_q, w_s, in_scale, _in_zp, azp_adj = kernel._get_layer_params(layer)
    if in_scale is not None or azp_adj is not None:
        raise NotImplementedError(
            "a PreQuant input fits only symmetric, dynamic per-token int8 activations; this "
            "layer uses a static input scale or an asymmetric zero point")
    return w_q, w_s


def _wrap_apply(cls: type, matmul: Callable) -> None:
    """Route cls.apply_weights(layer, x, bias): a PreQuant x goes to
    matmul(codes, w_q, scales, w_s, out_dtype, bias); any other x to the original method.
    Routing a class again replaces only the matmul, never wraps the router in itself."""
    original = _ROUTES.setdefault(cls, cls.apply_weights)

    def apply_weights(self, layer, x, bias=None):
        global PREQUANT_CALLS
        if not isinstance(x, PreQuant):
            return original(self, layer, x, bias)
        w_q, w_s = _scheme_operands(self, layer)
        PREQUANT_CALLS += 1
        return matmul(x.data, w_q, x.scale, w_s, x.dtype, bias)

    apply_weights.__wrapped__ = original
    cls.apply_weights = apply_weights


def _quantized_norm(norm, x: torch.Tensor, residual: torch.Tensor | None):
    """RMSNorm of x (plus the residual stream, when there is one) as a PreQuant, and the
    residual stream after it.  Without a residual, x itself starts the stream."""
    if residual is None:
        q, s = rmsnorm_quant_op(x, norm.weight, norm.variance_epsilon)
        return PreQuant(q, s, x.dtype), x
    q, s, residual = add_rmsnorm_quant_op(x, residual, norm.weight, norm.variance_epsilon)
    return PreQuant(q, s, x.dtype), residual


def _decoder_forward(self, positions, hidden_states, residual):
    """Qwen3DecoderLayer.forward with both norms producing the next linear's int8 input."""
    attn_in, residual = _quantized_norm(self.input_layernorm, hidden_states, residual)
    attn_out = self.self_attn(positions=positions, hidden_states=attn_in)
    mlp_in, residual = _quantized_norm(self.post_attention_layernorm, attn_out, residual)
    return self.mlp(mlp_in), residual


def _mlp_forward(self, x):
    """Qwen2MLP.forward with SiLU-and-mul producing down_proj's int8 input."""
    gate_up = self.gate_up_proj(x)[0]
    codes, scales = silu_mul_quant_op(gate_up)
    return self.down_proj(PreQuant(codes, scales, gate_up.dtype))[0]


def use_measured_numerics(path: Path = NUMERICS_PATH) -> None:
    """Apply a numerics record {"best_precise_div": bool, "best_round_silu": bool} to the
    custom ops' division and SiLU rounding (a missing file changes nothing)."""
    if not path.exists():
        return
    record = json.loads(path.read_text())
    fused_quant.PRECISE_DIV = bool(record["best_precise_div"])
    fused_quant.ROUND_SILU = bool(record["best_round_silu"])


def _consumer_routes():
    """(kernel class, matmul) for vLLM's int8 linear kernels.  The Triton kernel's matmul is
    looked up through its module at every call, so int8_linear.vllm_patch's swap of
    triton_scaled_mm (before or after this patch) is the matmul a PreQuant reaches."""
    from vllm import _custom_ops as ops
    from vllm.model_executor.kernels.linear.scaled_mm import cutlass
    from vllm.model_executor.kernels.linear.scaled_mm import triton as vllm_triton

    def via_triton(a, w, sa, sb, dt, bias):
        return vllm_triton.triton_scaled_mm(a, w, scale_a=sa, scale_b=sb, out_dtype=dt,
                                            bias=bias)

    def via_cutlass(a, w, sa, sb, dt, bias):
        return ops.cutlass_scaled_mm(a, w, scale_a=sa, scale_b=sb, out_dtype=dt, bias=bias)

    return [(vllm_triton.TritonInt8ScaledMMLinearKernel, via_triton),
            (cutlass.CutlassInt8ScaledMMLinearKernel, via_cutlass)]


def _producer_routes():
    from vllm.model_executor.models import qwen2, qwen3
    return [(qwen3.Qwen3DecoderLayer, "forward", _decoder_forward),
            (qwen2.Qwen2MLP, "forward", _mlp_forward)]


def patch_vllm() -> None:
    """Apply the measured numerics, then route vLLM's int8 kernels and Qwen3's producers."""
    use_measured_numerics()
    for cls, matmul in _consumer_routes():
        _wrap_apply(cls, matmul)
    for owner, attr, fn in _producer_routes():
        _PRODUCERS.setdefault((owner, attr), getattr(owner, attr))
        setattr(owner, attr, fn)


def unpatch_vllm() -> None:
    """Put back every method patch_vllm replaced."""
    for cls, original in _ROUTES.items():
        cls.apply_weights = original
    _ROUTES.clear()
    for (owner, attr), original in _PRODUCERS.items():
        setattr(owner, attr, original)
    _PRODUCERS.clear()
