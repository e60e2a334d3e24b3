"""Put this package's MI355X matmul behind vLLM's int8 Triton linear.

vLLM's `TritonInt8ScaledMMLinearKernel` reaches its GEMM through one module-level name,
``vllm.model_executor.kernels.linear.scaled_mm.triton.triton_scaled_mm(input, weight,
scale_a=, scale_b=, out_dtype=, bias=)``.  `patch_vllm` points that name at `scaled_mm`
below; weight loading, activation quantization and layer dispatch stay vLLM's own.

How a call travels:

* eager (no trace active): straight to `w8a8_mm`, which picks the tile configuration for
  this call's M through the C++ binding when it is built.  No torch op dispatch is paid;
* during a torch.compile trace: through the opaque custom op ``int8_linear::w8a8_mm``.  The
  compiled graph then calls the op at run time, so the configuration follows the live batch
  size instead of the one seen while tracing;
* declined (`NotSupported`: a K or N no tile divides, a dtype the kernels lack): to the
  `triton_scaled_mm` that `patch_vllm` displaced, counted in `FALLBACKS`.  With nothing
  displaced (the patch never ran) the exception propagates.

`CALLS`, `FALLBACKS` and `CONFIGS` ({(M, K, N): config name}) are process-wide counters.  HIP
graph replay runs no Python, so in a graph-captured model they only move during warm-up and
capture: a served model that shows `CALLS == 0` never reached this kernel.

vLLM must build the model in this process (VLLM_ENABLE_V1_MULTIPROCESSING=0) for the
rebinding to be seen.  Contract followed: AshrithaG/int8-linear int8_linear/vllm_patch.py:30-83.
"""

from typing import Optional

import torch

from int8_linear.kernel import NotSupported, choose_config, tuned_config, w8a8_mm

CALLS = 0
FALLBACKS = 0
CONFIGS: dict[tuple[int, int, int], str] = {}
# vLLM's own triton_scaled_mm, kept by patch_vllm for the shapes this kernel declines
_vllm_triton_scaled_mm = None


def _note(m: int, k: int, n: int) -> None:
    """Count the call and record which configuration (M, K, N) runs with."""
    global CALLS
    CALLS += 1
    if (m, k, n) not in CONFIGS:
        CONFIGS[(m, k, n)] = choose_config(m, n, k).name


def _run(a_q: torch.Tensor, b_q: torch.Tensor, scale_a: torch.Tensor, scale_b: torch.Tensor,
         out_dtype: torch.dtype, bias: Optional[torch.Tensor]) -> torch.Tensor:
    global FALLBACKS
    _note(a_q.shape[0], a_q.shape[1], b_q.shape[1])
    try:
        return w8a8_mm(a_q, b_q, scale_a, scale_b, out_dtype, bias)
    except NotSupported:
        displaced = _vllm_triton_scaled_mm
        if displaced is None:
            raise
        FALLBACKS += 1
        return displaced(a_q, b_q, scale_a, scale_b, out_dtype, bias)


@torch.library.custom_op("int8_linear::w8a8_mm", mutates_args=())
def w8a8_mm_op(a_q: torch.Tensor, b_q: torch.Tensor, scale_a: torch.Tensor,
               scale_b: torch.Tensor, out_dtype: torch.dtype,
               bias: Optional[torch.Tensor]) -> torch.Tensor:
    return _run(a_q, b_q, scale_a, scale_b, out_dtype, bias)


@w8a8_mm_op.register_fake
def _(a_q, b_q, scale_a, scale_b, out_dtype, bias):
    return a_q.new_empty((a_q.shape[0], b_q.shape[1]), dtype=out_dtype)


def scaled_mm(input: torch.Tensor, weight: torch.Tensor, scale_a: torch.Tensor,
              scale_b: torch.Tensor, out_dtype: torch.dtype,
              bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """vLLM's triton_scaled_mm signature: int8 input [M, K], K-contiguous int8 weight
    [K, N], fp32 scales per token / per channel (or scalars), optional bias."""
    if torch.compiler.is_compiling():
        return w8a8_mm_op(input, weight, scale_a, scale_b, out_dtype, bias)
    return _run(input, weight, scale_a, scale_b, out_dtype, bias)


def patch_vllm() -> None:
    """Point vLLM's triton_scaled_mm at scaled_mm; safe to call more than once."""
    global _vllm_triton_scaled_mm
    import vllm.model_executor.kernels.linear.scaled_mm.triton as vllm_triton

    current = vllm_triton.triton_scaled_mm
    if current is not scaled_mm:
        _vllm_triton_scaled_mm = current
    # Read the tuned table now: a compiled or captured region must not touch the file system.
    tuned_config(1, 1, 1)
    vllm_triton.triton_scaled_mm = scaled_mm
