"""The int8 linears of the benchmarked models, as (name, K, N) for C[M, N] = A[M, K] @ W[N, K]^T.

Each table is derived from the model's published dimensions (hidden size, MLP width,
attention heads and head size), either with every projection separate, as the checkpoint
stores them, or merged the way vLLM runs them (q, k, v in one qkv_proj; gate with up).  The
keys and names are the ones the reference's benchmarks use (AshrithaG/int8-linear
int8_linear/shapes.py), so a shape named there means the same matrix here.
"""

from __future__ import annotations

from typing import NamedTuple


class ModelDims(NamedTuple):
    hidden: int
    intermediate: int
    q_heads: int
    kv_heads: int
    head_dim: int


QWEN3_1_7B = ModelDims(hidden=2048, intermediate=6144, q_heads=16, kv_heads=8, head_dim=128)
LLAMA_3_8B = ModelDims(hidden=4096, intermediate=14336, q_heads=32, kv_heads=8, head_dim=128)


def separate_linears(d: ModelDims) -> list[tuple[str, int, int]]:
    """Distinct (K, N) of the unmerged projections; projections of one shape share a row."""
    q, kv = d.q_heads * d.head_dim, d.kv_heads * d.head_dim
    return [("q_proj, o_proj", d.hidden, q),
            ("k_proj, v_proj", d.hidden, kv),
            ("gate_proj, up_proj", d.hidden, d.intermediate),
            ("down_proj", d.intermediate, d.hidden)]


def merged_linears(d: ModelDims) -> list[tuple[str, int, int]]:
    """The four GEMMs of a decoder layer as vLLM executes them at tensor parallelism 1."""
    q, kv = d.q_heads * d.head_dim, d.kv_heads * d.head_dim
    return [("qkv_proj", d.hidden, q + 2 * kv),
            ("o_proj", q, d.hidden),
            ("gate_up_proj", d.hidden, 2 * d.intermediate),
            ("down_proj", d.intermediate, d.hidden)]


SHAPES = {
    "qwen3-1.7b": separate_linears(QWEN3_1_7B),
    "qwen3-1.7b-vllm": merged_linears(QWEN3_1_7B),
    "llama-3-8b": merged_linears(LLAMA_3_8B),
}
