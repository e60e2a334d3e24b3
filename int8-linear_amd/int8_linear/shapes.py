"""Linear-layer shapes, as (layers, K, N) for C[M, N] = A[M, K] @ W[N, K]^T.

The model dimensions are public model facts; the table is kept identical to the
reference's int8_linear/shapes.py (AshrithaG/int8-linear, 3-27) so that shape names agree.
"""

SHAPES = {
    # Qwen3-1.7B: hidden 2048, intermediate 6144, 16 query and 8 KV heads of 128.
    "qwen3-1.7b": [
        ("q_proj, o_proj", 2048, 2048),
        ("k_proj, v_proj", 2048, 1024),
        ("gate_proj, up_proj", 2048, 6144),
        ("down_proj", 6144, 2048),
    ],
    # What vLLM runs for Qwen3-1.7B: q, k, v merged into one projection, gate with up.
    "qwen3-1.7b-vllm": [
        ("qkv_proj", 2048, 4096),
        ("o_proj", 2048, 2048),
        ("gate_up_proj", 2048, 12288),
        ("down_proj", 6144, 2048),
    ],
    # Llama-3-8B at TP1, QKV and gate/up merged as vLLM runs them.
    "llama-3-8b": [
        ("qkv_proj", 4096, 6144),
        ("o_proj", 4096, 4096),
        ("gate_up_proj", 4096, 28672),
        ("down_proj", 14336, 4096),
    ],
}
