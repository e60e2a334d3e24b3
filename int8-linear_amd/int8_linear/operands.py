"""Seeded synthetic operands of the benchmark configurations.

Follows the reference's benchmark methodology (AshrithaG/int8-linear,
bench/bench_linear.py:146-167): bf16 activations x ~ N(0, 1) [M, K], bf16 weights
W ~ N(0, 0.02) [N, K] and optional bias ~ N(0, 0.01) [N], each quantized symmetrically per
row (per token for x, per output channel for W) with scale = max(absmax, 1e-8) / 127 and
q = clamp(round_half_even(x / scale), -127, 127).  The generator is a seeded CPU
torch.Generator, so the same seed gives the same operands on every machine; tensors are
moved to `device` afterwards.
"""

from __future__ import annotations

import torch


def quant_rows(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric int8 with one float32 scale per row (bench/bench_linear.py:146-150)."""
    scale = x.float().abs().amax(dim=1, keepdim=True).clamp_min(1e-8) / 127.0
    return (x.float() / scale).round().clamp(-127, 127).to(torch.int8), scale


def operands(m: int, k: int, n: int, seed: int, with_bias: bool = False,
             device: str | torch.device = "cpu", dtype: torch.dtype = torch.bfloat16) -> dict:
    """x, W, bias and their quantized forms; w_qt is the K-contiguous [K, N] view."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    a = torch.randn((m, k), generator=g).to(dtype)
    w = (torch.randn((n, k), generator=g) * 0.02).to(dtype)
    bias = (torch.randn((n,), generator=g) * 0.01).to(dtype) if with_bias else None
    a_q, a_s = quant_rows(a)
    w_q, w_s = quant_rows(w)
    d = {"a": a, "w": w, "bias": bias, "a_q": a_q, "a_s": a_s, "w_q": w_q, "w_s": w_s}
    d = {key: (v.to(device) if v is not None else None) for key, v in d.items()}
    d["w_qt"] = d["w_q"].t()
    return d


def seed_of(m: int, k: int, n: int) -> int:
    """Per-shape seed, as the reference's sweep derives one (bench/bench_linear.py:422)."""
    return m * 7919 + k * 31 + n
