"""Shared helpers of the test files: seeded CPU-generated inputs and bit-pattern views."""

from __future__ import annotations

import sys

import numpy as np
import torch


def say(msg: str) -> None:
    """Name the case about to run on the GPU (flushed, so it survives a lost box)."""
    print(f"[case] {msg}", file=sys.stderr, flush=True)


def ints(shape, seed: int, low: int = -127, high: int = 128, device: str = "cuda") -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randint(low, high, shape, dtype=torch.int8, generator=g).to(device)


def offset_ints(shape, seed: int) -> torch.Tensor:
    """int8 values stored one byte into their buffer, so the data pointer is odd."""
    flat = ints((shape[0] * shape[1] + 1,), seed)
    return flat[1:].view(shape)


def randn(shape, seed: int, scale: float = 1.0, dtype=torch.bfloat16, device: str = "cuda"):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype).to(device)


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw 16-bit patterns of a bf16/fp16 tensor as numpy uint16."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def np_(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().numpy()


def from_bits(h: np.ndarray, dtype=torch.bfloat16, device: str = "cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(h, np.uint16).view(np.int16)).view(dtype).to(device)
