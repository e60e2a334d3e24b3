"""The reference's torch restatement of its fused quantizers (AshrithaG/int8-linear
tests/test_fused_quant.py:26-51), on the CPU, with switches for the three steps where it and
this repository's canonical definitions part:

* division: the restatement writes ``127.0 / absmax`` and calls it an IEEE divide, but torch
  evaluates a Python number over a tensor as ``reciprocal(absmax) * 127``, two roundings.
  ``division="as_written"`` keeps that; ``"ieee"`` makes it the single IEEE division
  (``torch.full_like(absmax, 127.0) / absmax``), which is the reference kernel's PRECISE_DIV
  arithmetic (int8_linear/fused_quant.py:45-47);
* variance: ``xf.pow(2).mean(-1)`` sums in float32 in torch's order; ``canonical_var`` sums
  the squares exactly in float64 and rounds the mean once;
* rsqrt: ``torch.rsqrt`` (float32); ``canonical_rsqrt`` is 1/sqrt in float64 rounded once.

With all three canonical the restatement is the oracle's definition, element for element.
"""

from __future__ import annotations

import torch

EPS = 1e-6


def quant(yf: torch.Tensor, division: str = "as_written"):
    """(codes int8, scales fp32 [M, 1]) of float32 rows yf."""
    absmax = yf.abs().amax(-1, keepdim=True)
    if division == "as_written":
        ratio = 127.0 / absmax
    elif division == "ieee":
        ratio = torch.full_like(absmax, 127.0) / absmax
    else:
        raise ValueError(division)
    inv = torch.where(absmax == 0, torch.zeros_like(absmax), ratio)
    return torch.round(yf * inv).clamp(-128, 127).to(torch.int8), absmax / 127.0


def norm(x, r, w, division="as_written", canonical_var=False, canonical_rsqrt=False, eps=EPS):
    """(codes, scales, residual_out or None) of add+RMSNorm+quant (reference test lines 34-43)."""
    x, w = x.cpu(), w.cpu()
    xf = x.float()
    rout = None
    if r is not None:
        xf = xf + r.cpu().float()
        rout = xf.to(x.dtype)
    if canonical_var:
        var = (xf.double().pow(2).sum(-1, keepdim=True) / xf.shape[-1]).float()
    else:
        var = xf.pow(2).mean(-1, keepdim=True)
    if canonical_rsqrt:
        inv = (1.0 / torch.sqrt((var + eps).double())).float()
    else:
        inv = torch.rsqrt(var + eps)
    y = ((xf * inv).to(w.dtype) * w).to(x.dtype)
    return (*quant(y.float(), division), rout)


def silu(gu, round_silu, division="as_written"):
    """(codes, scales) of SiLU-and-mul+quant (reference test lines 46-51)."""
    gu = gu.cpu()
    i = gu.shape[1] // 2
    g, u = gu[:, :i].float(), gu[:, i:].float()
    a = g / (1.0 + torch.exp(-g))
    if round_silu:
        a = a.to(gu.dtype).float()
    return quant((a * u).to(gu.dtype).float(), division)


def differences(q, s, q0, s0) -> tuple[int, int, int]:
    """(codes that differ, largest code difference, scales whose bits differ)."""
    q, q0 = torch.as_tensor(q).int(), torch.as_tensor(q0).int()
    s, s0 = torch.as_tensor(s).float(), torch.as_tensor(s0).float()
    d = (q - q0).abs()
    return int(d.ne(0).sum()), int(d.max()) if d.numel() else 0, int(
        (s.view(torch.int32) != s0.view(torch.int32)).sum())
