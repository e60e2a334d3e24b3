"""The decoder stand-in on the GPU against the CPU oracle.

The reference's stand-in (bench/fuse_quant.py:184-240 of AshrithaG/int8-linear) chains the
fused quantizers and the four int8 linears of each Qwen3-1.7B layer.  Every kernel in the
chain is bit-exact against the oracle, so the whole chain is too: the final down_proj output,
the residual stream and every intermediate agree bit for bit after several layers, at decode
batch sizes and at a prefill-regime one.  The captured-graph replay the benchmark times must
equal the eager step.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits, np_, say
from int8_linear import fused_quant as fq
from int8_linear.standin import EPS, Q_COLS, DecoderStandIn
from oracle import oracle as o

pytestmark = pytest.mark.gpu


def oracle_step(stack: DecoderStandIn) -> tuple[np.ndarray, np.ndarray]:
    """The same chain on the CPU oracle: (last h bits, residual bits)."""
    x = bits(stack.x)
    gamma = bits(stack.norm)
    precise, round_silu = fq.PRECISE_DIV, fq.ROUND_SILU

    def mm(layer, name, q, s):
        w, ws = layer[name]
        return o.w8a8_mm(q, np_(w), s, np_(ws), out_dt=o.BF16)

    res = x
    q, s, _ = o.add_rmsnorm_quant(x, None, gamma, EPS, precise_div=precise)
    h = None
    for i, layer in enumerate(stack.layers):
        if i:
            q, s, res = o.add_rmsnorm_quant(h, res, gamma, EPS, precise_div=precise)
        a = mm(layer, "qkv_proj", q, s)
        q, s = o.quant_per_token(a[:, :Q_COLS], precise_div=precise)
        h = mm(layer, "o_proj", q, s)
        q, s, res = o.add_rmsnorm_quant(h, res, gamma, EPS, precise_div=precise)
        gu = mm(layer, "gate_up_proj", q, s)
        q, s = o.silu_mul_quant(gu, round_silu=round_silu, precise_div=precise)
        h = mm(layer, "down_proj", q, s)
    return h, res


@pytest.mark.parametrize("m,layers", [(1, 3), (8, 3), (17, 2), (128, 2), (300, 1)])
@pytest.mark.parametrize("round_silu", [False, True])
def test_standin_matches_oracle_bit_for_bit(m, layers, round_silu, monkeypatch):
    say(f"standin m={m} layers={layers} round_silu={round_silu}")
    monkeypatch.setattr(fq, "ROUND_SILU", round_silu)
    stack = DecoderStandIn(m, layers=layers, seed=m)
    h = stack.forward()
    torch.cuda.synchronize()
    h0, _ = oracle_step(stack)
    assert h.shape == (m, 2048) and h.dtype == torch.bfloat16
    assert np.array_equal(bits(h), h0)


def test_standin_graph_replay_equals_eager():
    say("standin graph replay")
    stack = DecoderStandIn(8, layers=2, seed=5)
    eager = stack.forward().clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        stack.forward()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = stack.forward()
    for seed in (6, 7):
        stack.x.copy_(torch.randn((8, 2048), generator=torch.Generator().manual_seed(seed))
                      .to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        again = stack.forward()
        torch.cuda.synchronize()
        assert torch.equal(out, again)
        assert not torch.equal(out, eager)
