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


def oracle_step(stack: DecoderStandIn, rows=None) -> tuple[np.ndarray, np.ndarray]:
    """The same chain on the CPU oracle: (last h bits, residual bits).  Every op of the chain
    works on each token row alone, so with `rows` given the oracle runs on those token rows
    only and its result is exactly those rows of the full step."""
    x = bits(stack.x) if rows is None else bits(stack.x)[rows]
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


@pytest.mark.parametrize("m,layers", [(1, 3), (2, 2), (4, 2), (8, 3), (17, 2), (32, 3), (128, 2),
                                      (300, 1)])
@pytest.mark.parametrize("round_silu", [False, True])
def test_standin_matches_oracle_bit_for_bit(m, layers, round_silu, monkeypatch):
    say(f"standin m={m} layers={layers} round_silu={round_silu}")
    monkeypatch.setattr(fq, "ROUND_SILU", round_silu)
    stack = DecoderStandIn(m, layers=layers, seed=m)
    h, res = stack.forward(with_residual=True)
    torch.cuda.synchronize()
    h0, r0 = oracle_step(stack)
    assert h.shape == (m, 2048) and h.dtype == torch.bfloat16
    assert np.array_equal(bits(h), h0)
    assert np.array_equal(bits(res), r0)


@pytest.mark.parametrize("round_silu", [False, True])
def test_prefill_step_matches_oracle_on_sampled_rows(round_silu, monkeypatch):
    """The 4096-token step the benchmark times (prefill regime: every GEMM on the macro-tile
    schedules), two layers, compared with the oracle on the first, last and tile-edge token
    rows and six random ones: final output and residual stream, bit for bit."""
    m = 4096
    say(f"standin prefill m={m} layers=2 round_silu={round_silu}, sampled rows")
    monkeypatch.setattr(fq, "ROUND_SILU", round_silu)
    stack = DecoderStandIn(m, layers=2, seed=4096)
    h, res = stack.forward(with_residual=True)
    torch.cuda.synchronize()
    rng = np.random.default_rng(7 + round_silu)
    rows = np.unique(np.concatenate([[0, 1, 127, 128, 255, 256, 2047, 4095],
                                     rng.choice(m, 6, replace=False)]))
    h0, r0 = oracle_step(stack, rows)
    idx = torch.from_numpy(rows).cuda()
    assert np.array_equal(bits(h[idx]), h0)
    assert np.array_equal(bits(res[idx]), r0)


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


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5])
@pytest.mark.parametrize("round_silu", [False, True])
def test_folded_kernels_give_the_same_step(m, round_silu, monkeypatch):
    """For few tokens the stand-in folds each add+RMSNorm+quant into the projection after it,
    the q-column quantizer into o_proj, and SiLU-and-mul+quant into down_proj or gate_up_proj's
    epilogue (4 kernels a layer at 1-3 tokens); the step's output and residual stream are the
    same bits with every fold and with none."""
    say(f"standin folds m={m} round_silu={round_silu}")
    monkeypatch.setattr(fq, "ROUND_SILU", round_silu)
    stack = DecoderStandIn(m, layers=3, seed=40 + m)
    assert stack.fused_norm == (m <= fq.NORM_MM_FOLD_M)
    assert stack.fused_silu == (fq.SILU_EPI_MIN_M <= m <= fq.SILU_EPI_MAX_M)
    h, res = stack.forward(with_residual=True)
    stack.use_fused_norm = stack.use_fused_silu = stack.use_fused_down = False
    monkeypatch.setattr(fq, "QUANT_MM_MAX_M", 0)
    assert not (stack.fused_norm or stack.fused_silu or stack.fused_down or stack.fused_o)
    h0, r0 = stack.forward(with_residual=True)
    torch.cuda.synchronize()
    assert torch.equal(h, h0) and torch.equal(res, r0)
