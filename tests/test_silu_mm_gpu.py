"""SiLU-and-mul+quant folded into the decode GEMM (fused_quant.silu_mul_quant_mm,
i8l_silu_mul_quant_mm) on the GPU: bit for bit the two launches it replaces, silu_mul_quant
then w8a8_mm, and through them the CPU oracle; every token count it takes, both SiLU
roundings, both division conventions, both activation dtypes, bias and output kinds, every
bf16 gate (extreme ones included), graph replay, and the cases it declines.

The reference issues these two kernels per down_proj in its stand-in (bench/fuse_quant.py:
238-240 of AshrithaG/int8-linear)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits, from_bits, np_, say
from int8_linear import fused_quant as fq
from int8_linear.kernel import Config, NotSupported, w8a8_mm
from oracle import oracle as o

pytestmark = pytest.mark.gpu

K, N = 6144, 2048          # Qwen3-1.7B down_proj: the intermediate size in, the hidden size out


def operands(m, seed, dtype=torch.bfloat16, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    gu = (torch.randn((m, 2 * K), generator=g) * scale).to(dtype).cuda()
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).cuda()
    sb = (torch.rand((N, 1), generator=g) * 1e-3 + 1e-4).cuda()
    return gu, w, sb, g


def two_calls(gu, w, sb, out_dtype=torch.bfloat16, bias=None, precise=True, round_silu=False):
    q, s = fq.silu_mul_quant(gu, precise, round_silu)
    return w8a8_mm(q, w.t(), s, sb, out_dtype, bias), s


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("round_silu", [False, True])
def test_equals_the_two_launches(m, round_silu, monkeypatch):
    monkeypatch.setattr(fq, "SILU_MM_MAX_M", 8)     # the kernel takes up to 8 rows
    say(f"silu_mul_quant_mm m={m} round_silu={round_silu}")
    gu, w, sb, _ = operands(m, 100 + m)
    assert fq.silu_mul_quant_mm_supported(m, N, K)
    got, s = fq.silu_mul_quant_mm(gu, w.t(), sb, round_silu=round_silu, return_scale=True)
    ref, s0 = two_calls(gu, w, sb, round_silu=round_silu)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(s, s0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("precise", [True, False])
def test_dtypes_division_bias_and_outputs(dtype, precise, monkeypatch):
    monkeypatch.setattr(fq, "SILU_MM_MAX_M", 8)
    say(f"silu_mul_quant_mm {dtype} precise={precise}")
    for m in (1, 7):
        gu, w, sb, g = operands(m, 7 * m + precise, dtype)
        for out_dtype, bias in ((torch.bfloat16, None),
                                (torch.bfloat16, torch.randn(N, generator=g).to(torch.bfloat16).cuda()),
                                (torch.float32, torch.randn(N, generator=g).cuda()),
                                (torch.float16, torch.randn(N, generator=g).to(torch.float16).cuda())):
            for rs in (False, True):
                got = fq.silu_mul_quant_mm(gu, w.t(), sb, out_dtype, bias, precise, rs)
                ref, _ = two_calls(gu, w, sb, out_dtype, bias, precise, rs)
                assert torch.equal(got, ref), (m, out_dtype, bias is not None, rs)


def test_matches_the_cpu_oracle(monkeypatch):
    monkeypatch.setattr(fq, "SILU_MM_MAX_M", 8)
    say("silu_mul_quant_mm vs oracle")
    gu, w, sb, _ = operands(3, 11)
    for rs in (False, True):
        got = fq.silu_mul_quant_mm(gu, w.t(), sb, round_silu=rs)
        q0, s0 = o.silu_mul_quant(bits(gu), o.BF16, rs, True)
        ref = o.w8a8_mm(q0, np_(w), s0, np_(sb), out_dt=o.BF16)
        assert np.array_equal(bits(got), ref)


def test_every_bf16_gate_and_the_extreme_ones(monkeypatch):
    """The gates of the rows run through every bf16 value with |g| < 2^124 (signed zeros,
    subnormals, -87 and below, where 1 + exp(-g) is huge or infinite): the folded kernel's
    SiLU gives the standalone kernel's codes and scales for each of them, on waves that take
    the fast quotient and on waves sent to IEEE division by an extreme gate."""
    monkeypatch.setattr(fq, "SILU_MM_MAX_M", 8)
    pats = np.arange(1 << 16, dtype=np.uint32)
    pats = pats[((pats >> 7) & 0xff) <= 250].astype(np.uint16)
    per_call = 8 * K
    for start in range(0, pats.size, per_call):
        say(f"silu_mul_quant_mm gates {start}..{min(start + per_call, pats.size)}")
        gu, w, sb, g = operands(8, 31 + start)
        gb = bits(gu).copy()
        chunk = pats[start:start + per_call]
        gate = gb[:, :K].reshape(-1)
        gate[:chunk.size] = chunk
        gb[:, :K] = gate.reshape(8, K)
        gu = from_bits(gb)
        for rs in (False, True):
            got, s = fq.silu_mul_quant_mm(gu, w.t(), sb, round_silu=rs, return_scale=True)
            ref, s0 = two_calls(gu, w, sb, round_silu=rs)
            assert torch.equal(s, s0)
            assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_zero_row_and_a_strided_gate_up(monkeypatch):
    monkeypatch.setattr(fq, "SILU_MM_MAX_M", 8)
    g = torch.Generator().manual_seed(3)
    wide = (torch.randn((4, 2 * K + 64), generator=g) * 2).to(torch.bfloat16).cuda()
    wide[2].zero_()                                  # absmax 0: codes and scale 0
    gu = wide[:, :2 * K]                             # rows 2K + 64 apart
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).cuda()
    sb = (torch.rand((N, 1), generator=g) * 1e-3 + 1e-4).cuda()
    got, s = fq.silu_mul_quant_mm(gu, w.t(), sb, return_scale=True)
    ref, s0 = two_calls(gu.contiguous(), w, sb)
    assert torch.equal(got, ref) and torch.equal(s, s0)
    assert s[2].item() == 0.0 and torch.all(got[2] == 0)


def test_replays_inside_a_hip_graph():
    say("silu_mul_quant_mm graph replay")
    gu, w, sb, _ = operands(fq.SILU_MM_MAX_M, 21)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fq.silu_mul_quant_mm(gu, w.t(), sb)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fq.silu_mul_quant_mm(gu, w.t(), sb)
    for seed in (1, 2, 3):
        gu.copy_((torch.randn(gu.shape, generator=torch.Generator().manual_seed(seed)) * 2)
                 .to(gu.dtype))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, two_calls(gu, w, sb)[0])


def test_declines_what_it_does_not_take():
    gu, w, sb, _ = operands(fq.SILU_MM_MAX_M + 1, 5)
    assert not fq.silu_mul_quant_mm_supported(fq.SILU_MM_MAX_M + 1, N, K)
    with pytest.raises(NotSupported):
        fq.silu_mul_quant_mm(gu, w.t(), sb)            # more tokens than it takes
    g = torch.Generator().manual_seed(6)
    gu2 = torch.randn((2, 4096), generator=g).to(torch.bfloat16).cuda()
    w2 = torch.randint(-127, 128, (N, 2048), generator=g, dtype=torch.int8).cuda()
    assert not fq.silu_mul_quant_mm_supported(2, N, 2048)
    with pytest.raises(NotSupported):
        fq.silu_mul_quant_mm(gu2, w2.t(), sb)          # no built tile for K = 2048
    gu, w, sb, _ = operands(2, 7)
    with pytest.raises(NotSupported):
        fq.silu_mul_quant_mm(gu.float(), w.t(), sb)    # fp32 activations
    with pytest.raises(NotSupported):
        fq.silu_mul_quant_mm(gu, w.t().contiguous(), sb)   # an N-contiguous weight
    with pytest.raises(ValueError):
        fq.silu_mul_quant_mm(gu[:, :K], w.t(), sb)     # gate_up narrower than 2K
    cfg = Config(16, 8, 512, 12, 3, 1)
    assert fq.silu_mul_quant_mm_supported(1, N, K, cfg)
    assert not fq.silu_mul_quant_mm_supported(1, N, K, Config(16, 16, 512, 12, 3, 1))
