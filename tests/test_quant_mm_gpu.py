"""The quantizer folded into the decode GEMM (fused_quant.quant_mm, i8l_w8a8_mm_dynq) on the
GPU: bit for bit the two launches it replaces, quant_per_token then w8a8_mm, and through them
the CPU oracle; every built tile, both activation dtypes, both division conventions, bias
kinds, column slices, zero rows, graph replay, and the cases it declines."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits, np_, say
from int8_linear import fused_quant as fq
from int8_linear.kernel import Config, NotSupported, w8a8_mm
from oracle import oracle as o

pytestmark = pytest.mark.gpu

# (NC, KS, W) of the built tiles; K = 64 * KS * W
TILES = [(8, 2, 16), (16, 2, 16), (32, 2, 16), (8, 4, 16), (16, 4, 16), (8, 8, 12)]


def operands(m, k, n, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn((m, k), generator=g) * 3).to(dtype).cuda()
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).cuda()
    sb = (torch.rand((n, 1), generator=g) * 1e-2 + 1e-3).cuda()
    return x, w, sb, g


def two_calls(x, w, sb, out_dtype=torch.bfloat16, bias=None, precise=True):
    q, s = fq.quant_per_token(x, precise)
    return w8a8_mm(q, w.t(), s, sb, out_dtype, bias), s


@pytest.mark.parametrize("tile", TILES, ids=lambda t: f"nc{t[0]}_ks{t[1]}_w{t[2]}")
@pytest.mark.parametrize("m", [1, 3, 7, 12, 16])
def test_every_tile_equals_the_two_launches(tile, m, monkeypatch):
    monkeypatch.setattr(fq, "QUANT_MM_MAX_M", 16)   # the kernel itself takes any M
    nc, ks, w_ = tile
    k, n = 64 * ks * w_, 1024
    say(f"quant_mm tile={tile} m={m}")
    cfg = Config(16, nc, 64 * ks, w_, 3, 1)
    if ks == 8 and m > 8:
        assert not fq.quant_mm_supported(m, n, k, cfg)   # 512-byte slices: 8 rows at most
        pytest.skip(f"{cfg.name} takes up to 8 tokens")
    x, w, sb, _ = operands(m, k, n, m + k)
    assert fq.quant_mm_supported(m, n, k, cfg)
    got, s = fq.quant_mm(x, w.t(), sb, config=cfg, return_scale=True)
    ref, s0 = two_calls(x, w, sb)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(s, s0)


@pytest.mark.parametrize("k,n", [(2048, 2048), (2048, 4096), (2048, 12288), (4096, 4096)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("precise", [True, False])
def test_default_tile_dtypes_and_division(k, n, dtype, precise):
    say(f"quant_mm k={k} n={n} {dtype} precise={precise}")
    for m in (1, fq.QUANT_MM_MAX_M):
        x, w, sb, g = operands(m, k, n, m * 3 + n, dtype)
        for out_dtype, bias in ((torch.bfloat16, None),
                                (torch.bfloat16, torch.randn(n, generator=g).to(torch.bfloat16).cuda()),
                                (torch.float32, torch.randn(n, generator=g).cuda()),
                                (torch.float16, None)):
            got = fq.quant_mm(x, w.t(), sb, out_dtype, bias, precise)
            ref, _ = two_calls(x, w, sb, out_dtype, bias, precise)
            assert torch.equal(got, ref), (m, out_dtype, bias is not None)


def test_matches_the_cpu_oracle():
    x, w, sb, _ = operands(5, 2048, 2048, 11)
    got = fq.quant_mm(x, w.t(), sb)
    q0, s0 = o.quant_per_token(bits(x), precise_div=True)
    ref = o.w8a8_mm(q0, np_(w), s0, np_(sb), out_dt=o.BF16)
    assert np.array_equal(bits(got), ref)


def test_column_slice_zero_row_and_scalar_scale():
    g = torch.Generator().manual_seed(3)
    qkv = torch.randn((8, 4096), generator=g).to(torch.bfloat16).cuda()
    qkv[4].zero_()                                   # absmax 0: codes and scale 0
    qkv[6, 100] = 3e4                                # one large value dominates its row
    x = qkv[:, :2048]
    w = torch.randint(-127, 128, (2048, 2048), generator=g, dtype=torch.int8).cuda()
    for sb in ((torch.rand((2048, 1), generator=g) + 0.5).cuda(), torch.tensor([0.02]).cuda()):
        got, s = fq.quant_mm(x, w.t(), sb, return_scale=True)
        ref, s0 = two_calls(x, w, sb)
        assert torch.equal(got, ref) and torch.equal(s, s0)
        assert s[4].item() == 0.0 and torch.all(got[4] == 0)


def test_replays_inside_a_hip_graph():
    x, w, sb, _ = operands(8, 2048, 4096, 21)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fq.quant_mm(x, w.t(), sb)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fq.quant_mm(x, w.t(), sb)
    for seed in (1, 2, 3):
        x.copy_(torch.randn(x.shape, generator=torch.Generator().manual_seed(seed)).to(x.dtype))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, two_calls(x, w, sb)[0])


def test_declines_what_it_does_not_take():
    x, w, sb, _ = operands(fq.QUANT_MM_MAX_M + 1, 2048, 2048, 5)
    with pytest.raises(NotSupported):
        fq.quant_mm(x, w.t(), sb)                      # more tokens than the host layer takes
    x, w, sb, _ = operands(4, 3072, 2048, 6)
    assert not fq.quant_mm_supported(4, 2048, 3072)
    with pytest.raises(NotSupported):
        fq.quant_mm(x, w.t(), sb)                      # no single-step tile for K = 3072
    with pytest.raises(NotSupported):
        fq.quant_mm(x.float(), w.t(), sb)
    x, w, sb, _ = operands(4, 2048, 2048, 7)
    with pytest.raises(NotSupported):
        fq.quant_mm(x, w.t().contiguous(), sb)         # an N-contiguous weight
