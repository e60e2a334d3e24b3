"""add + RMSNorm + quantize folded into the persistent decode GEMM
(fused_quant.add_rmsnorm_quant_mm, i8l_add_rmsnorm_quant_mm) on the GPU: bit for bit the two
launches it replaces, add_rmsnorm_quant then w8a8_mm (output, residual_out and scales), and
through them the CPU oracle; every built tile at every pass count, both activation dtypes,
both division conventions, with and without a residual, bias and output kinds, one and
several workgroups a compute unit, rows that hold zeros or one dominant value, graph replay,
and the cases it declines."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits, np_, say
from int8_linear import fused_quant as fq
from int8_linear.kernel import Config, NotSupported, w8a8_mm
from int8_linear.kernel import supported as kernel_supported
from oracle import oracle as o

pytestmark = pytest.mark.gpu

# (NC, KS, W) of the built tiles; K = 64 * KS * W
TILES = [(16, 8, 4), (16, 4, 8), (8, 8, 4), (8, 4, 8), (16, 8, 8), (8, 8, 8)]
EPS = 1e-6


def operands(m, k, n, seed, dtype=torch.bfloat16, residual=True):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn((m, k), generator=g) * 3).to(dtype).cuda()
    r = (torch.randn((m, k), generator=g)).to(dtype).cuda() if residual else None
    gamma = (1 + 0.1 * torch.randn(k, generator=g)).to(dtype).cuda()
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).cuda()
    sb = (torch.rand((n, 1), generator=g) * 1e-2 + 1e-3).cuda()
    return x, r, gamma, w, sb, g


def two_calls(x, r, gamma, w, sb, out_dtype=torch.bfloat16, bias=None, precise=True):
    q, s, rout = fq.add_rmsnorm_quant(x, r, gamma, EPS, precise)
    return w8a8_mm(q, w.t(), s, sb, out_dtype, bias), rout, s


def check(x, r, gamma, w, sb, cfg=None, out_dtype=torch.bfloat16, bias=None, precise=True):
    out, rout, s = fq.add_rmsnorm_quant_mm(x, r, gamma, EPS, w.t(), sb, out_dtype, bias,
                                           precise, config=cfg, return_scale=True)
    ref, rout0, s0 = two_calls(x, r, gamma, w, sb, out_dtype, bias, precise)
    assert torch.equal(out.view(torch.int16) if out.element_size() == 2 else out.view(torch.int32),
                       ref.view(torch.int16) if ref.element_size() == 2 else ref.view(torch.int32))
    assert torch.equal(s, s0)
    if r is None:
        assert rout is None
    else:
        assert torch.equal(rout.view(torch.int16), rout0.view(torch.int16))


@pytest.mark.parametrize("tile", TILES, ids=lambda t: f"nc{t[0]}_ks{t[1]}_w{t[2]}")
@pytest.mark.parametrize("per_cu", [1, 2])
def test_every_tile_equals_the_two_launches(tile, per_cu):
    nc, ks, w_ = tile
    k = 64 * ks * w_
    cfg = Config(16, nc, 64 * ks, w_, 4, per_cu)
    if not fq.add_rmsnorm_quant_mm_supported(1, 4096, k, cfg):
        pytest.skip(f"{cfg.name}: {per_cu} workgroups of this tile exceed a CU's LDS")
    for n in (1024, 4096):                       # fewer tiles than CUs, and several a CU
        for m in range(1, fq.NORM_MM_MAX_M + 1):   # every pass count
            for res in (True, False):
                say(f"norm_mm tile={tile} g={per_cu} n={n} m={m} residual={res}")
                x, r, gamma, w, sb, _ = operands(m, k, n, m + k + n, residual=res)
                assert fq.add_rmsnorm_quant_mm_supported(m, n, k, cfg)
                check(x, r, gamma, w, sb, cfg)


@pytest.mark.parametrize("k,n", [(2048, 4096), (2048, 12288), (4096, 6144), (4096, 28672)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("precise", [True, False])
def test_default_tile_dtypes_bias_and_division(k, n, dtype, precise):
    for m in (1, 5, fq.NORM_MM_MAX_M):
        say(f"norm_mm k={k} n={n} m={m} {dtype} precise={precise}")
        x, r, gamma, w, sb, g = operands(m, k, n, m * 3 + n, dtype)
        for out_dtype, bias in ((torch.bfloat16, None),
                                (torch.bfloat16, torch.randn(n, generator=g).to(torch.bfloat16).cuda()),
                                (torch.float32, torch.randn(n, generator=g).cuda()),
                                (torch.float16, torch.randn(n, generator=g).to(torch.float16).cuda())):
            check(x, r, gamma, w, sb, None, out_dtype, bias, precise)


def test_matches_the_cpu_oracle():
    for res in (True, False):
        x, r, gamma, w, sb, _ = operands(6, 2048, 4096, 11, residual=res)
        out, rout, s = fq.add_rmsnorm_quant_mm(x, r, gamma, EPS, w.t(), sb, return_scale=True)
        q0, s0, r0 = o.add_rmsnorm_quant(bits(x), bits(r) if res else None, bits(gamma), EPS)
        assert np.array_equal(np_(s).reshape(-1), s0.reshape(-1))
        assert np.array_equal(bits(out), o.w8a8_mm(q0, np_(w), s0, np_(sb), out_dt=o.BF16))
        if res:
            assert np.array_equal(bits(rout), r0)


def test_zero_row_dominant_value_and_scalar_scale():
    x, r, gamma, w, sb, g = operands(8, 2048, 4096, 3)
    x[4].zero_()
    r[4].zero_()                                    # a zero row: codes and scale 0
    x[6, 100] = 3e4                                 # one value dominates its row
    for sbv in (sb, torch.tensor([0.02]).cuda()):
        check(x, r, gamma, w, sbv)
    out, _, s = fq.add_rmsnorm_quant_mm(x, r, gamma, EPS, w.t(), sb, return_scale=True)
    assert s[4].item() == 0.0 and torch.all(out[4] == 0)


def test_replays_inside_a_hip_graph():
    x, r, gamma, w, sb, _ = operands(8, 2048, 12288, 21)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fq.add_rmsnorm_quant_mm(x, r, gamma, EPS, w.t(), sb)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out, rout = fq.add_rmsnorm_quant_mm(x, r, gamma, EPS, w.t(), sb)
    for seed in (1, 2, 3):
        gen = torch.Generator().manual_seed(seed)
        x.copy_(torch.randn(x.shape, generator=gen).to(x.dtype))
        r.copy_(torch.randn(r.shape, generator=gen).to(r.dtype))
        graph.replay()
        torch.cuda.synchronize()
        ref, rout0, _ = two_calls(x, r, gamma, w, sb)
        assert torch.equal(out, ref) and torch.equal(rout, rout0)


def test_declines_what_it_does_not_take():
    x, r, gamma, w, sb, _ = operands(fq.NORM_MM_MAX_M + 1, 2048, 2048, 5)
    with pytest.raises(NotSupported):
        fq.add_rmsnorm_quant_mm(x, r, gamma, EPS, w.t(), sb)   # more tokens than it takes
    x, r, gamma, w, sb, _ = operands(4, 6144, 2048, 6)
    assert not fq.add_rmsnorm_quant_mm_supported(4, 2048, 6144)
    with pytest.raises(NotSupported):
        fq.add_rmsnorm_quant_mm(x, r, gamma, EPS, w.t(), sb)   # K = 6144: no built tile
    x, r, gamma, w, sb, _ = operands(4, 2048, 2048, 7)
    with pytest.raises(NotSupported):
        fq.add_rmsnorm_quant_mm(x, r, gamma.float(), EPS, w.t(), sb)   # weight of another dtype
    with pytest.raises(NotSupported):
        fq.add_rmsnorm_quant_mm(x, r, gamma, EPS, w.t().contiguous(), sb)   # N-contiguous weight


@pytest.mark.parametrize("silu", [False, True])
def test_repeated_calls_with_tiles_in_flight(silu):
    """The cross-wave exchanges of the persistent kernel and of the fold's prologue meet at
    barriers that do not wait for the weight copies in flight (the next tile's, or the first
    tile's during the prologue): 40 calls in a row at shapes where every workgroup walks
    several column tiles and two workgroups share a CU, each against the first and against the
    two launches, and the plain persistent GEMM and the SiLU epilogue the same way."""
    k, n = 2048, 12288
    for m in (1, 2, 4, 8):
        say(f"norm_mm repeated silu={silu} m={m}")
        x, r, gamma, w, sb, _ = operands(m, k, n, 400 + m)
        for cfg in (None, Config(16, 16, 256, 8, 4, 2), Config(16, 16, 512, 4, 4, 2)):
            if cfg is not None and not fq.add_rmsnorm_quant_mm_supported(m, n, k, cfg):
                continue
            outs = [fq.add_rmsnorm_quant_mm(x, r, gamma, EPS, w.t(), sb, config=cfg,
                                            silu_mul=silu)[0] for _ in range(40)]
            torch.cuda.synchronize()
            assert all(torch.equal(o.view(torch.int16), outs[0].view(torch.int16)) for o in outs)
            q, s, _ = fq.add_rmsnorm_quant(x, r, gamma, EPS)
            ref = (fq.w8a8_mm_silu_mul(q, w.t(), s, sb) if silu
                   else w8a8_mm(q, w.t(), s, sb, torch.bfloat16))
            assert torch.equal(outs[0].view(torch.int16), ref.view(torch.int16))
            # the persistent GEMM (and its SiLU epilogue) alone, same tiles
            takes = cfg is not None and (fq.w8a8_mm_silu_mul_supported(m, n, k, cfg) if silu
                                         else kernel_supported(m, n, k, cfg))
            if takes:
                alone = [(fq.w8a8_mm_silu_mul(q, w.t(), s, sb, config=cfg) if silu
                          else w8a8_mm(q, w.t(), s, sb, torch.bfloat16, config=cfg))
                         for _ in range(40)]
                torch.cuda.synchronize()
                assert all(torch.equal(a.view(torch.int16), ref.view(torch.int16)) for a in alone)
