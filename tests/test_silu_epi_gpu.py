"""The SiLU-and-mul in the gate_up GEMM's epilogue (fused_quant.w8a8_mm_silu_mul,
i8l_w8a8_mm_silu_mul, and the norm-folded form add_rmsnorm_quant_mm(..., silu_mul=True)) on
the GPU.  The epilogue's y = bf16(silu(g) * u) from the bf16 gate_up products g | u must be
the values silu_mul_quant quantizes, bit for bit:
  * against a restatement from the oracle's pieces: the oracle's GEMM gives g | u, its
    canonical exp gives d = 1 + exp(-g), and silu(g) = g / d is IEEE division (numpy float32),
    rounded to bf16 where round_silu says, times u, rounded to bf16;
  * through quant_per_token(y): the codes and scales of silu_mul_quant on the unfused gate_up
    output;
for every built tile, one to sixteen tokens, both SiLU roundings, with and without a bias,
and gates below -87 (where exp(-g) overflows) so that the kernel takes its IEEE-division
path.  (Infinite and NaN values are outside the bit-exact contract: their NaN payloads
follow the hardware.)"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits, np_, say
from int8_linear import fused_quant as fq
from int8_linear import tune
from int8_linear.kernel import Config, NotSupported, w8a8_mm
from oracle import oracle as o

pytestmark = pytest.mark.gpu

# (NC, KS, W) of every built persistent tile with one 16-row block and 8 or 16 columns (the
# tiles the SiLU epilogue takes): K = 64 * KS * W
TILES = [(nc, ks, w) for mt, nc, ks, w in tune.WLDSP_TILES if mt == 1 and nc in (8, 16)]


def operands(m, k, n, seed, big_gates=False):
    g = torch.Generator().manual_seed(seed)
    a = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8).cuda()
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).cuda()
    sa = (torch.rand((m, 1), generator=g) * 1e-2 + 1e-3).cuda()
    sb = torch.rand((n, 1), generator=g) * 1e-5 + 1e-6
    if big_gates:       # gates of magnitude ~1e3 (some below -87: exp(-g) overflows)
        sb[: n // 2: 7] = 1.0
    return a, w, sa, sb.cuda(), g


def y_reference(gu_bits: np.ndarray, round_silu: bool) -> np.ndarray:
    """bf16 bits of silu(g) * u from the bf16 bits of g | u, as silu_mul_quant computes it."""
    i = gu_bits.shape[1] // 2
    g, u = o.bf16_to_f32(gu_bits[:, :i]), o.bf16_to_f32(gu_bits[:, i:])
    with np.errstate(all="ignore"):
        d = np.float32(1.0) + o.expf(-g)
        a = (g / d).astype(np.float32)
        if round_silu:
            a = o.bf16_to_f32(o.f32_to_bf16(a))
        return o.f32_to_bf16((a * u).astype(np.float32))


def check(a, w, sa, sb, bias, round_silu, cfg=None):
    y = fq.w8a8_mm_silu_mul(a, w.t(), sa, sb, round_silu, bias, config=cfg)
    gu = w8a8_mm(a, w.t(), sa, sb, torch.bfloat16, bias)
    assert np.array_equal(bits(y), y_reference(bits(gu), round_silu))
    q, s = fq.quant_per_token(y)
    q0, s0 = fq.silu_mul_quant(gu, True, round_silu)
    assert torch.equal(q, q0) and torch.equal(s, s0)


@pytest.mark.parametrize("tile", TILES, ids=lambda t: f"nc{t[0]}_ks{t[1]}_w{t[2]}")
def test_every_tile_against_the_restatement(tile):
    nc, ks, w_ = tile
    k, n = 64 * ks * w_, 2048
    for per_cu in (1, 2):
        cfg = Config(16, nc, 64 * ks, w_, 4, per_cu)
        if not fq.w8a8_mm_silu_mul_supported(1, n, k, cfg):
            continue
        for m in (1, 7, 16):
            for round_silu in (False, True):
                say(f"silu epilogue tile={tile} g={per_cu} m={m} round={round_silu}")
                a, w, sa, sb, _ = operands(m, k, n, m + k + nc)
                check(a, w, sa, sb, None, round_silu, cfg)


@pytest.mark.parametrize("round_silu", [False, True])
def test_qwen3_gate_up_bias_and_big_gates(round_silu):
    k, n = 2048, 12288
    for m in (1, 2, 4, 8):
        say(f"silu epilogue qwen3 gate_up m={m} round={round_silu}")
        a, w, sa, sb, g = operands(m, k, n, 100 + m, big_gates=True)
        check(a, w, sa, sb, None, round_silu)
        bias = (torch.randn(n, generator=g) * 0.5).to(torch.bfloat16).cuda()
        check(a, w, sa, sb, bias, round_silu)


@pytest.mark.parametrize("round_silu", [False, True])
def test_norm_fold_with_the_silu_epilogue(round_silu):
    """add_rmsnorm_quant_mm(..., silu_mul=True) equals add_rmsnorm_quant then
    w8a8_mm_silu_mul, with the residual stream bit for bit."""
    k, n = 2048, 12288
    for m in (1, 2, 3, 4, 8):
        say(f"norm fold + silu epilogue m={m} round={round_silu}")
        g = torch.Generator().manual_seed(200 + m)
        x = torch.randn((m, k), generator=g).to(torch.bfloat16).cuda()
        r = torch.randn((m, k), generator=g).to(torch.bfloat16).cuda()
        gamma = (1 + 0.1 * torch.randn(k, generator=g)).to(torch.bfloat16).cuda()
        w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).cuda()
        sb = (torch.rand((n, 1), generator=g) * 1e-3 + 1e-4).cuda()
        y, rout = fq.add_rmsnorm_quant_mm(x, r, gamma, 1e-6, w.t(), sb, silu_mul=True,
                                          round_silu=round_silu)
        q, s, rout0 = fq.add_rmsnorm_quant(x, r, gamma, 1e-6)
        y0 = fq.w8a8_mm_silu_mul(q, w.t(), s, sb, round_silu)
        assert torch.equal(y.view(torch.int16), y0.view(torch.int16))
        assert torch.equal(rout, rout0)


def test_quantized_down_projection_of_y():
    """quant_mm of y into down_proj (the 12-wave K = 6144 tile) equals quant_per_token then
    w8a8_mm, and the silu_mul_quant chain it replaces."""
    k, n, kd = 2048, 12288, 6144
    for m in (1, 4, 8):
        say(f"y into down_proj m={m}")
        a, w, sa, sb, g = operands(m, k, n, 300 + m)
        wd = torch.randint(-127, 128, (2048, kd), generator=g, dtype=torch.int8).cuda()
        sd = (torch.rand((2048, 1), generator=g) * 1e-3 + 1e-4).cuda()
        y = fq.w8a8_mm_silu_mul(a, w.t(), sa, sb, True)
        got = fq.quant_mm(y, wd.t(), sd)
        q, s = fq.quant_per_token(y)
        assert torch.equal(got, w8a8_mm(q, wd.t(), s, sd, torch.bfloat16))
        q0, s0 = fq.silu_mul_quant(w8a8_mm(a, w.t(), sa, sb, torch.bfloat16), True, True)
        assert torch.equal(got, w8a8_mm(q0, wd.t(), s0, sd, torch.bfloat16))


def test_declines_what_it_does_not_take():
    a, w, sa, sb, _ = operands(17, 2048, 2048, 5)
    with pytest.raises(NotSupported):
        fq.w8a8_mm_silu_mul(a, w.t(), sa, sb)             # more than one 16-row block
    a, w, sa, sb, _ = operands(4, 2048, 2048, 6)
    with pytest.raises(NotSupported):
        fq.w8a8_mm_silu_mul(a, w.t(), sa, sb, bias=torch.zeros(2048, device="cuda"))  # fp32 bias
    with pytest.raises(ValueError):
        fq.w8a8_mm_silu_mul(a, w.t(), sa, sb[:1])            # per-tensor scale_b
    cfg = Config(16, 32, 128, 16, 4, 1)                      # a 32-column tile: two fragments
    assert not fq.w8a8_mm_silu_mul_supported(4, 2048, 2048, cfg)
