"""W8A8 GEMM on the GPU against the CPU oracle, through the C ABI.

The cases mirror the reference's tests/test_kernel.py (AshrithaG/int8-linear): exact int32
products at ragged and even M (41-45), other tilings (48-53), scaled outputs against
float64 (56-75), the decline rule (78-82), graph replay (85-100) and an odd data pointer
(139-145).  Beyond them: every output is compared with the oracle bit for bit, the BASELINE
decode sweep (configs 0-1) at full size, and the prefill shapes (config 3) at full size
through size-independent checks (row and column checksums of the int32 product, plus full
rows compared exactly).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits, ints, np_, offset_ints, say
from int8_linear import Config, NotSupported, _lib, kernel, w8a8_mm
from int8_linear.operands import operands, seed_of
from int8_linear.shapes import SHAPES
from oracle import oracle as o

pytestmark = pytest.mark.gpu

CODE = {torch.bfloat16: o.BF16, torch.float16: o.F16, torch.float32: o.F32}


def oracle_out(a, w, sa, sb, bias, dtype):
    acc = o.gemm_i32(np_(a), np_(w))
    if bias is None:
        bias_np, bdt = None, o.NONE
    elif bias.dtype == torch.float32:
        bias_np, bdt = np_(bias), o.F32
    else:
        bias_np, bdt = bits(bias), CODE[bias.dtype]
    return o.epilogue(acc, np_(sa), np_(sb), bias_np, bdt, CODE[dtype])


def as_np(out: torch.Tensor) -> np.ndarray:
    return np_(out) if out.dtype in (torch.float32, torch.int32) else bits(out)


SHAPES_REF = [(1, 2048, 2048), (3, 2048, 1024), (17, 2048, 6144), (64, 2048, 2048),
              (100, 6144, 2048)]


@pytest.mark.parametrize("m,k,n", SHAPES_REF)
def test_int32_product_is_exact(m, k, n):
    say(f"w8a8_mm raw m={m} k={k} n={n}")
    a, w = ints((m, k), 1), ints((n, k), 2)
    one = torch.ones(1, device="cuda")
    got = w8a8_mm(a, w.t(), one, one, raw=True)
    ref = o.gemm_i32(np_(a), np_(w))
    assert got.dtype == torch.int32 and np.array_equal(np_(got), ref)
    assert np.array_equal(ref, (np_(a).astype(np.float64) @ np_(w).astype(np.float64).T).astype(np.int32))


TILINGS = [Config(16, 16, 64, 1, 1, 1), Config(32, 32, 256, 4, 1, 1), Config(64, 16, 512, 8, 1, 1),
           Config(128, 16, 256, 4, 1, 1), Config(16, 32, 512, 8, 1, 1),
           Config(16, 8, 256, 4, 1, 1), Config(32, 8, 512, 8, 1, 1), Config(16, 4, 128, 2, 1, 1),
           Config(128, 128, 64, 4, 2, 8), Config(256, 128, 64, 4, 2, 1),
           Config(128, 256, 64, 4, 2, 1), Config(128, 128, 128, 4, 2, 1),
           Config(256, 256, 64, 8, 2, 8), Config(256, 128, 64, 8, 2, 1),
           Config(128, 256, 128, 8, 2, 8),
           Config(256, 256, 64, 8, 3, 8), Config(256, 256, 64, 8, 4, 8),
           Config(256, 256, 64, 8, 5, 4), Config(256, 128, 64, 8, 6, 8),
           Config(256, 128, 64, 8, 4, 1), Config(128, 256, 128, 8, 3, 8),
           Config(128, 128, 64, 4, 4, 1), Config(128, 128, 64, 4, 8, 8),
           # overlapped fragment reads (stages = ring depth + 8)
           Config(256, 256, 64, 8, 11, 8), Config(256, 256, 64, 8, 12, 8),
           Config(256, 256, 64, 8, 13, 4), Config(256, 128, 64, 8, 12, 8),
           Config(128, 256, 64, 8, 12, 4), Config(128, 256, 128, 8, 11, 8),
           Config(256, 128, 128, 8, 11, 8), Config(128, 128, 64, 4, 12, 1),
           Config(128, 128, 128, 4, 12, 8), Config(64, 128, 128, 4, 12, 8),
           Config(64, 256, 128, 8, 11, 4), Config(64, 128, 64, 4, 14, 1),
           Config(64, 128, 128, 4, 14, 8), Config(64, 64, 128, 4, 12, 8),
           Config(128, 64, 128, 4, 12, 4),
           # double-buffered (ring of two) with 128-byte K steps
           Config(256, 256, 128, 8, 10, 4), Config(256, 128, 128, 8, 10, 8),
           Config(128, 256, 128, 8, 10, 1)]


@pytest.mark.parametrize("config", TILINGS, ids=lambda c: c.name.replace(" ", "_"))
@pytest.mark.parametrize("m", [256, 300])
def test_exact_under_other_tilings(config, m):
    k, n = 2048, 1024
    say(f"w8a8_mm raw m={m} k={k} n={n} config={config.name}")
    a, w = ints((m, k), 3), ints((n, k), 4)
    one = torch.ones(1, device="cuda")
    got = w8a8_mm(a, w.t(), one, one, raw=True, config=config)
    assert np.array_equal(np_(got), o.gemm_i32(np_(a), np_(w)))
    # and the scaled path of the same tiling
    sa = torch.rand((m, 1), device="cuda") * 1e-2 + 1e-3
    sb = torch.rand((n, 1), device="cuda") * 1e-2 + 1e-3
    out = w8a8_mm(a, w.t(), sa, sb, torch.bfloat16, config=config)
    assert np.array_equal(bits(out), oracle_out(a, w, sa, sb, None, torch.bfloat16))


# Regression test for a race in the prefill epilogue: its LDS staging stores were handed to the
# other waves by a barrier that did not wait for them, and with two workgroups a CU sharing the
# LDS about one call in ten returned 16x16 blocks of stale LDS bytes (M=700, K=N=2048, 64x64
# tiles).  Every repeated call must give the oracle's bits.
@pytest.mark.parametrize("config", [Config(64, 64, 128, 4, 12, 4), Config(128, 64, 128, 4, 12, 4),
                                    Config(128, 128, 64, 4, 2, 8), Config(128, 128, 64, 4, 4, 1)],
                         ids=lambda c: c.name.replace(" ", "_"))
def test_prefill_epilogue_is_repeatable(config):
    m, k, n = 700, 2048, 2048
    say(f"w8a8_mm repeated m={m} k={k} n={n} config={config.name}")
    a, w = ints((m, k), 11), ints((n, k), 12)
    sa = torch.rand((m, 1), device="cuda") * 1e-2 + 1e-3
    sb = torch.rand((n, 1), device="cuda") * 1e-2 + 1e-3
    first = w8a8_mm(a, w.t(), sa, sb, torch.bfloat16, config=config)
    assert np.array_equal(bits(first), oracle_out(a, w, sa, sb, None, torch.bfloat16))
    outs = [w8a8_mm(a, w.t(), sa, sb, torch.bfloat16, config=config) for _ in range(100)]
    torch.cuda.synchronize()
    assert sum(not torch.equal(o, first) for o in outs) == 0


def _prefill_tiles():
    from int8_linear import tune
    out = [Config(bm, bn, bk, w, st + tune.PIPELINED, 4) for bm, bn, bk, w, st in tune.DMAP_TILES]
    out += [Config(bm, bn, bk, w, st, 1) for bm, bn, bk, w, st in tune.DMA_TILES]
    out += [Config(bm, bn, bk, w, 2, 1) for bm, bn, bk, w in tune.STAGED_TILES]
    return out


@pytest.mark.parametrize("m,n", [(700, 2304), (300, 4608)])
def test_every_prefill_tile_is_repeatable(m, n):
    """Every prefill tile the tuner may pick, called 20 times in a row at a shape where two
    workgroups share a CU, gives the same bits each time and the oracle's bits; and its
    4-byte outputs (raw int32, fp32), which are staged through LDS in two halves of the
    tile's rows, give the oracle's values on every one of 5 calls."""
    k = 2048
    say(f"w8a8_mm every prefill tile repeated m={m} k={k} n={n}")
    a, w = ints((m, k), 13), ints((n, k), 14)
    sa = torch.rand((m, 1), device="cuda") * 1e-2 + 1e-3
    sb = torch.rand((n, 1), device="cuda") * 1e-2 + 1e-3
    one = torch.ones(1, device="cuda")
    want = oracle_out(a, w, sa, sb, None, torch.bfloat16)
    want_f32 = oracle_out(a, w, sa, sb, None, torch.float32)
    want_i32 = o.gemm_i32(np_(a), np_(w))
    for config in _prefill_tiles():
        if not kernel.supported(m, n, k, config):
            continue
        outs = [w8a8_mm(a, w.t(), sa, sb, torch.bfloat16, config=config) for _ in range(20)]
        raws = [w8a8_mm(a, w.t(), one, one, raw=True, config=config) for _ in range(5)]
        f32s = [w8a8_mm(a, w.t(), sa, sb, torch.float32, config=config) for _ in range(5)]
        torch.cuda.synchronize()
        assert np.array_equal(bits(outs[0]), want), config.name
        assert all(torch.equal(o, outs[0]) for o in outs), config.name
        assert all(np.array_equal(np_(r), want_i32) for r in raws), config.name
        assert all(np.array_equal(np_(f), want_f32) for f in f32s), config.name


@pytest.mark.parametrize("m", [16, 100])
def test_every_decode_tile_is_repeatable(m):
    """Every decode tile the tuner may pick (weights through LDS or streamed), called 10 times
    in a row, gives the same bits each time and the oracle's bits."""
    from int8_linear import tune
    k, n = 2048, 4096
    say(f"w8a8_mm every decode tile repeated m={m} k={k} n={n}")
    a, w = ints((m, k), 15), ints((n, k), 16)
    sa = torch.rand((m, 1), device="cuda") * 1e-2 + 1e-3
    sb = torch.rand((n, 1), device="cuda") * 1e-2 + 1e-3
    want = oracle_out(a, w, sa, sb, None, torch.bfloat16)
    configs = [Config(16 * mt, nc, 64 * ks, w_, 3, 1) for mt, nc, ks in tune.WLDS_TILES
               for w_ in (4, 8, 16)]
    configs += [Config(16 * mt, bn, 64 * w_, w_, 1, 1) for mt, bn in tune.STREAM_TILES
                for w_ in (1, 2, 4, 8, 16)]
    configs += [Config(16 * mt, nc, 64 * ks, w_, 4, 1) for mt, nc, ks, w_ in tune.WLDSP_TILES]
    checked = 0
    for config in configs:
        if not kernel.supported(m, n, k, config):
            continue
        outs = [w8a8_mm(a, w.t(), sa, sb, torch.bfloat16, config=config) for _ in range(10)]
        torch.cuda.synchronize()
        assert np.array_equal(bits(outs[0]), want), config.name
        assert all(torch.equal(o, outs[0]) for o in outs), config.name
        checked += 1
    assert checked >= 40


# The persistent single-step decode schedule (stages 4): every built tile on a shape with more
# column tiles than the launch has workgroups a row block (so each workgroup walks several,
# and the last walk is ragged), ragged M over one to three row blocks, every epilogue kind.
WLDSP = [(mt, nc, ks, w) for mt, nc, ks, w in
         [(1, 16, 2, 16), (2, 16, 2, 16), (1, 32, 2, 16), (1, 16, 4, 16),
          (1, 16, 4, 8), (2, 16, 4, 8), (4, 16, 4, 8), (1, 16, 8, 8),
          (4, 16, 2, 16), (8, 16, 4, 8), (4, 32, 2, 8), (1, 8, 2, 16), (1, 8, 4, 16),
          (1, 8, 8, 8), (1, 8, 16, 4), (1, 16, 16, 4), (1, 8, 8, 4), (1, 16, 8, 4),
          (1, 8, 6, 16), (2, 8, 6, 16), (1, 8, 12, 8), (1, 8, 4, 8)]]


@pytest.mark.parametrize("mt,nc,ks,w", WLDSP, ids=lambda v: str(v))
@pytest.mark.parametrize("m", [1, 17, 40, 100])
def test_persistent_decode_tiles_exact(mt, nc, ks, w, m):
    k, n = 64 * ks * w, 32 * 311                          # 622 or 311 column tiles
    config = Config(16 * mt, nc, 64 * ks, w, 4, 2 if kernel.supported(m, 32 * 311, k, Config(
        16 * mt, nc, 64 * ks, w, 4, 2)) and m % 2 else 1)   # two workgroups a CU where they fit
    say(f"w8a8_mm persistent m={m} k={k} n={n} config={config.name}")
    a, wt = ints((m, k), 21 + m), ints((n, k), 22)
    one = torch.ones(1, device="cuda")
    got = w8a8_mm(a, wt.t(), one, one, raw=True, config=config)
    assert np.array_equal(np_(got), o.gemm_i32(np_(a), np_(wt)))
    sa = torch.rand((m, 1), device="cuda") * 1e-2 + 1e-3
    sb = torch.rand((n, 1), device="cuda") * 1e-2 + 1e-3
    for dtype, bias in ((torch.bfloat16, None),
                        (torch.bfloat16, (torch.randn(n, device="cuda") * 0.01).to(torch.bfloat16)),
                        (torch.float16, torch.randn(n, device="cuda") * 0.01)):
        out = w8a8_mm(a, wt.t(), sa, sb, dtype, bias, config=config)
        assert np.array_equal(bits(out), oracle_out(a, wt, sa, sb, bias, dtype)), (dtype, bias is None)


@pytest.mark.parametrize("mt,nc,ks,w", WLDSP, ids=lambda v: str(v))
def test_persistent_decode_tiles_one_tile_a_workgroup(mt, nc, ks, w):
    """The straight single-tile form of the persistent tile (the launcher's choice when the
    grid covers the column tiles: N = NC x compute units, one row block), exact."""
    m, k = min(16 * mt, 9), 64 * ks * w
    n = nc * torch.cuda.get_device_properties(0).multi_processor_count
    config = Config(16 * mt, nc, 64 * ks, w, 4, 1)
    say(f"w8a8_mm persistent, one tile a workgroup m={m} k={k} n={n} config={config.name}")
    a, wt = ints((m, k), 31 + m), ints((n, k), 32)
    one = torch.ones(1, device="cuda")
    got = w8a8_mm(a, wt.t(), one, one, raw=True, config=config)
    assert np.array_equal(np_(got), o.gemm_i32(np_(a), np_(wt)))
    sa = torch.rand((m, 1), device="cuda") * 1e-2 + 1e-3
    sb = torch.rand((n, 1), device="cuda") * 1e-2 + 1e-3
    bias = (torch.randn(n, device="cuda") * 0.01).to(torch.bfloat16)
    out = w8a8_mm(a, wt.t(), sa, sb, torch.bfloat16, bias, config=config)
    assert np.array_equal(bits(out), oracle_out(a, wt, sa, sb, bias, torch.bfloat16))


# Tiles 384 and 192 columns wide (N a multiple of 192: Llama-3-8B qkv 6144, Qwen3 gate_up
# 12288), exact on N = 1536 with ragged M.
WIDE_TILINGS = [Config(128, 384, 64, 8, 11, 4), Config(128, 384, 64, 8, 12, 8),
                Config(128, 192, 64, 4, 12, 8), Config(256, 192, 64, 4, 12, 4),
                Config(256, 192, 128, 8, 10, 4)]


@pytest.mark.parametrize("config", WIDE_TILINGS, ids=lambda c: c.name.replace(" ", "_"))
@pytest.mark.parametrize("m", [256, 300])
def test_exact_under_wide_tilings(config, m):
    k, n = 2048, 1536
    say(f"w8a8_mm wide m={m} k={k} n={n} config={config.name}")
    a, w = ints((m, k), 5), ints((n, k), 6)
    one = torch.ones(1, device="cuda")
    got = w8a8_mm(a, w.t(), one, one, raw=True, config=config)
    assert np.array_equal(np_(got), o.gemm_i32(np_(a), np_(w)))
    sa = torch.rand((m, 1), device="cuda") * 1e-2 + 1e-3
    sb = torch.rand((n, 1), device="cuda") * 1e-2 + 1e-3
    bias = (torch.randn(n, device="cuda") * 0.01).to(torch.bfloat16)
    out = w8a8_mm(a, w.t(), sa, sb, torch.bfloat16, bias, config=config)
    assert np.array_equal(bits(out), oracle_out(a, w, sa, sb, bias, torch.bfloat16))


# The weights-through-LDS decode schedule (stages 3, bm <= 128): every built tile, with one,
# two, three and four K steps a wave (the ring's even and odd tails), 32/16/8/4 columns a
# workgroup, ragged M.
WLDS = [(mt, nc, ks) for mt, nc, ks in
        [(1, 16, 2), (1, 16, 4), (1, 16, 6), (1, 16, 8), (1, 8, 2), (1, 8, 4), (1, 8, 6),
         (1, 8, 8), (1, 4, 4), (1, 4, 8), (2, 16, 2), (2, 16, 4), (2, 8, 2), (2, 8, 4),
         (4, 16, 2), (4, 16, 4), (4, 8, 2), (4, 8, 4), (8, 16, 2), (8, 8, 2),
         (1, 32, 2), (1, 32, 4), (2, 32, 2), (2, 32, 4), (4, 32, 2), (4, 32, 4),
         (1, 64, 2), (2, 64, 2), (4, 64, 2), (1, 64, 4), (2, 64, 4)]]


@pytest.mark.parametrize("tile", WLDS, ids=lambda t: f"mt{t[0]}_nc{t[1]}_ks{t[2]}")
@pytest.mark.parametrize("steps", [1, 2, 3, 4, 5])
@pytest.mark.parametrize("waves", [4, 8, 12, 16])
@pytest.mark.parametrize("ring", [1, 3, 4], ids=["two_buffers", "three_buffers", "four_buffers"])
def test_weights_through_lds_schedule(tile, steps, waves, ring):
    """group_m 3 / 4: the three- / four-buffer ring of the activations-through-LDS tile (more
    than two / three steps a wave), whose loops and tails differ from the two-buffer one's."""
    mt, nc, ks = tile
    k, n = 64 * ks * waves * steps, 512
    cfg = Config(16 * mt, nc, 64 * ks, waves, 3, ring)
    if not kernel.supported(16 * mt, n, k, cfg):
        pytest.skip(f"{cfg.name} is not built for K={k}")
    for m in {1: (1, 5, 16), 2: (17, 32), 4: (33, 64), 8: (65, 100, 128)}[mt]:
        say(f"w8a8_mm wlds m={m} k={k} n={n} config={cfg.name}")
        a, w = ints((m, k), 11 + m), ints((n, k), 12)
        one = torch.ones(1, device="cuda")
        got = w8a8_mm(a, w.t(), one, one, raw=True, config=cfg)
        assert np.array_equal(np_(got), o.gemm_i32(np_(a), np_(w)))
        g = torch.Generator().manual_seed(m)
        sa = (torch.rand((m, 1), generator=g) * 1e-2 + 1e-3).cuda()
        sb = (torch.rand((n, 1), generator=g) * 1e-2 + 1e-3).cuda()
        for bias in (None, torch.randn(n, generator=g).to(torch.bfloat16).cuda()):
            out = w8a8_mm(a, w.t(), sa, sb, torch.bfloat16, bias, config=cfg)
            assert np.array_equal(bits(out), oracle_out(a, w, sa, sb, bias, torch.bfloat16))
        out = w8a8_mm(a, w.t(), sa, sb, torch.float16, config=cfg)     # the generic epilogue
        assert np.array_equal(bits(out), oracle_out(a, w, sa, sb, None, torch.float16))


def _wlds_a_lds(mt, nc, ks, w):
    """LDS bytes of the activations-through-LDS multi-step tile (two step buffers of weight
    and activation rows a wave, or the cross-wave reduction area, the larger)."""
    ring = w * 2 * (16 * mt + nc) * 64 * ks
    red = w * mt * (nc // 16 if nc > 16 else 1) * 1024
    return max(ring, red)


# (mt, nc, ks, waves): the first two copy the activations through LDS with the weights, the
# last two need more LDS than a CU has for that and load them into registers instead
MULTI_STEP = [(2, 32, 4, 4), (1, 16, 4, 4), (4, 64, 2, 8), (2, 32, 4, 8)]


@pytest.mark.parametrize("tile", MULTI_STEP, ids=lambda t: f"mt{t[0]}_nc{t[1]}_ks{t[2]}_w{t[3]}")
def test_multi_step_tiles_every_epilogue(tile):
    """Both multi-step decode kernels (gemm_wlds_a, and gemm_wlds where its rings do not fit)
    through every output dtype, bias dtype and scale layout, bit-exact against the oracle."""
    mt, nc, ks, w_ = tile
    assert (_wlds_a_lds(*tile) <= 160 * 1024) == (tile in MULTI_STEP[:2])
    m, k, n = 16 * mt - 3, 64 * ks * w_ * 3, 512
    cfg = Config(16 * mt, nc, 64 * ks, w_, 3, 1)
    assert kernel.supported(m, n, k, cfg), cfg.name
    a, w = ints((m, k), 41 + mt), ints((n, k), 42 + nc)
    g = torch.Generator().manual_seed(43)
    sa_row = (torch.rand((m, 1), generator=g) * 1e-2 + 1e-3).cuda()
    sb_col = (torch.rand((n, 1), generator=g) * 1e-2 + 1e-3).cuda()
    for dtype in (torch.bfloat16, torch.float16, torch.float32):
        for bias_dtype in (None, torch.bfloat16, torch.float16, torch.float32):
            say(f"multi-step {cfg.name} m={m} k={k} {dtype} bias={bias_dtype}")
            bias = torch.randn(n, generator=g).to(bias_dtype).cuda() if bias_dtype else None
            for sa, sb in ((sa_row, sb_col), (sa_row[:1].reshape(1), sb_col[:1].reshape(1))):
                out = w8a8_mm(a, w.t(), sa, sb, dtype, bias, config=cfg)
                assert np.array_equal(as_np(out), oracle_out(a, w, sa, sb, bias, dtype)), \
                    (dtype, bias_dtype, sa.numel(), sb.numel())


@pytest.mark.parametrize("m", [37, 13])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("per_row", [True, False])
@pytest.mark.parametrize("per_col", [True, False])
@pytest.mark.parametrize("bias_dtype", [None, torch.bfloat16, torch.float16, torch.float32])
def test_scaled_output_matches_oracle_and_float64(m, dtype, per_row, per_col, bias_dtype):
    k, n = 2048, 1024
    say(f"w8a8_mm scaled m={m} {dtype} row={per_row} col={per_col} bias={bias_dtype}")
    a, w = ints((m, k), 5), ints((n, k), 6)
    g = torch.Generator().manual_seed(7)
    sa = (torch.rand((m, 1) if per_row else (1,), generator=g) * 1e-2 + 1e-3).cuda()
    sb = (torch.rand((n, 1) if per_col else (1,), generator=g) * 1e-2 + 1e-3).cuda()
    bias = torch.randn(n, generator=g).to(bias_dtype).cuda() if bias_dtype else None
    got = w8a8_mm(a, w.t(), sa, sb, dtype, bias)
    assert got.dtype == dtype
    assert np.array_equal(as_np(got), oracle_out(a, w, sa, sb, bias, dtype))
    # the reference's own check (tests/test_kernel.py:68-75): rel < 1e-2 of max(|ref|,|term|)
    term = (np_(a).astype(np.float64) @ np_(w).astype(np.float64).T) * \
        np_(sa).astype(np.float64).reshape(-1, 1) * np_(sb).astype(np.float64).reshape(1, -1)
    ref = term + np_(bias.float()).astype(np.float64) if bias is not None else term
    scale = np.maximum(np.abs(ref), np.abs(term)).clip(1e-6)
    assert (np.abs(np_(got.float()).astype(np.float64) - ref) / scale).max() < 1e-2
    if bias is None and dtype == torch.bfloat16:
        # within one bf16 ulp of float64
        ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - 7)
        assert np.all(np.abs(np_(got.float()).astype(np.float64) - ref) <= ulp)


@pytest.mark.parametrize("nc", [4, 8, 16])
@pytest.mark.parametrize("m", [1, 7, 16])
def test_twelve_wave_tiles(nc, m):
    """Weights-through-LDS tiles with 12 waves (not a power of two; 256-byte steps, two a
    wave at K = 6144, a tuner candidate): every epilogue kind, bit-exact against the oracle."""
    k, n = 6144, 512
    cfg = Config(16, nc, 256, 12, 3, 1)
    assert kernel.supported(m, n, k, cfg)
    say(f"w8a8_mm {cfg.name} m={m} k={k} n={n}")
    a, w = ints((m, k), 61 + nc), ints((n, k), 62 + m)
    g = torch.Generator().manual_seed(63)
    sa = (torch.rand((m, 1), generator=g) * 1e-2 + 1e-3).cuda()
    sb = (torch.rand((n, 1), generator=g) * 1e-2 + 1e-3).cuda()
    one = torch.ones(1, device="cuda")
    assert np.array_equal(np_(w8a8_mm(a, w.t(), one, one, raw=True, config=cfg)),
                          o.gemm_i32(np_(a), np_(w)))
    for dtype, bias_dtype in ((torch.bfloat16, None), (torch.bfloat16, torch.bfloat16),
                              (torch.float32, torch.float16)):
        bias = torch.randn(n, generator=g).to(bias_dtype).cuda() if bias_dtype else None
        out = w8a8_mm(a, w.t(), sa, sb, dtype, bias, config=cfg)
        assert np.array_equal(as_np(out), oracle_out(a, w, sa, sb, bias, dtype)), (dtype, bias_dtype)


@pytest.mark.parametrize("m,n", [(5, 24), (40, 8), (100, 40), (300, 24), (1500, 12)])
def test_default_config_narrow_n(m, n):
    """N not a multiple of 16 takes the library default's 8- or 4-column streaming tiles."""
    k = 2112
    say(f"w8a8_mm default narrow N m={m} n={n} k={k}")
    a, w = ints((m, k), 51), ints((n, k), 52)
    sa = torch.rand((m, 1), device="cuda") * 1e-2 + 1e-3
    sb = torch.rand((n, 1), device="cuda") * 1e-2 + 1e-3
    assert kernel.default_config(m, n, k).bn == (8 if n % 8 == 0 else 4)
    out = w8a8_mm(a, w.t(), sa, sb, torch.bfloat16, config=kernel.default_config(m, n, k))
    assert np.array_equal(bits(out), oracle_out(a, w, sa, sb, None, torch.bfloat16))


def test_declines_shapes_the_tiles_do_not_divide():
    a, w = ints((4, 100), 8), ints((64, 100), 9)
    one = torch.ones(1, device="cuda")
    with pytest.raises(NotSupported):
        w8a8_mm(a, w.t(), one, one)


def test_replays_inside_a_hip_graph():
    m, k, n = 16, 2048, 2048
    say("w8a8_mm graph capture m=16")
    a, w = ints((m, k), 10), ints((n, k), 11)
    sa = torch.full((m, 1), 1e-2, device="cuda")
    sb = torch.full((n, 1), 1e-2, device="cuda")
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        w8a8_mm(a, w.t(), sa, sb)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = w8a8_mm(a, w.t(), sa, sb)
    for seed in (12, 13, 14):
        a.copy_(ints((m, k), seed))  # new input in the same buffer
        graph.replay()
        torch.cuda.synchronize()
        eager = w8a8_mm(a, w.t(), sa, sb)
        torch.cuda.synchronize()
        assert torch.equal(static_out, eager)
        assert np.array_equal(bits(eager), oracle_out(a, w, sa, sb, None, torch.bfloat16))


def test_exact_on_an_odd_pointer():
    m, k, n = 5, 2048, 1024
    say("w8a8_mm odd A pointer (generic schedule)")
    a, w = offset_ints((m, k), 23), ints((n, k), 24)
    assert a.data_ptr() % 2 == 1
    one = torch.ones(1, device="cuda")
    for _ in range(3):
        assert np.array_equal(np_(w8a8_mm(a, w.t(), one, one, raw=True)), o.gemm_i32(np_(a), np_(w)))


def test_exact_on_an_n_contiguous_weight():
    m, k, n = 9, 256, 48
    say("w8a8_mm N-contiguous B (generic schedule)")
    a = ints((m, k), 25)
    b = ints((k, n), 26)                      # [K, N] row-major: stride (N, 1)
    sa = torch.rand((m, 1), device="cuda") + 0.5
    sb = torch.rand((n, 1), device="cuda") + 0.5
    got = w8a8_mm(a, b, sa, sb, torch.float32)
    w = b.t().contiguous()
    assert np.array_equal(np_(got), oracle_out(a, w, sa, sb, None, torch.float32))


@pytest.mark.parametrize("m,k,n", [(1, 64, 16), (3, 128, 48), (65, 256, 80), (130, 2048, 256),
                                   (33, 512, 96), (200, 1024, 272), (7, 0, 16)])
@pytest.mark.parametrize("layout", ["a_t_b_n", "a_k_b_n", "a_t_b_k", "a_strided_b_strided"])
def test_generic_schedule_any_layout(m, k, n, layout):
    """The generic kernel (any strides; M, N and K that are not multiples of its 64 x 64 x 64
    tile, K = 0): transposed A (column-major), N-contiguous B, and both read through strided
    views, against the oracle, int32 and bf16 with a bias and scalar scales.  The shapes pass
    the reference's decline rule (N % bn, K % bk) under the default config."""
    say(f"w8a8_mm generic m={m} k={k} n={n} {layout}")
    a0, w0 = ints((m, k), 41 + m), ints((n, k), 42 + n)
    if layout.startswith("a_t"):
        a = a0.t().contiguous().t()                     # strides (1, M)
    elif layout.startswith("a_strided"):
        a = torch.zeros((m, 2 * k), dtype=torch.int8, device="cuda")[:, ::2]
        a.copy_(a0)
    else:
        a = a0
    if layout.endswith("b_n"):
        b = w0.t().contiguous()                         # [K, N] row-major: strides (N, 1)
    elif layout.endswith("b_strided"):
        b = torch.zeros((k, 3 * n), dtype=torch.int8, device="cuda")[:, ::3]
        b.copy_(w0.t())
    else:
        b = w0.t()                                      # K-contiguous (N, K) view
    one = torch.ones(1, device="cuda")
    acc = o.gemm_i32(np_(a0), np_(w0)) if k else np.zeros((m, n), np.int32)
    assert np.array_equal(np_(w8a8_mm(a, b, one, one, raw=True)), acc)
    g = torch.Generator().manual_seed(m * n + k)
    sa = (torch.rand((1,), generator=g) * 1e-2 + 1e-3).cuda()
    sb = (torch.rand((1,), generator=g) * 1e-2 + 1e-3).cuda()
    bias = torch.randn(n, generator=g).to(torch.bfloat16).cuda()
    out = w8a8_mm(a, b, sa, sb, torch.bfloat16, bias)
    ref = o.epilogue(acc, np_(sa), np_(sb), bits(bias), o.BF16, o.BF16)
    assert np.array_equal(bits(out), ref)


def test_generic_schedule_is_not_a_scalar_loop():
    """An N-contiguous weight at a decode shape takes the generic kernel; it must stay
    within a small factor of the fast schedule on the same product (the scalar per-output
    loop it replaced was ~100x slower)."""
    m, k, n = 64, 2048, 2048
    a, w = ints((m, k), 51), ints((n, k), 52)
    b_n = w.t().contiguous()
    one = torch.ones(1, device="cuda")
    assert torch.equal(w8a8_mm(a, b_n, one, one, raw=True), w8a8_mm(a, w.t(), one, one, raw=True))

    def timed(b):
        for _ in range(3):
            w8a8_mm(a, b, one, one, raw=True)
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(20):
            w8a8_mm(a, b, one, one, raw=True)
        e.record()
        e.synchronize()
        return s.elapsed_time(e) / 20
    fast, generic = timed(w.t()), timed(b_n)
    say(f"generic {generic * 1e3:.1f} us vs fast {fast * 1e3:.1f} us")
    assert generic < 20 * fast + 0.05


def test_empty_batch():
    a = torch.empty((0, 2048), dtype=torch.int8, device="cuda")
    w = ints((1024, 2048), 1)
    out = w8a8_mm(a, w.t(), torch.ones(1, device="cuda"), torch.ones(1, device="cuda"))
    assert out.shape == (0, 1024)


def test_golden_fixtures():
    from pathlib import Path
    gdir = Path(__file__).resolve().parent / "golden"
    for name in ("gemm_small", "gemm_config0"):
        say(f"w8a8_mm golden {name}")
        f = np.load(gdir / f"{name}.npz")
        a = torch.from_numpy(f["a"]).cuda()
        w = torch.from_numpy(f["w"]).cuda()
        sa, sb = torch.from_numpy(f["sa"]).cuda(), torch.from_numpy(f["sb"]).cuda()
        one = torch.ones(1, device="cuda")
        assert np.array_equal(np_(w8a8_mm(a, w.t(), one, one, raw=True)), f["raw"])
        assert np.array_equal(bits(w8a8_mm(a, w.t(), sa, sb)), f["out_bf16"])
        bias = torch.from_numpy(f["bias_bf16"].view(np.int16)).view(torch.bfloat16).cuda()
        key = "out_bf16_bias_bf16" if name == "gemm_small" else "out_bf16_bias"
        assert np.array_equal(bits(w8a8_mm(a, w.t(), sa, sb, torch.bfloat16, bias)), f[key])
        if name == "gemm_small":
            bf = torch.from_numpy(f["bias_f32"]).cuda()
            assert np.array_equal(bits(w8a8_mm(a, w.t(), sa, sb, torch.float16, bf)),
                                  f["out_f16_bias_f32"])
            out = w8a8_mm(a, w.t(), sa[:1, :1].reshape(1), sb[:1, :1].reshape(1), torch.float32)
            assert np.array_equal(np_(out), f["out_f32_scalar"])


# the four Qwen3-1.7B shapes at every decode M, bias off and on.
DECODE_M = [1, 2, 4, 8, 16, 17, 32, 64, 128]


@pytest.mark.parametrize("shape", SHAPES["qwen3-1.7b-vllm"], ids=lambda s: s[0])
@pytest.mark.parametrize("with_bias", [False, True])
def test_decode_sweep_is_bit_exact(shape, with_bias):
    _, k, n = shape
    for m in DECODE_M:
        say(f"decode sweep {shape[0]} m={m} bias={with_bias}")
        d = operands(m, k, n, seed_of(m, k, n), with_bias=with_bias, device="cuda")
        got = w8a8_mm(d["a_q"], d["w_qt"], d["a_s"], d["w_s"], torch.bfloat16, d["bias"])
        ref = oracle_out(d["a_q"], d["w_q"], d["a_s"], d["w_s"], d["bias"], torch.bfloat16)
        assert np.array_equal(bits(got), ref), (shape, m, with_bias)


def matvec(w: np.ndarray, v: np.ndarray) -> np.ndarray:
    """Exact int64 W[N,K] @ v[K] in row chunks (no full int64 copy of W)."""
    return np.concatenate([w[i:i + 2048].astype(np.int64) @ v for i in range(0, w.shape[0], 2048)])


# Llama-3-8B shapes at prefill M, full size, on BASELINE's operands
# (x ~ N(0,1), W ~ N(0,0.02), bias ~ N(0,0.01), each quantized per row as the reference's
# bench/bench_linear.py:146-167 does).
def _baseline_weight(k, n, seed):
    """W ~ N(0, 0.02) [N, K] and bias ~ N(0, 0.01) [N] in bf16, quantized per output channel."""
    from int8_linear.operands import quant_rows
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn((n, k), generator=g) * 0.02).to(torch.bfloat16)
    bias = (torch.randn((n,), generator=g) * 0.01).to(torch.bfloat16)
    w_q, w_s = quant_rows(w)
    return w_q, w_s, bias


def _baseline_acts(m, k, seed):
    from int8_linear.operands import quant_rows
    g = torch.Generator().manual_seed(seed)
    return quant_rows(torch.randn((m, k), generator=g).to(torch.bfloat16))


def _sample_rows(m, rng, tile=256, count=32):
    """The first and last row of the first, second and last row tiles (and of the middle
    one), row M-1, then random rows up to `count`."""
    edges = {0, tile - 1, tile, 2 * tile - 1, m // 2 - 1, m // 2, m - tile, m - 1}
    rows = {r for r in edges if 0 <= r < m}
    while len(rows) < count:
        rows.add(int(rng.integers(m)))
    return np.array(sorted(rows))


@pytest.mark.parametrize("shape", SHAPES["llama-3-8b"], ids=lambda s: s[0])
def test_prefill_full_size_checksums_and_rows(shape):
    """Exact int32 row and column checksums of the whole product, then 32 rows per M (tile
    edges included) compared bit for bit in int32 and, with bias, in bf16."""
    _, k, n = shape
    rng = np.random.default_rng(k + n)
    w_q, w_s, bias = _baseline_weight(k, n, k * 7 + n)
    w_np = np_(w_q)
    wsum_k = w_np.sum(axis=0, dtype=np.int64)     # [K]: sum over n of W[n, k]
    w, ws, bias_d = w_q.cuda(), w_s.cuda(), bias.cuda()
    one = torch.ones(1, device="cuda")
    for m in (512, 1024, 2048, 4096):
        say(f"prefill {shape[0]} m={m} k={k} n={n} (BASELINE operands, bias)")
        a_q, a_s = _baseline_acts(m, k, m + k)
        a, sa = a_q.cuda(), a_s.cuda()
        a_np = np_(a_q).astype(np.int64)
        got = w8a8_mm(a, w.t(), one, one, raw=True)
        # row checksums: sum_n C[m,n] = A[m,:] . (sum_n W[n,:]); column checksums likewise
        assert np.array_equal(np_(got.sum(dim=1, dtype=torch.int64)), a_np @ wsum_k)
        assert np.array_equal(np_(got.sum(dim=0, dtype=torch.int64)), matvec(w_np, a_np.sum(axis=0)))
        rows = _sample_rows(m, rng)
        idx = torch.from_numpy(rows).cuda()
        acc = o.gemm_i32(np_(a_q)[rows], w_np)
        assert np.array_equal(np_(got[idx]), acc)
        out = w8a8_mm(a, w.t(), sa, ws, torch.bfloat16, bias_d)
        ref = o.epilogue(acc, np_(a_s)[rows], np_(w_s), bits(bias), o.BF16, o.BF16)
        assert np.array_equal(bits(out[idx]), ref)
        out = w8a8_mm(a, w.t(), sa, ws, torch.bfloat16)
        ref = o.epilogue(acc, np_(a_s)[rows], np_(w_s), None, o.NONE, o.BF16)
        assert np.array_equal(bits(out[idx]), ref)
        del got, out


# The prefill tiles' epilogue in every output dtype, bias dtype and scale shape (the decode
# tiles take these at M = 13 and 37 in test_scaled_output_matches_oracle_and_float64): one
# tile of each prefill schedule (overlapped ring, ring, register-staged) and a 192-wide one.
PREFILL_EPILOGUE_TILES = [Config(128, 128, 128, 4, 12, 8), Config(256, 256, 64, 8, 12, 4),
                          Config(256, 192, 64, 4, 12, 4), Config(256, 256, 64, 8, 3, 8),
                          Config(128, 128, 64, 4, 2, 8), Config(256, 256, 128, 8, 10, 4),
                          Config(256, 192, 128, 8, 10, 4)]


@pytest.mark.parametrize("config", PREFILL_EPILOGUE_TILES, ids=lambda c: c.name.replace(" ", "_"))
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_prefill_epilogue_every_dtype_bias_and_scale(config, dtype):
    m, k, n = 300, 2048, 1536
    a, w = ints((m, k), 31), ints((n, k), 32)
    g = torch.Generator().manual_seed(33)
    for per_row, per_col in ((True, True), (True, False), (False, True)):
        sa = (torch.rand((m, 1) if per_row else (1,), generator=g) * 1e-2 + 1e-3).cuda()
        sb = (torch.rand((n, 1) if per_col else (1,), generator=g) * 1e-2 + 1e-3).cuda()
        for bias_dtype in (None, torch.bfloat16, torch.float16, torch.float32):
            say(f"prefill epilogue {config.name} {dtype} row={per_row} col={per_col} "
                f"bias={bias_dtype}")
            bias = torch.randn(n, generator=g).to(bias_dtype).cuda() if bias_dtype else None
            got = w8a8_mm(a, w.t(), sa, sb, dtype, bias, config=config)
            assert got.dtype == dtype
            assert np.array_equal(as_np(got), oracle_out(a, w, sa, sb, bias, dtype)), \
                (per_row, per_col, bias_dtype)


def test_long_prefill_offsets_pass_two_to_the_31():
    """M * K > 2^31 (M = 150000, K = 14336, Llama-3-8B down_proj): the reference indexes A
    with int64 for this case (int8_linear/kernel.py:85-86).  Rows on both sides of
    m * K = 2^31 and the last row tile are compared exactly with the oracle, in int32 and in
    bf16 with bias; the column checksums cover every row of the product."""
    m, k, n = 150_000, 14336, 4096
    assert m * k > 2 ** 31
    say(f"long prefill m={m} k={k} n={n} (M*K = {m * k})")
    w_q, w_s, bias = _baseline_weight(k, n, 77)
    w_np = np_(w_q)
    w, ws, bias_d = w_q.cuda(), w_s.cuda(), bias.cuda()
    g = torch.Generator(device="cuda").manual_seed(78)
    a = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8, device="cuda")
    sa = torch.rand((m, 1), generator=g, device="cuda") * 1e-2 + 1e-3
    one = torch.ones(1, device="cuda")
    got = w8a8_mm(a, w.t(), one, one, raw=True)
    edge = 2 ** 31 // k
    rows = np.array(sorted({0, 1, edge - 1, edge, edge + 1, m - 257, m - 256, m - 2, m - 1,
                            m // 2}))
    idx = torch.from_numpy(rows).cuda()
    a_rows = np_(a[idx])
    acc = o.gemm_i32(a_rows, w_np)
    assert np.array_equal(np_(got[idx]), acc)
    # column checksums: sum_m C[m, n] = (sum_m A[m, :]) . W[n, :], exact in int64
    a_colsum = np_(a.sum(dim=0, dtype=torch.int64))
    assert np.array_equal(np_(got.sum(dim=0, dtype=torch.int64)), matvec(w_np, a_colsum))
    del got
    out = w8a8_mm(a, w.t(), sa, ws, torch.bfloat16, bias_d)
    ref = o.epilogue(acc, np_(sa)[rows], np_(w_s), bits(bias), o.BF16, o.BF16)
    assert np.array_equal(bits(out[idx]), ref)


# The split of K across workgroups (stages 5): tiles up to 64 columns with K in 2, 4 and 8
# parts of one or two steps a wave, ragged M; the int32 product exact, then every output
# dtype, bias dtype and scale layout through the sum kernel's epilogue.
SPLIT_TILES = [(1, 16, 2), (2, 32, 2), (4, 32, 2), (8, 16, 2), (1, 64, 2), (2, 64, 2),
               (4, 64, 2), (2, 64, 4)]


@pytest.mark.parametrize("tile", SPLIT_TILES, ids=lambda t: f"mt{t[0]}_nc{t[1]}_ks{t[2]}")
@pytest.mark.parametrize("parts", [2, 4, 8])
@pytest.mark.parametrize("waves,n", [(4, 512), (8, 512), (4, 192)])
def test_split_of_k_is_exact(tile, parts, waves, n):
    """n = 512 gives the sum kernel its XCD-local order (N / bn a multiple of 8), n = 192 the
    plain one; 8 waves put the reduction area over the whole weight ring."""
    mt, nc, ks = tile
    if n % nc:
        pytest.skip(f"N={n} is not whole {nc}-column tiles")
    for steps in (1, 2):
        k = 64 * ks * waves * steps * parts
        cfg = Config(16 * mt, nc, 64 * ks, waves, 5, parts)
        if not kernel.supported(16 * mt, n, k, cfg):
            assert waves == 8, cfg.name       # every 4-wave split tile is built
            pytest.skip(f"{cfg.name} is not built for K={k}")
        for m in sorted({1, 16 * mt - 3, 16 * mt}):
            say(f"w8a8_mm split m={m} k={k} n={n} config={cfg.name}")
            a, w = ints((m, k), 21 + m), ints((n, k), 22 + steps)
            one = torch.ones(1, device="cuda")
            acc = o.gemm_i32(np_(a), np_(w))
            assert np.array_equal(np_(w8a8_mm(a, w.t(), one, one, raw=True, config=cfg)), acc)
            g = torch.Generator().manual_seed(m + parts)
            sa = (torch.rand((m, 1), generator=g) * 1e-2 + 1e-3).cuda()
            sb = (torch.rand((n, 1), generator=g) * 1e-2 + 1e-3).cuda()
            for dtype, bias in ((torch.bfloat16, None),
                                (torch.bfloat16, torch.randn(n, generator=g).to(torch.bfloat16)),
                                (torch.float16, torch.randn(n, generator=g).to(torch.float16)),
                                (torch.float32, torch.randn(n, generator=g))):
                bias = bias.cuda() if bias is not None else None
                out = w8a8_mm(a, w.t(), sa, sb, dtype, bias, config=cfg)
                assert np.array_equal(as_np(out), oracle_out(a, w, sa, sb, bias, dtype)), \
                    (dtype, bias is not None)
            sb1 = sb[:1].reshape(1)
            out = w8a8_mm(a, w.t(), sa, sb1, torch.bfloat16, config=cfg)   # scalar scale_b
            assert np.array_equal(bits(out), oracle_out(a, w, sa, sb1, None, torch.bfloat16))


@pytest.mark.parametrize("m,k,n,cfg", [
    (128, 6144, 2048, Config(64, 64, 128, 4, 5, 4)),      # Qwen3 down_proj
    (64, 6144, 2048, Config(64, 64, 128, 6, 5, 8)),
    (128, 14336, 4096, Config(64, 64, 128, 4, 5, 4)),     # Llama-3-8B down_proj
    (32, 14336, 4096, Config(32, 64, 128, 4, 5, 4)),
], ids=["qwen_down_128", "qwen_down_64", "llama_down_128", "llama_down_32"])
def test_split_of_k_at_decode_shapes(m, k, n, cfg):
    """The BASELINE operand distributions (x ~ N(0,1), W ~ N(0,0.02), both quantized per row)
    with a bias, at the down_proj shapes the split is for; bit-exact against the oracle and
    the unsplit schedule."""
    say(f"split decode shape m={m} k={k} n={n} {cfg.name}")
    d = operands(m, k, n, seed_of(m, k, n), with_bias=True, device="cuda")
    got = w8a8_mm(d["a_q"], d["w_qt"], d["a_s"], d["w_s"], torch.bfloat16, d["bias"], config=cfg)
    ref = oracle_out(d["a_q"], d["w_q"], d["a_s"], d["w_s"], d["bias"], torch.bfloat16)
    assert np.array_equal(bits(got), ref)
    unsplit = w8a8_mm(d["a_q"], d["w_qt"], d["a_s"], d["w_s"], torch.bfloat16, d["bias"],
                      config=Config(cfg.bm, cfg.bn, cfg.bk, 4, 3, 1))
    assert torch.equal(got, unsplit)


def test_split_of_k_needs_a_workspace_and_replays_in_a_graph():
    """The workspace-less entry declines a split (it cannot allocate), the workspace entry
    rejects one too small; under graph capture the partial planes come from the graph's
    pool and every replay sums the current inputs."""
    m, k, n = 48, 4096, 1024
    cfg = Config(32, 64, 128, 4, 5, 4)
    a, w = ints((m, k), 3), ints((n, k), 4)
    one = torch.ones(1, device="cuda")
    out = torch.empty((m, n), dtype=torch.int32, device="cuda")
    L = _lib.lib()
    args = (a.data_ptr(), a.stride(0), 1, w.data_ptr(), 1, w.stride(0), one.data_ptr(), 1,
            one.data_ptr(), 1, None, _lib.DTYPE_NONE, out.data_ptr(), n, _lib.I32, m, n, k)
    c = kernel._cconfig(cfg)
    st = L.i8l_w8a8_mm(*args, c, _lib.stream_of(a))
    assert st == _lib.UNSUPPORTED and "workspace" in _lib.last_error()
    need = L.i8l_w8a8_mm_workspace_bytes(m, n, k, c)
    assert need == 4 * m * n * 4
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    assert L.i8l_w8a8_mm_ws(*args, ws.data_ptr(), need - 16, c, _lib.stream_of(a)) == _lib.INVALID_ARG
    assert L.i8l_w8a8_mm_ws(*args, ws.data_ptr(), need, c, _lib.stream_of(a)) == _lib.OK
    torch.cuda.synchronize()
    assert np.array_equal(np_(out), o.gemm_i32(np_(a), np_(w)))

    sa = torch.full((m, 1), 1e-3, device="cuda")
    sb = torch.full((n, 1), 2e-3, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        w8a8_mm(a, w.t(), sa, sb, torch.bfloat16, config=cfg)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = w8a8_mm(a, w.t(), sa, sb, torch.bfloat16, config=cfg)
    for seed in (5, 6, 7):
        a.copy_(ints((m, k), seed))
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(got), oracle_out(a, w, sa, sb, None, torch.bfloat16)), seed


def test_random_configs_against_the_oracle():
    """Seeded random cases over the whole built configuration space: a random shape, a
    random configuration from the tuner's candidates for it (every schedule family: weight
    streaming, weights through LDS, persistent, split of K, prefill tiles), random scale
    layouts, bias and output dtype; each output against the oracle bit for bit."""
    from int8_linear.tune import candidate_configs
    rng = np.random.default_rng(2026)
    ks = [1024, 2048, 3072, 4096, 6144]
    ns = [256, 512, 768, 1024, 2048]
    ms = [1, 2, 3, 7, 16, 17, 31, 48, 64, 100, 128, 200, 256, 300, 513]
    cases = 0
    families = set()
    while cases < 120:
        m, k, n = int(rng.choice(ms)), int(rng.choice(ks)), int(rng.choice(ns))
        cands = candidate_configs(m, k, n)
        if not cands:
            continue
        cfg = cands[int(rng.integers(len(cands)))]
        families.add(cfg.stages if cfg.stages < 10 else 10)
        say(f"random case {cases}: m={m} k={k} n={n} {cfg.name}")
        a, w = ints((m, k), 1000 + cases), ints((n, k), 2000 + cases)
        g = torch.Generator().manual_seed(cases)
        per_row, per_col = bool(rng.integers(2)), bool(rng.integers(2))
        sa = (torch.rand((m, 1) if per_row else (1,), generator=g) * 1e-2 + 1e-3).cuda()
        sb = (torch.rand((n, 1) if per_col else (1,), generator=g) * 1e-2 + 1e-3).cuda()
        dtype = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(3))]
        bias_dt = [None, torch.bfloat16, torch.float32][int(rng.integers(3))]
        bias = torch.randn(n, generator=g).to(bias_dt).cuda() if bias_dt else None
        out = w8a8_mm(a, w.t(), sa, sb, dtype, bias, config=cfg)
        assert np.array_equal(as_np(out), oracle_out(a, w, sa, sb, bias, dtype)), (m, k, n, cfg)
        cases += 1
    assert families >= {1, 3, 4, 5, 10}, families
