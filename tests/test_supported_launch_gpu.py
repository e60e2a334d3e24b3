"""Every configuration a support check accepts launches and gives the default's result.

The tuner offers each shape every built configuration its support check accepts
(tune.candidate_configs), and the in-situ tuner every built tile of the folded kernels
(situ_tune.folded_candidates).  A tile the check accepts but no launcher instantiates would
raise RuntimeError at the launch instead of NotSupported before it, so here each of them runs
at decode and prefill shapes and must give the default configuration's output bit for bit:
the int32 product for w8a8_mm, the bf16 output and residual for the norm-folded projection,
y = silu(gate) * up for the SiLU epilogue."""

from __future__ import annotations

import pytest
import torch

from helpers import ints, randn, say
from int8_linear import fused_quant as fq
from int8_linear import situ_tune, tune
from int8_linear.kernel import w8a8_mm

pytestmark = pytest.mark.gpu


def scales(rows: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.rand((rows, 1), generator=g) * 1e-3 + 1e-4).cuda()


@pytest.mark.parametrize("m,k,n", [(1, 2048, 4096), (8, 2048, 12288), (17, 2048, 2048),
                                   (64, 6144, 2048), (128, 2048, 4096), (512, 4096, 4096)])
def test_every_candidate_config_launches(m, k, n):
    a, w = ints((m, k), m + k), ints((n, k), n + k + 1)
    sa, sb = scales(m, m), scales(n, n)
    ref = w8a8_mm(a, w.t(), sa, sb, raw=True)
    cands = tune.candidate_configs(m, k, n)
    say(f"supported launches: w8a8_mm m={m} k={k} n={n}, {len(cands)} configs")
    assert cands
    for cfg in cands:
        got = w8a8_mm(a, w.t(), sa, sb, raw=True, config=cfg)
        assert torch.equal(got, ref), cfg.name


@pytest.mark.parametrize("m", [1, 4, 8])
def test_every_norm_fold_tile_launches(m):
    k, n = 2048, 4096
    x, r = randn((m, k), m), randn((m, k), m + 1)
    gamma = (1 + randn((k,), 7, 0.1, torch.float32)).to(torch.bfloat16)
    w, sb = ints((n, k), n), scales(n, n)
    ref, rref = fq.add_rmsnorm_quant_mm(x, r, gamma, 1e-6, w.t(), sb)
    cands = situ_tune.folded_candidates("norm", m, n, k)
    say(f"supported launches: norm fold m={m}, {len(cands)} tiles")
    assert cands
    for cfg in cands:
        out, rout = fq.add_rmsnorm_quant_mm(x, r, gamma, 1e-6, w.t(), sb, config=cfg)
        assert torch.equal(out, ref) and torch.equal(rout, rref), cfg.name


@pytest.mark.parametrize("m,k,n", [(1, 2048, 12288), (8, 2048, 12288), (8, 6144, 2048)])
def test_every_silu_epilogue_tile_launches(m, k, n):
    a, w = ints((m, k), m + k), ints((n, k), n + k)
    sa, sb = scales(m, m), scales(n, n)
    ref = fq.w8a8_mm_silu_mul(a, w.t(), sa, sb)
    cands = situ_tune.folded_candidates("silu", m, n, k)
    say(f"supported launches: SiLU epilogue m={m} k={k} n={n}, {len(cands)} tiles")
    assert cands
    for cfg in cands:
        assert torch.equal(fq.w8a8_mm_silu_mul(a, w.t(), sa, sb, config=cfg), ref), cfg.name
