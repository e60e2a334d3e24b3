"""Every configuration of the shipped MI355X tuned table (int8_linear/tuned_configs.json), on
its own weight shape, is bit-exact against the CPU oracle: the table picks among the built
schedules per (K, N, M bucket), so each entry is a launch users get.  M is the entry's
bucket, capped at 64 tokens to keep the oracle's work small (the schedules' arithmetic does
not depend on M; the row tails of ragged M are covered by the tiling tests)."""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from helpers import bits, np_, say
from int8_linear import Config, kernel, w8a8_mm
from int8_linear.operands import operands, seed_of
from oracle import oracle as o

pytestmark = pytest.mark.gpu


def table_entries():
    tables = json.loads(kernel.TUNED_PATH.read_text())
    seen, out = set(), []
    for device, shapes in sorted(tables.items()):
        for kn, buckets in sorted(shapes.items()):
            for m, row in sorted(buckets.items(), key=lambda kv: int(kv[0])):
                cfg = Config(**row["config"])
                if (kn, cfg) in seen:
                    continue
                seen.add((kn, cfg))
                k, n = map(int, kn.split("x"))
                out.append((k, n, min(int(m), 64), cfg))
    return out


@pytest.mark.parametrize("k,n,m,cfg", table_entries(),
                         ids=lambda v: v.name.replace(" ", "_") if isinstance(v, Config) else str(v))
def test_tuned_entry_is_bit_exact(k, n, m, cfg):
    say(f"tuned entry K={k} N={n} M={m} {cfg.name}")
    d = operands(m, k, n, seed_of(m, k, n), with_bias=True, device="cuda")
    got = w8a8_mm(d["a_q"], d["w_qt"], d["a_s"], d["w_s"], torch.bfloat16, d["bias"], config=cfg)
    acc = o.gemm_i32(np_(d["a_q"]), np_(d["w_q"]))
    ref = o.epilogue(acc, np_(d["a_s"]), np_(d["w_s"]), bits(d["bias"]), o.BF16, o.BF16)
    assert np.array_equal(bits(got), ref)


def test_tuner_keeps_the_stored_entry_without_a_clear_gain(monkeypatch):
    """A re-tune times the stored entry among its finalists and, under --min-gain, keeps it
    unless a candidate beats it by that fraction (here 99%, which none does)."""
    from int8_linear import tune
    k, n, m = 2048, 1024, 16
    stored = kernel.default_config(m, n, k)
    say(f"tune_shape keeps {stored.name} at m={m} k={k} n={n}")
    monkeypatch.setattr(kernel, "tuned_config", lambda mm, nn, kk: stored)
    rows = tune.tune_shape(k, n, [m], torch.device("cuda:0"), log=lambda *a: None,
                           refine=True, min_gain=0.99)
    row = rows[str(m)]
    assert Config(**row["config"]) == stored
    assert row["graph_us"] == row["table_us"] > 0
