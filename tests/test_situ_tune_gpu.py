"""In-situ tuning in the decoder stand-in (reference bench/situ_tune.py:214-255 of
AshrithaG/int8-linear): one pass over the four linears on a short stand-in, the chosen set
made only of built configurations, kept only when the alternating confirmation shows it
faster, and a stand-in step under the chosen set bit-identical to the step under the
starting set (a configuration changes speed, never results)."""

from __future__ import annotations

import pytest
import torch

from helpers import say
from int8_linear import Config, kernel, situ_tune
from int8_linear.standin import SHAPES, DecoderStandIn

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,top", [(4, 0), (8, 0), (32, 2)])
def test_situ_tune_pass(m, top):
    """At 4 tokens the norm-folded qkv and gate_up are tuned (o_proj and down_proj run the
    folded quantizers' own tiles), at 8 qkv on w8a8_mm and gate_up with the SiLU epilogue, at
    32 all four on w8a8_mm."""
    say(f"situ_tune m={m} top={top}")
    stack = DecoderStandIn(m, layers=2)
    base = stack.forward().clone()
    entry = situ_tune.situ_tune(m, layers=2, top=top, rounds=1, windows=2, stack=stack,
                                log=lambda *a: None)
    kinds = entry["kernels"]
    assert entry["batch"] == m and set(entry["chosen"]) == set(SHAPES)
    assert kinds == situ_tune.kernels(stack)
    tried = {t["layer"] for t in entry["trials"]}
    assert tried == {name for name, kind in kinds.items() if kind is not None}
    chosen = {name: Config(**c) if c is not None else None for name, c in entry["chosen"].items()}
    for name, (k, n) in SHAPES.items():
        if kinds[name] is None:
            assert chosen[name] is None
            continue
        assert situ_tune.kind_supported(kinds[name], m, n, k, chosen[name]), name
        # each chosen configuration is the fastest trial of its layer
        rows = [t for t in entry["trials"] if t["layer"] == name]
        label = chosen[name].name if chosen[name] is not None else "default"
        assert label == min(rows, key=lambda t: t["us"])["config"]
    if entry["chosen"] == entry["start"]:
        assert not entry["kept"] and "confirm_us" not in entry
    else:
        t = entry["confirm_us"]
        assert entry["kept"] == (t["chosen"] < t["start"] * (1 - situ_tune.ACCEPT))
    rows = situ_tune.table_rows(entry)
    assert set(rows) == ({f"{k}x{n}" for name, (k, n) in SHAPES.items() if kinds[name] == "mm"}
                         if entry["kept"] else set())
    situ_tune.apply(stack, chosen, kinds)
    assert torch.equal(stack.forward(), base)
