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


@pytest.mark.parametrize("m,top", [(4, 0), (32, 2)])
def test_situ_tune_pass(m, top):
    say(f"situ_tune m={m} top={top}")
    stack = DecoderStandIn(m, layers=2)
    base = stack.forward().clone()
    entry = situ_tune.situ_tune(m, layers=2, top=top, rounds=1, windows=2, stack=stack,
                                log=lambda *a: None)
    assert entry["batch"] == m and set(entry["chosen"]) == set(SHAPES)
    tried = {t["layer"] for t in entry["trials"]}
    assert tried == set(SHAPES) - ({"o_proj"} if stack.fused_o else set())
    chosen = {name: Config(**c) for name, c in entry["chosen"].items()}
    for name, (k, n) in SHAPES.items():
        assert kernel.supported(m, n, k, chosen[name]), (name, chosen[name].name)
        # each chosen configuration is the fastest trial of its layer
        rows = [t for t in entry["trials"] if t["layer"] == name]
        if rows:
            assert chosen[name].name == min(rows, key=lambda t: t["us"])["config"]
    if entry["chosen"] == entry["start"]:
        assert not entry["kept"] and "confirm_us" not in entry
    else:
        t = entry["confirm_us"]
        assert entry["kept"] == (t["chosen"] < t["start"] * (1 - situ_tune.ACCEPT))
    rows = situ_tune.table_rows(entry)
    assert bool(rows) == entry["kept"]
    stack.configs = chosen
    assert torch.equal(stack.forward(), base)
