"""In-situ tuning: each linear's configuration chosen by the 28-layer stand-in's step time.

The reference tunes in a stand-in for the served model because isolated per-layer timings
mispredicted it (AshrithaG/int8-linear, bench/situ_tune.py:1-34 and 214-255; README
"in-situ tuning"): one kernel replayed on one weight, back to back, is not the served
decode step, where 28 layers with their own weights run with the quantizers between them.

For a batch of m tokens this makes one pass over the four linears of the stand-in
(int8_linear.standin): each linear tries its current configuration (the tuned table's or the
library default's), the library default and the `top` fastest configurations of an
isolated sweep of that shape, with the other three fixed, and keeps whichever makes the
stand-in's step (one HIP graph of all 28 layers) fastest.  The chosen set is then timed
against the starting set in alternating fresh captures, and kept only if it is at least
ACCEPT faster (reference situ_tune.py:237-246).  Kept sets can be merged into the tuned
table, each entry carrying its stand-in time.  A configuration never changes a result, only
its speed.

Not done here: the reference's check of its stand-in against two served vLLM runs
(situ_tune.py:172-211), which needs vLLM and the served models.  o_proj is not tuned when
the stand-in folds its quantizer into the GEMM (fused_quant.quant_mm, up to
fused_quant.QUANT_MM_MAX_M tokens), since that kernel takes its own tile.

    python -m int8_linear.situ_tune --m 1,8,32,128 [--top 4] [--merge]
"""

from __future__ import annotations

import argparse
import json
import statistics
import sys
from dataclasses import asdict

import torch

from int8_linear import tune
from int8_linear.kernel import Config, choose_config, default_config, supported, w8a8_mm
from int8_linear.operands import operands, seed_of
from int8_linear.standin import SHAPES, DecoderStandIn, per_layer_us

ACCEPT = 0.01  # a chosen set must beat the starting one by this fraction to be kept


def isolated_top(m: int, k: int, n: int, top: int, device) -> list[Config]:
    """The `top` fastest built configurations of one shape timed alone (cold weights, one
    window each): the candidates an isolated sweep would offer (reference: the per-layer
    sweep's best rows, situ_tune.py:220-224)."""
    if top <= 0:
        return []
    d = operands(m, k, n, seed_of(m, k, n), device=device)
    copies = max(2, -(-tune.ROTATE_BYTES // (k * n)))
    ws = [d["w_q"]] + [d["w_q"].clone() for _ in range(copies - 1)]
    timed = []
    for cfg in tune.candidate_configs(m, k, n):
        us = tune.time_cold_us(lambda i, c=cfg: w8a8_mm(d["a_q"], ws[i % copies].t(), d["a_s"],
                                                        d["w_s"], torch.bfloat16, config=c),
                               copies, windows=1)
        timed.append((us, cfg))
    del ws
    torch.cuda.empty_cache()
    return [c for _, c in sorted(timed, key=lambda t: t[0])[:top]]


def step_us(stack: DecoderStandIn, configs: dict, windows: int) -> float:
    """Microseconds per layer of the stand-in's step under `configs` (a fresh capture)."""
    stack.configs = dict(configs)
    try:
        return per_layer_us(stack, windows)
    finally:
        stack.configs = {}


def alternating(stack: DecoderStandIn, options: dict, rounds: int, windows: int) -> dict:
    """Each option timed in fresh captures, in rotation; the median over the rounds."""
    times: dict = {key: [] for key in options}
    for _ in range(rounds):
        for key, configs in options.items():
            times[key].append(step_us(stack, configs, windows))
    return {key: statistics.median(v) for key, v in times.items()}


def situ_tune(m: int, layers: int = 28, top: int = 4, rounds: int = 5, windows: int = 5,
              stack: DecoderStandIn | None = None, device="cuda", log=print) -> dict:
    """One in-situ pass for batch m.  Returns {"batch", "start", "chosen" (Config dicts),
    "trials", "confirm_us" (start/chosen, when they differ), "kept"}."""
    stack = stack or DecoderStandIn(m, layers=layers, device=device)
    start = {name: choose_config(m, n, k) for name, (k, n) in SHAPES.items()}
    tunable = [name for name in SHAPES if not (name == "o_proj" and stack.fused_o)]
    current = dict(start)
    trials = []
    for name in tunable:
        k, n = SHAPES[name]
        options = list(dict.fromkeys([current[name], default_config(m, n, k),
                                      *isolated_top(m, k, n, top, device)]))
        best = None
        for cfg in options:
            if not supported(m, n, k, cfg):
                continue
            us = step_us(stack, {**current, name: cfg}, windows)
            trials.append({"layer": name, "config": cfg.name, "us": round(us, 3)})
            log(f"M={m} {name} {cfg.name}: {us:.2f} us a layer")
            if best is None or us < best[1]:
                best = (cfg, us)
        current[name] = best[0]
    entry = {"batch": m, "start": {k: asdict(v) for k, v in start.items()},
             "chosen": {k: asdict(v) for k, v in current.items()}, "trials": trials,
             "kept": False}
    if current != start:
        t = alternating(stack, {"start": start, "chosen": current}, rounds, windows)
        entry["confirm_us"] = {key: round(v, 3) for key, v in t.items()}
        entry["kept"] = t["chosen"] < t["start"] * (1 - ACCEPT)
    log(f"M={m}: " + ", ".join(f"{name} {start[name].name} -> {current[name].name}"
                               for name in SHAPES if start[name] != current[name])
        + f"; confirm {entry.get('confirm_us')}; kept {entry['kept']}")
    return entry


def table_rows(entry: dict) -> dict:
    """A kept entry as tuned-table rows {"KxN": {str(m): {"config", "stand_in_us"}}}."""
    if not entry["kept"]:
        return {}
    return {f"{k}x{n}": {str(entry["batch"]): {"config": entry["chosen"][name],
                                                "stand_in_us": entry["confirm_us"]["chosen"]}}
            for name, (k, n) in SHAPES.items()}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--m", default="1,8,32,128", help="comma-separated batch sizes")
    ap.add_argument("--layers", type=int, default=28)
    ap.add_argument("--top", type=int, default=4, help="isolated-sweep candidates per linear")
    ap.add_argument("--rounds", type=int, default=5)
    ap.add_argument("--windows", type=int, default=5)
    ap.add_argument("--merge", action="store_true", help="write kept sets into tuned_configs.json")
    ap.add_argument("--out", default=None, help="also write the entries to this JSON file")
    args = ap.parse_args()
    dev = torch.device("cuda:0")
    arch = torch.cuda.get_device_properties(dev).gcnArchName.split(":")[0]
    entries, table = [], {}
    stack = None
    for m in tune.parse_ms(args.m):
        stack = stack.with_batch(m) if stack is not None else DecoderStandIn(m, args.layers,
                                                                             device=dev)
        e = situ_tune(m, args.layers, args.top, args.rounds, args.windows, stack, dev,
                      log=lambda *a: print(*a, file=sys.stderr, flush=True))
        entries.append(e)
        for kn, rows in table_rows(e).items():
            table.setdefault(kn, {}).update(rows)
    if args.out:
        with open(args.out, "w") as f:
            json.dump({arch: entries}, f, indent=1)
    if args.merge and table:
        tune.merge(table, arch)
    print(json.dumps({arch: {"entries": entries, "kept": table}}))
    return 0


if __name__ == "__main__":
    sys.exit(main())
