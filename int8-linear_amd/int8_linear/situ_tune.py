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

Each linear is tuned in the kernel the stand-in runs for it at that batch (`kernel_of`):
w8a8_mm ("mm", DecoderStandIn.configs), or for few tokens the norm-folded projection
("norm", fused_quant.add_rmsnorm_quant_mm, DecoderStandIn.norm_configs: its built tiles) or
gate_up with the SiLU-and-mul epilogue ("silu", fused_quant.w8a8_mm_silu_mul,
DecoderStandIn.silu_configs: the built persistent tiles of 8 and 16 columns).  A linear
whose quantizer is folded in front of it (fused_quant.quant_mm, silu_mul_quant_mm) takes
that kernel's own tile and is not tuned.  Only "mm" choices become tuned-table rows; the
folded kernels' choices are reported beside them.

Not done here: the reference's check of its stand-in against two served vLLM runs
(situ_tune.py:172-211), which needs vLLM and the served models.

    python -m int8_linear.situ_tune --m 1,8,32,128 [--top 4] [--merge]
"""

from __future__ import annotations

import argparse
import json
import statistics
import sys
from dataclasses import asdict

import torch

from int8_linear import fused_quant as fq
from int8_linear import tune
from int8_linear.kernel import Config, choose_config, default_config, supported, w8a8_mm
from int8_linear.operands import operands, seed_of
from int8_linear.standin import HIDDEN, INTER, SHAPES, DecoderStandIn, per_layer_us

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


# (NC, KS, W) of the built norm-folded tiles (bm 16, stages 4), as the library lists them
NORM_TILES = [(16, 8, 4), (16, 4, 8), (8, 8, 4), (8, 4, 8), (16, 8, 8), (8, 8, 8)]


def kernel_of(name: str, fused_norm: bool, fused_silu: bool, fused_down: bool, fused_o: bool,
              quant_down: bool) -> str | None:
    """The kernel the stand-in runs for linear `name` under its fold flags (DecoderStandIn.
    fused_norm, fused_silu, fused_down, fused_o, and whether down_proj takes quant_mm after
    the SiLU epilogue): "mm", "norm", "silu", or None where a folded quantizer's own tile
    runs (DecoderStandIn.forward)."""
    if name == "qkv_proj":
        return "norm" if fused_norm else "mm"
    if name == "o_proj":
        return None if fused_o else "mm"
    if name == "gate_up_proj":
        return "norm" if fused_norm else ("silu" if fused_silu else "mm")
    if fused_silu:
        return None if quant_down else "mm"
    return None if fused_down else "mm"


def kernels(stack: DecoderStandIn) -> dict:
    """kernel_of for each linear of the stand-in at its batch size."""
    quant_down = stack.fused_silu and fq.quant_mm_supported(stack.m, HIDDEN, INTER)
    return {name: kernel_of(name, stack.fused_norm, stack.fused_silu, stack.fused_down,
                            stack.fused_o, quant_down) for name in SHAPES}


def kind_supported(kind: str, m: int, n: int, k: int, cfg: Config | None) -> bool:
    """Whether the kernel `kind` takes `cfg` (None: its library default) for this shape."""
    if kind == "norm":
        return fq.add_rmsnorm_quant_mm_supported(m, n, k, cfg)
    if kind == "silu":
        return fq.w8a8_mm_silu_mul_supported(m, n, k, cfg)
    return cfg is not None and supported(m, n, k, cfg)


def folded_candidates(kind: str, m: int, n: int, k: int) -> list[Config]:
    """Every built tile of a folded kernel that takes the shape."""
    if kind == "norm":
        tiles = [(nc, ks, w) for nc, ks, w in NORM_TILES]
    else:
        tiles = [(nc, ks, w) for mt, nc, ks, w in tune.WLDSP_TILES if mt == 1 and nc in (8, 16)]
    out = []
    for nc, ks, w in tiles:
        for g in (1, 2, 4):
            cfg = Config(16, nc, 64 * ks, w, 4, g)
            if kind_supported(kind, m, n, k, cfg):
                out.append(cfg)
    return out


def apply(stack: DecoderStandIn, chosen: dict, kinds: dict) -> None:
    """Set the stand-in's configurations: each linear's in the dict of the kernel it runs."""
    stack.configs, stack.norm_configs, stack.silu_configs = {}, {}, {}
    target = {"mm": stack.configs, "norm": stack.norm_configs, "silu": stack.silu_configs}
    for name, cfg in chosen.items():
        if kinds.get(name) in target and cfg is not None:
            target[kinds[name]][name] = cfg


def step_us(stack: DecoderStandIn, configs: dict, windows: int, kinds: dict | None = None
            ) -> float:
    """Microseconds per layer of the stand-in's step under `configs` ({linear: Config or
    None}, each set for the kernel `kinds` names; all w8a8_mm when not given), a fresh
    capture."""
    apply(stack, configs, kinds if kinds is not None else dict.fromkeys(configs, "mm"))
    try:
        return per_layer_us(stack, windows)
    finally:
        stack.configs, stack.norm_configs, stack.silu_configs = {}, {}, {}


def alternating(stack: DecoderStandIn, options: dict, rounds: int, windows: int,
                kinds: dict | None = None) -> dict:
    """Each option timed in fresh captures, in rotation; the median over the rounds."""
    times: dict = {key: [] for key in options}
    for _ in range(rounds):
        for key, configs in options.items():
            times[key].append(step_us(stack, configs, windows, kinds))
    return {key: statistics.median(v) for key, v in times.items()}


def situ_tune(m: int, layers: int = 28, top: int = 4, rounds: int = 5, windows: int = 5,
              stack: DecoderStandIn | None = None, device="cuda", log=print) -> dict:
    """One in-situ pass for batch m.  Returns {"batch", "start", "chosen" (Config dicts),
    "trials", "confirm_us" (start/chosen, when they differ), "kept"}."""
    stack = stack or DecoderStandIn(m, layers=layers, device=device)
    kinds = kernels(stack)
    # w8a8_mm linears start from the table's choice, the folded kernels from their default
    start = {name: choose_config(m, n, k) if kinds[name] == "mm" else None
             for name, (k, n) in SHAPES.items()}
    current = dict(start)
    trials = []
    for name in [name for name in SHAPES if kinds[name] is not None]:
        k, n = SHAPES[name]
        kind = kinds[name]
        if kind == "mm":
            options = [current[name], default_config(m, n, k), *isolated_top(m, k, n, top, device)]
        else:
            options = [None, *folded_candidates(kind, m, n, k)]
        best = None
        for cfg in dict.fromkeys(options):
            if not kind_supported(kind, m, n, k, cfg):
                continue
            us = step_us(stack, {**current, name: cfg}, windows, kinds)
            label = cfg.name if cfg is not None else "default"
            trials.append({"layer": name, "kernel": kind, "config": label, "us": round(us, 3)})
            log(f"M={m} {name} ({kind}) {label}: {us:.2f} us a layer")
            if best is None or us < best[1]:
                best = (cfg, us)
        current[name] = best[0]

    def dicts(sel):
        return {k: asdict(v) if v is not None else None for k, v in sel.items()}

    entry = {"batch": m, "kernels": kinds, "start": dicts(start), "chosen": dicts(current),
             "trials": trials, "kept": False}
    if current != start:
        t = alternating(stack, {"start": start, "chosen": current}, rounds, windows, kinds)
        entry["confirm_us"] = {key: round(v, 3) for key, v in t.items()}
        entry["kept"] = t["chosen"] < t["start"] * (1 - ACCEPT)

    def label(c):
        return c.name if c is not None else "default"

    log(f"M={m}: " + ", ".join(f"{name} {label(start[name])} -> {label(current[name])}"
                               for name in SHAPES if start[name] != current[name])
        + f"; confirm {entry.get('confirm_us')}; kept {entry['kept']}")
    return entry


def table_rows(entry: dict) -> dict:
    """A kept entry as tuned-table rows {"KxN": {str(m): {"config", "stand_in_us"}}}: one
    for each linear that runs w8a8_mm at the batch (the table holds w8a8_mm configurations;
    an entry without "kernels" has every linear on w8a8_mm)."""
    if not entry["kept"]:
        return {}
    kinds = entry.get("kernels") or dict.fromkeys(SHAPES, "mm")
    return {f"{k}x{n}": {str(entry["batch"]): {"config": entry["chosen"][name],
                                                "stand_in_us": entry["confirm_us"]["chosen"]}}
            for name, (k, n) in SHAPES.items() if kinds.get(name) == "mm"}


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
