"""Measure every built GEMM configuration per (K, N, M) on this GPU and store the fastest in
tuned_configs.json, which tuned_config() reads with the reference's semantics: device ->
"KxN" -> largest tuned M bucket at or below M (AshrithaG/int8-linear kernel.py:137-148; the
reference's sweep and merge are bench/bench_linear.py:213-227, 385-389).

    python -m int8_linear.tune --shapes qwen3-1.7b-vllm --m 1,2,4,8,16,17,32,64,128
    python -m int8_linear.tune --shapes llama-3-8b --m 512,1024,2048,4096 --merge
    python -m int8_linear.tune --shapes qwen3-1.7b-vllm --m capture --merge
    python -m int8_linear.tune --ring-costs [--kn 8192x8192,...] [--m 48,96,...]

`--ring-costs` times the overlapped-ring tiles the library default chooses among (their
per-wave costs are the constants of that rule) and checks the default's pick against the
fastest of them.  `--m capture` is vLLM's CUDA-graph batch sizes (1, 2, 4, 8 to 248 by 8, 256 to 512 by 16)
plus three prefill sizes, the M values a served decode step is padded to (the reference's
tools/run_e2e_vm.sh:60-67).

Timing is graph replay of back-to-back calls whose weights rotate through >= 512 MiB of
copies, so each call reads its weights from HBM rather than from the 256 MiB Infinity
Cache, as in a served model.  Every candidate's int32 product must equal the default
configuration's before it is timed.  Tables are stored under the architecture name
(gfx950), which every MI355X reports.
"""

from __future__ import annotations

import argparse
import json
import statistics
import sys
import time
from dataclasses import asdict

import torch

from int8_linear.kernel import TUNED_PATH, Config, default_config, supported, w8a8_mm
from int8_linear.operands import operands, seed_of

ROTATE_BYTES = 512 << 20
# (MT, bn) of the built weight-streaming tiles: bm = 16*MT tokens, bn output columns
STREAM_TILES = [(1, 16), (2, 16), (4, 16), (8, 16), (1, 32), (2, 32), (4, 32), (1, 8), (2, 8),
                (1, 4)]
# (BM, BN, BK, waves) of the built staged tiles
STAGED_TILES = [(128, 128, 64, 4), (256, 128, 64, 4), (128, 256, 64, 4), (128, 128, 128, 4),
                (256, 256, 64, 8), (256, 128, 64, 8), (128, 256, 64, 8), (256, 128, 128, 8),
                (128, 256, 128, 8)]


# (BM, BN, BK, waves, ring depth) of the built direct-to-LDS tiles
DMA_TILES = [(256, 256, 64, 8, 3), (256, 256, 64, 8, 4), (256, 128, 64, 8, 4),
             (128, 256, 64, 8, 4), (256, 128, 128, 8, 3), (128, 256, 128, 8, 3),
             (128, 128, 128, 4, 4), (128, 128, 64, 4, 4), (256, 256, 64, 8, 5),
             (256, 128, 64, 8, 6), (128, 256, 64, 8, 6), (128, 128, 64, 4, 8)]
# the same with fragment reads overlapped with the MFMAs: stages = ring depth + 8
PIPELINED = 8
DMAP_TILES = [(256, 256, 64, 8, 3), (256, 256, 64, 8, 4), (256, 256, 64, 8, 5),
              (256, 128, 64, 8, 4), (128, 256, 64, 8, 4), (128, 256, 128, 8, 3),
              (256, 128, 128, 8, 3), (128, 128, 64, 4, 4), (128, 128, 128, 4, 4),
              (64, 128, 128, 4, 4), (64, 256, 128, 8, 3), (64, 128, 64, 4, 6),
              (64, 128, 128, 4, 6), (64, 64, 128, 4, 4), (128, 64, 128, 4, 4),
              (128, 384, 64, 8, 3), (128, 384, 64, 8, 4), (128, 192, 64, 4, 4),
              (256, 192, 64, 4, 4), (64, 192, 64, 4, 4), (64, 192, 128, 4, 4),
              (256, 256, 128, 8, 2), (256, 128, 128, 8, 2), (128, 256, 128, 8, 2),
              (256, 192, 128, 8, 2)]


# (MT, NC, KS, W) of the built persistent single-step decode tiles (stages 4): K = 64*KS*W
WLDSP_TILES = [(1, 16, 2, 16), (2, 16, 2, 16), (1, 32, 2, 16), (1, 16, 4, 16),
               (1, 16, 4, 8), (2, 16, 4, 8), (4, 16, 4, 8), (1, 16, 8, 8),
               (4, 16, 2, 16), (8, 16, 4, 8), (4, 32, 2, 8), (1, 8, 2, 16), (1, 8, 4, 16),
               (1, 8, 8, 8), (1, 8, 16, 4), (1, 16, 16, 4), (1, 8, 8, 4), (1, 16, 8, 4),
               (1, 8, 6, 16), (2, 8, 6, 16), (1, 8, 12, 8), (1, 8, 4, 8)]

# (MT, NC, KS) of the built weights-through-LDS decode tiles: bm = 16*MT, bn = NC, bk = 64*KS
WLDS_TILES = [(1, 16, 2), (1, 16, 4), (1, 16, 6), (1, 16, 8), (1, 8, 2), (1, 8, 4), (1, 8, 6),
              (1, 8, 8), (1, 4, 4), (1, 4, 8), (2, 16, 2), (2, 16, 4), (2, 8, 2), (2, 8, 4),
              (4, 16, 2), (4, 16, 4), (4, 8, 2), (4, 8, 4), (8, 16, 2), (8, 8, 2),
              (1, 32, 2), (1, 32, 4), (2, 32, 2), (2, 32, 4), (4, 32, 2), (4, 32, 4),
              (1, 64, 2), (2, 64, 2), (4, 64, 2), (1, 64, 4), (2, 64, 4)]
# The tiles worth splitting K for (stages 5, K in group_m parts): wide ones, whose L2-to-CU
# traffic per output is lowest but which give fewer workgroups than there are CUs.
SPLIT_TILES = [(1, 32, 2), (2, 32, 2), (4, 32, 2), (2, 32, 4), (1, 64, 2), (2, 64, 2),
               (4, 64, 2), (1, 64, 4), (2, 64, 4), (8, 16, 2)]


CAPTURE_SIZES = [1, 2, 4, *range(8, 256, 8), *range(256, 513, 16), 1024, 2048, 4096]


def parse_ms(spec: str) -> list[int]:
    """A comma-separated list of M values, or `capture` for vLLM's graph batch sizes."""
    return list(CAPTURE_SIZES) if spec == "capture" else [int(x) for x in spec.split(",")]


def candidate_configs(m: int, k: int, n: int) -> list[Config]:
    """Every built configuration that takes (M, N, K)."""
    out: list[Config] = []
    if m <= 128:
        need = next(mt for mt in (1, 2, 4, 8) if 16 * mt >= m)
        for mt, nc, ks in WLDS_TILES:
            if mt > need:
                continue  # one row block covering M, or several smaller ones
            for w in (4, 8, 12, 16):
                for g in (1, 3, 4):          # group_m 3 / 4: the three- / four-buffer ring
                    cfg = Config(16 * mt, nc, 64 * ks, w, 3, g)
                    if supported(m, n, k, cfg):
                        out.append(cfg)
        for mt, nc, ks, w in WLDSP_TILES:
            if mt > need:
                continue
            for g in (1, 2, 4):              # workgroups a compute unit
                cfg = Config(16 * mt, nc, 64 * ks, w, 4, g)
                if supported(m, n, k, cfg):
                    out.append(cfg)
        for mt, nc, ks in SPLIT_TILES:
            tiles = -(-m // (16 * mt)) * (n // nc)
            if mt > need or tiles >= 512:
                continue  # enough workgroups without a split
            for parts in (2, 4, 8):
                if tiles * parts > 1024:
                    continue
                for w in (4, 8):
                    cfg = Config(16 * mt, nc, 64 * ks, w, 5, parts)
                    if supported(m, n, k, cfg):
                        out.append(cfg)
    if m <= 256:
        need = next(mt for mt in (1, 2, 4, 8) if 16 * mt >= min(m, 128))
        for mt, bn in STREAM_TILES:
            if mt > need:
                continue  # one row block covering M, or several smaller ones
            for w in (1, 2, 4, 8, 16):
                cfg = Config(16 * mt, bn, 64 * w, w, 1, 1)
                if supported(m, n, k, cfg):
                    out.append(cfg)
    if m >= 33:
        for bm, bn, bk, w in STAGED_TILES:
            for g in (1, 8):
                cfg = Config(bm, bn, bk, w, 2, g)
                if supported(m, n, k, cfg):
                    out.append(cfg)
        for bm, bn, bk, w, st in DMA_TILES:
            for g in (1, 8):
                cfg = Config(bm, bn, bk, w, st, g)
                if supported(m, n, k, cfg):
                    out.append(cfg)
        for bm, bn, bk, w, st in DMAP_TILES:
            for g in (4, 8):
                cfg = Config(bm, bn, bk, w, st + PIPELINED, g)
                if supported(m, n, k, cfg):
                    out.append(cfg)
    return out


FINALISTS = 4      # candidates timed again, in turn, before one is chosen
FINAL_ROUNDS = 2   # extra timings of each finalist


def time_cold_us(call, copies: int, windows: int = 3) -> float:
    """Median us per call of 2*copies back-to-back calls in one HIP graph."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call(0)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    n = 2 * copies
    with torch.cuda.graph(g):
        for i in range(n):
            call(i)
    g.replay()
    torch.cuda.synchronize()
    # After the GPU has idled, sustained matrix work runs up to ~15% slower for the first
    # ~20 ms while the clocks settle: replay for 30 ms first, so every candidate is timed in
    # the steady state rather than the first ones at a disadvantage.
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.03:
        g.replay()
        torch.cuda.synchronize()
    res = []
    for _ in range(windows):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        b.synchronize()
        res.append(a.elapsed_time(b) * 1e3 / n)
    del g
    return statistics.median(res)


def refine_candidates(m: int, k: int, n: int, stages=(3, 5)) -> list[Config]:
    """The configuration tuned_config holds now (else the default) and the decode schedules of
    the given stages that changed after the table was made: by default every
    weights-through-LDS tile (stages 3: 64-column tiles, 8 or more waves now that the
    reduction area shares the ring, activations copied through LDS) and the split of K
    (stages 5); stages 4 is the persistent tile (its cross-wave exchanges no longer wait for
    the next tile's weights).  Timing only these against the entry they would replace updates
    a table without re-timing every candidate of every bucket."""
    from int8_linear.kernel import tuned_config
    cur = tuned_config(m, n, k) or default_config(m, n, k)
    # bn <= 64 at stages 3-5: wider tiles at those stages are prefill rings (gemm_dma)
    new = [c for c in candidate_configs(m, k, n) if c.stages in stages and c.bn <= 64]
    return [cur] + [c for c in new if c != cur]


def tune_shape(k: int, n: int, ms: list[int], device, log=print, refine: bool = False,
               min_gain: float = 0.0, refine_stages=(3, 5)) -> dict:
    """{str(M): {"config": {...}, "graph_us": t, "default_us": t0}} for one weight shape.

    The configuration the stored table gives now (tuned_config) is always among the
    finalists, and a row with one also records its time as "table_us"; with min_gain > 0 the
    stored configuration is kept unless the best finalist is that fraction faster, so that
    re-tuning a table does not trade entries on timing noise."""
    from int8_linear.kernel import tuned_config
    d = operands(16, k, n, seed_of(16, k, n), device=device)
    copies = max(2, -(-ROTATE_BYTES // (k * n)))
    ws = [d["w_q"]] + [d["w_q"].clone() for _ in range(copies - 1)]
    w_s = d["w_s"]
    rows = {}
    for m in ms:
        a = operands(m, k, n, seed_of(m, k, n), device=device)
        a_q, a_s = a["a_q"], a["a_s"]
        one = torch.ones(1, device=device)
        ref = w8a8_mm(a_q, ws[0].t(), one, one, raw=True, config=default_config(m, n, k))
        t0 = None
        timed = []
        for cfg in (refine_candidates(m, k, n, refine_stages) if refine
                    else candidate_configs(m, k, n)):
            got = w8a8_mm(a_q, ws[0].t(), one, one, raw=True, config=cfg)
            if not torch.equal(got, ref):
                raise RuntimeError(f"config {cfg.name} gives a different product at M={m} K={k} N={n}")
            us = time_cold_us(lambda i, c=cfg: w8a8_mm(a_q, ws[i % copies].t(), a_s, w_s,
                                                       torch.bfloat16, config=c), copies)
            if cfg == default_config(m, n, k):
                t0 = us
            timed.append((us, cfg))
        # One pass ranks candidates only to within a few percent (clock and cache state drift
        # over the sweep): the FINALISTS fastest are timed again, in turn, and the best median
        # of their timings wins.
        timed.sort(key=lambda t: t[0])
        finals = {c: [us] for us, c in timed[:FINALISTS]}
        cur = tuned_config(m, n, k)
        if cur is not None and cur not in finals and supported(m, n, k, cur):
            # the stored entry is kept or re-recorded only if its product is checked too
            got = w8a8_mm(a_q, ws[0].t(), one, one, raw=True, config=cur)
            if not torch.equal(got, ref):
                raise RuntimeError(f"stored config {cur.name} gives a different product at "
                                   f"M={m} K={k} N={n}")
            finals[cur] = [next((us for us, c in timed if c == cur), None) or time_cold_us(
                lambda i: w8a8_mm(a_q, ws[i % copies].t(), a_s, w_s, torch.bfloat16,
                                  config=cur), copies)]
        for _ in range(FINAL_ROUNDS):
            for c in finals:
                finals[c].append(time_cold_us(lambda i, c=c: w8a8_mm(
                    a_q, ws[i % copies].t(), a_s, w_s, torch.bfloat16, config=c), copies))
        med = {c: statistics.median(v) for c, v in finals.items()}
        best = min(med.items(), key=lambda t: t[1])
        if cur in med and best[1] > med[cur] * (1.0 - min_gain):
            best = (cur, med[cur])
        if t0 is None:
            t0 = time_cold_us(lambda i: w8a8_mm(a_q, ws[i % copies].t(), a_s, w_s, torch.bfloat16,
                                                config=default_config(m, n, k)), copies)
        table = f", table {cur.name} {med[cur]:.2f} us" if cur in med else ""
        log(f"K={k} N={n} M={m}: best {best[0].name} {best[1]:.2f} us (default {t0:.2f} us{table})")
        rows[str(m)] = {"config": asdict(best[0]), "graph_us": round(best[1], 3),
                        "default_us": round(t0, 3)}
        if cur in med:
            rows[str(m)]["table_us"] = round(med[cur], 3)
    del ws
    torch.cuda.empty_cache()
    return rows


def merge(table: dict, device_key: str, path=TUNED_PATH) -> None:
    """Merge {"KxN": {M: row}} into the stored tables under device_key."""
    tables = json.loads(path.read_text()) if path.exists() else {}
    dev = tables.setdefault(device_key, {})
    for kn, rows in table.items():
        dev.setdefault(kn, {}).update(rows)
    path.write_text(json.dumps(tables, indent=1, sort_keys=True) + "\n")


# (bm, bn, bk, warps, stages, group_m) of the overlapped-ring tiles i8l_default_config
# chooses among above the decode rules (csrc/i8l_gemm.hip)
RING = [(64, 64, 128, 4, 12, 8), (128, 64, 128, 4, 12, 8), (64, 128, 128, 4, 12, 8),
        (128, 128, 128, 4, 12, 8), (64, 256, 128, 8, 11, 8), (256, 128, 128, 8, 11, 8),
        (128, 256, 128, 8, 11, 8), (256, 192, 128, 8, 10, 4), (256, 256, 128, 8, 10, 4)]
RING_SHAPES = ("8192x10240,8192x8192,8192x57344,28672x8192,5120x5120,5120x27648,27648x5120,"
               "5120x7168,4096x6144,2048x12288,4096x28672,14336x4096,2048x2048,6144x2048,"
               "4096x4096")
RING_MS = "48,96,160,200,272,400,512,768,1024,1536,2048,4096"


def ring_costs(shapes: str = RING_SHAPES, ms: str = RING_MS, log=print) -> dict:
    """Time the overlapped-ring tiles the library default chooses among, and check the default.

    Every tile of RING is timed per (K x N, M) as a candidate is (time_cold_us).  Logged: one
    line a case with the fastest tile and the default's time against it; then each tile's
    time for one wave of workgroups (one a CU) per K byte, the median over the cases (the
    per-tile constants of the default rule, relative to the 64x64 tile); then the default's
    geometric-mean and worst ratio to the fastest tile over the cases it takes from RING.
    """
    import math

    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    log(f"{torch.cuda.get_device_name(dev)}: {cus} CUs")
    cases = []
    for spec in shapes.split(","):
        k, n = map(int, spec.lower().split("x"))
        g = torch.Generator().manual_seed(k * 31 + n)
        copies = max(2, -(-(768 << 20) // (k * n)))
        ws = [torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(dev)
              for _ in range(copies)]
        for m in map(int, ms.split(",")):
            a = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8).to(dev)
            sa = torch.rand((m, 1), generator=g).to(dev)
            sb = torch.rand((n, 1), generator=g).to(dev)
            t = {}
            for c in RING:
                cfg = Config(*c)
                if supported(m, n, k, cfg):
                    t[c] = time_cold_us(lambda i, cfg=cfg: w8a8_mm(
                        a, ws[i % copies].t(), sa, sb, torch.bfloat16, None, config=cfg), copies)
            d = default_config(m, n, k)
            dc = (d.bm, d.bn, d.bk, d.warps, d.stages, d.group_m)
            best = min(t, key=t.get)
            rel = f"{t[dc] / t[best]:.3f}" if dc in t else "not a ring tile"
            log(f"K={k} N={n} M={m}: fastest {Config(*best).name} {t[best]:.2f} us; "
                f"default {Config(*dc).name} {rel}")
            cases.append((k, n, m, t, dc))
        del ws
        torch.cuda.empty_cache()
    per = {c: [] for c in RING}
    for k, n, m, t, _ in cases:
        for c, us in t.items():
            waves = math.ceil(math.ceil(m / c[0]) * (n // c[1]) / cus)
            per[c].append(us * 1e3 / (k * waves))
    base = statistics.median(per[RING[0]]) if per[RING[0]] else float("nan")
    log("one wave's time per K byte (median over the cases), relative to 64x64:")
    costs = {}
    for c in RING:
        if per[c]:
            med = statistics.median(per[c])
            costs[Config(*c).name] = round(med, 4)
            log(f"  {c[0]}x{c[1]}: {med:.3f} ns ({100 * med / base:.0f})")
    out = {"wave_ns_per_k_byte": costs}
    ratios = [t[dc] / min(t.values()) for _, _, _, t, dc in cases if dc in t]
    if ratios:
        out["default_vs_fastest_geomean"] = round(
            math.exp(sum(map(math.log, ratios)) / len(ratios)), 4)
        out["default_vs_fastest_worst"] = round(max(ratios), 4)
        log(f"default against the fastest ring tile over {len(ratios)} cases: geometric mean "
            f"{out['default_vs_fastest_geomean']:.3f}, worst {out['default_vs_fastest_worst']:.3f}")
    return out


def main() -> int:
    from int8_linear.shapes import SHAPES
    ap = argparse.ArgumentParser()
    ap.add_argument("--ring-costs", action="store_true",
                    help="time the default rule's overlapped-ring tiles (--kn: K x N shapes, "
                         "--m: token counts; defaults: 15 shapes at 48-4096 tokens)")
    ap.add_argument("--shapes", default="qwen3-1.7b-vllm")
    ap.add_argument("--m", default="1,2,4,8,16,17,32,64,128",
                    help="comma-separated M values, or capture (vLLM graph batch sizes)")
    ap.add_argument("--kn", default=None,
                    help="comma-separated KxN shapes of the preset to tune (default: all)")
    ap.add_argument("--merge", action="store_true", help="write the result into tuned_configs.json")
    ap.add_argument("--refine", action="store_true",
                    help="time only the current table entry against the weights-through-LDS "
                         "tiles and the split of K (stages 3 and 5)")
    ap.add_argument("--refine-stages", default="3,5",
                    help="with --refine: the stages whose tiles are timed against the entry "
                         "(comma-separated; 4 = the persistent decode tile)")
    ap.add_argument("--min-gain", type=float, default=0.0,
                    help="keep the stored entry unless a candidate is this fraction faster "
                         "(e.g. 0.02)")
    ap.add_argument("--out", default=None, help="also write the result to this JSON file")
    args = ap.parse_args()
    if args.ring_costs:
        res = ring_costs(args.kn or RING_SHAPES,
                         RING_MS if args.m == ap.get_default("m") else args.m,
                         log=lambda *a: print(*a, file=sys.stderr, flush=True))
        print(json.dumps(res))
        return 0
    dev = torch.device("cuda:0")
    arch = torch.cuda.get_device_properties(dev).gcnArchName.split(":")[0]
    ms = parse_ms(args.m)
    table = {}
    only = set(args.kn.split(",")) if args.kn else None
    for label, k, n in SHAPES[args.shapes]:
        if only is not None and f"{k}x{n}" not in only:
            continue
        table[f"{k}x{n}"] = tune_shape(k, n, ms, dev, log=lambda *a: print(*a, file=sys.stderr, flush=True),
                                       refine=args.refine, min_gain=args.min_gain,
                                       refine_stages=tuple(int(x) for x in
                                                           args.refine_stages.split(",")))
    if args.out:
        with open(args.out, "w") as f:
            json.dump({arch: table}, f, indent=1)
    if args.merge:
        merge(table, arch)
    print(json.dumps({arch: table}))
    return 0


if __name__ == "__main__":
    sys.exit(main())
