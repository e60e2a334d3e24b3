"""Time the overlapped-ring tiles the library default chooses among, and check the default.

    python3 int8-linear_amd/probes/ring_costs.py [--shapes 8192x8192,...] [--ms 48,96,...]

For each weight shape (K x N) and token count, every tile of the library default's ring table
(i8l_default_config, csrc/i8l_gemm.hip) is timed as the tuner times a candidate (HIP graph of
back-to-back calls, weights rotating through copies of at least 768 MiB, so they come from
HBM).  Printed: one line a case with the fastest tile and the default's time against it; then
each tile's time for one wave of workgroups (one a CU) per K byte, the median over the cases
(the costs that table holds, relative to the 64x64 tile); then the default's geometric-mean
and worst ratio to the fastest tile over the cases it takes from that table.
"""

from __future__ import annotations

import argparse
import math
import os
import statistics
import sys

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), ".."))

import torch  # noqa: E402

from int8_linear.kernel import Config, default_config, supported, w8a8_mm  # noqa: E402
from int8_linear.tune import time_cold_us  # noqa: E402

# (bm, bn, bk, warps, stages, group_m) of the ring table in i8l_default_config
RING = [(64, 64, 128, 4, 12, 8), (128, 64, 128, 4, 12, 8), (64, 128, 128, 4, 12, 8),
        (128, 128, 128, 4, 12, 8), (64, 256, 128, 8, 11, 8), (256, 128, 128, 8, 11, 8),
        (128, 256, 128, 8, 11, 8), (256, 192, 128, 8, 10, 4), (256, 256, 128, 8, 10, 4)]
SHAPES = ("8192x10240,8192x8192,8192x57344,28672x8192,5120x5120,5120x27648,27648x5120,"
          "5120x7168,4096x6144,2048x12288,4096x28672,14336x4096,2048x2048,6144x2048,4096x4096")
MS = "48,96,160,200,272,400,512,768,1024,1536,2048,4096"


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--shapes", default=SHAPES, help="K x N of the weights, comma-separated")
    ap.add_argument("--ms", default=MS, help="token counts, comma-separated")
    args = ap.parse_args()
    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    print(f"{torch.cuda.get_device_name(dev)}: {cus} CUs", flush=True)
    cases = []
    for spec in args.shapes.split(","):
        k, n = map(int, spec.lower().split("x"))
        g = torch.Generator().manual_seed(k * 31 + n)
        copies = max(2, -(-(768 << 20) // (k * n)))
        ws = [torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(dev)
              for _ in range(copies)]
        for m in map(int, args.ms.split(",")):
            a = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8).to(dev)
            sa = torch.rand((m, 1), generator=g).to(dev)
            sb = torch.rand((n, 1), generator=g).to(dev)
            t = {}
            for c in RING:
                cfg = Config(*c)
                if supported(m, n, k, cfg):
                    t[c] = time_cold_us(lambda i: w8a8_mm(a, ws[i % copies].t(), sa, sb,
                                                          torch.bfloat16, None, config=cfg),
                                        copies)
            d = default_config(m, n, k)
            dc = (d.bm, d.bn, d.bk, d.warps, d.stages, d.group_m)
            best = min(t, key=t.get)
            rel = f"{t[dc] / t[best]:.3f}" if dc in t else "not a ring tile"
            print(f"K={k} N={n} M={m}: fastest {Config(*best).name} {t[best]:.2f} us; "
                  f"default {Config(*dc).name} {rel}", flush=True)
            cases.append((k, n, m, t, dc))
        del ws
        torch.cuda.empty_cache()
    print("\none wave's time per K byte (median over the cases), relative to 64x64:")
    per = {c: [] for c in RING}
    for k, n, m, t, _ in cases:
        for c, us in t.items():
            waves = math.ceil(math.ceil(m / c[0]) * (n // c[1]) / cus)
            per[c].append(us * 1e3 / (k * waves))
    base = statistics.median(per[RING[0]]) if per[RING[0]] else float("nan")
    for c in RING:
        if per[c]:
            med = statistics.median(per[c])
            print(f"  {c[0]}x{c[1]}: {med:.3f} ns ({100 * med / base:.0f})")
    ratios = [t[dc] / min(t.values()) for _, _, _, t, dc in cases if dc in t]
    if ratios:
        geo = math.exp(sum(map(math.log, ratios)) / len(ratios))
        print(f"\ndefault against the fastest ring tile over {len(ratios)} cases: "
              f"geometric mean {geo:.3f}, worst {max(ratios):.3f}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
