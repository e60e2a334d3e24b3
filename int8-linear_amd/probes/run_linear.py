"""Run one W8A8 linear repeatedly, for a profiler to watch (rocprofv3 --kernel-trace / --pmc).

    python3 int8-linear_amd/probes/run_linear.py --kn 14336x4096 --m 64 [--config 32,32,256,4,3,1]

Random int8 operands of the shape, fp32 per-token and per-channel scales, bf16 output;
`int8_linear.kernel.w8a8_mm` with the given config (bm,bn,bk,warps,stages,group_m) or, by
default, the one the library chooses (the shipped table).  The weights rotate through copies
filling at least 768 MiB, so every launch reads them from HBM as the bench does; --reps passes
over the copies.  No output check: the GPU tests cover every config against the oracle.
"""

from __future__ import annotations

import argparse
import os
import sys

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), ".."))

import torch  # noqa: E402

from int8_linear.kernel import Config, choose_config, w8a8_mm  # noqa: E402


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--kn", required=True, help="K x N of the weight, e.g. 14336x4096")
    ap.add_argument("--m", type=int, required=True, help="tokens")
    ap.add_argument("--config", default=None, help="bm,bn,bk,warps,stages,group_m")
    ap.add_argument("--reps", type=int, default=3)
    args = ap.parse_args()
    k, n = map(int, args.kn.lower().split("x"))
    m = args.m
    cfg = Config(*map(int, args.config.split(","))) if args.config else choose_config(m, n, k)
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(m * 7919 + k * 31 + n)
    copies = max(2, -(-(768 << 20) // (k * n)))
    ws = [torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(dev)
          for _ in range(copies)]
    a = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8).to(dev)
    sa = (torch.rand((m, 1), generator=g) * 1e-2).to(dev)
    sb = (torch.rand((n, 1), generator=g) * 1e-2).to(dev)
    for _ in range(args.reps):
        for w in ws:
            w8a8_mm(a, w.t(), sa, sb, torch.bfloat16, config=cfg)
    torch.cuda.synchronize()
    print(f"ran {args.reps * copies} launches: M={m} K={k} N={n} {cfg.name}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
