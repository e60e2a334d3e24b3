#!/usr/bin/env python3
"""Benchmark of the MI355X W8A8 linear path (one GPU).

    python bench.py [--steps K] [--warmup W] [--gpus 1]

Workload (the decode sweep): the four Qwen3-1.7B linear shapes as vLLM
runs them (qkv 2048->4096, o_proj 2048->2048, gate_up 2048->12288, down 6144->2048) at
M in {1,2,4,8,16,17,32,64,128}, bias off and on: 72 W8A8 linears.  One step replays all
72 as one HIP graph.  Operands are the benchmark's seeded synthetic data (x ~ N(0,1),
W ~ N(0,0.02), bias ~ N(0,0.01), bf16, quantized per token / per channel), already in HBM.
Weights rotate through enough distinct copies (>= 512 MiB) that no call finds its weights
in the 256 MiB Infinity Cache.  `value` is the mean microseconds per linear over the sweep.

After the timed steps (not inside them): per-call graph-replay times of every sweep point,
the roofline object of the dominant kernel (HIP events on the launch stream, algorithmic
bytes per launch), the fused quantizers (config 2), the prefill shapes (config 3), the
28-layer decoder stand-in in microseconds per layer (config 4), the CPU baseline (the
oracle's CPU restatement of the reference's path, on a bounded sample) and, beside it, the
reference's own CPU path as torch ops (`cpu_reference_path`: torch._int_mm and an int32
matmul with the fp32 dequant for config 0, the torch quantizers at 1024 tokens).

    python bench.py --roofline-only      # only the config-0 launches (for rocprofv3)
    python bench.py --only standin       # one extra section alone
                                         # (quant|prefill|standin|launch|llama_decode)
Every GPU output is checked against a float64 reference before it is timed, after the
output buffer has been poisoned.  Prints ONE JSON line.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "int8-linear_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
INT8_PEAK_TOPS = 5000.0      # MI355X dense int8 MFMA, TOP/s
DECODE_M = [1, 2, 4, 8, 16, 17, 32, 64, 128]
PREFILL_M = [512, 1024, 2048, 4096]
QUANT_M = [1, 16, 128, 1024, 4096]
STANDIN_M = [1, 8, 32, 128]
STANDIN_PREFILL_M = 4096
ROTATE_BYTES = 768 << 20
METRIC = "W8A8 linear µs & % of HBM/int8 roofline, M=1-4096; µs per decoder-layer stand-in"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemm_bytes(m: int, k: int, n: int, bias: bool) -> int:
    """Algorithmic HBM bytes of one W8A8 linear: int8 A and B, fp32 scales, bf16 out/bias."""
    return m * k + k * n + 4 * m + 4 * n + 2 * m * n + (2 * n if bias else 0)


def norm_bytes(m: int, h: int, residual: bool = True) -> int:
    return (7 if residual else 3) * m * h + 2 * h + 4 * m


def silu_bytes(m: int, i: int) -> int:
    return 5 * m * i + 4 * m


def warm_up(g, seconds: float = 0.03) -> None:
    """Replays a graph for `seconds` before it is timed.  After the GPU has idled (operand
    set-up on the host), sustained matrix work runs up to ~15% slower for the first ~20 ms
    while the clocks settle; the timed windows then see the steady state."""
    import torch
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        g.replay()
        torch.cuda.synchronize()


def graph_time_us(fn, calls: int, windows: int = 5) -> float:
    """Median microseconds per call of `calls` back-to-back calls captured in one graph."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn(0)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(calls):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    warm_up(g)
    out = []
    for _ in range(windows):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        g.replay()
        e.record()
        e.synchronize()
        out.append(s.elapsed_time(e) * 1e3 / calls)
    del g
    return statistics.median(out)


def check_linear(out, d) -> float:
    """Max relative error against float64, relative to max(|ref|, |term|) (reference rule)."""
    import torch
    term = (d["a_q"].double() @ d["w_q"].double().t()) * d["a_s"].double() * d["w_s"].double().t()
    ref = term + d["bias"].double() if d["bias"] is not None else term
    scale = torch.maximum(ref.abs(), term.abs()).clamp_min(1e-6)
    return ((out.double() - ref).abs() / scale).max().item()


class Sweep:
    """The decode sweep's operands.  Each shape has one weight (seeded as the benchmark's
    M=16 point) held in several copies that calls rotate through; each (M, bias) point
    has its own seeded activations and bias."""

    def __init__(self, shapes, ms, device):
        import torch

        from int8_linear.operands import operands, seed_of
        per_set = sum(k * n for _, k, n in shapes)
        self.copies = max(2, -(-ROTATE_BYTES // per_set))
        self.weights = {}   # (k, n) -> ([w_q copies], w_s)
        for _, k, n in shapes:
            d = operands(16, k, n, seed_of(16, k, n), device=device)
            self.weights[(k, n)] = ([d["w_q"]] + [d["w_q"].clone() for _ in range(self.copies - 1)],
                                    d["w_s"])
        self.points = []    # (label, m, k, n, bias, operand dict)
        for label, k, n in shapes:
            for m in ms:
                for bias in (False, True):
                    d = operands(m, k, n, seed_of(m, k, n), with_bias=bias, device=device)
                    d["w_q"], d["w_s"] = self.weights[(k, n)][0][0], self.weights[(k, n)][1]
                    del d["w_qt"], d["w"]
                    self.points.append((label, m, k, n, bias, d))
        torch.cuda.synchronize()

    def call(self, idx: int, copy: int):
        from int8_linear import w8a8_mm
        import torch
        label, m, k, n, bias, d = self.points[idx]
        ws, w_s = self.weights[(k, n)]
        return w8a8_mm(d["a_q"], ws[copy % self.copies].t(), d["a_s"], w_s, torch.bfloat16,
                       d["bias"])


TRAFFIC_PATH = ROOT / "profiles" / "traffic_config0.json"


def roofline_config0(dev, launches: int = 0) -> dict:
    """Roofline object of the dominant kernel: the decode GEMM at BASELINE config 0 (qkv_proj,
    M=16, K=2048, N=4096, no bias, bf16 out), weights rotating through >= 768 MiB of copies.
    `achieved` = algorithmic bytes per launch / average launch time of back-to-back launches
    in a HIP graph, timed with HIP events on the stream the graph is launched on."""
    import torch

    from int8_linear import w8a8_mm
    from int8_linear.kernel import choose_config
    from int8_linear.operands import operands, seed_of
    m, k, n = 16, 2048, 4096
    d = operands(m, k, n, seed_of(m, k, n), device=dev)
    copies = max(2, -(-ROTATE_BYTES // (k * n)))
    ws = [d["w_q"]] + [d["w_q"].clone() for _ in range(copies - 1)]
    cfg = choose_config(m, n, k)
    reps = launches or 2 * copies
    us = graph_time_us(lambda i: w8a8_mm(d["a_q"], ws[i % copies].t(), d["a_s"], d["w_s"],
                                         torch.bfloat16), reps)
    b0 = gemm_bytes(m, k, n, False)
    ach = b0 / (us * 1e-6) / 1e9
    traffic = None
    if TRAFFIC_PATH.exists():
        rec = json.loads(TRAFFIC_PATH.read_text())
        if rec.get("config") == cfg.name:
            traffic = rec["bytes_per_launch"]
    return {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic,
            "kernel": f"{schedule_of(cfg, k)}, config {cfg.name} "
                      "(BASELINE config 0: M=16 K=2048 N=4096)",
            "bytes_per_launch": b0, "avg_launch_us": round(us, 3), "launches": reps}


def schedule_of(cfg, k: int) -> str:
    """The kernel a config launches (its name in a rocprofv3 kernel trace)."""
    if cfg.stages == 1:
        return "gemm_stream"
    if cfg.stages == 2:
        return "gemm_staged"
    if cfg.stages == 3 and cfg.bn <= 32:
        return "gemm_wlds1" if k == cfg.bk * cfg.warps else "gemm_wlds"
    if cfg.stages == 4 and cfg.bn <= 32:
        return "gemm_wlds1p"
    return "gemm_dmap" if cfg.stages >= 11 else "gemm_dma"


def copy_calibration(dev, mib: int = 256) -> dict:
    """A plain device copy of known size (for scaling FETCH_SIZE / WRITE_SIZE counters)."""
    import torch
    src = torch.empty(mib << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    return {"copy_bytes": mib << 20, "copies": 3}


def cpu_baseline() -> dict:
    """The oracle's CPU restatement of the reference's path (exact int32 product + fp32
    dequant + bf16 cast) on the config-0 shape, repeated for about 10 s."""
    import numpy as np

    from int8_linear.operands import operands, seed_of
    from oracle import oracle as o
    m, k, n = 16, 2048, 4096
    d = operands(m, k, n, seed_of(m, k, n))
    a, w = d["a_q"].numpy(), d["w_q"].numpy()
    sa, sb = d["a_s"].numpy(), d["w_s"].numpy()
    o.w8a8_mm(a, w, sa, sb)                     # warm-up
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < 10.0 or reps < 5:
        o.w8a8_mm(a, w, sa, sb)
        reps += 1
    us = (time.perf_counter() - t0) / reps * 1e6
    threads = int(os.environ.get("OMP_NUM_THREADS", len(os.sched_getaffinity(0))))
    return {"value": round(us, 2), "unit": "us per linear", "cores": threads,
            "kind": "port",
            "sample": f"config 0 (M=16, K=2048, N=4096, bf16 out), {reps} calls of the C oracle "
                      f"(int32 GEMM + fp32 dequant), OpenMP threads={threads}"}


def cpu_reference_path(seconds: float = 2.0) -> dict:
    """The reference's CPU path as torch ops on the host cores (each leg repeated for about
    `seconds`): the int32 product of config 0 by torch's int8 matmul (torch._int_mm) and by
    an int32 matmul, each with the fp32 dequant and bf16 cast (kernel.py:105-120); and the
    reference's torch restatements of the fused quantizers (tests/test_fused_quant.py:26-51)
    at config 2's 1024 tokens.  Reported beside the oracle's time, not as a target."""
    import torch

    from int8_linear.operands import operands, seed_of

    def per_call_us(fn) -> tuple[float, int]:
        fn()
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds or reps < 3:
            fn()
            reps += 1
        return (time.perf_counter() - t0) / reps * 1e6, reps

    m, k, n = 16, 2048, 4096
    d = operands(m, k, n, seed_of(m, k, n))
    a, w, sa, sb = d["a_q"], d["w_q"], d["a_s"], d["w_s"].view(1, -1)

    def dequant(acc):
        return (acc.float() * sa * sb).to(torch.bfloat16)

    def quant(yf):
        absmax = yf.abs().amax(-1, keepdim=True)
        inv = torch.where(absmax == 0, torch.zeros_like(absmax), 127.0 / absmax)
        return torch.round(yf * inv).clamp(-128, 127).to(torch.int8), absmax / 127.0

    g = torch.Generator().manual_seed(1)
    mq, h, inter = 1024, 2048, 6144
    x = torch.randn((mq, h), generator=g).to(torch.bfloat16)
    r = torch.randn((mq, h), generator=g).to(torch.bfloat16)
    gamma = (1 + 0.1 * torch.randn(h, generator=g)).to(torch.bfloat16)
    gu = torch.randn((mq, 2 * inter), generator=g).to(torch.bfloat16)

    def norm():
        xf = x.float() + r.float()
        var = xf.pow(2).mean(-1, keepdim=True)
        y = ((xf * torch.rsqrt(var + 1e-6)).to(gamma.dtype) * gamma).to(x.dtype)
        return quant(y.float()), xf.to(x.dtype)

    def silu():
        gf, uf = gu[:, :inter].float(), gu[:, inter:].float()
        act = (gf / (1.0 + torch.exp(-gf))).to(gu.dtype).float()
        return quant((act * uf).to(gu.dtype).float())

    legs = {"gemm_int_mm": lambda: dequant(torch._int_mm(a, w.t())),
            "gemm_int32_matmul": lambda: dequant(a.int() @ w.int().t()),
            "add_rmsnorm_quant": norm, "silu_mul_quant": silu}
    out = {"unit": "us per call", "threads": torch.get_num_threads(),
           "sample": f"config 0 GEMM (M=16, K=2048, N=4096) and config 2 quantizers at M={mq} "
                     f"(H={h}, I={inter}), torch CPU ops, about {seconds:g} s a leg"}
    for name, fn in legs.items():
        us, reps = per_call_us(fn)
        out[name] = round(us, 2)
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-extra", action="store_true", help="skip configs 2-3 and per-point table")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the config-0 roofline launches (and a copy of known size), for "
                         "rocprofv3 kernel-trace and counter runs")
    ap.add_argument("--only", choices=["quant", "prefill", "standin", "launch", "llama_decode"],
                    default=None,
                    help="run one extra section alone (for profiling) and print its JSON")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (each GPU box has "
              "one MI355X); run with --gpus 1", file=sys.stderr)
        return 2

    import torch
    from int8_linear import _lib
    from int8_linear.shapes import SHAPES

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log("library:", _lib.lib().i8l_version().decode(), "device:", torch.cuda.get_device_name())
    if args.roofline_only:
        rf = roofline_config0(dev)
        cal = copy_calibration(dev)
        print(json.dumps({"roofline": rf, "calibration": cal}), flush=True)
        return 0
    if args.only:
        fn = {"quant": bench_quant, "prefill": bench_prefill, "standin": bench_standin,
              "launch": bench_launch, "llama_decode": bench_llama_decode}[args.only]
        print(json.dumps({args.only: fn(dev)}), flush=True)
        return 0
    shapes = SHAPES["qwen3-1.7b-vllm"]
    sw = Sweep(shapes, DECODE_M, dev)
    log(f"sweep: {len(sw.points)} linears, {sw.copies} weight copies")

    # correctness first, into poisoned outputs
    worst = 0.0
    for i, (label, m, k, n, bias, d) in enumerate(sw.points):
        torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=dev)
        out = sw.call(i, 0)
        err = check_linear(out, d)
        worst = max(worst, err)
        if not err <= 1e-2:
            raise SystemExit(f"FAIL: {label} M={m} bias={bias}: max rel err {err}")
    log(f"sweep checked against float64: worst rel err {worst:.3g}")

    # one step = the whole sweep, each call on its own weight copy, one graph
    def step_calls(rep: int):
        for i in range(len(sw.points)):
            sw.call(i, rep * len(sw.points) + i)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step_calls(0)
    torch.cuda.current_stream().wait_stream(side)
    graphs = []
    for rep in range(2):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step_calls(rep)
        graphs.append(g)
    for i in range(args.warmup):
        graphs[i % 2].replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(args.steps):
        graphs[i % 2].replay()
    stop.record()
    torch.cuda.synchronize()
    ms_per_step = start.elapsed_time(stop) / args.steps
    n_calls = len(sw.points)
    us_per_linear = ms_per_step * 1e3 / n_calls
    sweep_bytes = sum(gemm_bytes(m, k, n, b) for _, m, k, n, b, _ in sw.points)
    log(f"step: {ms_per_step * 1e3:.1f} us for {n_calls} linears = {us_per_linear:.2f} us each; "
        f"{sweep_bytes / (ms_per_step * 1e-3) / 1e9:.0f} GB/s")
    del graphs

    result = {
        "metric": METRIC, "value": round(us_per_linear, 3), "unit": "us per linear (mean over decode sweep)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8xint8->int32, bf16 out", "data": "synthetic",
        "config": {"workload": "BASELINE config 1: decode sweep, Qwen3-1.7B vLLM shapes "
                               "(qkv 2048->4096, o 2048->2048, gate_up 2048->12288, "
                               "down 6144->2048) x M{1,2,4,8,16,17,32,64,128} x bias{off,on}",
                   "linears_per_step": n_calls, "weight_copies": sw.copies,
                   "sweep_GBps": round(sweep_bytes / (ms_per_step * 1e-3) / 1e9, 1)},
    }

    result["roofline"] = roofline_config0(dev)
    log(f"roofline config0: {result['roofline']['avg_launch_us']:.2f} us, "
        f"{result['roofline']['achieved']:.0f} GB/s ({result['roofline']['frac']:.1%})")

    if not args.no_extra:
        table = []
        for i, (label, m, k, n, bias, d) in enumerate(sw.points):
            us = graph_time_us(lambda j, i=i: sw.call(i, j), 2 * sw.copies, windows=3)
            gbs = gemm_bytes(m, k, n, bias) / (us * 1e-6) / 1e9
            table.append([label, m, int(bias), round(us, 2), round(gbs / HBM_PEAK_GBS, 3)])
        result["decode_points"] = {"cols": ["shape", "M", "bias", "us", "hbm_frac"], "rows": table}
        result["quant"] = bench_quant(dev)
        result["llama_decode"] = bench_llama_decode(dev)
        result["prefill"] = bench_prefill(dev)
        result["standin"] = bench_standin(dev)
        result["launch"] = bench_launch(dev)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline()
        result["cpu_reference_path"] = cpu_reference_path()
    print(json.dumps(result), flush=True)
    return 0


def bench_quant(dev) -> dict:
    """the two fused quantizers at H=2048 / I=6144."""
    import torch

    from int8_linear import fused_quant as fq
    rows = []
    for m in QUANT_M:
        g = torch.Generator().manual_seed(m)
        copies = max(2, -(-ROTATE_BYTES // (m * 2048 * 7 + 1)))
        copies = min(copies, 64)
        xs = [torch.randn((m, 2048), generator=g).to(torch.bfloat16).to(dev) for _ in range(2)]
        rs = [torch.randn((m, 2048), generator=g).to(torch.bfloat16).to(dev) for _ in range(copies)]
        w = (1 + 0.1 * torch.randn(2048, generator=g)).to(torch.bfloat16).to(dev)
        us_n = graph_time_us(lambda i: fq.add_rmsnorm_quant(xs[i % 2], rs[i % copies], w, 1e-6), 2 * copies, 3)
        copies_s = min(64, max(2, -(-ROTATE_BYTES // (m * 12288 * 2 + 1))))
        gus = [torch.randn((m, 12288), generator=g).to(torch.bfloat16).to(dev) for _ in range(copies_s)]
        us_s = graph_time_us(lambda i: fq.silu_mul_quant(gus[i % copies_s], True, True), 2 * copies_s, 3)
        rows.append([m, round(us_n, 2), round(norm_bytes(m, 2048) / (us_n * 1e-6) / 1e9 / HBM_PEAK_GBS, 3),
                     round(us_s, 2), round(silu_bytes(m, 6144) / (us_s * 1e-6) / 1e9 / HBM_PEAK_GBS, 3)])
        del xs, rs, gus
    return {"cols": ["M", "add_rmsnorm_quant_us", "hbm_frac", "silu_mul_quant_us", "hbm_frac"],
            "rows": rows}


def bench_standin(dev) -> dict:
    """the 28-layer Qwen3-1.7B decoder stand-in, one step per graph
    replay, microseconds per decoder layer, at decode M and one 4096-token prefill."""
    import torch

    from int8_linear import standin
    base = standin.DecoderStandIn(1, generator_device="cuda")   # 1.41 GB of layer weights
    wbytes = base.weight_bytes() / len(base.layers)
    rows = []
    for m in STANDIN_M + [STANDIN_PREFILL_M]:
        st = base.with_batch(m, seed=m)
        us = standin.per_layer_us(st, windows=5)
        rows.append([m, round(us, 2), round(wbytes / (us * 1e-6) / 1e9, 1)])
        log(f"standin M={m}: {us:.2f} us per layer")
        del st
    del base
    torch.cuda.empty_cache()
    return {"cols": ["M", "us_per_layer", "weight_GBps"], "rows": rows,
            "layers": standin.LAYERS, "weight_bytes_per_layer": int(wbytes),
            "step": "add_rmsnorm_quant > qkv > quant(q cols) > o > add_rmsnorm_quant > gate_up "
                    "> silu_mul_quant > down, one HIP graph per 28-layer step"}


LLAMA_DECODE_M = [1, 4, 16]


def bench_llama_decode(dev) -> dict:
    """Decode on the Llama-3-8B shapes (the larger of the two models BASELINE names for the
    HBM target at M <= 16): µs per linear and fraction of 8 TB/s, weights rotating through
    >= 768 MiB of copies so every call reads them from HBM."""
    import torch

    from int8_linear import w8a8_mm
    from int8_linear.operands import operands, seed_of
    from int8_linear.shapes import SHAPES
    rows = []
    for label, k, n in SHAPES["llama-3-8b"]:
        d = operands(16, k, n, seed_of(16, k, n), device=dev)
        copies = max(2, -(-ROTATE_BYTES // (k * n)))
        ws = [d["w_q"]] + [d["w_q"].clone() for _ in range(copies - 1)]
        w_s = d["w_s"]
        for m in LLAMA_DECODE_M:
            a = operands(m, k, 64, seed_of(m, k, n), device=dev)
            a_q, a_s = a["a_q"], a["a_s"]
            out = w8a8_mm(a_q, ws[0].t(), a_s, w_s, torch.bfloat16)
            term = (a_q.double() @ ws[0].double().t()) * a_s.double() * w_s.double().t()
            err = ((out.double() - term).abs() / term.abs().clamp_min(1e-6)).max().item()
            if not err <= 1e-2:
                raise SystemExit(f"FAIL llama decode {label} M={m}: rel err {err}")
            us = graph_time_us(lambda i: w8a8_mm(a_q, ws[i % copies].t(), a_s, w_s,
                                                 torch.bfloat16), 2 * copies, 3)
            frac = gemm_bytes(m, k, n, False) / (us * 1e-6) / 1e9 / HBM_PEAK_GBS
            rows.append([label, m, round(us, 2), round(frac, 3)])
            log(f"llama decode {label} M={m}: {us:.2f} us, {frac:.1%} of HBM")
        del ws, d
        torch.cuda.empty_cache()
    return {"cols": ["shape", "M", "us", "hbm_frac"], "rows": rows}


LAUNCH_SHAPES = [("q_proj, o_proj", 2048, 2048), ("gate_up_proj", 2048, 12288)]
LAUNCH_M = [1, 4, 16]


def time_host_us(fn, iters: int, windows: int) -> list[float]:
    """CPU microseconds per call, nothing synchronized inside a window (the host cost)."""
    import torch
    fn()
    torch.cuda.synchronize()
    out = []
    for _ in range(windows):
        t0 = time.perf_counter()
        for _ in range(iters):
            fn()
        out.append((time.perf_counter() - t0) / iters * 1e6)
        torch.cuda.synchronize()
    return out


def time_eager_us(fn, iters: int, windows: int) -> list[float]:
    """Microseconds per call between HIP events around `iters` back-to-back eager calls."""
    import torch
    out = []
    for _ in range(windows):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(iters):
            fn()
        b.record()
        b.synchronize()
        out.append(a.elapsed_time(b) * 1e3 / iters)
    return out


class _ctypes_only:
    """Inside: the Python wrappers launch through ctypes (the C++ binding is set aside)."""

    def __enter__(self):
        from int8_linear import _lib
        self.saved = _lib.fast()
        _lib._fast_mod = None

    def __exit__(self, *exc):
        from int8_linear import _lib
        _lib._fast_mod = self.saved


def bench_launch(dev, iters: int = 300, windows: int = 5) -> dict:
    """Host cost of one eager call (the reference's bench/launch_overhead.py:52-153 on the
    same shapes and batch sizes): CPU time per call, back-to-back time between HIP events
    (a step without graphs), and graph replay (the GPU work alone), per launch path."""
    import torch
    import torch.nn.functional as F

    from int8_linear import fused_quant as fq
    from int8_linear import vllm_patch
    from int8_linear.kernel import w8a8_mm
    from int8_linear.operands import operands, seed_of

    def ctypes_path(fn):
        def run():
            with _ctypes_only():
                return fn()
        return run

    rows = []
    for label, k, n in LAUNCH_SHAPES:
        for m in LAUNCH_M:
            d = operands(m, k, n, seed_of(m, k, n), device=dev)
            a, wb = d["a"], d["w"]
            q = (d["a_q"], d["w_qt"], d["a_s"], d["w_s"], torch.bfloat16, None)
            provs = [
                ("bf16 F.linear (torch, hipBLASLt)", lambda: F.linear(a, wb)),
                ("int8 torch._int_mm (hipBLASLt, int32 out, no scales)",
                 lambda: torch._int_mm(d["a_q"], d["w_qt"])),
                ("ours, ctypes", ctypes_path(lambda: w8a8_mm(*q))),
                ("ours, C++ binding", lambda: w8a8_mm(*q)),
                ("ours, custom op", lambda: torch.ops.int8_linear.w8a8_mm(*q)),
                ("ours, vLLM entry", lambda: vllm_patch.scaled_mm(*q)),
            ]
            ref = None
            for name, fn in provs:
                row = {"shape": label, "k": k, "n": n, "m": m, "provider": name}
                try:
                    out = fn()
                    torch.cuda.synchronize()
                except Exception as e:  # a vendor path that does not take this shape
                    row["status"] = f"{type(e).__name__}: {str(e).splitlines()[0][:80]}"
                    rows.append(row)
                    continue
                if name.startswith("ours"):
                    ref = out if ref is None else ref
                    if not torch.equal(out, ref):
                        raise SystemExit(f"FAIL launch paths differ: {name} {label} M={m}")
                h = time_host_us(fn, iters, windows)
                e = time_eager_us(fn, iters, windows)
                try:
                    g = graph_time_us(lambda i: fn(), 100, windows)
                except Exception as ex:
                    g = None
                    row["graph_status"] = type(ex).__name__
                row.update(status="ok", host_us=round(statistics.median(h), 2),
                           eager_us=round(statistics.median(e), 2),
                           graph_us=round(g, 2) if g is not None else None)
                rows.append(row)
                log(f"launch {label} M={m} {name}: host {row['host_us']} eager "
                    f"{row['eager_us']} graph {row['graph_us']} us")
    # the fused quantizers of one decode token row set, ctypes vs the binding
    for m in LAUNCH_M:
        x = torch.randn((m, 2048), device=dev).to(torch.bfloat16)
        r = torch.randn((m, 2048), device=dev).to(torch.bfloat16)
        w = torch.ones(2048, device=dev, dtype=torch.bfloat16)
        gu = torch.randn((m, 12288), device=dev).to(torch.bfloat16)
        ops = [("add_rmsnorm_quant", lambda: fq.add_rmsnorm_quant(x, r, w, 1e-6)),
               ("silu_mul_quant", lambda: fq.silu_mul_quant(gu))]
        for opname, fn in ops:
            for name, f in (("ours, ctypes", ctypes_path(fn)), ("ours, C++ binding", fn)):
                h = time_host_us(f, iters, windows)
                e = time_eager_us(f, iters, windows)
                g = graph_time_us(lambda i: f(), 100, windows)
                rows.append({"shape": opname, "k": 2048, "n": 2048 if opname[0] == "a" else 6144,
                             "m": m, "provider": name, "status": "ok",
                             "host_us": round(statistics.median(h), 2),
                             "eager_us": round(statistics.median(e), 2), "graph_us": round(g, 2)})
                log(f"launch {opname} M={m} {name}: host {rows[-1]['host_us']} eager "
                    f"{rows[-1]['eager_us']} graph {rows[-1]['graph_us']} us")
    cols = ["shape", "m", "provider", "host_us", "eager_us", "graph_us"]
    return {"cols": cols, "rows": [[r.get(c, r.get("status")) for c in cols] for r in rows],
            "iters": iters, "windows": windows}


def bench_prefill(dev) -> dict:
    """Llama-3-8B shapes at prefill M; int8 TOP/s and MFMA fraction."""
    import torch

    from int8_linear import w8a8_mm
    from int8_linear.operands import quant_rows
    from int8_linear.shapes import SHAPES
    rows = []
    for label, k, n in SHAPES["llama-3-8b"]:
        g = torch.Generator().manual_seed(k + n)
        w = (torch.randn((n, k), generator=g) * 0.02).to(torch.bfloat16)
        w_q, w_s = quant_rows(w)
        w_q, w_s = w_q.to(dev), w_s.to(dev)
        del w
        for m in PREFILL_M:
            x = torch.randn((m, k), generator=g).to(torch.bfloat16)
            a_q, a_s = quant_rows(x)
            a_q, a_s = a_q.to(dev), a_s.to(dev)
            out = w8a8_mm(a_q, w_q.t(), a_s, w_s, torch.bfloat16)
            term = (a_q[:64].double() @ w_q.double().t()) * a_s[:64].double() * w_s.double().t()
            err = ((out[:64].double() - term).abs() / term.abs().clamp_min(1e-6)).max().item()
            if not err <= 1e-2:
                raise SystemExit(f"FAIL prefill {label} M={m}: rel err {err}")
            us = graph_time_us(lambda i: w8a8_mm(a_q, w_q.t(), a_s, w_s, torch.bfloat16), 10, 3)
            tops = 2 * m * n * k / (us * 1e-6) / 1e12
            rows.append([label, m, round(us, 2), round(tops, 1), round(tops / INT8_PEAK_TOPS, 3)])
            log(f"prefill {label} M={m}: {us:.1f} us {tops:.0f} TOP/s")
        del w_q, w_s
    return {"cols": ["shape", "M", "us", "TOPs", "mfma_frac"], "rows": rows}


if __name__ == "__main__":
    sys.exit(main())
