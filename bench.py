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
28-layer decoder stand-in in microseconds per layer (config 4), Llama-3-8B decode, the eager
host cost per call, the hardware floors measured by probe kernels the same way (empty-kernel
launch, cold HBM reads, sustained int8 MFMA rate), and on the host cores the CPU baseline:
the reference's CPU path as torch ops (`cpu_baseline`: torch._int_mm with the fp32 dequant
for config 0; `cpu_reference_path`: an int32 matmul and the torch quantizers at 1024 tokens)
and the C oracle (`cpu_oracle`), each on a bounded sample.

    python bench.py --roofline-only      # only the config-0 launches (for rocprofv3)
    python bench.py --only standin       # one extra section alone
                         # (quant|prefill|standin|launch|llama_decode|floors|linear)
    python bench.py --only prefill --prefill-m 4096   # config 3 at M=4096 only
    python bench.py --only linear --kn 14336x4096 --m 64 [--config 32,32,256,4,3,1]
                         # one linear launched repeatedly, for a profiler to watch
    python bench.py --details out.json   # also every per-point table, in one file

Every timed output is checked before it is timed, with its output buffer poisoned first:
the linears against float64, the quantizers and every op of the stand-in against the
reference's CPU arithmetic.  The last line printed is the one-line JSON result, with only
scalar fields in each section; the per-point tables are printed on the lines before it
({"detail": name, "data": ...}).
"""

from __future__ import annotations

import argparse
import collections
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


def checked_mm(d, cfg=None, copy=None):
    """The linear of operand dict d (a_q, w_q [N,K], a_s, w_s, bias) written into an output
    buffer filled with NaN first: the same C entry point and configuration as the timed calls
    (i8l_w8a8_mm_ws, cfg or choose_config), with the output passed in, so every element the
    check reads was written by the kernel (a skipped element stays NaN and fails the check)."""
    import torch

    from int8_linear import _lib
    from int8_linear.kernel import _cconfig, choose_config
    a, w = d["a_q"], d["w_q"] if copy is None else copy
    m, k = a.shape
    n = w.shape[0]
    cfg = cfg or choose_config(m, n, k)
    out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=a.device)
    sa, sb = d["a_s"].reshape(-1).contiguous(), d["w_s"].reshape(-1).contiguous()
    bias = d.get("bias")
    ws_bytes = _lib.lib().i8l_w8a8_mm_workspace_bytes(m, n, k, _cconfig(cfg))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=a.device) if ws_bytes else None
    st = _lib.lib().i8l_w8a8_mm_ws(
        a.data_ptr(), a.stride(0), a.stride(1), w.data_ptr(), 1, w.stride(0),
        sa.data_ptr(), sa.numel(), sb.data_ptr(), sb.numel(),
        bias.data_ptr() if bias is not None else None,
        _lib.BF16 if bias is not None else _lib.DTYPE_NONE,
        out.data_ptr(), out.stride(0), _lib.BF16, m, n, k,
        ws.data_ptr() if ws is not None else None, ws_bytes, _cconfig(cfg), _lib.stream_of(a))
    _lib.check(st, RuntimeError)
    torch.cuda.synchronize()
    return out


def check_linear(out, d) -> float:
    """Max relative error against float64, relative to max(|ref|, |term|) (reference rule)."""
    import torch
    term = (d["a_q"].double() @ d["w_q"].double().t()) * d["a_s"].double() * d["w_s"].double().t()
    ref = term + d["bias"].double() if d["bias"] is not None else term
    scale = torch.maximum(ref.abs(), term.abs()).clamp_min(1e-6)
    return ((out.double() - ref).abs() / scale).max().item()


# ---------------------------------------------------------------- output checks
# The reference's CPU arithmetic, restated in torch ops on the host, checks the quantizer leg
# and the stand-in before they are timed.  The division is the IEEE one the reference kernel
# specifies (PRECISE_DIV, int8_linear/fused_quant.py:45-47); the sum of squares, rsqrt and
# exp are torch's float32 ones, which is why the checks carry the reference test's tolerance
# (tests/test_fused_quant.py:54-61) rather than bit equality.

def ref_quant(yf):
    """(codes, scales) of float32 rows: absmax/127 and round(y * 127/absmax), IEEE division
    (reference fused_quant.py:41-53)."""
    import torch
    absmax = yf.abs().amax(-1, keepdim=True)
    inv = torch.where(absmax == 0, torch.zeros_like(absmax),
                      torch.full_like(absmax, 127.0) / absmax)
    return torch.round(yf * inv).clamp(-128, 127).to(torch.int8), absmax / 127.0


def ref_norm(x, r, w, eps: float = 1e-6):
    """add+RMSNorm+quant (reference fused_quant.py:56-73): (codes, scales, residual_out)."""
    import torch
    xf = x.float()
    rout = None
    if r is not None:
        xf = xf + r.float()
        rout = xf.to(x.dtype)
    var = xf.pow(2).mean(-1, keepdim=True)
    y = ((xf * torch.rsqrt(var + eps)).to(w.dtype) * w).to(x.dtype)
    return (*ref_quant(y.float()), rout)


def ref_silu(gu, round_silu: bool):
    """SiLU-and-mul+quant (reference fused_quant.py:76-88): (codes, scales)."""
    import torch
    i = gu.shape[1] // 2
    g, u = gu[:, :i].float(), gu[:, i:].float()
    a = g / (1.0 + torch.exp(-g))
    if round_silu:
        a = a.to(gu.dtype).float()
    return ref_quant((a * u).to(gu.dtype).float())


def ref_mm(q, s, w, ws):
    """The reference's CPU path of one linear: exact int32 product (torch._int_mm), then
    acc * scale_a * scale_b in float32 and one cast (kernel.py:105-120)."""
    import torch
    acc = torch._int_mm(q, w.t())
    return (acc.float() * s.reshape(-1, 1) * ws.reshape(1, -1)).to(torch.bfloat16)


def check_quant(q, s, q0, s0, what: str) -> None:
    """The reference test's tolerance (tests/test_fused_quant.py:54-61): codes within one
    step, at most max(8, 0.1%) of them different, scales within 1e-5 relative.  A few rows
    (at most max(1, rows/512)) may have their scale one bf16 step of the row's absmax away
    (at most 2^-7 relative): the restatement's float32 sum of squares and rsqrt round a row's
    largest value the other way now and then, where the kernel's are exact."""
    d = (q.cpu().int() - q0.int()).abs()
    bad = int(d.ne(0).sum())
    if d.numel() and (int(d.max()) > 1 or bad > max(8, d.numel() // 1000)):
        raise SystemExit(f"FAIL {what}: {bad} codes differ, largest by {int(d.max())}")
    if not s0.numel():
        return
    rel = ((s.cpu().float().reshape(-1) - s0.reshape(-1)).abs()
           / s0.reshape(-1).abs().clamp_min(1e-30))
    off = rel.ge(1e-5) | rel.isnan()
    if int(off.sum()) > max(1, rel.numel() // 512) or not bool((rel[off] <= 2.0 ** -7).all()):
        raise SystemExit(f"FAIL {what}: scales differ by {rel.max().item():.3g} relative "
                         f"({int(off.sum())} rows beyond 1e-5)")


def check_standin(stack, rows, h_step) -> int:
    """Checks the stand-in step the bench times, h_step being its output (the last down_proj
    output of the captured graph's replay):
      * an eager run of the same chain with every op launched on its own (the folded kernels
        are bit-identical to the launches they replace) ends in h_step bit for bit;
      * along that run, each op's output on the token rows `rows`, computed on the host from
        that op's own GPU inputs in the reference's CPU arithmetic: the GEMMs (exact int32
        product, fp32 dequant, one cast) and the residual adds bit for bit, the quantizers
        within the reference test's tolerance.  (Every op works on each token row alone.)
    Checking op by op rather than the chain's end: one code that rounds the other way early in
    28 layers moves the end by a few percent, so only per-op checks have a tight bar.
    Returns the number of ops checked."""
    import torch

    from int8_linear import fused_quant as fq
    from int8_linear.kernel import w8a8_mm
    from int8_linear.standin import EPS, Q_COLS
    gamma = stack.norm.cpu()
    ops = 0

    def rows_of(t):
        return t[rows].cpu()

    def norm(x, r):
        nonlocal ops
        q, s, rout = fq.add_rmsnorm_quant(x, r, stack.norm, EPS, fq.PRECISE_DIV)
        q0, s0, r0 = ref_norm(rows_of(x), rows_of(r) if r is not None else None, gamma, EPS)
        check_quant(rows_of(q), rows_of(s), q0, s0, f"stand-in add_rmsnorm_quant layer {i}")
        if r is not None and not torch.equal(rows_of(rout), r0):
            raise SystemExit(f"FAIL stand-in residual add layer {i}")
        ops += 1
        return q, s, rout

    def mm(name, q, s):
        nonlocal ops
        w, ws = stack.layers[i][name]
        out = w8a8_mm(q, w.t(), s, ws, torch.bfloat16, config=stack.configs.get(name))
        if not torch.equal(rows_of(out), ref_mm(rows_of(q), rows_of(s), w.cpu(), ws.cpu())):
            raise SystemExit(f"FAIL stand-in {name} layer {i}")
        ops += 1
        return out

    res = stack.x
    i = 0
    q, s, _ = norm(stack.x, None)
    h = None
    for i in range(len(stack.layers)):
        if i:
            q, s, res = norm(h, res)
        a = mm("qkv_proj", q, s)
        q, s = fq.quant_per_token(a[:, :Q_COLS], fq.PRECISE_DIV)
        q0, s0 = ref_quant(rows_of(a[:, :Q_COLS]).float())
        check_quant(rows_of(q), rows_of(s), q0, s0, f"stand-in quant_per_token layer {i}")
        h = mm("o_proj", q, s)
        q, s, res = norm(h, res)
        gu = mm("gate_up_proj", q, s)
        q, s = fq.silu_mul_quant(gu, fq.PRECISE_DIV, fq.ROUND_SILU)
        q0, s0 = ref_silu(rows_of(gu), fq.ROUND_SILU)
        check_quant(rows_of(q), rows_of(s), q0, s0, f"stand-in silu_mul_quant layer {i}")
        h = mm("down_proj", q, s)
        ops += 2
    if not torch.equal(h, h_step):
        raise SystemExit("FAIL stand-in: the timed graph's output differs from the op-by-op run")
    return ops


class Sweep:
    """The decode sweep's operands.  Each shape has one weight (seeded as the benchmark's
    M=16 point) held in enough copies of its own (>= ROTATE_BYTES per shape) that a copy is
    read again only after at least 768 MiB of other weights; each (M, bias) point has its own
    seeded activations and bias."""

    def __init__(self, shapes, ms, device):
        import torch

        from int8_linear.operands import operands, seed_of
        self.weights = {}   # (k, n) -> ([w_q copies], w_s)
        self.copies = {}    # (k, n) -> number of copies
        for _, k, n in shapes:
            d = operands(16, k, n, seed_of(16, k, n), device=device)
            c = self.copies[(k, n)] = max(2, -(-ROTATE_BYTES // (k * n)))
            self.weights[(k, n)] = ([d["w_q"]] + [d["w_q"].clone() for _ in range(c - 1)],
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
        return w8a8_mm(d["a_q"], ws[copy % len(ws)].t(), d["a_s"], w_s, torch.bfloat16,
                       d["bias"])

    def min_reuse_bytes(self, plan: list[list[int]]) -> int:
        """Fewest weight bytes read between two reads of one copy when the steps of `plan`
        replay in turn, repeatedly (the timed loop alternates them)."""
        seq = [(self.points[i][2], self.points[i][3], c) for row in plan
               for i, c in enumerate(row)]
        seq = seq + seq                     # the cycle, twice: reuses across the wrap too
        last, best, total = {}, None, 0
        for k, n, c in seq:
            key = (k, n, c % self.copies[(k, n)])
            if key in last:
                gap = total - last[key]
                best = gap if best is None else min(best, gap)
            total += k * n
            last[key] = total
        return best or 0

    def step_copies(self, reps: int) -> list[list[int]]:
        """For `reps` consecutive steps over every point, the copy each call reads: a shape's
        calls take its copies in turn, so between two reads of one copy lie all the others."""
        seen = {kn: 0 for kn in self.copies}
        out = []
        for _ in range(reps):
            row = []
            for _, _, k, n, _, _ in self.points:
                row.append(seen[(k, n)])
                seen[(k, n)] += 1
            out.append(row)
        return out


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
    if cfg.stages == 3 and cfg.bn <= 64:
        return "gemm_wlds1" if k == cfg.bk * cfg.warps else "gemm_wlds"
    if cfg.stages == 4 and cfg.bn <= 32:
        return "gemm_wlds1p"
    if cfg.stages == 5 and cfg.bn <= 64:
        return "gemm_wlds + splitk_sum"
    return "gemm_dmap" if cfg.stages >= 10 else "gemm_dma"


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

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)     # pinned: every leg runs on the same thread count

    def per_call_us(fn) -> tuple[float, int]:
        """Median over 5 windows of about seconds/5 each (after two warm-up calls)."""
        fn()
        fn()
        windows, total = [], 0
        for _ in range(5):
            reps, t0 = 0, time.perf_counter()
            while time.perf_counter() - t0 < seconds / 5 or reps < 2:
                fn()
                reps += 1
            windows.append((time.perf_counter() - t0) / reps * 1e6)
            total += reps
        return statistics.median(windows), total

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
                     f"(H={h}, I={inter}), torch CPU ops on {threads} threads, median of 5 "
                     f"windows, about {seconds:g} s a leg"}
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
    ap.add_argument("--only", choices=["quant", "prefill", "standin", "launch", "llama_decode",
                                       "floors", "linear", "decode_points"],
                    default=None,
                    help="run one extra section alone (for profiling) and print its JSON")
    ap.add_argument("--calibrate", action="store_true",
                    help="with --only: also run three 256 MiB device copies (counter scale)")
    ap.add_argument("--prefill-m", type=int, nargs="+", default=None,
                    help="with --only prefill: the token counts to run (default 512-4096)")
    ap.add_argument("--quant-m", type=int, nargs="+", default=None,
                    help="with --only quant: the token counts to run (default 1-4096)")
    ap.add_argument("--mark", action="store_true",
                    help="launch a one-element marker kernel just before and just after the "
                         "timed sweep steps, so a kernel trace shows where they lie")
    ap.add_argument("--details", default=None,
                    help="also write the result with every per-point table to this JSON file")
    ap.add_argument("--kn", default=None, help="with --only linear: K x N of the weight")
    ap.add_argument("--m", type=int, default=None, help="with --only linear: tokens")
    ap.add_argument("--config", default=None,
                    help="with --only linear: bm,bn,bk,warps,stages,group_m (default: the "
                         "library's choice)")
    ap.add_argument("--trace-summary", nargs=2, metavar=("SWEEP_CSV", "POINTS_CSV"),
                    default=None,
                    help="summarize two rocprofv3 kernel traces (the sweep run with --mark, "
                         "--only decode_points --mark) into in-graph against alone kernel "
                         "times per point, on the host (no GPU); --steps as in the sweep run")
    ap.add_argument("--traffic-summary", nargs=4,
                    metavar=("KIND", "FETCH_CSV", "WRITE_CSV", "RUN_JSON"), default=None,
                    help="HBM traffic per launch (KIND config0 or prefill) from a FETCH_SIZE and "
                         "a WRITE_SIZE counter run of the same command and that command's "
                         "output line, on the host (no GPU)")
    args = ap.parse_args()
    if args.traffic_summary:
        print(json.dumps(traffic_summary(*args.traffic_summary), indent=1))
        return 0
    if args.trace_summary:
        print(json.dumps({"trace_summary": trace_summary(*args.trace_summary, args.steps)}))
        return 0
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
        fn = {"quant": lambda d: bench_quant(d, args.quant_m),
              "prefill": lambda d: bench_prefill(d, args.prefill_m),
              "standin": bench_standin, "launch": bench_launch,
              "llama_decode": bench_llama_decode, "floors": bench_floors,
              "linear": lambda d: run_linear(d, args.kn, args.m, args.config),
              "decode_points": lambda d: decode_points(d, mark=args.mark)}[args.only]
        res = {args.only: fn(dev)}
        if args.calibrate:
            res["calibration"] = copy_calibration(dev)
        print(json.dumps(res), flush=True)
        return 0
    shapes = SHAPES["qwen3-1.7b-vllm"]
    sw = Sweep(shapes, DECODE_M, dev)
    log(f"sweep: {len(sw.points)} linears, weight copies per shape {sorted(sw.copies.values())}")

    # correctness first: each point through the C entry into a poisoned output, checked
    # against float64, and the timed call path (the binding) must give the same bits
    worst = 0.0
    for i, (label, m, k, n, bias, d) in enumerate(sw.points):
        out = checked_mm(d)
        err = check_linear(out, d)
        worst = max(worst, err)
        if not err <= 1e-2:
            raise SystemExit(f"FAIL: {label} M={m} bias={bias}: max rel err {err}")
        if not torch.equal(sw.call(i, 0), out):
            raise SystemExit(f"FAIL: {label} M={m} bias={bias}: the timed path differs")
    log(f"sweep checked against float64: worst rel err {worst:.3g}")

    # one step = the whole sweep, each call on its own weight copy, one graph (two graphs
    # alternate, so consecutive steps read different copies too)
    plan = sw.step_copies(2)

    def step_calls(rep: int):
        for i in range(len(sw.points)):
            sw.call(i, plan[rep][i])

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
    mark = torch.zeros(1, dtype=torch.int16, device=dev)   # its add is the trace's marker
    torch.cuda.synchronize()
    if args.mark:
        mark.add_(1)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(args.steps):
        graphs[i % 2].replay()
    stop.record()
    if args.mark:
        mark.add_(1)
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
        "config": {"workload": "BASELINE config 1: decode sweep, 4 Qwen3-1.7B linears x "
                               "M{1,2,4,8,16,17,32,64,128} x bias{off,on}",
                   "linears_per_step": n_calls,
                   "min_reuse_MiB": round(sw.min_reuse_bytes(plan) / 2 ** 20, 1),
                   "sweep_GBps": round(sweep_bytes / (ms_per_step * 1e-3) / 1e9, 1)},
    }
    details = {"weight_copies": {f"{k}x{n}": c for (k, n), c in sw.copies.items()}}

    result["roofline"] = roofline_config0(dev)
    log(f"roofline config0: {result['roofline']['avg_launch_us']:.2f} us, "
        f"{result['roofline']['achieved']:.0f} GB/s ({result['roofline']['frac']:.1%})")

    if not args.no_extra:
        details["decode_points"] = decode_points(dev, sw)
        result["decode"] = summary_decode(details["decode_points"]["rows"])
        for name, fn in (("quant", bench_quant), ("llama_decode", bench_llama_decode),
                         ("prefill", bench_prefill), ("standin", bench_standin),
                         ("launch", bench_launch), ("floors", bench_floors)):
            details[name] = fn(dev)
            summary = SUMMARIES[name](details[name])
            if summary:
                result[name] = summary
        result["checks"] = ("every timed output checked first (poisoned outputs): sweep, Llama "
                            "decode and prefill against float64; quantizers and every op of the "
                            "stand-in against the reference's CPU arithmetic")
    if not args.no_cpu_baseline:
        ref_path = cpu_reference_path()
        details["cpu_reference_path"] = ref_path
        result["cpu_baseline"] = {
            "value": ref_path["gemm_int_mm"], "unit": "us per linear", "cores": ref_path["threads"],
            "kind": "port",
            "sample": "config 0 (M=16 K=2048 N=4096): the reference's CPU path in torch ops, "
                      "torch._int_mm + fp32 dequant + bf16 cast (kernel.py:105-120), median of "
                      "5 windows of ~0.4 s"}
        result["cpu_reference_path"] = {k: v for k, v in ref_path.items()
                                        if k not in ("sample", "unit")}
        result["cpu_oracle"] = cpu_baseline()
    # the per-point tables on lines of their own, then the one-line result (last line)
    for name, obj in details.items():
        print(json.dumps({"detail": name, "data": obj}), flush=True)
    if args.details:
        Path(args.details).write_text(json.dumps({**result, "details": details}, indent=1) + "\n")
    print(json.dumps(result), flush=True)
    return 0


# ---------------------------------------------------------------- one-line summaries
# The result line keeps only scalars in each section (the driver's record keeps a section's
# scalar fields), the tables go on the lines before it.

def summary_decode(table) -> dict:
    """us and HBM fraction per Qwen3 shape at 1, 16 and 128 tokens (no bias), and the mean
    HBM fraction over 1-16 tokens."""
    out = {}
    for label in dict.fromkeys(r[0] for r in table):
        rows = {r[1]: r for r in table if r[0] == label and r[2] == 0}
        short = label.replace("_proj", "")
        for m in (1, 16, 128):
            if m in rows:
                out[f"{short}_m{m}_us"] = rows[m][3]
        small = [rows[m][4] for m in rows if m <= 16]
        if small:
            out[f"{short}_m1_16_hbm_frac"] = round(sum(small) / len(small), 3)
    return out


def summary_prefill(pf) -> dict:
    """The dominant launch's roofline fields, then the MFMA fraction of every shape and M."""
    out = dict(pf.get("roofline", {}))
    for label, m, us, tops, frac in pf["rows"]:
        out[f"{label.replace('_proj', '')}_m{m}_frac"] = frac
    return out


def summary_quant(q) -> dict:
    out = {}
    for m, us_n, f_n, us_s, f_s in q["rows"]:
        if m in (1, 4096):
            out.update({f"add_rmsnorm_quant_m{m}_us": us_n, f"add_rmsnorm_quant_m{m}_frac": f_n,
                        f"silu_mul_quant_m{m}_us": us_s, f"silu_mul_quant_m{m}_frac": f_s})
    return out


def summary_standin(st) -> dict:
    out = {f"m{m}_us_per_layer": us for m, us, _ in st["rows"]}
    out["ops_checked"] = st.get("ops_checked")
    return out


def summary_llama(ld) -> dict:
    return {f"{label.replace('_proj', '')}_m{m}_frac": frac
            for label, m, us, frac, _ in ld["rows"] if m in (1, 16, 64)}


def summary_floors(fl) -> dict:
    out = {"empty_kernel_us": min(r[2] for r in fl["empty_kernel"]["rows"])}
    for mib, cache, us, gbs, frac, *_ in fl["read"]["rows"]:
        out[f"read_{mib}MiB_{cache}_us"] = us
    for name, operands, us, tops, frac in fl["mfma"]["rows"]:
        out[f"mfma_{name.split('_')[3]}_{operands}_TOPs"] = tops
    return out


SUMMARIES = {"quant": summary_quant, "llama_decode": summary_llama, "prefill": summary_prefill,
             "standin": summary_standin, "launch": lambda _: None, "floors": summary_floors}


def trace_summary(sweep_csv: str, points_csv: str, steps: int) -> dict:
    """In-graph against alone, per decode-sweep point, from two rocprofv3 kernel traces (CSV):
    the sweep run with --mark (the timed steps lie between two marker dispatches, each step
    the 72 points in order, a split of K being two dispatches) and --only decode_points --mark
    (each point's own graph replays after a marker dispatch).  Kernel durations are the
    trace's end - start of each dispatch: in the graph, the mean over the timed steps; alone,
    the median over the point's replays."""
    import csv

    from int8_linear.shapes import SHAPES

    def dispatches(path):
        rows = list(csv.DictReader(open(path)))
        rows.sort(key=lambda r: int(r["Start_Timestamp"]))
        return [(r["Kernel_Name"], (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
                for r in rows]

    def is_mark(name):     # the in-place add on the one-element int16 marker tensor
        return "elementwise" in name and "add" in name.lower() and "short" in name

    def short(name):
        return name.split("(")[0].replace("void ", "").replace("i8l::", "")

    labels = [(lbl, m, b) for lbl, k, n in SHAPES["qwen3-1.7b-vllm"] for m in DECODE_M
              for b in (0, 1)]
    sw = dispatches(sweep_csv)
    marks = [i for i, (nm, _) in enumerate(sw) if is_mark(nm)]
    inner = sw[marks[-2] + 1: marks[-1]]
    per_step = len(inner) // steps
    if per_step * steps != len(inner):
        raise SystemExit(f"{len(inner)} dispatches between the marks do not make {steps} steps")
    in_graph = []   # per point: (kernel names, summed mean us)
    pos = 0
    step0 = inner[:per_step]
    for _ in labels:
        names, idx = [short(step0[pos][0])], [pos]
        pos += 1
        if pos < per_step and "splitk_sum" in step0[pos][0]:
            names.append(short(step0[pos][0]))
            idx.append(pos)
            pos += 1
        us = sum(statistics.mean(inner[s * per_step + i][1] for s in range(steps)) for i in idx)
        in_graph.append((" + ".join(names), us))
    if pos != per_step:
        raise SystemExit(f"the step's {per_step} dispatches do not map onto {len(labels)} points")
    pt = dispatches(points_csv)
    pmarks = [i for i, (nm, _) in enumerate(pt) if is_mark(nm)] + [len(pt)]
    alone = []
    for a, b in zip(pmarks[:-1], pmarks[1:]):
        seg = [d for d in pt[a + 1: b] if "splitk_sum" not in d[0]]
        sk = [d for d in pt[a + 1: b] if "splitk_sum" in d[0]]
        us = statistics.median(d[1] for d in seg) + (statistics.median(d[1] for d in sk) if sk else 0)
        alone.append(us)
    if len(alone) != len(labels):
        raise SystemExit(f"{len(alone)} marked segments for {len(labels)} points")
    rows = [[lbl, m, b, names, round(g, 3), round(al, 3), round(g - al, 3)]
            for (lbl, m, b), (names, g), al in zip(labels, in_graph, alone)]
    return {"cols": ["shape", "M", "bias", "kernel", "in_graph_us", "alone_us", "diff_us"],
            "rows": rows, "mean_in_graph_us": round(statistics.mean(r[4] for r in rows), 3),
            "mean_alone_us": round(statistics.mean(r[5] for r in rows), 3)}


PREFILL_SHAPES = {"qkv_proj": (4096, 6144), "o_proj": (4096, 4096),
                  "gate_up_proj": (4096, 28672), "down_proj": (14336, 4096)}


def traffic_summary(kind: str, fetch_csv: str, write_csv: str, run_json: str) -> dict:
    """HBM bytes per launch from two rocprofv3 counter runs (CSV) of the same command, one with
    FETCH_SIZE and one with WRITE_SIZE (KiB a dispatch): kind "config0" for `--roofline-only`,
    "prefill" for `--only prefill --prefill-m 4096 --calibrate`; `run_json` is that command's
    last stdout line (the configs it ran).  Each counter is scaled by what it reads for the
    run's 256 MiB device copies (the largest copy dispatches); the GEMM dispatches (the
    library's kernels, in order) fall into one group per shape, where the kernel or its grid
    changes, and each group's mean per dispatch is its launch's traffic."""
    import csv

    def load(path):
        val, meta = collections.defaultdict(float), {}
        for r in csv.DictReader(open(path)):
            d = int(r["Dispatch_Id"])
            val[d] += float(r["Counter_Value"])
            meta[d] = (r["Kernel_Name"], int(r["Grid_Size"]))
        ds = sorted(val)
        # the calibration copies are the largest copy dispatches (other copies, e.g. of the
        # rotating weight buffers, may share their kernel and grid)
        copies = [val[d] for d in ds if "copyBuffer" in meta[d][0]]
        top = max(copies, default=0.0)
        copy = statistics.mean(v for v in copies if v >= 0.99 * top) if copies else 0.0
        groups, prev = [], None
        for d in ds:
            if "i8l::" not in meta[d][0] or "gemm" not in meta[d][0]:
                continue
            if meta[d] != prev:
                groups.append([])
                prev = meta[d]
            groups[-1].append(val[d])
        return [statistics.mean(g) for g in groups], copy, [meta[d][0] for d in ds]

    fetch, fcopy, _ = load(fetch_csv)
    write, wcopy, _ = load(write_csv)
    if not fcopy or not wcopy:
        raise SystemExit("no device copy in the runs: add --calibrate")
    cmd = {"config0": "--roofline-only", "prefill": "--only prefill --prefill-m 4096 --calibrate"}[kind]
    commands = [f"rocprofv3 --pmc {c} --output-format csv -d DIR/{c} -o c -- python3 bench.py "
                f"{cmd} > DIR/{c}.out" for c in ("FETCH_SIZE", "WRITE_SIZE")]
    commands.append(f"python3 bench.py --traffic-summary {kind} "
                    "DIR/FETCH_SIZE/c_counter_collection.csv "
                    "DIR/WRITE_SIZE/c_counter_collection.csv DIR/FETCH_SIZE.out")
    copy_bytes = 256 << 20
    fs, ws = copy_bytes / (fcopy * 1024), copy_bytes / (wcopy * 1024)
    run = json.loads(open(run_json).read().strip().splitlines()[-1])
    cal = {"copy_bytes": copy_bytes, "fetch_kib": round(fcopy, 2), "write_kib": round(wcopy, 2),
           "fetch_scale": round(fs, 4), "write_scale": round(ws, 4)}
    note = ("FETCH_SIZE counts bytes the L2 fetches from the fabric (Infinity Cache or HBM), so "
            "these are an upper bound on HBM bytes")

    def record(f, w, algorithmic):
        return {"fetch_kib_per_launch": round(f, 2), "write_kib_per_launch": round(w, 2),
                "bytes_per_launch": int(round(f * 1024 * fs + w * 1024 * ws)),
                "algorithmic_bytes_per_launch": algorithmic}

    if kind == "config0":
        if len(fetch) != 1 or len(write) != 1:
            raise SystemExit(f"expected one GEMM launch group, found {len(fetch)} / {len(write)}")
        rf = run["roofline"]
        out = {"config": rf["kernel"].split("config ")[1].split(" (")[0],
               "workload": "BASELINE config 0 (M=16, K=2048, N=4096, no bias, bf16 out), cold "
                           "weights", "copy_calibration": cal, "note": note,
               "commands": commands}
        out.update(record(fetch[0], write[0], rf["bytes_per_launch"]))
        return out
    per = run["prefill"]["per_shape"]
    if len(fetch) != len(PREFILL_SHAPES) or len(write) != len(PREFILL_SHAPES):
        raise SystemExit(f"expected {len(PREFILL_SHAPES)} GEMM launch groups, found "
                         f"{len(fetch)} / {len(write)}")
    out = {"workload": "BASELINE config 3 at M=4096 (Llama-3-8B shapes, bench.py --only "
                       "prefill --prefill-m 4096)", "copy_calibration": cal, "note": note,
           "commands": commands, "shapes": {}}
    m = 4096
    for i, (lbl, (k, n)) in enumerate(PREFILL_SHAPES.items()):
        rec = {"config": per[lbl]["kernel"].split("config ")[1].split(" (")[0]}
        rec.update(record(fetch[i], write[i], m * k + k * n + 4 * m + 4 * n + 2 * m * n))
        out["shapes"][lbl] = rec
    return out


def decode_points(dev, sw=None, mark: bool = False) -> dict:
    """Each point of the decode sweep timed on its own: a HIP graph of back-to-back calls of
    that point alone, its weight rotating through the shape's copies (checked first when the
    sweep is built here)."""
    import torch
    if sw is None:
        from int8_linear.shapes import SHAPES
        sw = Sweep(SHAPES["qwen3-1.7b-vllm"], DECODE_M, dev)
        for i, (label, m, k, n, bias, d) in enumerate(sw.points):
            out = checked_mm(d)
            if not check_linear(out, d) <= 1e-2 or not torch.equal(sw.call(i, 0), out):
                raise SystemExit(f"FAIL: {label} M={m} bias={bias}")
    table = []
    marker = torch.zeros(1, dtype=torch.int16, device=dev)
    for i, (label, m, k, n, bias, d) in enumerate(sw.points):
        if mark:                 # one dispatch before each point's launches, for a trace
            marker.add_(1)
        us = graph_time_us(lambda j, i=i: sw.call(i, j), 2 * sw.copies[(k, n)], windows=3)
        gbs = gemm_bytes(m, k, n, bias) / (us * 1e-6) / 1e9
        table.append([label, m, int(bias), round(us, 2), round(gbs / HBM_PEAK_GBS, 3)])
    return {"cols": ["shape", "M", "bias", "us", "hbm_frac"], "rows": table}


def bench_quant(dev, ms=None) -> dict:
    """the two fused quantizers at H=2048 / I=6144.  Each size is checked
    first: the C entry point writes into poisoned outputs (codes 99, NaN scales and residual),
    which are compared with the reference's CPU arithmetic (ref_norm, ref_silu)."""
    import torch

    from int8_linear import _lib
    from int8_linear import fused_quant as fq

    def poisoned(shape, dtype=None):
        if dtype == torch.int8:
            return torch.full(shape, 99, dtype=torch.int8, device=dev)
        return torch.full(shape, float("nan"), device=dev,
                          dtype=torch.float32 if shape[1] == 1 else torch.bfloat16)
    rows = []
    for m in ms or QUANT_M:
        g = torch.Generator().manual_seed(m)
        copies = max(2, -(-ROTATE_BYTES // (m * 2048 * 7 + 1)))
        copies = min(copies, 64)
        xs = [torch.randn((m, 2048), generator=g).to(torch.bfloat16).to(dev) for _ in range(2)]
        rs = [torch.randn((m, 2048), generator=g).to(torch.bfloat16).to(dev) for _ in range(copies)]
        w = (1 + 0.1 * torch.randn(2048, generator=g)).to(torch.bfloat16).to(dev)
        # checked first: outputs poisoned, then against the reference's CPU arithmetic
        q, s, rout = poisoned((m, 2048), torch.int8), poisoned((m, 1)), poisoned((m, 2048))
        _lib.check(_lib.lib().i8l_add_rmsnorm_quant(
            xs[0].data_ptr(), rs[0].data_ptr(), w.data_ptr(), 1e-6, q.data_ptr(), s.data_ptr(),
            rout.data_ptr(), m, 2048, _lib.BF16, _lib.BF16, 1, _lib.stream_of(q)), RuntimeError)
        q0, s0, r0 = ref_norm(xs[0].cpu(), rs[0].cpu(), w.cpu(), 1e-6)
        check_quant(q, s, q0, s0, f"add_rmsnorm_quant M={m}")
        if not torch.equal(rout.cpu(), r0):
            raise SystemExit(f"FAIL add_rmsnorm_quant M={m}: residual_out differs")
        us_n = graph_time_us(lambda i: fq.add_rmsnorm_quant(xs[i % 2], rs[i % copies], w, 1e-6), 2 * copies, 3)
        copies_s = min(64, max(2, -(-ROTATE_BYTES // (m * 12288 * 2 + 1))))
        gus = [torch.randn((m, 12288), generator=g).to(torch.bfloat16).to(dev) for _ in range(copies_s)]
        q, s = poisoned((m, 6144), torch.int8), poisoned((m, 1))
        _lib.check(_lib.lib().i8l_silu_mul_quant(gus[0].data_ptr(), q.data_ptr(), s.data_ptr(), m,
                                                 6144, _lib.BF16, 1, 1, _lib.stream_of(q)),
                   RuntimeError)
        q0, s0 = ref_silu(gus[0].cpu(), True)
        check_quant(q, s, q0, s0, f"silu_mul_quant M={m}")
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

    from int8_linear import fused_quant as fq
    from int8_linear import standin
    base = standin.DecoderStandIn(1, generator_device="cuda")   # 1.41 GB of layer weights
    wbytes = base.weight_bytes() / len(base.layers)
    rows = []
    checked = 0
    for m in STANDIN_M + [STANDIN_PREFILL_M]:
        st = base.with_batch(m, seed=m)
        # every token row up to 128 tokens, 16 spread rows of the 4096-token step
        rows_m = slice(None) if m <= 128 else torch.linspace(0, m - 1, 16).long()

        def check(h, st=st, rows_m=rows_m):
            nonlocal checked
            checked += check_standin(st, rows_m, h)

        us = standin.per_layer_us(st, windows=5, check=check)
        rows.append([m, round(us, 2), round(wbytes / (us * 1e-6) / 1e9, 1)])
        log(f"standin M={m}: {us:.2f} us per layer (checked)")
        del st
    del base
    torch.cuda.empty_cache()
    return {"cols": ["M", "us_per_layer", "weight_GBps"], "rows": rows, "ops_checked": checked,
            "layers": standin.LAYERS, "weight_bytes_per_layer": int(wbytes),
            "step": "add_rmsnorm_quant > qkv > quant(q cols) > o > add_rmsnorm_quant > gate_up "
                    "> silu_mul_quant > down, one HIP graph per 28-layer step; folded into one "
                    "launch each where few tokens make it pay: norm+qkv and norm+gate_up up to "
                    f"{fq.NORM_MM_FOLD_M} tokens, quant+o up to {fq.QUANT_MM_MAX_M}, "
                    f"silu_mul_quant+down up to {fq.SILU_MM_MAX_M} except at "
                    f"{fq.SILU_EPI_MIN_M}-{fq.SILU_EPI_MAX_M} tokens, where gate_up writes "
                    "silu(gate)*up and down quantizes it"}


LLAMA_DECODE_M = [1, 4, 16, 64, 128]


def bench_llama_decode(dev) -> dict:
    """Decode on the Llama-3-8B shapes (the larger of the two models BASELINE names for the
    HBM target at M <= 16, and at 64 and 128 tokens, where down_proj splits K across
    workgroups): µs per linear, fraction of 8 TB/s and the configuration, weights rotating
    through >= 768 MiB of copies so every call reads them from HBM."""
    import torch

    from int8_linear import w8a8_mm
    from int8_linear.kernel import choose_config
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
            dd = {"a_q": a_q, "w_q": ws[0], "a_s": a_s, "w_s": w_s, "bias": None}
            out = checked_mm(dd)
            err = check_linear(out, dd)
            if not err <= 1e-2 or not torch.equal(
                    w8a8_mm(a_q, ws[0].t(), a_s, w_s, torch.bfloat16), out):
                raise SystemExit(f"FAIL llama decode {label} M={m}: rel err {err}")
            us = graph_time_us(lambda i: w8a8_mm(a_q, ws[i % copies].t(), a_s, w_s,
                                                 torch.bfloat16), 2 * copies, 3)
            frac = gemm_bytes(m, k, n, False) / (us * 1e-6) / 1e9 / HBM_PEAK_GBS
            cfg = choose_config(m, n, k)
            rows.append([label, m, round(us, 2), round(frac, 3), f"{schedule_of(cfg, k)} {cfg.name}"])
            log(f"llama decode {label} M={m}: {us:.2f} us, {frac:.1%} of HBM ({cfg.name})")
        del ws, d
        torch.cuda.empty_cache()
    return {"cols": ["shape", "M", "us", "hbm_frac", "kernel"], "rows": rows}


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


PREFILL_TRAFFIC_PATH = ROOT / "profiles" / "traffic_prefill_config3.json"


def bench_prefill(dev, ms=None) -> dict:
    """Llama-3-8B shapes at prefill M, int8 TOP/s against the 5.0 POP/s
    dense int8 MFMA peak.  `roofline` is the dominant launch (gate_up at M=4096, the longest),
    `per_shape` the same object for each shape at M=4096; `achieved` = 2*M*N*K ops per launch
    / the average launch time of back-to-back launches in a HIP graph (HIP events on the
    launch stream)."""
    import torch

    from int8_linear import w8a8_mm
    from int8_linear.kernel import choose_config
    from int8_linear.operands import quant_rows
    from int8_linear.shapes import SHAPES
    ms = ms or PREFILL_M
    traffic = {}
    if PREFILL_TRAFFIC_PATH.exists():
        traffic = json.loads(PREFILL_TRAFFIC_PATH.read_text()).get("shapes", {})
    rows, per_shape = [], {}
    for label, k, n in SHAPES["llama-3-8b"]:
        g = torch.Generator().manual_seed(k + n)
        w = (torch.randn((n, k), generator=g) * 0.02).to(torch.bfloat16)
        w_q, w_s = quant_rows(w)
        w_q, w_s = w_q.to(dev), w_s.to(dev)
        del w
        for m in ms:
            x = torch.randn((m, k), generator=g).to(torch.bfloat16)
            a_q, a_s = quant_rows(x)
            a_q, a_s = a_q.to(dev), a_s.to(dev)
            out = checked_mm({"a_q": a_q, "w_q": w_q, "a_s": a_s, "w_s": w_s, "bias": None})
            # float64 on 64 rows spread over M (several in every 256-row tile block);
            # every element must have been written (no NaN left)
            rows_m = torch.linspace(0, m - 1, 64).long().to(dev)
            term = (a_q[rows_m].double() @ w_q.double().t()) * a_s[rows_m].double() * \
                w_s.double().t()
            err = ((out[rows_m].double() - term).abs() / term.abs().clamp_min(1e-6)).max().item()
            if not err <= 1e-2 or bool(out.isnan().any()) or not torch.equal(
                    w8a8_mm(a_q, w_q.t(), a_s, w_s, torch.bfloat16), out):
                raise SystemExit(f"FAIL prefill {label} M={m}: rel err {err}")
            us = graph_time_us(lambda i: w8a8_mm(a_q, w_q.t(), a_s, w_s, torch.bfloat16), 10, 3)
            ops = 2 * m * n * k
            tops = ops / (us * 1e-6) / 1e12
            rows.append([label, m, round(us, 2), round(tops, 1), round(tops / INT8_PEAK_TOPS, 3)])
            log(f"prefill {label} M={m}: {us:.1f} us {tops:.0f} TOP/s")
            if m == max(ms):
                cfg = choose_config(m, n, k)
                rec = traffic.get(label, {})
                per_shape[label] = {
                    "bound": "mfma", "achieved": round(tops, 1), "peak": INT8_PEAK_TOPS,
                    "unit": "TOP/s", "frac": round(tops / INT8_PEAK_TOPS, 4),
                    "traffic": rec.get("bytes_per_launch") if rec.get("config") == cfg.name
                    else None,
                    "kernel": f"{schedule_of(cfg, k)}, config {cfg.name} "
                              f"(Llama-3-8B {label}: M={m} K={k} N={n})",
                    "ops_per_launch": ops, "avg_launch_us": round(us, 3), "launches": 10}
        del w_q, w_s
    out = {"cols": ["shape", "M", "us", "TOPs", "mfma_frac"], "rows": rows,
           "per_shape": per_shape}
    if per_shape:
        dominant = max(per_shape, key=lambda lbl: per_shape[lbl]["avg_launch_us"])
        out["roofline"] = per_shape[dominant]
    return out


PROBES_LIB = ROOT / "int8-linear_amd" / "probes" / "libi8l_floors.so"


def run_linear(dev, kn: str, m: int, config: str | None, reps: int = 3) -> dict:
    """One W8A8 linear launched repeatedly, for a profiler to watch (rocprofv3 kernel trace or
    counters): random int8 operands of the shape, fp32 per-token and per-channel scales, bf16
    out, the given config (bm,bn,bk,warps,stages,group_m) or the library's choice.  The
    weights rotate through copies filling >= 768 MiB, so every launch reads them from HBM;
    the first output is checked against float64 before the profiled launches."""
    import torch

    from int8_linear.kernel import Config, choose_config, w8a8_mm
    k, n = map(int, kn.lower().split("x"))
    cfg = Config(*map(int, config.split(","))) if config else choose_config(m, n, k)
    g = torch.Generator().manual_seed(m * 7919 + k * 31 + n)
    copies = max(2, -(-ROTATE_BYTES // (k * n)))
    ws = [torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(dev)
          for _ in range(copies)]
    a = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8).to(dev)
    sa = (torch.rand((m, 1), generator=g) * 1e-2).to(dev)
    sb = (torch.rand((n, 1), generator=g) * 1e-2).to(dev)
    d = {"a_q": a, "w_q": ws[0], "a_s": sa, "w_s": sb, "bias": None}
    err = check_linear(checked_mm(d, cfg), d)
    if not err <= 1e-2:
        raise SystemExit(f"FAIL linear {kn} M={m} {cfg.name}: rel err {err}")
    for _ in range(reps):
        for w in ws:
            w8a8_mm(a, w.t(), sa, sb, torch.bfloat16, config=cfg)
    torch.cuda.synchronize()
    log(f"ran {reps * copies} launches: M={m} K={k} N={n} {cfg.name}")
    return {"kn": kn, "m": m, "config": cfg.name, "launches": reps * copies,
            "kernel": schedule_of(cfg, k)}


def bench_floors(dev) -> dict:
    """What the hardware gives a kernel of each regime, measured the way the kernels are
    (back-to-back launches in a HIP graph, HIP events on the launch stream), by the probe
    kernels of int8-linear_amd/probes/i8l_floors.hip:
      * an empty kernel at three grid shapes (the decode GEMM's is 256 x 512 threads);
      * a read of 4 / 8 / 12 / 16 / 24 / 120 MiB (the weights of Qwen3 o_proj, config 0,
        Qwen3 down_proj, Llama-3-8B o_proj, Qwen3 gate_up, Llama-3-8B gate_up) rotating
        through >= 768 MiB of buffers so every read comes from HBM, and 8 MiB hot; the best
        of 1, 2, 4 and 8 loads a thread;
      * back-to-back int8 MFMAs on every SIMD: the rate sustained under load, on constant
        operands and on random ones (toggling data costs power, and the clock follows);
      * the rate at which CUs take in L2-resident bytes (each workgroup re-reading 64 KiB
        windows that stay in its XCD's L2), into registers and straight into LDS;
      * the LDS read rate of 16-byte-a-lane reads (the GEMMs' MFMA fragment reads) at 8 and
        32 waves a CU."""
    import ctypes

    import torch

    from int8_linear import _lib
    _lib.lib()                               # torch's HIP runtime first
    L = ctypes.CDLL(str(PROBES_LIB))
    L.fl_empty.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    L.fl_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                          ctypes.c_void_p]
    L.fl_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                          ctypes.c_void_p, ctypes.c_void_p]
    L.fl_ingest.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                            ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    L.fl_lds.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                         ctypes.c_void_p]

    def stream():
        return torch.cuda.current_stream(dev).cuda_stream

    def ok(rc):
        if rc != 0:
            raise SystemExit(f"FAIL floor probe launch: status {rc}")

    sink = torch.zeros(16, dtype=torch.int32, device=dev)
    empty = []
    for blocks, threads in ((1, 64), (256, 512), (1024, 256)):
        us = graph_time_us(lambda i: ok(L.fl_empty(blocks, threads, stream())), 200)
        empty.append([blocks, threads, round(us, 3)])
        log(f"floor empty kernel {blocks}x{threads}: {us:.2f} us")
    reads = []
    for mib, cold in ((4, True), (8, True), (12, True), (16, True), (24, True), (120, True),
                      (8, False)):
        size = mib << 20
        copies = max(2, -(-ROTATE_BYTES // size)) if cold else 1
        bufs = [torch.zeros(size, dtype=torch.uint8, device=dev) for _ in range(copies)]
        per_unroll = {}
        for unroll in (1, 2, 4, 8):
            per_unroll[unroll] = graph_time_us(
                lambda i: ok(L.fl_read(bufs[i % copies].data_ptr(), size, sink.data_ptr(),
                                       unroll, stream())), 2 * copies if cold else 50)
        best = min(per_unroll, key=per_unroll.get)
        us = per_unroll[best]
        gbs = size / (us * 1e-6) / 1e9
        reads.append([mib, "cold" if cold else "hot", round(us, 3), round(gbs, 1),
                      round(gbs / HBM_PEAK_GBS, 3), best,
                      {u: round(t, 3) for u, t in per_unroll.items()}])
        log(f"floor read {mib} MiB {'cold' if cold else 'hot'}: {us:.2f} us {gbs:.0f} GB/s "
            f"(loads a thread {best}; all: {per_unroll})")
        del bufs
    mfma = []
    props = torch.cuda.get_device_properties(dev)
    blocks, iters = 8 * props.multi_processor_count, 1000
    rnd = torch.randint(-128, 128, (4096,), dtype=torch.int8,
                        generator=torch.Generator().manual_seed(0)).to(dev)
    for kind, ops_each in ((32, 65536), (16, 32768)):
        for operands, data in (("constant", None), ("random", rnd.data_ptr())):
            us = graph_time_us(lambda i: ok(L.fl_mfma(kind, blocks, iters, data,
                                                      sink.data_ptr(), stream())), 5)
            tops = blocks * 4 * iters * 4 * ops_each / (us * 1e-6) / 1e12
            name = "v_mfma_i32_32x32x32_i8" if kind == 32 else "v_mfma_i32_16x16x64_i8"
            mfma.append([name, operands, round(us, 1), round(tops, 1),
                         round(tops / INT8_PEAK_TOPS, 3)])
            log(f"floor {name} {operands} operands: {tops:.0f} TOP/s")
    ingest = []
    window = torch.randint(-128, 128, (2 << 20,), dtype=torch.int8,
                           generator=torch.Generator().manual_seed(1)).to(dev)
    cus = props.multi_processor_count
    for direct in (0, 1):
        for blocks in (cus, 2 * cus):
            iters = 128
            us = graph_time_us(lambda i: ok(L.fl_ingest(window.data_ptr(), 32, blocks, 8, direct,
                                                        iters, sink.data_ptr(), stream())), 5)
            total = blocks * iters * 65536
            ingest.append(["lds" if direct else "registers", blocks, round(us, 1),
                           round(total / (us * 1e-6) / 1e12, 2),
                           round(total / (us * 1e-6) / 1e9 / cus, 1)])
            log(f"floor L2 ingest into {'LDS' if direct else 'registers'}, {blocks} workgroups: "
                f"{total / (us * 1e-6) / 1e9 / cus:.0f} GB/s per CU")
    lds = []
    for blocks in (cus, 4 * cus):
        iters = 4096
        us = graph_time_us(lambda i: ok(L.fl_lds(blocks, 512, iters, sink.data_ptr(),
                                                 stream())), 3)
        total = blocks * 512 * 16 * 8 * iters
        lds.append([blocks * 8 // cus, round(us, 1), round(total / (us * 1e-6) / 1e9 / cus, 1)])
        log(f"floor LDS reads, {blocks * 8 // cus} waves a CU: "
            f"{total / (us * 1e-6) / 1e9 / cus:.0f} GB/s per CU")
    torch.cuda.empty_cache()
    return {"empty_kernel": {"cols": ["blocks", "threads", "us"], "rows": empty},
            "lds_read": {"cols": ["waves_per_CU", "us", "GBps_per_CU"], "rows": lds,
                         "read": "ds_read_b128, 8 in flight a wave, conflict-free"},
            "l2_ingest": {"cols": ["into", "workgroups", "us", "TBps", "GBps_per_CU"],
                          "rows": ingest, "waves_per_workgroup": 8, "window_KiB": 64},
            "read": {"cols": ["MiB", "cache", "us", "GBps", "hbm_frac", "loads_per_thread",
                              "us_by_loads_per_thread"], "rows": reads},
            "mfma": {"cols": ["instruction", "operands", "us", "TOPs", "frac_of_5000"],
                     "rows": mfma,
                     "waves": blocks * 4, "mfmas_per_wave": iters * 4},
            "compute_units": props.multi_processor_count}


if __name__ == "__main__":
    sys.exit(main())
