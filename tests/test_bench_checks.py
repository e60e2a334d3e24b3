"""The bench's own output checks, on the CPU: the reference's CPU arithmetic that bench.py
compares the timed quantizers and stand-in ops with (ref_mm, ref_norm, ref_silu, ref_quant,
check_quant) must accept the oracle's outputs, which the GPU matches bit for bit, and must
reject a planted mistake; and the one-line result keeps only scalars in each section (the
driver's record keeps a section's scalar fields).
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

import bench
from helpers import from_bits
from oracle import oracle as o


def _bf16(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_ref_mm_is_the_oracle_bit_for_bit():
    """The reference's CPU path of a linear (torch._int_mm, fp32 dequant, one cast) is the
    oracle's epilogue order, so the bench's GEMM check is bit equality."""
    g = torch.Generator().manual_seed(3)
    for m, k, n in ((1, 2048, 4096), (8, 6144, 2048), (5, 256, 96)):
        q = torch.randint(-128, 128, (m, k), dtype=torch.int8, generator=g)
        w = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=g)
        s = torch.rand((m, 1), generator=g) * 1e-2 + 1e-3
        ws = torch.rand((n, 1), generator=g) * 1e-3 + 1e-4
        got = bench.ref_mm(q, s, w, ws)
        ref = o.w8a8_mm(q.numpy(), w.numpy(), s.numpy(), ws.numpy(), out_dt=o.BF16)
        assert np.array_equal(_bits(got), ref)


def test_quantizer_checks_accept_the_oracle():
    x, r = _bf16((64, 2048), 1), _bf16((64, 2048), 2)
    gamma = (1 + 0.1 * torch.randn(2048, generator=torch.Generator().manual_seed(3))).to(
        torch.bfloat16)
    q, s, rout = o.add_rmsnorm_quant(_bits(x), _bits(r), _bits(gamma), 1e-6)
    q0, s0, r0 = bench.ref_norm(x, r, gamma, 1e-6)
    bench.check_quant(torch.from_numpy(q), torch.from_numpy(s), q0, s0, "norm")
    assert torch.equal(from_bits(rout, device="cpu"), r0)
    gu = _bf16((64, 12288), 4)
    for round_silu in (False, True):
        q, s = o.silu_mul_quant(_bits(gu), round_silu=round_silu)
        q0, s0 = bench.ref_silu(gu, round_silu)
        bench.check_quant(torch.from_numpy(q), torch.from_numpy(s), q0, s0, "silu")
    y = _bf16((16, 2048), 5).float()
    q, s = o.quant_per_token(_bits(y.to(torch.bfloat16)))
    q0, s0 = bench.ref_quant(y.to(torch.bfloat16).float())
    bench.check_quant(torch.from_numpy(q), torch.from_numpy(s), q0, s0, "quant")


def test_quantizer_check_rejects_planted_mistakes():
    gu = _bf16((16, 12288), 6)
    q, s = (torch.from_numpy(a) for a in o.silu_mul_quant(_bits(gu), round_silu=True))
    q0, s0 = bench.ref_silu(gu, True)
    bench.check_quant(q, s, q0, s0, "silu")
    two = q.clone()
    two[3, 7] = (two[3, 7].int() + 2).clamp(-128, 127).to(torch.int8)
    with pytest.raises(SystemExit):
        bench.check_quant(two, s, q0, s0, "code off by two")
    many = q.clone()
    many[:, :100] = (many[:, :100].int() + 1).clamp(-128, 126).to(torch.int8)
    with pytest.raises(SystemExit):
        bench.check_quant(many, s, q0, s0, "1600 codes off by one")
    with pytest.raises(SystemExit):
        bench.check_quant(q, s * (1 + 1e-4), q0, s0, "scales off")
    one = s.clone()
    one[5] = one[5] * (1 + 2.0 ** -8)                     # one row a bf16 step of absmax away
    bench.check_quant(q, one, q0, s0, "one row's scale a bf16 step away")
    one[5] = s[5] * (1 + 2.0 ** -5)                       # too far
    with pytest.raises(SystemExit):
        bench.check_quant(q, one, q0, s0, "one row's scale far off")
    two = s.clone()
    two[1:3] = two[1:3] * (1 + 2.0 ** -8)                 # two of 16 rows: more than allowed
    with pytest.raises(SystemExit):
        bench.check_quant(q, two, q0, s0, "two rows' scales off")
    with pytest.raises(SystemExit):
        bench.check_quant(q, torch.full_like(s, float("nan")), q0, s0, "scales never written")


def test_result_sections_are_scalars():
    """Each summary section of the one-line result holds scalars only, from tables shaped
    as the bench's legs return them."""
    decode = [["qkv_proj", m, b, 3.5, 0.3] for m in bench.DECODE_M for b in (0, 1)]
    prefill = {"rows": [["qkv_proj", m, 100.0, 2000.0, 0.4] for m in bench.PREFILL_M],
               "roofline": {"bound": "mfma", "achieved": 2000.0, "peak": 5000.0,
                            "unit": "TOP/s", "frac": 0.4, "traffic": None, "kernel": "k"}}
    quant = {"rows": [[m, 2.0, 0.1, 3.0, 0.2] for m in bench.QUANT_M]}
    standin = {"rows": [[m, 25.0, 2000.0] for m in bench.STANDIN_M + [4096]], "ops_checked": 9}
    llama = {"rows": [["gate_up_proj", m, 19.0, 0.76, "k"] for m in bench.LLAMA_DECODE_M]}
    floors = {"empty_kernel": {"rows": [[1, 64, 1.6]]},
              "read": {"rows": [[8, "cold", 2.9, 2900.0, 0.36, 4, {}]]},
              "mfma": {"rows": [["v_mfma_i32_32x32x32_i8", "random", 1.0, 3500.0, 0.7]]}}
    for fn, table in ((bench.summary_decode, decode), (bench.summary_prefill, prefill),
                      (bench.summary_quant, quant), (bench.summary_standin, standin),
                      (bench.summary_llama, llama), (bench.summary_floors, floors)):
        out = fn(table)
        assert out and all(isinstance(v, (int, float, str, type(None))) for v in out.values()), fn
        json.dumps(out)
    assert bench.summary_prefill(prefill)["qkv_m4096_frac"] == 0.4
    assert bench.summary_standin(standin)["m1_us_per_layer"] == 25.0


def test_trace_summary_maps_dispatches_onto_sweep_points(tmp_path):
    """bench.py --trace-summary on synthetic kernel traces shaped as the two runs make them:
    the timed steps between marker dispatches (a split of K being two dispatches), and each
    point's replays after its own marker."""
    import csv as csvmod

    n_points = 4 * len(bench.DECODE_M) * 2
    split = {5, 40}                                  # points launched as two kernels
    head = ["Kernel_Name", "Start_Timestamp", "End_Timestamp"]

    def write(path, events):
        t = 0
        with open(path, "w", newline="") as f:
            w = csvmod.writer(f)
            w.writerow(head)
            for name, dur in events:
                w.writerow([name, t, t + int(dur * 1000)])
                t += int(dur * 1000) + 500

    mark = ("void at::native::vectorized_elementwise_kernel<4, CUDAFunctorOnSelf_add<short>>()", 1)
    step = []
    for p in range(n_points):
        step.append((f"void i8l::gemm_k{p}(int)", 2.0 + p / 100))
        if p in split:
            step.append(("void i8l::splitk_sum<2>(int)", 1.0))
    steps = 3
    write(tmp_path / "sweep.csv", [("void warm()", 5)] + [mark] + step * steps + [mark] + step)
    pts = [("void check()", 3)]
    for p in range(n_points):
        pts.append(mark)
        for _ in range(5):
            pts.append((f"void i8l::gemm_k{p}(int)", 1.5 + p / 100))
            if p in split:
                pts.append(("void i8l::splitk_sum<2>(int)", 0.5))
    write(tmp_path / "points.csv", pts)
    out = bench.trace_summary(str(tmp_path / "sweep.csv"), str(tmp_path / "points.csv"), steps)
    rows = out["rows"]
    assert len(rows) == n_points
    assert rows[5][3] == "gemm_k5 + splitk_sum<2>" and rows[5][4] == 3.05 and rows[5][5] == 2.05
    assert rows[6][3] == "gemm_k6" and rows[6][4] == 2.06 and rows[6][5] == 1.56
    assert all(abs(r[6] - (r[4] - r[5])) < 1e-9 for r in rows)


def test_traffic_summary_groups_launches_and_scales_by_the_copies(tmp_path):
    """bench.py --traffic-summary on synthetic counter runs shaped as rocprofv3 writes them:
    GEMM dispatches grouped by shape where the kernel or grid changes (o_proj and down_proj
    share a kernel and grid, with gate_up between them), scaled by the 256 MiB copies'
    readings, and the configs taken from the run's output line."""
    import csv as csvmod

    head = ["Dispatch_Id", "Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"]
    kernels = [("void i8l::gemm_dmap<256, 192>(int)", 98304, 90000.0, 49152.0),
               ("void i8l::gemm_dmap<256, 256>(int)", 131072, 50000.0, 32768.0),
               ("void i8l::gemm_dmap<256, 256>(int)", 229376, 340000.0, 229376.0),
               ("void i8l::gemm_dmap<256, 256>(int)", 131072, 170000.0, 32768.0)]

    def write(path, col, scale):
        rows, did = [], 0
        for name, grid, f, w in kernels:
            for _ in range(3):                                  # a check and two timed launches
                did += 1
                rows.append([did, name, grid, col, (f if col == "FETCH_SIZE" else w) * scale])
        for _ in range(3):                                      # the three calibration copies
            did += 1
            val = 131072.0 if col == "FETCH_SIZE" else 262144.0
            rows.append([did, "__amd_rocclr_copyBuffer", 131072, col, val])
        for _ in range(5):                                      # small copies, same grid
            did += 1
            rows.append([did, "__amd_rocclr_copyBuffer", 131072, col, 4096.0])
        with open(path, "w", newline="") as fh:
            wr = csvmod.writer(fh)
            wr.writerow(head)
            wr.writerows(rows)

    write(tmp_path / "f.csv", "FETCH_SIZE", 1.0)
    write(tmp_path / "w.csv", "WRITE_SIZE", 1.0)
    cfgs = ["256x192x128 w8 s10 g4", "256x256x128 w8 s10 g8", "256x256x128 w8 s10 g4",
            "256x256x128 w8 s10 g4"]
    run = {"prefill": {"per_shape": {lbl: {"kernel": f"gemm_dmap, config {c} (x)"}
                                     for lbl, c in zip(bench.PREFILL_SHAPES, cfgs)}}}
    (tmp_path / "run.out").write_text("log line\n" + json.dumps(run) + "\n")
    out = bench.traffic_summary("prefill", str(tmp_path / "f.csv"), str(tmp_path / "w.csv"),
                                str(tmp_path / "run.out"))
    assert out["copy_calibration"]["fetch_scale"] == 2.0
    assert out["copy_calibration"]["write_scale"] == 1.0
    sh = out["shapes"]
    assert list(sh) == list(bench.PREFILL_SHAPES)
    assert sh["o_proj"]["config"] == cfgs[1] and sh["down_proj"]["config"] == cfgs[3]
    assert sh["gate_up_proj"]["bytes_per_launch"] == 340000 * 1024 * 2 + 229376 * 1024
    assert sh["down_proj"]["fetch_kib_per_launch"] == 170000.0
    m, k, n = 4096, 4096, 6144
    assert sh["qkv_proj"]["algorithmic_bytes_per_launch"] == m * k + k * n + 4 * m + 4 * n + 2 * m * n
