"""Pins of the CPU oracle (oracle/i8l_oracle.c) against mathematics that does not depend on
the restatement, before anything is checked against it.  CPU only.

Each oracle function is checked against an independent source chosen so that a plausible
mistake (a dropped term, a transposed operand, a wrong rounding) fails:
  * the exact int32 product against int64 numpy matmul and brute force;
  * the epilogue against float64 (<= 1 bf16 ulp) and exact power-of-two cases;
  * bf16/fp16 conversions against torch's casts;
  * exp against math.exp, rsqrt against 40-digit decimal arithmetic;
  * the quantizers against the reference's own torch restatements
    (AshrithaG/int8-linear tests/test_fused_quant.py:26-51) under its tolerance, against
    closed forms, and against hand-built tie cases;
  * the committed golden fixtures, which the oracle must still reproduce exactly.
"""

from __future__ import annotations

import decimal
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as o

GOLDEN = Path(__file__).resolve().parent / "golden"
EPS = 1e-6


def bits_to_bf16(h: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(h, np.uint16).view(np.int16)).view(torch.bfloat16)


def bf16_to_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


# ------------------------------------------------------------------ GEMM
@pytest.mark.parametrize("m,k,n", [(1, 64, 16), (3, 100, 7), (17, 2048, 64), (64, 6144, 32)])
def test_gemm_matches_int64_matmul(m, k, n):
    rng = np.random.default_rng(m * 1000 + k + n)
    a = rng.integers(-128, 128, (m, k), dtype=np.int8)
    w = rng.integers(-128, 128, (n, k), dtype=np.int8)
    ref = a.astype(np.int64) @ w.astype(np.int64).T
    assert np.array_equal(o.gemm_i32(a, w), ref.astype(np.int32))


def test_gemm_brute_force_and_float64():
    rng = np.random.default_rng(5)
    a = rng.integers(-127, 128, (4, 9), dtype=np.int8)
    w = rng.integers(-127, 128, (3, 9), dtype=np.int8)
    got = o.gemm_i32(a, w)
    for i in range(4):
        for j in range(3):
            assert got[i, j] == sum(int(a[i, kk]) * int(w[j, kk]) for kk in range(9))
    # float64 matmul of int8 values is exact (tests/test_kernel.py:36-38 of the reference)
    assert np.array_equal(got, (a.astype(np.float64) @ w.astype(np.float64).T).astype(np.int32))


def test_gemm_extreme_values_do_not_overflow():
    k = 14336
    a = np.full((2, k), -128, np.int8)
    w = np.full((2, k), -128, np.int8)
    assert o.gemm_i32(a, w)[0, 0] == 128 * 128 * k


def test_gemm_strided_layouts():
    rng = np.random.default_rng(8)
    M, N, K = 5, 6, 33
    a = rng.integers(-127, 128, (K, M), dtype=np.int8)        # A stored transposed
    b = rng.integers(-127, 128, (K, N), dtype=np.int8)        # B stored N-contiguous
    got = o.gemm_i32_strided(a.reshape(-1), 1, M, b.reshape(-1), N, 1, M, N, K)
    assert np.array_equal(got, a.T.astype(np.int64) @ b.astype(np.int64))


# ------------------------------------------------------------------ epilogue
def _ulp_bf16(x: np.ndarray) -> np.ndarray:
    e = np.floor(np.log2(np.maximum(np.abs(x), 1e-30)))
    return 2.0 ** (e - 7)


def test_epilogue_within_one_bf16_ulp_of_float64():
    rng = np.random.default_rng(11)
    M, N = 33, 257
    acc = rng.integers(-3_000_000, 3_000_000, (M, N)).astype(np.int32)
    sa = (rng.random((M, 1)) * 1e-2 + 1e-3).astype(np.float32)
    sb = (rng.random((N, 1)) * 1e-2 + 1e-3).astype(np.float32)
    out = o.bf16_to_f32(o.epilogue(acc, sa, sb, None, o.NONE, o.BF16)).astype(np.float64)
    ref = acc.astype(np.float64) * sa.astype(np.float64) * sb.astype(np.float64).T
    assert np.all(np.abs(out - ref) <= _ulp_bf16(ref))


def test_epilogue_bias_follows_the_reference_tolerance():
    # tests/test_kernel.py:68-75 of the reference: rel < 1e-2 of max(|ref|, |term|)
    rng = np.random.default_rng(12)
    M, N = 37, 128
    acc = rng.integers(-2_000_000, 2_000_000, (M, N)).astype(np.int32)
    sa = (rng.random((M, 1)) * 1e-2 + 1e-3).astype(np.float32)
    sb = (rng.random((N, 1)) * 1e-2 + 1e-3).astype(np.float32)
    for bias_dt, bias in ((o.F32, rng.standard_normal(N).astype(np.float32)),
                          (o.BF16, o.f32_to_bf16(rng.standard_normal(N)))):
        for out_dt in (o.BF16, o.F16, o.F32):
            out = o.epilogue(acc, sa, sb, bias, bias_dt, out_dt)
            outf = out if out_dt == o.F32 else o.act_to_f32(out, out_dt)
            b64 = bias.astype(np.float64) if bias_dt == o.F32 else o.bf16_to_f32(bias).astype(np.float64)
            term = acc.astype(np.float64) * sa.astype(np.float64) * sb.astype(np.float64).T
            ref = term + b64
            scale = np.maximum(np.abs(ref), np.abs(term)).clip(1e-6)
            assert (np.abs(outf.astype(np.float64) - ref) / scale).max() < 1e-2


def test_epilogue_exact_for_power_of_two_scales():
    acc = np.array([[3, -5, 1 << 20, -(1 << 23)]], np.int32)
    out = o.epilogue(acc, np.array([[0.5]], np.float32), np.array([0.25, 2, 1, 4], np.float32),
                     np.array([1, 1, 0, 0], np.float32), o.F32, o.F32)
    assert np.array_equal(out, np.array([[1.375, -4.0, 2.0 ** 19, -(2.0 ** 24)]], np.float32))


def test_epilogue_order_is_left_to_right():
    # (acc*sa)*sb differs from acc*(sa*sb) for these values; the reference multiplies by
    # sa first (int8_linear/kernel.py:109-117).
    acc = np.array([[1_000_003]], np.int32)
    sa, sb = np.float32(0.1), np.float32(0.3)
    out = o.epilogue(acc, np.array([sa]), np.array([sb]), None, o.NONE, o.F32)[0, 0]
    assert out == np.float32(np.float32(np.float32(1_000_003) * sa) * sb)


def test_raw_epilogue_is_identity():
    acc = np.arange(-6, 6, dtype=np.int32).reshape(3, 4)
    assert np.array_equal(o.epilogue(acc, np.ones(1), np.ones(1), None, o.NONE, o.I32), acc)


# ------------------------------------------------------------------ conversions
EDGE = np.array([0.0, -0.0, 1.0, -1.0, 1.00390625, 1.005859375, 3.0e38, -3.4e38, 1e-40,
                 -1e-45, 65504.0, 65519.0, 65520.0, 6.1e-5, 5.96e-8, 2.98e-8, 1e-8,
                 float("inf"), -float("inf"), 0.1, 1 / 3], np.float32)


def test_bf16_conversion_matches_torch():
    rng = np.random.default_rng(3)
    x = np.concatenate([EDGE, rng.standard_normal(100_000).astype(np.float32) * 100,
                        (rng.random(10_000) * 2 ** 8).astype(np.float32)])
    # values exactly half-way between two bf16 numbers
    ties = ((rng.integers(0, 1 << 16, 4096).astype(np.uint32) << 16) | 0x8000).view(np.float32)
    x = np.concatenate([x, ties[np.isfinite(ties)]])
    ref = bf16_to_bits(torch.from_numpy(x).to(torch.bfloat16))
    assert np.array_equal(o.f32_to_bf16(x), ref)
    # NaN: a quiet NaN with the input's sign and top payload bits (the gfx950 conversion's
    # rule); torch's canonical NaN 0x7FC0 is the case of a payload-free positive NaN
    nans = np.array([0x7FC00000, 0xFFC00001, 0x7F800001, 0xFF800001, 0x7FFFFFFF, 0x7FA51234],
                    np.uint32).view(np.float32)
    assert o.f32_to_bf16(nans).tolist() == [0x7FC0, 0xFFC0, 0x7FC0, 0xFFC0, 0x7FFF, 0x7FE5]
    assert o.f32_to_bf16(np.array([np.nan], np.float32))[0] == 0x7FC0


def test_f16_conversion_matches_torch():
    rng = np.random.default_rng(4)
    x = np.concatenate([EDGE, rng.standard_normal(100_000).astype(np.float32) * 1000,
                        rng.standard_normal(10_000).astype(np.float32) * 1e-6])
    ties = ((rng.integers(0, 1 << 19, 4096).astype(np.uint32) << 13) | 0x1000).view(np.float32)
    x = np.concatenate([x, ties[np.isfinite(ties)]])
    ref = torch.from_numpy(x).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(o.f32_to_f16(x), ref)
    back = torch.from_numpy(ref.view(np.int16)).view(torch.float16).float().numpy()
    assert np.array_equal(o.f16_to_f32(ref), back)


# ------------------------------------------------------------------ exp / rsqrt
def test_expf_within_one_ulp_of_math_exp():
    x = np.concatenate([np.linspace(-87.0, 88.7, 400_001, dtype=np.float32),
                        np.linspace(-1, 1, 100_001, dtype=np.float32)])
    got = o.expf(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - ref) <= ulp)
    # fp32 Horner evaluation: about 94% of results are the correctly rounded float
    assert np.mean(got == ref.astype(np.float32).astype(np.float64)) > 0.9


def test_expf_special_values():
    y = o.expf(np.array([0.0, -0.0, 1.0, -87.5, -1000.0, 88.8, 1000.0, np.nan], np.float32))
    assert y[0] == 1.0 and y[1] == 1.0
    assert y[2] == np.float32(math.e)
    assert y[3] == 0.0 and y[4] == 0.0
    assert np.isinf(y[5]) and np.isinf(y[6]) and np.isnan(y[7])


def test_rsqrtf_against_40_digit_decimal():
    rng = np.random.default_rng(6)
    v = np.concatenate([rng.random(2000).astype(np.float32) * 10,
                        (2.0 ** rng.integers(-60, 60, 500)).astype(np.float32) *
                        rng.random(500).astype(np.float32) + np.float32(1e-6),
                        np.array([1e-6, 1.0, 4.0, 2.0, 0.5, 3.0], np.float32)])
    got = o.rsqrtf(v)
    decimal.getcontext().prec = 40
    bad = 0
    for vi, gi in zip(v.tolist(), got.tolist()):
        exact = decimal.Decimal(1) / decimal.Decimal(vi).sqrt()
        cr = np.float32(float(exact))  # double then float: flagged below if that double-rounds
        if gi != cr:
            lo, hi = np.nextafter(cr, np.float32(0)), np.nextafter(cr, np.float32(np.inf))
            assert gi in (lo, hi)
            bad += 1
    assert bad <= 2  # double rounding may differ from the correctly rounded float, rarely


# ------------------------------------------------------------------ quantizer
def ref_quant(yf: torch.Tensor):
    """The reference's restatement of vLLM's quantizer (tests/test_fused_quant.py:26-31)."""
    absmax = yf.abs().amax(-1, keepdim=True)
    inv = torch.where(absmax == 0, torch.zeros_like(absmax), 127.0 / absmax)
    return torch.round(yf * inv).clamp(-128, 127).to(torch.int8), absmax / 127.0


def np_quant(y: np.ndarray):
    """The same restatement with numpy's float32 ops, which are IEEE-correctly rounded on
    every CPU (torch's CPU division can differ by an ulp between CPU builds)."""
    absmax = np.abs(y).max(-1, keepdims=True)
    inv = np.where(absmax == 0, np.float32(0), np.float32(127) / np.maximum(absmax, np.float32(1e-38)))
    q = np.clip(np.rint(y * inv.astype(np.float32)), -128, 127).astype(np.int8)
    return q, (absmax / np.float32(127)).astype(np.float32)


def test_quantize_row_matches_reference_restatement():
    rng = np.random.default_rng(7)
    for n in (1, 7, 2048, 6144):
        y = o.bf16_to_f32(o.f32_to_bf16(rng.standard_normal(n) * 3))
        q, s = o.quantize_row(y)
        q1, s1 = np_quant(y[None])
        assert np.array_equal(q, q1[0]) and s == s1[0, 0]
        q0, s0 = ref_quant(torch.from_numpy(y)[None])
        assert np.abs(q.astype(int) - q0[0].numpy().astype(int)).max() <= 1
        assert abs(s - s0.item()) <= np.spacing(np.float32(s))


def test_quantize_row_special_cases():
    q, s = o.quantize_row(np.zeros(64, np.float32))
    assert s == 0.0 and not q.any()
    q, s = o.quantize_row(np.array([-3.0, 1.0, 2.0], np.float32))
    assert q[0] == -127 and s == np.float32(3.0) / np.float32(127.0)
    # max exactly 127 -> inv == 1: half-way values round to even
    y = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5], np.float32)
    q, _ = o.quantize_row(y)
    assert q.tolist() == [127, 0, 2, 2, 0, -2, -2, 126]


def test_quantize_row_approximate_division_stays_close():
    rng = np.random.default_rng(9)
    y = rng.standard_normal(4096).astype(np.float32)
    q1, s1 = o.quantize_row(y, True)
    q0, s0 = o.quantize_row(y, False)
    assert np.abs(q1.astype(int) - q0.astype(int)).max() <= 1
    assert abs(s1 - s0) <= np.spacing(s1)


# ------------------------------------------------------------------ fused quantizers
def ref_norm(x, r, w):
    """tests/test_fused_quant.py:34-43 of the reference."""
    xf = x.float()
    rout = None
    if r is not None:
        xf = xf + r.float()
        rout = xf.to(x.dtype)
    var = xf.pow(2).mean(-1, keepdim=True)
    y = ((xf * torch.rsqrt(var + EPS)).to(w.dtype) * w).to(x.dtype)
    return (*ref_quant(y.float()), rout)


def ref_silu(gu, round_silu):
    """tests/test_fused_quant.py:46-51 of the reference."""
    i = gu.shape[1] // 2
    g, u = gu[:, :i].float(), gu[:, i:].float()
    a = g / (1.0 + torch.exp(-g))
    if round_silu:
        a = a.to(gu.dtype).float()
    return ref_quant((a * u).to(gu.dtype).float())


def assert_close_int8(q, s, q0, s0):
    """The reference's tolerance (tests/test_fused_quant.py:54-61)."""
    d = np.abs(q.astype(np.int32) - q0.astype(np.int32))
    assert d.max() <= 1
    assert np.count_nonzero(d) <= max(8, 1e-3 * d.size)
    assert (np.abs(s - s0) / np.maximum(np.abs(s0), 1e-30)).max() < 1e-5


def randn_bf16(shape, seed, scale=1.0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("m,k", [(1, 2048), (7, 2048), (64, 1024), (300, 2048), (5, 1000)])
@pytest.mark.parametrize("has_res", [False, True])
def test_add_rmsnorm_quant_against_reference_restatement(m, k, has_res):
    x = randn_bf16((m, k), m)
    r = randn_bf16((m, k), m + 1) if has_res else None
    w = randn_bf16((k,), 99, 0.1) + 1.0
    q, s, rout = o.add_rmsnorm_quant(bf16_to_bits(x), None if r is None else bf16_to_bits(r),
                                     bf16_to_bits(w), EPS)
    q0, s0, r0 = ref_norm(x, r, w)
    assert_close_int8(q, s, q0.numpy(), s0.numpy())
    if has_res:
        assert np.array_equal(rout, bf16_to_bits(r0))


def test_add_rmsnorm_quant_constant_row_closed_form():
    # x = c everywhere: var = c^2 exactly, xn = c/sqrt(c^2+eps) -> bf16 1.0 for c = 3,
    # y = 1.0 * w, so with w = 1 every code is 127 and the scale is 1/127
    H = 2048
    x = np.full((2, H), o.f32_to_bf16(np.float32(3.0)), np.uint16)
    x[1] = o.f32_to_bf16(np.float32(-3.0))
    w = np.full(H, o.f32_to_bf16(np.float32(1.0)), np.uint16)
    q, s, _ = o.add_rmsnorm_quant(x, None, w, EPS)
    assert (q[0] == 127).all() and (q[1] == -127).all()
    assert s[0, 0] == np.float32(1.0) / np.float32(127.0)


def test_add_rmsnorm_quant_sum_of_squares_is_exact_for_small_integers():
    # integer rows: sum x^2 is exact in double, so var is the correctly rounded mean; compare
    # the whole pipeline with the same steps done in Python integers/floats
    rng = np.random.default_rng(21)
    H = 1000
    xi = rng.integers(-20, 21, (3, H)).astype(np.float32)
    x = o.f32_to_bf16(xi)
    w = o.f32_to_bf16(np.ones(H, np.float32))
    q, s, _ = o.add_rmsnorm_quant(x, None, w, EPS)
    for row in range(3):
        ss = sum(int(v) * int(v) for v in xi[row])
        var = np.float32(ss / H)  # correctly rounded: ss and H are exact doubles
        rs = np.float32(1.0 / math.sqrt(float(np.float32(var + np.float32(EPS)))))
        y = o.bf16_to_f32(o.f32_to_bf16(o.bf16_to_f32(o.f32_to_bf16(xi[row] * rs))))
        q0, s0 = o.quantize_row(y)
        assert np.array_equal(q[row], q0) and s[row, 0] == s0


def test_fp16_activations_against_reference_restatement():
    g = torch.Generator().manual_seed(3)
    x = torch.randn((9, 2048), generator=g).to(torch.float16)
    r = torch.randn((9, 2048), generator=g).to(torch.float16)
    w = (torch.randn(2048, generator=g) * 0.1 + 1).to(torch.float16)
    xb = x.view(torch.int16).numpy().view(np.uint16)
    rb = r.view(torch.int16).numpy().view(np.uint16)
    wb = w.view(torch.int16).numpy().view(np.uint16)
    q, s, rout = o.add_rmsnorm_quant(xb, rb, wb, EPS, o.F16, o.F16)
    q0, s0, r0 = ref_norm(x, r, w)
    assert_close_int8(q, s, q0.numpy(), s0.numpy())
    assert np.array_equal(rout, r0.view(torch.int16).numpy().view(np.uint16))


@pytest.mark.parametrize("m,i", [(1, 6144), (33, 6144), (8, 1000)])
@pytest.mark.parametrize("round_silu", [False, True])
def test_silu_mul_quant_against_reference_restatement(m, i, round_silu):
    gu = randn_bf16((m, 2 * i), m, 2.0)
    q, s = o.silu_mul_quant(bf16_to_bits(gu), round_silu=round_silu)
    q0, s0 = ref_silu(gu, round_silu)
    assert_close_int8(q, s, q0.numpy(), s0.numpy())


def test_silu_saturates_at_127():
    gu = randn_bf16((16, 2 * 512), 5, 3.0)
    q, _ = o.silu_mul_quant(bf16_to_bits(gu))
    assert (np.abs(q.astype(int)).max(-1) == 127).all()


def test_quant_per_token_matches_reference_restatement():
    x = randn_bf16((6, 2048), 17, 2.0)
    q, s = o.quant_per_token(bf16_to_bits(x))
    q1, s1 = np_quant(x.float().numpy())
    assert np.array_equal(q, q1) and np.array_equal(s, s1)
    assert_close_int8(q, s, *(t.numpy() for t in ref_quant(x.float())))


def test_quant_rows_div_matches_the_operand_generator():
    from int8_linear.operands import quant_rows
    w = (torch.randn((64, 2048), generator=torch.Generator().manual_seed(2)) * 0.02).to(torch.bfloat16)
    q, s = o.quant_rows_div(bf16_to_bits(w))
    q0, s0 = quant_rows(w)
    assert np.array_equal(q, q0.numpy()) and np.array_equal(s, s0.numpy())
    assert np.abs(q.astype(int)).max() == 127


# ------------------------------------------------------------------ golden fixtures
def test_oracle_reproduces_golden_gemm_fixtures():
    for name in ("gemm_small", "gemm_config0"):
        f = np.load(GOLDEN / f"{name}.npz")
        acc = o.gemm_i32(f["a"], f["w"])
        assert np.array_equal(acc, f["raw"])
        assert np.array_equal(acc, (f["a"].astype(np.float64) @ f["w"].astype(np.float64).T).astype(np.int32))
        assert np.array_equal(o.epilogue(acc, f["sa"], f["sb"], None, o.NONE, o.BF16), f["out_bf16"])
    f = np.load(GOLDEN / "gemm_small.npz")
    acc = f["raw"]
    assert np.array_equal(o.epilogue(acc, f["sa"], f["sb"], f["bias_bf16"], o.BF16, o.BF16),
                          f["out_bf16_bias_bf16"])
    assert np.array_equal(o.epilogue(acc, f["sa"], f["sb"], f["bias_f32"], o.F32, o.F16),
                          f["out_f16_bias_f32"])


def test_oracle_reproduces_golden_quantizer_fixtures():
    f = np.load(GOLDEN / "quantizers.npz")
    q, s, rout = o.add_rmsnorm_quant(f["x"], f["r"], f["gamma"], EPS)
    assert np.array_equal(q, f["q_res"]) and np.array_equal(s, f["s_res"])
    assert np.array_equal(rout, f["rout"])
    q, s, _ = o.add_rmsnorm_quant(f["x"], None, f["gamma"], EPS)
    assert np.array_equal(q, f["q_nores"]) and np.array_equal(s, f["s_nores"])
    for key, rs in (("silu", False), ("silu_round", True)):
        q, s = o.silu_mul_quant(f["gu"], round_silu=rs)
        assert np.array_equal(q, f[f"q_{key}"]) and np.array_equal(s, f[f"s_{key}"])
    q, s = o.quant_per_token(f["xp"])
    assert np.array_equal(q, f["q_plain"]) and np.array_equal(s, f["s_plain"])
    assert f["q_plain"][2, :8].tolist() == [127, 0, 2, 2, 0, -2, -2, 126]
    assert f["s_plain"][1, 0] == 0 and not f["q_plain"][1].any()


# ------------------------------------------------------------------ BASELINE config 2 against
# the reference's restatement (tests/test_fused_quant.py:26-51), at full size.  The oracle and
# the GPU kernels agree bit for bit (tests/test_quant_gpu.py), so these counts are the GPU's.
CONFIG2_M = [1, 16, 128, 1024, 4096]


def _config2_norm_inputs(m):
    return randn_bf16((m, 2048), 10 + m), randn_bf16((m, 2048), 20 + m), \
        randn_bf16((2048,), 98, 0.1) + 1.0


def test_restatement_divides_by_a_reciprocal_product():
    """torch evaluates `127.0 / t` as reciprocal(t) * 127: bit for bit equal to that product,
    and not always the IEEE quotient.  This is why the restatement as written and the
    reference kernel's IEEE division (fused_quant.py:45-47) can part by one code."""
    rng = np.random.default_rng(5)
    t = torch.from_numpy((np.abs(rng.standard_normal(1 << 16)) * 4 + 1e-3).astype(np.float32))
    as_written = (127.0 / t).numpy()
    assert np.array_equal(as_written, (t.reciprocal() * 127.0).numpy())
    ieee = np.float32(127.0) / t.numpy()
    assert np.array_equal((torch.full_like(t, 127.0) / t).numpy(), ieee)
    assert 0 < np.count_nonzero(as_written != ieee) < t.numel() // 2


@pytest.mark.parametrize("m", CONFIG2_M)
def test_config2_restatement_made_canonical_is_the_oracle(m):
    """With IEEE division, float64 variance and a correctly rounded rsqrt substituted, the
    reference's restatement gives the oracle's codes and scales exactly, for both fused
    quantizers, with and without the residual, SiLU rounded or not."""
    import restated as rs
    x, r, w = _config2_norm_inputs(m)
    for res in (r, None):
        q, s, _ = o.add_rmsnorm_quant(bf16_to_bits(x), None if res is None else bf16_to_bits(res),
                                      bf16_to_bits(w), EPS)
        q0, s0, _ = rs.norm(x, res, w, "ieee", canonical_var=True, canonical_rsqrt=True)
        assert rs.differences(q, s, q0, s0) == (0, 0, 0)
    gu = randn_bf16((m, 12288), 30 + m)
    for round_silu in (True, False):
        q, s = o.silu_mul_quant(bf16_to_bits(gu), round_silu=round_silu)
        q0, s0 = rs.silu(gu, round_silu, "ieee")
        assert rs.differences(q, s, q0, s0) == (0, 0, 0)


@pytest.mark.parametrize("m", CONFIG2_M)
def test_config2_restatement_with_ieee_division(m):
    """The restatement with the IEEE division it describes (torch's float32 variance, rsqrt and
    exp kept): scales identical, SiLU codes identical, add+RMSNorm codes off by one in at most
    4 of M x 2048 (measured: 0-3, from the float32 variance and rsqrt roundings)."""
    import restated as rs
    x, r, w = _config2_norm_inputs(m)
    for res in (r, None):
        q, s, _ = o.add_rmsnorm_quant(bf16_to_bits(x), None if res is None else bf16_to_bits(res),
                                      bf16_to_bits(w), EPS)
        n, dmax, sdiff = rs.differences(q, s, *rs.norm(x, res, w, "ieee")[:2])
        assert sdiff == 0 and dmax <= 1 and n <= 4, (m, res is not None, n)
    gu = randn_bf16((m, 12288), 30 + m)
    for round_silu in (True, False):
        q, s = o.silu_mul_quant(bf16_to_bits(gu), round_silu=round_silu)
        assert rs.differences(q, s, *rs.silu(gu, round_silu, "ieee")) == (0, 0, 0)


# codes that differ from the restatement as written, per M: norm with/without residual, SiLU
# rounded/not (measured with this oracle, which the GPU matches bit for bit)
AS_WRITTEN = {1: (0, 0, 0, 0), 16: (5, 10, 2, 4), 128: (36, 31, 16, 14),
              1024: (278, 304, 92, 97), 4096: (1131, 1162, 377, 348)}


@pytest.mark.parametrize("m", CONFIG2_M)
def test_config2_restatement_as_written(m):
    """Against the restatement exactly as the reference wrote it: scales identical, codes off
    by at most one in at most 0.015% of elements (16 allowed in small tensors), every such code
    explained by the reciprocal-product division (the oracle's precise_div=False mode, which
    multiplies by the IEEE reciprocal, gives the restatement's SiLU codes exactly)."""
    import restated as rs
    x, r, w = _config2_norm_inputs(m)
    counts = []
    for res in (r, None):
        xb, rb = bf16_to_bits(x), None if res is None else bf16_to_bits(res)
        q, s, _ = o.add_rmsnorm_quant(xb, rb, bf16_to_bits(w), EPS)
        q0, s0, _ = rs.norm(x, res, w)
        n, dmax, sdiff = rs.differences(q, s, q0, s0)
        assert sdiff == 0 and dmax <= 1 and n <= max(16, 1.5e-4 * q.size)
        counts.append(n)
    gu = randn_bf16((m, 12288), 30 + m)
    for round_silu in (True, False):
        q, s = o.silu_mul_quant(bf16_to_bits(gu), round_silu=round_silu)
        q0, s0 = rs.silu(gu, round_silu)
        n, dmax, sdiff = rs.differences(q, s, q0, s0)
        assert sdiff == 0 and dmax <= 1 and n <= max(16, 1.5e-4 * q.size)
        counts.append(n)
        # (its scales are absmax * (1/127), so only the codes are compared)
        qr, _ = o.silu_mul_quant(bf16_to_bits(gu), round_silu=round_silu, precise_div=False)
        assert np.array_equal(qr, q0.numpy())
    # the recorded counts, with slack for another CPU's torch kernels
    for got, want in zip(counts, AS_WRITTEN[m]):
        assert abs(got - want) <= max(4, want // 20), (m, counts)
