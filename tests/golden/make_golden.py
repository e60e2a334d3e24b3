"""Write the golden fixtures of tests/golden/*.npz from the CPU oracle.

    python tests/golden/make_golden.py

The reference (AshrithaG/int8-linear) holds no tensor fixtures, so these are produced by
this repository's oracle (oracle/i8l_oracle.c) on seeded inputs and committed.  Before
they are trusted, tests/test_oracle.py pins the oracle itself against independent
mathematics; tests/test_oracle.py then checks that the oracle still reproduces every
fixture, and the GPU tests check the HIP kernels against them bit for bit.

Inputs come from numpy's PCG64 (np.random.default_rng) and from the package's own seeded
operand generator (int8_linear.operands, a CPU torch.Generator), both stable across
machines; the inputs are stored in the fixtures as well, so nothing is regenerated when
the fixtures are read.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path[:0] = [str(ROOT), str(ROOT / "int8-linear_amd")]

from oracle import oracle as o  # noqa: E402

EPS = 1e-6


def bf16_bits(x: np.ndarray) -> np.ndarray:
    return o.f32_to_bf16(np.asarray(x, np.float32))


def gemm_small() -> dict:
    """Ragged M, both scale kinds, bias dtypes and output dtypes at a small shape."""
    rng = np.random.default_rng(1234)
    M, K, N = 17, 512, 64
    a = rng.integers(-127, 128, (M, K), dtype=np.int8)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    sa = (rng.random((M, 1), dtype=np.float32) * 1e-2 + 1e-3).astype(np.float32)
    sb = (rng.random((N, 1), dtype=np.float32) * 1e-2 + 1e-3).astype(np.float32)
    bias_f32 = (rng.standard_normal(N) * 0.5).astype(np.float32)
    bias_bf16 = bf16_bits(bias_f32)
    acc = o.gemm_i32(a, w)
    return {
        "a": a, "w": w, "sa": sa, "sb": sb, "bias_bf16": bias_bf16, "bias_f32": bias_f32,
        "raw": acc,
        "out_bf16": o.epilogue(acc, sa, sb, None, o.NONE, o.BF16),
        "out_bf16_bias_bf16": o.epilogue(acc, sa, sb, bias_bf16, o.BF16, o.BF16),
        "out_f16_bias_f32": o.epilogue(acc, sa, sb, bias_f32, o.F32, o.F16),
        "out_f32_scalar": o.epilogue(acc, sa[:1, :1], sb[:1, :1], None, o.NONE, o.F32),
    }


def gemm_config0() -> dict:
    """BASELINE config 0 (Qwen3-1.7B qkv, M=16, K=2048) restricted to the first 128 output
    channels, from the benchmark's own operand generator (seed as the sweep derives it)."""
    import torch

    from int8_linear.operands import operands, seed_of
    M, K, N = 16, 2048, 4096
    d = operands(M, K, N, seed_of(M, K, N), with_bias=True)
    a = d["a_q"].numpy()
    w = d["w_q"][:128].numpy()
    sa = d["a_s"].numpy()
    sb = d["w_s"][:128].numpy()
    bias = d["bias"][:128].view(torch.int16).numpy().view(np.uint16)
    acc = o.gemm_i32(a, w)
    return {"a": a, "w": w, "sa": sa, "sb": sb, "bias_bf16": bias, "raw": acc,
            "out_bf16": o.epilogue(acc, sa, sb, None, o.NONE, o.BF16),
            "out_bf16_bias": o.epilogue(acc, sa, sb, bias, o.BF16, o.BF16)}


def quantizers() -> dict:
    rng = np.random.default_rng(99)
    H, I = 2048, 6144
    x = bf16_bits(rng.standard_normal((7, H)))
    r = bf16_bits(rng.standard_normal((7, H)))
    gamma = bf16_bits(1.0 + 0.1 * rng.standard_normal(H))
    q1, s1, rout = o.add_rmsnorm_quant(x, r, gamma, EPS)
    q0, s0, _ = o.add_rmsnorm_quant(x, None, gamma, EPS)
    gu = bf16_bits(2.0 * rng.standard_normal((5, 2 * I)))
    qs0, ss0 = o.silu_mul_quant(gu, round_silu=False)
    qs1, ss1 = o.silu_mul_quant(gu, round_silu=True)
    # plain quantizer rows: normal data, a zero row, and a row whose max is exactly 127
    # with half-way values (y*inv = k + 0.5 exactly) that round half to even
    xp = rng.standard_normal((4, H)).astype(np.float32)
    xp[1] = 0.0
    xp[2] = 0.0
    xp[2, :8] = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5]
    xp_bits = bf16_bits(xp)
    qp, sp = o.quant_per_token(xp_bits)
    return {"x": x, "r": r, "gamma": gamma, "q_res": q1, "s_res": s1, "rout": rout,
            "q_nores": q0, "s_nores": s0, "gu": gu, "q_silu": qs0, "s_silu": ss0,
            "q_silu_round": qs1, "s_silu_round": ss1, "xp": xp_bits, "q_plain": qp,
            "s_plain": sp}


def main() -> None:
    for name, fn in (("gemm_small", gemm_small), ("gemm_config0", gemm_config0),
                     ("quantizers", quantizers)):
        np.savez_compressed(HERE / f"{name}.npz", **fn())
        print("wrote", HERE / f"{name}.npz")


if __name__ == "__main__":
    main()
