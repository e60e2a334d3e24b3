"""Every tensor a launch reads must be on the launching device, checked on the host before
anything is launched.

A host scale or bias handed to the kernel would be read through a host address on the GPU.
The reference's Triton launcher refuses such a call with a ValueError; here the Python
wrappers do the same.  The C++ binding declines such calls (it compares every device), so
they reach the Python checks.  The library's launch entry points are replaced by a stub that
fails the test if it is reached, so no kernel ever runs on a host pointer in these tests.
"""

from __future__ import annotations

import pytest
import torch

from helpers import ints, randn, say
from int8_linear import _lib
from int8_linear import fused_quant as fq
from int8_linear.kernel import w8a8_mm

pytestmark = pytest.mark.gpu

LAUNCHES = ("i8l_w8a8_mm", "i8l_add_rmsnorm_quant", "i8l_silu_mul_quant",
            "i8l_quant_per_token", "i8l_w8a8_mm_dynq")


class _NoLaunch:
    """The real library, except that its launch entry points fail the test."""

    def __init__(self, real):
        self._real = real

    def __getattr__(self, name):
        if name in LAUNCHES:
            def refuse(*args):
                raise AssertionError(f"{name} was reached with an argument off the device")
            return refuse
        return getattr(self._real, name)


@pytest.fixture
def no_launch(monkeypatch):
    stub = _NoLaunch(_lib.lib())
    monkeypatch.setattr(_lib, "lib", lambda: stub)
    return stub


def _gemm_operands(m=16, k=2048, n=1024):
    a, w = ints((m, k), 1), ints((n, k), 2)
    sa = torch.rand((m, 1), device="cuda") * 1e-2 + 1e-3
    sb = torch.rand((n, 1), device="cuda") * 1e-2 + 1e-3
    bias = (torch.randn(n, device="cuda") * 0.01).to(torch.bfloat16)
    return a, w.t(), sa, sb, bias


@pytest.mark.parametrize("which", ["scale_a", "scale_b", "bias"])
def test_w8a8_mm_refuses_a_host_tensor(no_launch, which):
    say(f"device check w8a8_mm host {which}")
    a, b, sa, sb, bias = _gemm_operands()
    args = {"scale_a": sa, "scale_b": sb, "bias": bias}
    args[which] = args[which].cpu()
    with pytest.raises(ValueError, match=which):
        w8a8_mm(a, b, args["scale_a"], args["scale_b"], torch.bfloat16, args["bias"])


def test_w8a8_mm_refuses_a_host_weight(no_launch):
    a, b, sa, sb, _ = _gemm_operands()
    from int8_linear import NotSupported
    with pytest.raises((ValueError, NotSupported)):
        w8a8_mm(a, b.cpu(), sa, sb, torch.bfloat16)


@pytest.mark.parametrize("which", ["residual", "weight"])
def test_add_rmsnorm_quant_refuses_a_host_tensor(no_launch, which):
    say(f"device check add_rmsnorm_quant host {which}")
    x, r = randn((4, 2048), 3), randn((4, 2048), 4)
    w = randn((2048,), 5, 0.1) + 1.0
    args = {"residual": r, "weight": w}
    args[which] = args[which].cpu()
    from int8_linear import NotSupported
    with pytest.raises((ValueError, NotSupported)):
        fq.add_rmsnorm_quant(x, args["residual"], args["weight"], 1e-6)


@pytest.mark.parametrize("which", ["b_q", "scale_b", "bias"])
def test_quant_mm_refuses_a_host_tensor(no_launch, which):
    say(f"device check quant_mm host {which}")
    x = randn((4, 2048), 6)
    _, b, _, sb, bias = _gemm_operands(4, 2048, 2048)
    args = {"b_q": b, "scale_b": sb, "bias": bias}
    args[which] = args[which].cpu()
    from int8_linear import NotSupported
    with pytest.raises((ValueError, NotSupported)):
        fq.quant_mm(x, args["b_q"], args["scale_b"], torch.bfloat16, args["bias"])


def test_the_same_calls_launch_with_every_tensor_on_the_device():
    """The checks pass the ordinary call: all on one device, results as before."""
    a, b, sa, sb, bias = _gemm_operands()
    out = w8a8_mm(a, b, sa, sb, torch.bfloat16, bias)
    assert out.device == a.device and out.shape == (16, 1024)
    x, r = randn((4, 2048), 3), randn((4, 2048), 4)
    w = randn((2048,), 5, 0.1) + 1.0
    q, s, rout = fq.add_rmsnorm_quant(x, r, w, 1e-6)
    assert q.device == x.device and rout.device == x.device
