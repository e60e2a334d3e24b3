"""The C++ eager binding (csrc/i8l_torch.cpp) on the GPU: every call it takes launches the
same kernel as the ctypes path and gives the same bits; every call it declines comes back
to the Python path, with the reference's errors; it honours the caller's stream and graph
capture.  The launch counter shows which path ran."""

from __future__ import annotations

import pytest
import torch

from helpers import ints, say
from int8_linear import _lib, kernel
from int8_linear import fused_quant as fq
from int8_linear import vllm_patch
from int8_linear.kernel import NotSupported, choose_config, w8a8_mm

pytestmark = pytest.mark.gpu


@pytest.fixture
def ctypes_only(monkeypatch):
    """Set the binding aside: the wrappers then launch through ctypes."""
    def off():
        monkeypatch.setattr(_lib, "_fast_mod", None)
    return off


def fast():
    f = _lib.fast()
    assert f is not None, "the binding is built with the library"
    return f


@pytest.mark.parametrize("m,k,n", [(1, 2048, 4096), (16, 2048, 2048), (37, 2048, 12288),
                                   (96, 6144, 2048), (300, 2048, 2048), (1024, 4096, 4096),
                                   (96, 14336, 4096)])   # the last: a split of K (workspace)
@pytest.mark.parametrize("bias_dtype", [None, torch.bfloat16, torch.float32])
def test_mm_binding_equals_ctypes_path(m, k, n, bias_dtype, ctypes_only):
    say(f"binding mm m={m} k={k} n={n} bias={bias_dtype}")
    a, w = ints((m, k), m), ints((n, k), n)
    g = torch.Generator().manual_seed(m + n)
    sa = (torch.rand((m, 1), generator=g) * 1e-2 + 1e-3).cuda()
    sb = (torch.rand((n, 1), generator=g) * 1e-2 + 1e-3).cuda()
    bias = torch.randn(n, generator=g).to(bias_dtype).cuda() if bias_dtype else None
    before = fast().launches()
    got = w8a8_mm(a, w.t(), sa, sb, torch.bfloat16, bias)
    assert fast().launches() == before + 1
    cfg = choose_config(m, n, k)
    assert fast().config_for(a.get_device(), m, n, k) == (cfg.bm, cfg.bn, cfg.bk, cfg.warps,
                                                          cfg.stages, cfg.group_m)
    if (m, k, n) == (96, 14336, 4096):
        assert cfg.stages == 5, cfg.name      # the shipped table splits K here
    ctypes_only()
    ref = w8a8_mm(a, w.t(), sa, sb, torch.bfloat16, bias)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_mm_binding_declines_to_the_python_path():
    a, w = ints((8, 2048), 1), ints((2048, 2048), 2)
    sa2 = torch.rand((8, 2), device="cuda") + 0.5
    sb = torch.rand((2048,), device="cuda") + 0.5
    before = fast().launches()
    # a strided scale view: the Python path copies it, with the same result
    got = w8a8_mm(a, w.t(), sa2[:, :1], sb, torch.bfloat16)
    ref = w8a8_mm(a, w.t(), sa2[:, :1].contiguous(), sb, torch.bfloat16)
    assert fast().launches() == before + 1          # only the contiguous call was taken
    assert torch.equal(got, ref)
    with pytest.raises(NotSupported):                # dtype errors keep their exception
        w8a8_mm(a, w.t(), sa2[:, 0].double(), sb)
    with pytest.raises(ValueError):
        w8a8_mm(a, w.t(), torch.ones(3, device="cuda"), sb)
    with pytest.raises(NotSupported):
        w8a8_mm(a, w.t(), sa2[:, 0].contiguous(), sb, torch.int8)
    with pytest.raises(ValueError):
        w8a8_mm(a, w.t(), sa2[:, 0].contiguous(), sb, torch.bfloat16, torch.ones(7, device="cuda"))


def test_binding_launches_on_the_current_stream_and_under_capture():
    a, w = ints((16, 2048), 3), ints((4096, 2048), 4)
    sa = torch.rand((16, 1), device="cuda") + 0.5
    sb = torch.rand((4096, 1), device="cuda") + 0.5
    ref = w8a8_mm(a, w.t(), sa, sb)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        out = w8a8_mm(a, w.t(), sa, sb)
    side.synchronize()
    assert torch.equal(out, ref)
    graph = torch.cuda.CUDAGraph()
    before = fast().launches()
    with torch.cuda.graph(graph):
        cap = w8a8_mm(a, w.t(), sa, sb)
    assert fast().launches() == before + 1
    for seed in (5, 6, 7):
        a.copy_(ints((16, 2048), seed))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(cap, w8a8_mm(a, w.t(), sa, sb))


@pytest.mark.parametrize("m", [1, 16, 300])
def test_quantizer_bindings_equal_ctypes_path(m, ctypes_only):
    say(f"binding quantizers m={m}")
    g = torch.Generator().manual_seed(m)
    x = torch.randn((m, 2048), generator=g).to(torch.bfloat16).cuda()
    r = torch.randn((m, 2048), generator=g).to(torch.bfloat16).cuda()
    w = (1 + 0.1 * torch.randn(2048, generator=g)).to(torch.bfloat16).cuda()
    gu = torch.randn((m, 12288), generator=g).to(torch.bfloat16).cuda()
    qkv = torch.randn((m, 4096), generator=g).to(torch.bfloat16).cuda()
    before = fast().launches()
    got = [fq.add_rmsnorm_quant(x, r, w, 1e-6), fq.add_rmsnorm_quant(x, None, w, 1e-6, False),
           fq.silu_mul_quant(gu, True, True), fq.silu_mul_quant(gu, False, False),
           fq.quant_per_token(qkv[:, :2048]), fq.quant_per_token(x, False)]
    assert fast().launches() == before + len(got)
    ctypes_only()
    ref = [fq.add_rmsnorm_quant(x, r, w, 1e-6), fq.add_rmsnorm_quant(x, None, w, 1e-6, False),
           fq.silu_mul_quant(gu, True, True), fq.silu_mul_quant(gu, False, False),
           fq.quant_per_token(qkv[:, :2048]), fq.quant_per_token(x, False)]
    torch.cuda.synchronize()
    for g_, r_ in zip(got, ref):
        assert len(g_) == len(r_)
        for a_, b_ in zip(g_, r_):
            assert (a_ is None and b_ is None) or torch.equal(a_, b_)


def test_vllm_entry_uses_the_binding_and_records_configs():
    a, w = ints((4, 2048), 8), ints((2048, 2048), 9)
    sa = torch.rand((4, 1), device="cuda") + 0.5
    sb = torch.rand((2048, 1), device="cuda") + 0.5
    calls, before = vllm_patch.CALLS, fast().launches()
    out = vllm_patch.scaled_mm(a, w.t(), sa, sb, torch.bfloat16)
    assert vllm_patch.CALLS == calls + 1 and fast().launches() == before + 1
    assert vllm_patch.CONFIGS[(4, 2048, 2048)] == choose_config(4, 2048, 2048).name
    assert torch.equal(out, kernel.w8a8_mm(a, w.t(), sa, sb, config=choose_config(4, 2048, 2048)))
