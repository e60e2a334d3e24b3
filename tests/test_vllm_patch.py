"""The vLLM-facing boundary: scaled_mm / the custom op / the fallback, and the PreQuant
routing of the fused quantizers.  Mirrors the reference's tests/test_vllm_patch.py and
tests/test_fused_quant.py:108-139 (AshrithaG/int8-linear).  vLLM itself is never imported:
plain classes and monkeypatches stand in for it, as in the reference."""

from __future__ import annotations

import pytest
import torch

from helpers import ints, say
from int8_linear import vllm_fuse_patch as vfp
from int8_linear import vllm_patch
from int8_linear.kernel import w8a8_mm


def operands(m, k, n, seed, low=-127, high=128):
    g = torch.Generator().manual_seed(seed)
    a = torch.randint(low, high, (m, k), dtype=torch.int8, generator=g)
    w = torch.randint(low, high, (n, k), dtype=torch.int8, generator=g)
    sa = torch.rand((m, 1), generator=g) * 1e-2 + 1e-3
    sb = torch.rand((n, 1), generator=g) * 1e-2 + 1e-3
    return a.cuda(), w.t().cuda(), sa.cuda(), sb.cuda()


# ------------------------------------------------------------------ GPU
@pytest.mark.gpu
def test_op_matches_kernel():
    say("scaled_mm vs w8a8_mm m=64")
    a, w, sa, sb = operands(64, 2048, 4096, 1)
    got = vllm_patch.scaled_mm(a, w, scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16)
    assert torch.equal(got, w8a8_mm(a, w, sa, sb, torch.bfloat16))
    via_op = vllm_patch.w8a8_mm_op(a, w, sa, sb, torch.bfloat16, None)
    assert torch.equal(via_op, got)


@pytest.mark.gpu
def test_compiled_op_configures_from_runtime_batch():
    # If the configuration were chosen at trace time, both batch sizes would share it.
    say("torch.compile scaled_mm m=3 and m=700")

    def layer(a, w, sa, sb):
        return vllm_patch.scaled_mm(a, w, scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16)

    compiled = torch.compile(layer, fullgraph=True, dynamic=True)
    vllm_patch.CONFIGS.clear()
    for m in (3, 700):
        ops = operands(m, 2048, 2048, m)
        assert torch.equal(compiled(*ops), w8a8_mm(*ops, torch.bfloat16))
    chosen = {m: name for (m, _, _), name in vllm_patch.CONFIGS.items()}
    assert chosen[3] != chosen[700], chosen


@pytest.mark.gpu
def test_eager_calls_skip_the_custom_op(monkeypatch):
    def custom_op(*args):
        raise AssertionError("an eager call went through the custom op")

    monkeypatch.setattr(vllm_patch, "w8a8_mm_op", custom_op)
    a, w, sa, sb = operands(16, 2048, 2048, 4)
    got = vllm_patch.scaled_mm(a, w, scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16)
    assert torch.equal(got, w8a8_mm(a, w, sa, sb, torch.bfloat16))


@pytest.mark.gpu
def test_declined_shapes_go_to_the_replaced_kernel(monkeypatch):
    seen = []

    def replaced(a, w, sa, sb, out_dtype, bias):
        seen.append(tuple(a.shape))
        return torch.zeros((a.shape[0], w.shape[1]), dtype=out_dtype, device=a.device)

    monkeypatch.setattr(vllm_patch, "_vllm_triton_scaled_mm", replaced)
    before = vllm_patch.FALLBACKS
    a, w, sa, sb = operands(4, 100, 64, 2)  # K=100 divides no tile
    out = vllm_patch.scaled_mm(a, w, scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16)
    assert seen == [(4, 100)] and vllm_patch.FALLBACKS == before + 1
    assert tuple(out.shape) == (4, 64)


@pytest.mark.gpu
def test_declined_shapes_raise_without_a_replaced_kernel(monkeypatch):
    from int8_linear import NotSupported
    monkeypatch.setattr(vllm_patch, "_vllm_triton_scaled_mm", None)
    a, w, sa, sb = operands(4, 100, 64, 2)
    with pytest.raises(NotSupported):
        vllm_patch.scaled_mm(a, w, scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16)


@pytest.mark.gpu
def test_prequant_feeds_the_kernel_end_to_end():
    """add_rmsnorm_quant -> PreQuant -> wrapped apply_weights -> scaled_mm, as the patched
    Qwen3 layer runs it, equals quantizing separately and calling the kernel."""
    from int8_linear import fused_quant as fq
    say("prequant end to end")

    class Kernel:
        def __init__(self, w_q, w_s):
            self.w_q, self.w_s = w_q, w_s

        def _get_layer_params(self, layer):
            return self.w_q, self.w_s, None, None, None

        def apply_weights(self, layer, x, bias=None):
            raise AssertionError("a PreQuant must not reach the original apply_weights")

    vfp._wrap_apply(Kernel, lambda a, w, sa, sb, dt, b: vllm_patch.scaled_mm(
        a, w, scale_a=sa, scale_b=sb, out_dtype=dt, bias=b))
    g = torch.Generator().manual_seed(3)
    x = torch.randn((8, 2048), generator=g).to(torch.bfloat16).cuda()
    r = torch.randn((8, 2048), generator=g).to(torch.bfloat16).cuda()
    gamma = torch.ones(2048, dtype=torch.bfloat16, device="cuda")
    w_q = ints((4096, 2048), 5).t()
    w_s = torch.rand((4096, 1), device="cuda") * 1e-3 + 1e-4
    q, s, res = fq.add_rmsnorm_quant_op(x, r, gamma, 1e-6)
    got = Kernel(w_q, w_s).apply_weights(None, vfp.PreQuant(q, s, torch.bfloat16))
    assert torch.equal(got, w8a8_mm(q, w_q, s, w_s, torch.bfloat16))


# ------------------------------------------------------------------ CPU (routing only)
def test_prequant_routing():
    """A PreQuant goes straight to the matmul; a plain tensor takes the original path."""
    calls = []

    class Kernel:
        def _get_layer_params(self, layer):
            return "w_q", "w_s", None, None, None

        def apply_weights(self, layer, x, bias=None):
            calls.append("original")
            return "orig"

    vfp._wrap_apply(Kernel, lambda a, w, sa, sb, dt, b: calls.append((a, w, sa, sb, dt, b)) or "fast")
    before = vfp.PREQUANT_CALLS
    k = Kernel()
    assert k.apply_weights(None, vfp.PreQuant("q", "s", torch.bfloat16), "b") == "fast"
    assert calls[-1] == ("q", "w_q", "s", "w_s", torch.bfloat16, "b")
    assert vfp.PREQUANT_CALLS == before + 1
    assert k.apply_weights(None, torch.zeros(1)) == "orig"


def test_prequant_rejects_static_or_asymmetric():
    class Kernel:
        def _get_layer_params(self, layer):
            return "w_q", "w_s", "static_scale", None, None

        def apply_weights(self, layer, x, bias=None):
            return "orig"

    vfp._wrap_apply(Kernel, lambda *a: "fast")
    with pytest.raises(NotImplementedError):
        Kernel().apply_weights(None, vfp.PreQuant("q", "s", torch.bfloat16))


def test_use_measured_numerics(tmp_path):
    import json
    from int8_linear import fused_quant as fq
    saved = fq.PRECISE_DIV, fq.ROUND_SILU
    try:
        p = tmp_path / "n.json"
        p.write_text(json.dumps({"best_precise_div": False, "best_round_silu": True}))
        vfp.use_measured_numerics(p)
        assert (fq.PRECISE_DIV, fq.ROUND_SILU) == (False, True)
        vfp.use_measured_numerics()   # the shipped record: IEEE division, rounded SiLU
        assert (fq.PRECISE_DIV, fq.ROUND_SILU) == (True, True)
    finally:
        fq.PRECISE_DIV, fq.ROUND_SILU = saved


def test_run_counts_calls_and_configs(monkeypatch):
    from int8_linear.kernel import Config
    monkeypatch.setattr(vllm_patch, "choose_config", lambda m, n, k: Config(16, 16, 64, 1, 1, 1))
    monkeypatch.setattr(vllm_patch, "w8a8_mm", lambda *a, **kw: "out")
    vllm_patch.CONFIGS.clear()
    before = vllm_patch.CALLS
    a = torch.zeros((3, 64), dtype=torch.int8)
    b = torch.zeros((64, 32), dtype=torch.int8)
    assert vllm_patch.scaled_mm(a, b, torch.ones(1), torch.ones(1), torch.bfloat16) == "out"
    assert vllm_patch.CALLS == before + 1
    assert vllm_patch.CONFIGS == {(3, 64, 32): "16x16x64 w1 s1 g1"}


def test_patch_vllm_rebinds_the_module_name(monkeypatch):
    import sys
    import types
    names = ["vllm", "vllm.model_executor", "vllm.model_executor.kernels",
             "vllm.model_executor.kernels.linear", "vllm.model_executor.kernels.linear.scaled_mm",
             "vllm.model_executor.kernels.linear.scaled_mm.triton"]
    mods = {n: types.ModuleType(n) for n in names}
    original = object()
    mods[names[-1]].triton_scaled_mm = original
    for n in names:
        monkeypatch.setitem(sys.modules, n, mods[n])
    for parent, child in zip(names, names[1:]):
        setattr(mods[parent], child.rsplit(".", 1)[1], mods[child])
    monkeypatch.setattr(vllm_patch, "tuned_config", lambda *a: None)
    monkeypatch.setattr(vllm_patch, "_vllm_triton_scaled_mm", None)
    vllm_patch.patch_vllm()
    assert mods[names[-1]].triton_scaled_mm is vllm_patch.scaled_mm
    assert vllm_patch._vllm_triton_scaled_mm is original
    vllm_patch.patch_vllm()            # idempotent: the saved original is kept
    assert vllm_patch._vllm_triton_scaled_mm is original
