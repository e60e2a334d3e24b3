"""The vLLM-facing boundary: scaled_mm / the custom op / the fallback, and the PreQuant
routing of the fused quantizers.  Mirrors the reference's tests/test_vllm_patch.py and
tests/test_fused_quant.py:108-139 (AshrithaG/int8-linear).  vLLM itself is never imported:
plain classes and monkeypatches stand in for it, as in the reference."""

from __future__ import annotations

import numpy as np
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


class _Int8Kernel:
    """Stands in for one of vLLM's int8 linear kernels: its own apply_weights quantizes the
    bf16 input per token and calls the matmul, as vLLM's does (scaled_int8_quant then
    triton_scaled_mm); _get_layer_params hands out the layer's int8 weight and scales."""

    def _get_layer_params(self, layer):
        return layer.w_qt, layer.w_s, None, None, None

    def apply_weights(self, layer, x, bias=None):
        from int8_linear import fused_quant as fq
        q, s = fq.quant_per_token(x)
        return vllm_patch.scaled_mm(q, layer.w_qt, scale_a=s, scale_b=layer.w_s,
                                    out_dtype=x.dtype, bias=bias)


class _Linear:
    """vLLM's linear module surface: forward returns (output, output_bias)."""

    kernel = _Int8Kernel()

    def __init__(self, w_q, w_s):
        self.w_q, self.w_qt, self.w_s = w_q, w_q.t(), w_s

    def __call__(self, x):
        return self.kernel.apply_weights(self, x, None), None


class _Norm:
    def __init__(self, weight, eps):
        self.weight, self.variance_epsilon = weight, eps


class _Attention:
    """Attention left out as in the decoder stand-in: the q columns of qkv_proj's output
    feed o_proj, which quantizes its own input (no kernel before it to fuse into)."""

    def __init__(self, qkv, o):
        self.qkv_proj, self.o_proj = qkv, o

    def __call__(self, positions, hidden_states):
        qkv = self.qkv_proj(hidden_states)[0]
        return self.o_proj(qkv[:, :2048])[0]


class _MLP:
    def __init__(self, gate_up, down):
        self.gate_up_proj, self.down_proj = gate_up, down

    def __call__(self, x):
        return vfp._mlp_forward(self, x)


class _DecoderLayer:
    def __init__(self, gen):
        def linear(k, n):
            w = torch.randint(-127, 128, (n, k), generator=gen, dtype=torch.int8)
            s = torch.rand((n, 1), generator=gen) * 1e-3 + 1e-4
            return _Linear(w.cuda(), s.cuda())

        one = torch.ones(2048, dtype=torch.bfloat16, device="cuda")
        self.input_layernorm = _Norm(one, 1e-6)
        self.post_attention_layernorm = _Norm(one, 1e-6)
        self.self_attn = _Attention(linear(2048, 4096), linear(2048, 2048))
        self.mlp = _MLP(linear(2048, 12288), linear(6144, 2048))

    def forward(self, positions, hidden_states, residual):
        return vfp._decoder_forward(self, positions, hidden_states, residual)


def _oracle_layers(layers, x_bits):
    """The routed layers' arithmetic on the CPU oracle: (hidden bits, residual bits)."""
    from int8_linear import fused_quant as fq
    from oracle import oracle as o
    from helpers import bits, np_

    precise = fq.PRECISE_DIV

    def mm(lin, q, s):
        return o.w8a8_mm(q, np_(lin.w_q), s, np_(lin.w_s), out_dt=o.BF16)

    h, res = x_bits, None
    for layer in layers:
        gamma = bits(layer.input_layernorm.weight)
        if res is None:
            q, s, _ = o.add_rmsnorm_quant(h, None, gamma, 1e-6, precise_div=precise)
            res = h
        else:
            q, s, res = o.add_rmsnorm_quant(h, res, gamma, 1e-6, precise_div=precise)
        qkv = mm(layer.self_attn.qkv_proj, q, s)
        q, s = o.quant_per_token(qkv[:, :2048], precise_div=precise)
        h = mm(layer.self_attn.o_proj, q, s)
        q, s, res = o.add_rmsnorm_quant(h, res, bits(layer.post_attention_layernorm.weight),
                                        1e-6, precise_div=precise)
        gu = mm(layer.mlp.gate_up_proj, q, s)
        q, s = o.silu_mul_quant(gu, round_silu=fq.ROUND_SILU, precise_div=precise)
        h = mm(layer.mlp.down_proj, q, s)
    return h, res


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 8, 32])
@pytest.mark.parametrize("round_silu", [False, True])
def test_routed_decoder_layers_match_the_oracle_chain(m, round_silu, monkeypatch):
    """Two Qwen3 decoder layers run through the routing (the norms and SiLU-and-mul hand
    qkv_proj, gate_up_proj and down_proj a PreQuant; the wrapped apply_weights sends it to
    scaled_mm) equal the oracle's chain of add_rmsnorm_quant, w8a8_mm, quant_per_token and
    silu_mul_quant bit for bit: final hidden state and residual stream."""
    from int8_linear import fused_quant as fq
    from helpers import bits
    say(f"routed decoder layers m={m} round_silu={round_silu}")
    monkeypatch.setattr(fq, "ROUND_SILU", round_silu)
    monkeypatch.setitem(vfp._ROUTES, _Int8Kernel, _Int8Kernel.apply_weights)
    monkeypatch.setattr(_Int8Kernel, "apply_weights", _Int8Kernel.apply_weights)
    vfp._wrap_apply(_Int8Kernel, lambda a, w, sa, sb, dt, b: vllm_patch.scaled_mm(
        a, w, scale_a=sa, scale_b=sb, out_dtype=dt, bias=b))
    gen = torch.Generator().manual_seed(100 + m)
    layers = [_DecoderLayer(gen) for _ in range(2)]
    x = torch.randn((m, 2048), generator=gen).to(torch.bfloat16).cuda()
    before = vfp.PREQUANT_CALLS
    h, res = x, None
    for layer in layers:
        h, res = layer.forward(None, h, res)
    torch.cuda.synchronize()
    assert vfp.PREQUANT_CALLS == before + 3 * len(layers)     # qkv, gate_up, down per layer
    h0, r0 = _oracle_layers(layers, bits(x))
    assert np.array_equal(bits(h), h0)
    assert np.array_equal(bits(res), r0)


@pytest.mark.gpu
def test_prequant_feeds_the_kernel_end_to_end():
    """add_rmsnorm_quant -> PreQuant -> wrapped apply_weights -> scaled_mm equals the
    oracle's add_rmsnorm_quant followed by its w8a8_mm, bit for bit."""
    from int8_linear import fused_quant as fq
    from oracle import oracle as o
    from helpers import bits, np_
    say("prequant end to end vs oracle")

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
    x = torch.randn((8, 2048), generator=g).to(torch.bfloat16)
    r = torch.randn((8, 2048), generator=g).to(torch.bfloat16)
    gamma = (1 + 0.1 * torch.randn(2048, generator=g)).to(torch.bfloat16)
    w = torch.randint(-127, 128, (4096, 2048), generator=g, dtype=torch.int8)
    w_s = torch.rand((4096, 1), generator=g) * 1e-3 + 1e-4
    bias = (torch.randn(4096, generator=g) * 0.01).to(torch.bfloat16)
    q, s, res = fq.add_rmsnorm_quant_op(x.cuda(), r.cuda(), gamma.cuda(), 1e-6)
    got = Kernel(w.cuda().t(), w_s.cuda()).apply_weights(
        None, vfp.PreQuant(q, s, torch.bfloat16), bias.cuda())
    q0, s0, r0 = o.add_rmsnorm_quant(bits(x), bits(r), bits(gamma), 1e-6,
                                     precise_div=fq.PRECISE_DIV)
    want = o.w8a8_mm(q0, np_(w), s0, np_(w_s), bits(bias), o.BF16, o.BF16)
    assert np.array_equal(bits(got), want)
    assert np.array_equal(bits(res), r0)


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


def _fake_vllm(monkeypatch):
    """Minimal vllm modules with the classes patch_vllm routes (no vLLM is installed)."""
    import sys
    import types

    class Kernel:
        def apply_weights(self, layer, x, bias=None):
            return "original"

    class Triton(Kernel):
        pass

    class Cutlass(Kernel):
        def apply_weights(self, layer, x, bias=None):
            return "cutlass original"

    class Decoder:
        def forward(self, *a):
            return "decoder original"

    class MLP:
        def forward(self, *a):
            return "mlp original"

    tree = {"vllm": {}, "vllm._custom_ops": {"cutlass_scaled_mm": lambda *a, **k: "cutlass"},
            "vllm.model_executor": {}, "vllm.model_executor.kernels": {},
            "vllm.model_executor.kernels.linear": {},
            "vllm.model_executor.kernels.linear.scaled_mm": {},
            "vllm.model_executor.kernels.linear.scaled_mm.triton": {
                "TritonInt8ScaledMMLinearKernel": Triton,
                "triton_scaled_mm": lambda *a, **k: "triton"},
            "vllm.model_executor.kernels.linear.scaled_mm.cutlass": {
                "CutlassInt8ScaledMMLinearKernel": Cutlass},
            "vllm.model_executor.models": {},
            "vllm.model_executor.models.qwen3": {"Qwen3DecoderLayer": Decoder},
            "vllm.model_executor.models.qwen2": {"Qwen2MLP": MLP}}
    mods = {}
    for name, attrs in tree.items():
        mod = types.ModuleType(name)
        for k, v in attrs.items():
            setattr(mod, k, v)
        mods[name] = mod
        monkeypatch.setitem(sys.modules, name, mod)
    for name, mod in mods.items():
        if "." in name:
            parent, child = name.rsplit(".", 1)
            setattr(mods[parent], child, mod)
    return Triton, Cutlass, Decoder, MLP


def test_fuse_patch_is_idempotent_and_undone(monkeypatch):
    from int8_linear import fused_quant as fq
    triton_k, cutlass_k, decoder, mlp = _fake_vllm(monkeypatch)
    monkeypatch.setattr(fq, "PRECISE_DIV", fq.PRECISE_DIV)
    monkeypatch.setattr(fq, "ROUND_SILU", fq.ROUND_SILU)
    originals = (triton_k.apply_weights, cutlass_k.apply_weights, decoder.forward, mlp.forward)
    vfp.patch_vllm()
    routed = triton_k.apply_weights
    vfp.patch_vllm()                                   # twice: the router does not nest
    assert triton_k.apply_weights.__wrapped__ is originals[0]
    assert cutlass_k.apply_weights.__wrapped__ is originals[1]
    assert routed.__wrapped__ is triton_k.apply_weights.__wrapped__
    assert decoder.forward is vfp._decoder_forward and mlp.forward is vfp._mlp_forward
    assert triton_k().apply_weights(None, torch.zeros(1)) == "original"
    assert cutlass_k().apply_weights(None, torch.zeros(1)) == "cutlass original"
    vfp.unpatch_vllm()
    assert (triton_k.apply_weights, cutlass_k.apply_weights, decoder.forward,
            mlp.forward) == originals


def test_prequant_reaches_the_swapped_triton_matmul(monkeypatch):
    """The Triton route looks triton_scaled_mm up at call time, so a PreQuant reaches
    whatever the module holds then (vllm_patch's scaled_mm once that patch is applied)."""
    import sys
    from int8_linear import fused_quant as fq
    triton_k, *_ = _fake_vllm(monkeypatch)
    monkeypatch.setattr(fq, "PRECISE_DIV", fq.PRECISE_DIV)
    monkeypatch.setattr(fq, "ROUND_SILU", fq.ROUND_SILU)
    vfp.patch_vllm()
    try:
        mod = sys.modules["vllm.model_executor.kernels.linear.scaled_mm.triton"]
        seen = []
        mod.triton_scaled_mm = lambda a, w, **kw: seen.append((a, w, kw)) or "swapped"
        k = triton_k()
        k._get_layer_params = lambda layer: ("w_q", "w_s", None, None, None)
        assert k.apply_weights(None, vfp.PreQuant("q", "s", torch.bfloat16), "b") == "swapped"
        assert seen == [("q", "w_q", {"scale_a": "s", "scale_b": "w_s",
                                      "out_dtype": torch.bfloat16, "bias": "b"})]
    finally:
        vfp.unpatch_vllm()
