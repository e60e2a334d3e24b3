"""The 28-layer Qwen3-1.7B decoder stand-in, built from this package's kernels.

The reference measures its kernels in a stand-in for the served model's decode step
(AshrithaG/int8-linear, bench/fuse_quant.py:184-240, Stack.fused; also
bench/situ_tune.py:77-104).  The stand-in has 28 decoder layers of the model's four int8
linears, each layer with its own weights, with the fused quantizers and residual adds
between them. Attention is left out: the q columns of the qkv projection go straight to
o_proj. Per layer:

    add_rmsnorm_quant -> qkv_proj -> quant_per_token(q columns) -> o_proj
    -> add_rmsnorm_quant -> gate_up_proj -> silu_mul_quant -> down_proj

The first layer normalizes without a residual, as `rmsnorm_quant` does.

The reference slices the q columns with .contiguous() and then quantizes them
(bench/fuse_quant.py:233-234). Here the per-token quantizer reads the slice in place, so
each layer issues 8 kernels instead of 9, and the values are the same.  Up to
fused_quant.QUANT_MM_MAX_M tokens, the quantizer and o_proj are one kernel
(fused_quant.quant_mm), and for the few tokens fused_quant.silu_mul_quant_mm takes,
SiLU-and-mul+quant and down_proj are one kernel too, and up to
fused_quant.NORM_MM_FOLD_M tokens each add+RMSNorm+quant is folded into the projection
after it (fused_quant.add_rmsnorm_quant_mm), and from fused_quant.SILU_EPI_MIN_M to
SILU_EPI_MAX_M tokens gate_up_proj writes silu(gate) * up itself
(fused_quant.w8a8_mm_silu_mul) for down_proj to quantize; each gives the same bits as the
kernels it replaces: 4 kernels a layer at 1-5 tokens, 6 at 6-8.

Operands follow the reference's stand-in (bench/fuse_quant.py:186-198):
  * x ~ N(0, 1) bf16;
  * norm weight all ones;
  * per layer and linear, int8 weights uniform in [-127, 127] and per-channel scales
    rand * 1e-3 + 1e-4, all from one seeded generator.
A layer carries 50.3 MB of weights, so 28 layers (1.41 GB) cannot stay in the 256 MB
Infinity Cache: every step streams them from HBM, as the served model does.
"""

from __future__ import annotations

import torch

from int8_linear import fused_quant as fq
from int8_linear.kernel import w8a8_mm

HIDDEN = 2048
INTER = 6144
Q_COLS = 2048          # q heads x head dim: the slice of qkv that feeds o_proj
LAYERS = 28
EPS = 1e-6
# (K, N) of each linear, as vLLM runs Qwen3-1.7B (merged qkv and gate/up)
SHAPES = {"qkv_proj": (HIDDEN, 4096), "o_proj": (HIDDEN, HIDDEN),
          "gate_up_proj": (HIDDEN, 2 * INTER), "down_proj": (INTER, HIDDEN)}


class DecoderStandIn:
    """`layers` decoder layers' linears and quantizers for a batch of m tokens."""

    def __init__(self, m: int, layers: int = LAYERS, seed: int = 0,
                 device: str | torch.device = "cuda", generator_device: str = "cpu"):
        g = torch.Generator(device=generator_device).manual_seed(seed)
        dev = torch.device(device)
        self.m = m
        # per-linear configurations ({name: Config}); a linear not named takes choose_config
        self.configs: dict = {}
        # the same for the norm-folded linears ({name: Config}, else the library's choice)
        self.norm_configs: dict = {}
        # and for gate_up_proj with the SiLU-and-mul epilogue
        self.silu_configs: dict = {}
        # fold silu_mul_quant into down_proj where the library takes it (fused_down)
        self.use_fused_down = True
        # fold add_rmsnorm_quant into qkv_proj and gate_up_proj where the library takes it
        self.use_fused_norm = True
        # the SiLU-and-mul in gate_up_proj's epilogue (and the quantizer into down_proj)
        self.use_fused_silu = True
        self.x = torch.randn((m, HIDDEN), generator=g, device=generator_device).to(
            torch.bfloat16).to(dev)
        self.norm = torch.ones(HIDDEN, dtype=torch.bfloat16, device=dev)
        self.layers: list[dict[str, tuple[torch.Tensor, torch.Tensor]]] = []
        for _ in range(layers):
            layer = {}
            for name, (k, n) in SHAPES.items():
                w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8,
                                  device=generator_device).to(dev)
                s = (torch.rand((n, 1), generator=g, device=generator_device) * 1e-3
                     + 1e-4).to(dev)
                layer[name] = (w, s)
            self.layers.append(layer)

    def with_batch(self, m: int, seed: int = 0) -> "DecoderStandIn":
        """The same layers (weights shared, not copied) with a new batch of m tokens."""
        other = object.__new__(DecoderStandIn)
        other.__dict__.update(self.__dict__)
        g = torch.Generator().manual_seed(seed)
        other.m = m
        other.x = torch.randn((m, HIDDEN), generator=g).to(torch.bfloat16).to(self.x.device)
        return other

    @property
    def fused_o(self) -> bool:
        """Whether o_proj takes its input unquantized (quantizer folded into the GEMM)."""
        return fq.quant_mm_supported(self.m, HIDDEN, Q_COLS)

    @property
    def fused_down(self) -> bool:
        """Whether down_proj takes gate_up's output directly (SiLU-and-mul and its quantizer
        folded into the GEMM), for few tokens; otherwise silu_mul_quant runs on its own."""
        return self.use_fused_down and fq.silu_mul_quant_mm_supported(self.m, HIDDEN, INTER)

    @property
    def fused_norm(self) -> bool:
        """Whether qkv_proj and gate_up_proj take the hidden state unnormalized (add+RMSNorm+
        quant folded into the GEMM), for few tokens; otherwise add_rmsnorm_quant runs alone."""
        return self.use_fused_norm and self.m <= fq.NORM_MM_FOLD_M and all(
            fq.add_rmsnorm_quant_mm_supported(self.m, SHAPES[name][1], HIDDEN)
            for name in ("qkv_proj", "gate_up_proj"))

    @property
    def fused_silu(self) -> bool:
        """Whether gate_up_proj writes silu(gate) * up itself (w8a8_mm_silu_mul, or with the
        norm folded in too), so that down_proj only quantizes it; for few tokens."""
        return self.use_fused_silu and fq.SILU_EPI_MIN_M <= self.m <= fq.SILU_EPI_MAX_M and \
            fq.w8a8_mm_silu_mul_supported(self.m, 2 * INTER, HIDDEN)

    def weight_bytes(self) -> int:
        return sum(w.numel() + 4 * s.numel() for layer in self.layers for w, s in layer.values())

    def mm(self, layer, name: str, q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
        w, ws = layer[name]
        return w8a8_mm(q, w.t(), s, ws, torch.bfloat16, config=self.configs.get(name))

    def norm_mm(self, layer, name: str, x: torch.Tensor, res: torch.Tensor | None,
                silu: bool = False):
        """add_rmsnorm_quant then the linear, as one kernel: (output, residual_out); with
        silu, the output is gate_up's silu(gate) * up."""
        w, ws = layer[name]
        return fq.add_rmsnorm_quant_mm(x, res, self.norm, EPS, w.t(), ws, torch.bfloat16, None,
                                       fq.PRECISE_DIV, config=self.norm_configs.get(name),
                                       silu_mul=silu, round_silu=fq.ROUND_SILU)

    def forward(self, with_residual: bool = False):
        """One step through every layer; returns the last down_proj output [m, HIDDEN] (and
        the residual stream entering the last layer's MLP norm, with_residual=True)."""
        fused_o, fused_down, fused_norm = self.fused_o, self.fused_down, self.fused_norm
        fused_silu = self.fused_silu
        quant_down = fused_silu and fq.quant_mm_supported(self.m, HIDDEN, INTER)
        res = self.x
        if not fused_norm:
            q, s, _ = fq.add_rmsnorm_quant(self.x, None, self.norm, EPS, fq.PRECISE_DIV)
        h = None
        for i, layer in enumerate(self.layers):
            if fused_norm:
                a, rout = self.norm_mm(layer, "qkv_proj", h if i else self.x, res if i else None)
                res = rout if i else res
            else:
                if i:
                    q, s, res = fq.add_rmsnorm_quant(h, res, self.norm, EPS, fq.PRECISE_DIV)
                a = self.mm(layer, "qkv_proj", q, s)
            if fused_o:
                w, ws = layer["o_proj"]
                h = fq.quant_mm(a[:, :Q_COLS], w.t(), ws, torch.bfloat16, None, fq.PRECISE_DIV)
            else:
                q, s = fq.quant_per_token(a[:, :Q_COLS], fq.PRECISE_DIV)
                h = self.mm(layer, "o_proj", q, s)
            if fused_norm:
                gu, res = self.norm_mm(layer, "gate_up_proj", h, res, silu=fused_silu)
            else:
                q, s, res = fq.add_rmsnorm_quant(h, res, self.norm, EPS, fq.PRECISE_DIV)
                if fused_silu:
                    w, ws = layer["gate_up_proj"]
                    gu = fq.w8a8_mm_silu_mul(q, w.t(), s, ws, fq.ROUND_SILU,
                                             config=self.silu_configs.get("gate_up_proj"))
                else:
                    gu = self.mm(layer, "gate_up_proj", q, s)
            if fused_silu:   # gu holds silu(gate) * up: quantize it into down_proj
                w, ws = layer["down_proj"]
                if quant_down:
                    h = fq.quant_mm(gu, w.t(), ws, torch.bfloat16, None, fq.PRECISE_DIV)
                else:
                    q, s = fq.quant_per_token(gu, fq.PRECISE_DIV)
                    h = self.mm(layer, "down_proj", q, s)
            elif fused_down:
                w, ws = layer["down_proj"]
                h = fq.silu_mul_quant_mm(gu, w.t(), ws, torch.bfloat16, None, fq.PRECISE_DIV,
                                         fq.ROUND_SILU)
            else:
                q, s = fq.silu_mul_quant(gu, fq.PRECISE_DIV, fq.ROUND_SILU)
                h = self.mm(layer, "down_proj", q, s)
        return (h, res) if with_residual else h


def per_layer_us(stack: DecoderStandIn, windows: int = 5, min_window_ms: float = 20.0,
                 check=None) -> float:
    """Median microseconds per decoder layer, with the whole step captured as one HIP graph
    and replayed (the reference's discipline, bench/situ_tune.py:127-154).  `check`, if
    given, is called with the step's output after the graph's first replay, before timing."""
    import statistics

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        stack.forward()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        h = stack.forward()
    h.fill_(float("nan"))   # eager, outside the graph: the replay must write every element
    graph.replay()
    torch.cuda.synchronize()
    if check is not None:
        check(h)

    def window(reps: int) -> float:
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            graph.replay()
        stop.record()
        stop.synchronize()
        return start.elapsed_time(stop) * 1e3 / reps / len(stack.layers)

    one_ms = window(1) * len(stack.layers) / 1e3
    reps = max(3, int(min_window_ms / max(one_ms, 1e-3)))
    times = [window(reps) for _ in range(windows)]
    del graph
    return statistics.median(times)
