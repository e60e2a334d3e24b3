"""The allocation-free GEMM entry (i8l_w8a8_mm_noalloc) on the GPU, through the C ABI: a
split of K with its partial planes in the library's own device array gives the workspace
entry's output (i8l_w8a8_mm_ws, the caller's workspace) bit for bit, and through it the CPU
oracle's, on two calls in a row, the second with fewer tokens; a config that needs more
than the array holds is declined with an error, and a config without a split runs too.

The entry has no counterpart in the reference: it exists for callers that cannot allocate."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from helpers import bits, ints, np_, say
from int8_linear import Config, _lib, kernel
from oracle import oracle as o

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20


def _call(entry, a, w, sa, sb, bias, out, out_code, cfg, ws=None):
    m, k = a.shape
    n = w.shape[0]
    args = [a.data_ptr(), a.stride(0), 1, w.data_ptr(), 1, w.stride(0),
            sa.data_ptr(), sa.numel(), sb.data_ptr(), sb.numel(),
            bias.data_ptr() if bias is not None else None,
            _lib.BF16 if bias is not None else _lib.DTYPE_NONE,
            out.data_ptr(), out.stride(0), out_code, m, n, k]
    if ws is not None:
        args += [ws.data_ptr(), ws.numel()]
    return entry(*args, ctypes.byref(kernel._cconfig(cfg)) if cfg else None, _lib.stream_of(a))


def test_noalloc_equals_the_workspace_entry_twice():
    L = _lib.lib()
    k, n = 14336, 4096
    cfg = Config(64, 64, 128, 4, 5, 4)
    w = ints((n, k), 91)
    g = torch.Generator().manual_seed(92)
    sb = (torch.rand((n,), generator=g) * 1e-3 + 1e-4).cuda()
    bias = torch.randn(n, generator=g).to(torch.bfloat16).cuda()
    for m in (128, 37):                       # the second call smaller than the first
        say(f"noalloc m={m} k={k} n={n} {cfg.name}")
        a = ints((m, k), 93 + m)
        sa = (torch.rand((m,), generator=g) * 1e-2 + 1e-3).cuda()
        need = L.i8l_w8a8_mm_workspace_bytes(m, n, k, ctypes.byref(kernel._cconfig(cfg)))
        assert 0 < need <= SCRATCH_BYTES
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        ref = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
        got = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
        assert _call(L.i8l_w8a8_mm_ws, a, w, sa, sb, bias, ref, _lib.BF16, cfg, ws) == _lib.OK
        assert _call(L.i8l_w8a8_mm_noalloc, a, w, sa, sb, bias, got, _lib.BF16, cfg) == _lib.OK, \
            _lib.last_error()
        raw = torch.empty((m, n), dtype=torch.int32, device="cuda")
        assert _call(L.i8l_w8a8_mm_noalloc, a, w, sa, sb, None, raw, _lib.I32, cfg) == _lib.OK
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
        acc = o.gemm_i32(np_(a), np_(w))
        assert np.array_equal(np_(raw), acc)
        assert np.array_equal(bits(got), o.epilogue(acc, np_(sa), np_(sb), bits(bias), o.BF16,
                                                    o.BF16))


def test_noalloc_declines_beyond_its_scratch_and_runs_unsplit_configs():
    L = _lib.lib()
    m, k, n = 128, 4096, 12288
    cfg = Config(64, 64, 128, 4, 5, 4)         # 4 * 128 * 12288 * 4 = 24 MiB > 16 MiB
    assert L.i8l_w8a8_mm_workspace_bytes(m, n, k, ctypes.byref(kernel._cconfig(cfg))) > SCRATCH_BYTES
    a, w = ints((m, k), 5), ints((n, k), 6)
    one = torch.ones(1, device="cuda")
    out = torch.empty((m, n), dtype=torch.int32, device="cuda")
    assert _call(L.i8l_w8a8_mm_noalloc, a, w, one, one, None, out, _lib.I32, cfg) == _lib.UNSUPPORTED
    assert "scratch" in _lib.last_error()
    for c in (None, Config(32, 32, 128, 4, 3, 1)):   # no split: the scratch is not used
        say(f"noalloc unsplit {c.name if c else 'default'}")
        out.fill_(-1)
        assert _call(L.i8l_w8a8_mm_noalloc, a, w, one, one, None, out, _lib.I32, c) == _lib.OK
        torch.cuda.synchronize()
        assert np.array_equal(np_(out), o.gemm_i32(np_(a), np_(w)))


def test_python_wrapper_matches_w8a8_mm():
    """int8_linear.kernel.w8a8_mm_noalloc (into the caller's out) gives w8a8_mm's bits, with
    a split of K and without, and refuses operands it would have to copy."""
    kernel.init()                             # the set-up entry, current GPU and by index
    kernel.init(torch.cuda.current_device())
    k, n = 6144, 2048
    w = ints((n, k), 71)
    g = torch.Generator().manual_seed(72)
    sb = (torch.rand((n,), generator=g) * 1e-3 + 1e-4).cuda()
    for m, cfg in ((64, Config(64, 64, 128, 4, 5, 4)), (9, None)):
        say(f"noalloc wrapper m={m} {cfg.name if cfg else 'default'}")
        a = ints((m, k), 73 + m)
        sa = (torch.rand((m,), generator=g) * 1e-2 + 1e-3).cuda()
        out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
        got = kernel.w8a8_mm_noalloc(a, w.t(), sa, sb, out, config=cfg)
        assert got is out
        ref = kernel.w8a8_mm(a, w.t(), sa, sb, torch.bfloat16, config=cfg)
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    with pytest.raises(ValueError):
        kernel.w8a8_mm_noalloc(a, w.t(), torch.rand((m, 2), device="cuda")[:, 0], sb, out)


# A fresh process whose first use of the library is an allocation-free split-of-K call under
# HIP graph capture (so the device's scratch address is looked up inside the capture, unless
# argv[2] is "init": then i8l_init sets the device up before the capture), then replays with
# new activations checked against the workspace entry.
_CAPTURE = r"""
import ctypes, sys
sys.path[:0] = [sys.argv[1], sys.argv[1] + "/int8-linear_amd"]
import torch
from int8_linear import Config, _lib, kernel
L = _lib.lib()
dev = torch.device("cuda:0")
m, k, n = 96, 14336, 4096
cfg = Config(64, 64, 128, 4, 5, 4)
c = kernel._cconfig(cfg)
g = torch.Generator().manual_seed(5)
w = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=g).to(dev)
a = torch.empty((m, k), dtype=torch.int8, device=dev)
sa = (torch.rand((m,), generator=g) * 1e-2 + 1e-3).to(dev)
sb = (torch.rand((n,), generator=g) * 1e-3 + 1e-4).to(dev)
out = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
def call(entry, o, *ws):
    return entry(a.data_ptr(), k, 1, w.data_ptr(), 1, k, sa.data_ptr(), m, sb.data_ptr(), n,
                 None, _lib.DTYPE_NONE, o.data_ptr(), n, _lib.BF16, m, n, k, *ws,
                 ctypes.byref(c), torch.cuda.current_stream().cuda_stream)
if sys.argv[2] == "init":
    assert L.i8l_init(-1) == _lib.OK, _lib.last_error()
    assert L.i8l_init(0) == _lib.OK, _lib.last_error()       # again, by index: no-op
    assert L.i8l_init(torch.cuda.device_count()) == _lib.INVALID_ARG
    print("init", flush=True)
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    st = call(L.i8l_w8a8_mm_noalloc, out)
assert st == _lib.OK, _lib.last_error()
print("captured", flush=True)
need = L.i8l_w8a8_mm_workspace_bytes(m, n, k, ctypes.byref(c))
ws = torch.empty(need, dtype=torch.uint8, device=dev)
ref = torch.empty_like(out)
for r in range(4):
    a.copy_(torch.randint(-127, 128, (m, k), dtype=torch.int8, generator=g).to(dev))
    out.fill_(float("nan"))
    graph.replay()
    torch.cuda.synchronize()
    assert call(L.i8l_w8a8_mm_ws, ref, ws.data_ptr(), need) == _lib.OK, _lib.last_error()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"replay {r} differs"
    print("replay", r, "equal", flush=True)
print("ok", flush=True)
"""


@pytest.mark.parametrize("setup", ["lazy", "init"])
def test_first_call_inside_a_graph_capture(setup):
    import subprocess
    import sys
    from pathlib import Path
    root = str(Path(__file__).resolve().parents[1])
    say(f"noalloc: first call of a fresh process under graph capture ({setup}), 4 replays")
    r = subprocess.run([sys.executable, "-c", _CAPTURE, root, setup], capture_output=True,
                       text=True, timeout=150)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), (r.stdout[-2000:],
                                                                  r.stderr[-2000:])
