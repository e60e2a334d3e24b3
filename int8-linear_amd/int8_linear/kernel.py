"""W8A8 int8 matmul with the dequantization fused in, on MI355X (gfx950) HIP kernels.

    C[M, N] = (A_q[M, K] @ W_q[K, N]) * scale_a[M] * scale_b[N] + bias[N]

The same Python surface as the reference's int8_linear/kernel.py (AshrithaG/int8-linear):
Config, NotSupported, default_config, tuned_config, choose_config and w8a8_mm, with the
same argument meaning, validation order and exceptions (kernel.py:45-60, 127-160, 202-242).
The kernel itself is hand-written HIP in csrc/i8l_gemm*.hip, reached through the C ABI of
include/int8_linear_amd.h: an int8 MFMA (v_mfma_i32_16x16x64_i8 / 32x32x32_i8) product
accumulated exactly in int32, then acc * scale_a * scale_b + bias in fp32 and one cast.

W_q is the transposed [K, N] view of an [N, K] nn.Linear weight (K-contiguous), which is
how vLLM passes it.  Launches go on the caller's current stream and allocate nothing but
the output, so calls can be captured into a HIP graph.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from functools import lru_cache
from pathlib import Path

import torch

from int8_linear import _lib

TUNED_PATH = Path(__file__).with_name("tuned_configs.json")


class NotSupported(Exception):
    """The kernel does not take this shape or dtype, so the caller should fall back."""


@dataclass(frozen=True)
class Config:
    """One GEMM launch configuration (reference kernel.py:49-60), in MI355X terms.

    Decode schedules (bm <= 128 tokens a workgroup, bn <= 64 columns):
      stages == 1: weights streamed into MFMA registers; `warps` waves split K in 64-byte
        steps, so bk == 64 * warps.
      stages == 3: weights copied through LDS with direct-to-LDS loads; each of the
        `warps` waves owns one K slice taken bk bytes per step (K a multiple of bk * warps);
        group_m == 3 keeps two steps in flight (three step buffers a wave; more than two
        steps a wave), group_m == 4 three (four buffers; more than three steps), else one.
      stages == 4: the same with one K step a wave (K == bk * warps), each workgroup walking
        several column tiles with its activations held in registers.
      stages == 5: the stages-3 tile (up to 64 columns) with K split into group_m (2, 4 or 8)
        parts, one workgroup each, and the int32 partials summed by a second kernel; the
        call allocates the partials' workspace (group_m * M * N * 4 bytes).
    Prefill schedules (bm x bn macro tiles of 64 to 256, K in bk-byte steps, `group_m`
    rows of tiles walked together):
      stages == 2: double-buffered LDS staged through registers;
      3 <= stages <= 8, bm >= 128: a ring of `stages` LDS buffers filled by direct-to-LDS
        loads;
      stages >= 10: a ring of stages - 8 buffers (2 is a double buffer) with the LDS
        fragment reads of each MFMA substep overlapped with the MFMAs of the one before.
    A configuration the library was not built with raises NotSupported.
    """

    bm: int
    bn: int
    bk: int
    warps: int = 4
    stages: int = 2
    group_m: int = 1

    @property
    def name(self) -> str:
        return f"{self.bm}x{self.bn}x{self.bk} w{self.warps} s{self.stages} g{self.group_m}"


_cstructs: dict[Config, _lib.CConfig] = {}


def _cconfig(cfg: Config) -> _lib.CConfig:
    c = _cstructs.get(cfg)
    if c is None:
        c = _cstructs[cfg] = _lib.CConfig(cfg.bm, cfg.bn, cfg.bk, cfg.warps, cfg.stages,
                                          cfg.group_m)
    return c


def default_config(m: int, n: int, k: int) -> Config:
    """The untuned choice (the library's own rule, i8l_default_config): weights through LDS
    up to 32 tokens (the persistent tile on many column tiles), 32x32 weights-through-LDS
    tiles up to 128 tokens below N = 8192, and above that the overlapped-ring tile (64x64
    up to 256x256) with the least waves of workgroups times one wave's measured time."""
    c = _lib.CConfig()
    _lib.check(_lib.lib().i8l_default_config(m, n, k, c), NotSupported)
    return Config(c.bm, c.bn, c.bk, c.warps, c.stages, c.group_m)


@lru_cache(maxsize=None)
def _tuned_table(device_name: str) -> dict:
    tables = json.loads(TUNED_PATH.read_text()) if TUNED_PATH.exists() else {}
    return tables.get(device_name, {})


@lru_cache(maxsize=None)
def _device_table(device: int) -> dict:
    """The tuned table of this device: by marketing name as the reference keys it, else by
    the architecture name (gfx950), which is what some ROCm installs report instead of the
    product name."""
    table = _tuned_table(torch.cuda.get_device_name(device))
    if not table:
        arch = getattr(torch.cuda.get_device_properties(device), "gcnArchName", "")
        table = _tuned_table(arch.split(":")[0])
    return table


def tuned_config(m: int, n: int, k: int) -> Config | None:
    """The fastest measured config for this GPU and shape, from the largest tuned batch
    bucket at or below M, or None if nothing has been tuned (reference kernel.py:143-148)."""
    table = _device_table(torch.cuda.current_device()).get(f"{k}x{n}", {})
    fits = [int(bucket) for bucket in table if int(bucket) <= m]
    return Config(**table[str(max(fits))]["config"]) if fits else None


_chosen: dict[tuple[int, int, int, int], Config] = {}


def choose_config(m: int, n: int, k: int) -> Config:
    """tuned_config, else default_config, remembered per device and shape."""
    key = (torch.cuda.current_device(), m, n, k)
    cfg = _chosen.get(key)
    if cfg is None:
        cfg = _chosen[key] = tuned_config(m, n, k) or default_config(m, n, k)
    return cfg


def _table_rows(device: int) -> list[list[int]]:
    """This device's tuned table as rows (k, n, m, bm, bn, bk, warps, stages, group_m), for the
    C++ binding's configuration lookup."""
    rows = []
    for kn, buckets in _device_table(device).items():
        k, n = map(int, kn.split("x"))
        for m, row in buckets.items():
            c = Config(**row["config"])
            rows.append([k, n, int(m), c.bm, c.bn, c.bk, c.warps, c.stages, c.group_m])
    return rows


def _fast_mm(a_q, b_q, scale_a, scale_b, out_dtype, bias):
    """The launch through the C++ binding, or None (not built, or not the plain case)."""
    f = _lib.fast()
    if f is None:
        return None
    try:
        out = f.mm(a_q, b_q, scale_a, scale_b, out_dtype, bias)
        if out is None and a_q.is_cuda and not f.has_table(a_q.get_device()):
            # first call on this device: hand its tuned table over, then try again
            f.set_table(a_q.get_device(), _table_rows(a_q.get_device()))
            out = f.mm(a_q, b_q, scale_a, scale_b, out_dtype, bias)
    except (TypeError, AttributeError):
        return None  # not tensors or dtypes: the Python path reports it
    return out


def same_device(device: torch.device, **tensors) -> None:
    """Raise ValueError unless every tensor given (None entries are skipped) is on `device`."""
    for name, t in tensors.items():
        if t is not None and t.device != device:
            raise ValueError(f"{name} is on {t.device}, the launch is on {device}")


def supported(m: int, n: int, k: int, config: Config | None = None) -> bool:
    """Whether w8a8_mm takes (M, N, K) under `config` (default: choose_config)."""
    cfg = config or default_config(m, n, k)
    return _lib.lib().i8l_w8a8_mm_supported(m, n, k, _cconfig(cfg)) == _lib.OK


def w8a8_mm(
    a_q: torch.Tensor,
    b_q: torch.Tensor,
    scale_a: torch.Tensor,
    scale_b: torch.Tensor,
    out_dtype: torch.dtype = torch.bfloat16,
    bias: torch.Tensor | None = None,
    *,
    config: Config | None = None,
    raw: bool = False,
    cached_launch: bool = True,
) -> torch.Tensor:
    """(A_q @ B_q) * scale_a * scale_b + bias, for int8 A_q [M, K] and B_q [K, N].

    scale_a is per row ([M] or [M, 1]) or a scalar, scale_b per column ([N] or [N, 1]) or
    a scalar, both float32.  With raw=True the exact int32 product is returned and the
    scales and bias are ignored.  cached_launch is accepted for API compatibility; every
    launch is a direct C call already.

    Without an explicit config the call goes through the C++ binding when it is built,
    which chooses the same configuration (by the operands' device) and launches the same
    kernel; anything but the plain case comes back here.
    """
    if config is None and not raw:
        out = _fast_mm(a_q, b_q, scale_a, scale_b, out_dtype, bias)
        if out is not None:
            return out
    if a_q.dtype != torch.int8 or b_q.dtype != torch.int8:
        raise NotSupported(f"int8 operands only, got {a_q.dtype} and {b_q.dtype}")
    if a_q.dim() != 2 or b_q.dim() != 2 or a_q.shape[1] != b_q.shape[0]:
        raise ValueError(f"cannot multiply {tuple(a_q.shape)} by {tuple(b_q.shape)}")
    if not (a_q.is_cuda and b_q.is_cuda):
        raise NotSupported("operands must be on a HIP device")
    # Every pointer the kernel reads must live on the launching device: a host scale or a
    # tensor on another GPU would be dereferenced as a device address.
    same_device(a_q.device, b_q=b_q, scale_a=scale_a, scale_b=scale_b, bias=bias)
    m, k = a_q.shape
    n = b_q.shape[1]
    cfg = config or choose_config(m, n, k)
    if n % cfg.bn or k % cfg.bk:
        raise NotSupported(f"N={n} and K={k} must divide the {cfg.name} tile")
    # Scales and bias are read as flat stride-1 arrays; contiguous() is free when they
    # already are, and a copy only for a slice or a transpose.
    sa, sb = scale_a.reshape(-1).contiguous(), scale_b.reshape(-1).contiguous()
    if sa.dtype != torch.float32 or sb.dtype != torch.float32:
        raise NotSupported(f"float32 scales only, got {sa.dtype} and {sb.dtype}")
    if sa.numel() not in (1, m) or sb.numel() not in (1, n):
        raise ValueError(f"scale sizes {sa.numel()} and {sb.numel()} fit neither {m} nor {n}")
    if bias is not None and tuple(bias.shape) != (n,):
        raise ValueError(f"bias must have shape ({n},), got {tuple(bias.shape)}")
    if bias is not None:
        bias = bias.contiguous()
        bias_code = _lib.DTYPE_CODE.get(bias.dtype)
        if bias_code not in (_lib.BF16, _lib.F16, _lib.F32):
            raise NotSupported(f"bias dtype {bias.dtype} is not supported")
    else:
        bias_code = _lib.DTYPE_NONE
    if raw:
        out_code = _lib.I32
    else:
        out_code = _lib.DTYPE_CODE.get(out_dtype)
        if out_code not in (_lib.BF16, _lib.F16, _lib.F32):
            raise NotSupported(f"output dtype {out_dtype} is not supported")

    out = torch.empty((m, n), dtype=torch.int32 if raw else out_dtype, device=a_q.device)
    # A split of K writes int32 partial planes to a workspace from the caching allocator
    # (stream-ordered, and from the graph's pool under capture).
    ws_bytes = _lib.lib().i8l_w8a8_mm_workspace_bytes(m, n, k, _cconfig(cfg))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=a_q.device) if ws_bytes else None
    status = _lib.lib().i8l_w8a8_mm_ws(
        a_q.data_ptr(), a_q.stride(0), a_q.stride(1),
        b_q.data_ptr(), b_q.stride(0), b_q.stride(1),
        sa.data_ptr(), sa.numel(), sb.data_ptr(), sb.numel(),
        bias.data_ptr() if bias is not None else None, bias_code,
        out.data_ptr(), out.stride(0), out_code,
        m, n, k, ws.data_ptr() if ws is not None else None, ws_bytes,
        _cconfig(cfg), _lib.stream_of(a_q))
    _lib.check(status, NotSupported)
    return out


def init(device: torch.device | int | None = None) -> None:
    """Set up the library on one GPU (default: the current one): the C entry i8l_init, which
    looks up the device address of the array w8a8_mm_noalloc keeps its split-of-K partials
    in.  Optional (the first w8a8_mm_noalloc call on a GPU does it otherwise); call it before
    capturing that first call into a HIP graph.  No counterpart in the reference."""
    idx = -1
    if device is not None:
        d = torch.device("cuda", device) if isinstance(device, int) else torch.device(device)
        idx = -1 if d.index is None else d.index
    _lib.check(_lib.lib().i8l_init(idx), NotSupported)


def w8a8_mm_noalloc(a_q: torch.Tensor, b_q: torch.Tensor, scale_a: torch.Tensor,
                    scale_b: torch.Tensor, out: torch.Tensor, bias: torch.Tensor | None = None,
                    *, config: Config | None = None) -> torch.Tensor:
    """w8a8_mm into the caller's `out` ([M, N] bf16/fp16/fp32, or int32 for the raw product),
    allocating no device memory: the C entry i8l_w8a8_mm_noalloc, for callers that cannot
    allocate (code under HIP graph capture, serving loops that forbid it).  It has no
    counterpart in the reference.

    A split of K (stages 5) keeps its int32 partial planes in the library's own 16 MiB device
    array of the GPU, which every call of this entry on that GPU shares.  Calls that can
    overlap in time on one GPU (launched on two streams with no ordering between them) race
    on it and give wrong results: order them (one stream, or events).  Configurations whose
    planes exceed 16 MiB raise NotSupported (use w8a8_mm).  Scales and bias are taken as they
    are: contiguous float32 scales and a contiguous bias, or ValueError (no copies are made).
    The first call on a GPU looks up that array's device address unless init() did.
    """
    if a_q.dtype != torch.int8 or b_q.dtype != torch.int8:
        raise NotSupported(f"int8 operands only, got {a_q.dtype} and {b_q.dtype}")
    if a_q.dim() != 2 or b_q.dim() != 2 or a_q.shape[1] != b_q.shape[0]:
        raise ValueError(f"cannot multiply {tuple(a_q.shape)} by {tuple(b_q.shape)}")
    m, k = a_q.shape
    n = b_q.shape[1]
    if tuple(out.shape) != (m, n) or out.stride(1) != 1:
        raise ValueError(f"out must be a row-major [{m}, {n}] tensor")
    same_device(a_q.device, b_q=b_q, scale_a=scale_a, scale_b=scale_b, bias=bias, out=out)
    for name, t in (("scale_a", scale_a), ("scale_b", scale_b), ("bias", bias)):
        if t is not None and not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous (this entry makes no copies)")
    if scale_a.dtype != torch.float32 or scale_b.dtype != torch.float32:
        raise NotSupported(f"float32 scales only, got {scale_a.dtype} and {scale_b.dtype}")
    out_code = _lib.DTYPE_CODE.get(out.dtype)
    bias_code = _lib.DTYPE_CODE.get(bias.dtype) if bias is not None else _lib.DTYPE_NONE
    status = _lib.lib().i8l_w8a8_mm_noalloc(
        a_q.data_ptr(), a_q.stride(0), a_q.stride(1), b_q.data_ptr(), b_q.stride(0),
        b_q.stride(1), scale_a.data_ptr(), scale_a.numel(), scale_b.data_ptr(), scale_b.numel(),
        bias.data_ptr() if bias is not None else None, bias_code, out.data_ptr(),
        out.stride(0), out_code if out_code is not None else -1, m, n, k,
        _cconfig(config) if config is not None else None, _lib.stream_of(a_q))
    _lib.check(status, NotSupported)
    return out
