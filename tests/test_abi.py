"""The C-ABI library without a GPU: it loads, exports every entry point include/*.h declares,
and its host-only entry points (config choice, the decline rule) behave.  CPU only."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from int8_linear import Config, NotSupported, _lib, default_config, kernel

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols() -> set[str]:
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(i8l_\w+)\s*\(", text))
    return names


def test_library_loads_and_exports_every_declared_symbol():
    L = _lib.lib()
    declared = declared_symbols()
    assert declared >= set(_lib.EXPORTS)
    for name in declared:
        assert hasattr(L, name), name
    assert L.i8l_version().decode().startswith("int8_linear_amd")


def test_library_binary_is_built_for_gfx950_only():
    # the offload bundle names its targets; only gfx950 is built
    data = _lib.LIB_PATH.read_bytes()
    assert b"gfx950" in data
    for other in (b"gfx942", b"gfx90a", b"gfx1100"):
        assert b"amdgcn-amd-amdhsa--" + other not in data


def test_default_config_regimes():
    d = default_config(16, 4096, 2048)                      # weights through LDS
    assert d.stages == 3 and d.bm == 16 and 2048 % (d.bk * d.warps) == 0
    assert default_config(17, 4096, 2048).bm == 32          # one tile covers M=17
    assert default_config(1, 2048, 6144).bn == 8            # narrow N: 8 columns a workgroup
    s = default_config(64, 4096, 2048)                      # 32x32 tiles through LDS
    assert (s.bm, s.bn, s.stages, s.warps) == (32, 32, 3, 16)
    assert (default_config(128, 2048, 6144).bk, default_config(128, 2048, 6144).warps) == (256, 4)
    s = default_config(64, 4096, 2056)                      # odd K: register-streamed weights
    assert s.stages == 1 and s.bm == 64 and s.bk == 64 * s.warps
    s = default_config(64, 4104, 2048)                      # N = 8 mod 16: 8-column stream tiles
    assert (s.stages, s.bm, s.bn) == (1, 32, 8) and kernel.supported(64, 4104, 2048, s)
    p = default_config(4096, 28672, 4096)
    assert p.stages >= 2 and (p.bm, p.bn) == (256, 256)
    assert default_config(300, 2048, 2048).stages >= 2
    # 9-32 tokens on many column tiles: the persistent tile, two workgroups a CU
    assert default_config(16, 12288, 2048) == Config(16, 16, 256, 8, 4, 2)
    assert default_config(24, 12288, 2048) == Config(32, 16, 256, 8, 4, 2)
    assert default_config(16, 28672, 4096) == Config(16, 8, 512, 8, 4, 2)
    assert default_config(4, 12288, 2048).stages == 3     # few tokens: A is small
    assert default_config(24, 28672, 4096).stages == 3    # no 32-row 8-column persistent tile
    # From 129 tokens (33 on wide N) the overlapped-ring tile with the least waves x wave
    # time, one workgroup a CU on a 256-CU part: small tiles while few tokens leave CUs idle,
    # the largest tile that still fills one wave once it does.
    bmn = lambda m, n, k: (default_config(m, n, k).bm, default_config(m, n, k).bn)
    assert default_config(96, 12288, 2048) == Config(128, 64, 128, 4, 12, 8)
    assert bmn(512, 4096, 4096) == (128, 64)              # 256 tiles of 128x64 (one wave)
    assert bmn(1024, 4096, 4096) == (128, 128)            # 256 tiles of 128x128
    assert bmn(400, 2048, 6144) == (64, 64)               # 224 tiles: anything larger idles CUs
    assert bmn(272, 6144, 4096) == (64, 128)              # 240 of 64x128 beat 288 of 128x64
    assert default_config(288, 12288, 2048) == Config(64, 256, 128, 8, 11, 8)
    assert default_config(400, 28672, 4096) == Config(256, 256, 128, 8, 10, 4)
    assert bmn(2048, 2048, 2048) == (128, 128)            # 256x256 would leave 3/4 of the CUs idle
    assert bmn(2048, 4096, 4096) == (256, 128)
    assert default_config(96, 4096, 2048).bn == 32          # narrower N: 32-column tiles
    for m, n, k in ((300, 2048, 2048), (4096, 4096, 14336), (700, 6144, 4096), (200, 48, 256)):
        assert kernel.supported(m, n, k, default_config(m, n, k)), (m, n, k)


def test_default_config_takes_every_aligned_shape():
    """The library default is a built, supported configuration for every M and every N, K
    the fast schedules can take (N a multiple of 4, K of 64): narrow N included, where it
    falls back to 8- or 4-column streaming tiles."""
    ms = (1, 7, 16, 17, 32, 33, 64, 65, 128, 129, 300, 512, 1025, 4096, 16384)
    ks = (64, 192, 640, 2048, 2112, 5120, 14336)
    ns = (4, 8, 12, 24, 40, 48, 96, 320, 2304, 6144, 57344)
    for m in ms:
        for k in ks:
            for n in ns:
                assert kernel.supported(m, n, k, default_config(m, n, k)), (m, n, k)


def test_every_tuner_candidate_tile_is_built():
    """The tuner's tile lists and the library's built tiles stay in step: each listed tile
    is taken for a shape it divides."""
    from int8_linear import tune
    n, k = 2 * 3 * 128 * 8, 4096                            # divisible by every tile width
    for bm, bn, bk, w, st in tune.DMAP_TILES:
        assert kernel.supported(1024, n, k, Config(bm, bn, bk, w, st + tune.PIPELINED, 4)), bn
    for bm, bn, bk, w, st in tune.DMA_TILES:
        assert kernel.supported(1024, n, k, Config(bm, bn, bk, w, st, 1)), (bm, bn, bk, st)
    for bm, bn, bk, w in tune.STAGED_TILES:
        assert kernel.supported(1024, n, k, Config(bm, bn, bk, w, 2, 1)), (bm, bn, bk)
    for mt, nc, ks, w in tune.WLDSP_TILES:                  # persistent: one K step a wave
        assert kernel.supported(16 * mt, n, w * 64 * ks, Config(16 * mt, nc, 64 * ks, w, 4, 1))
        assert not kernel.supported(16 * mt, n, 2 * w * 64 * ks,
                                    Config(16 * mt, nc, 64 * ks, w, 4, 1))
    for mt, nc, ks in tune.WLDS_TILES:                     # one or more K steps a wave
        assert any(kernel.supported(16 * mt, n, steps * w * 64 * ks,
                                    Config(16 * mt, nc, 64 * ks, w, 3, 1))
                   for w in (4, 8, 16) for steps in (1, 2)), (mt, nc, ks)


def test_deeper_rings_take_only_what_they_can_keep_in_flight():
    """group_m 3 / 4 of the stages-3 tile keep two / three K steps in flight: each needs more
    steps a wave than that, its buffers within the LDS, and its outstanding copies (steps in
    flight x the step's 1 KiB copy instructions) below the 64 the vmcnt counter holds."""
    n = 4096
    for g, need in ((3, 3), (4, 4)):
        cfg = Config(16, 64, 128, 4, 3, g)      # 80 rows x 128 bytes: 10 copies a step
        for steps in range(1, 7):
            assert kernel.supported(16, n, steps * 4 * 128, cfg) == (steps >= need), (g, steps)
    # 96 rows x 256 bytes: 24 copies a step, so two steps (48) fit the counter, three (72) not
    cfg3, cfg4 = Config(32, 64, 256, 1, 3, 3), Config(32, 64, 256, 1, 3, 4)
    assert kernel.supported(32, n, 5 * 256, cfg3) and not kernel.supported(32, n, 5 * 256, cfg4)
    # four buffers of 32 rows x 512 bytes a wave over 4 waves: 256 KiB, beyond the LDS
    assert not kernel.supported(1, n, 5 * 4 * 512, Config(16, 16, 512, 4, 3, 4))


def test_supported_decline_rule_matches_reference():
    # kernel.py:228-229 of the reference: N % bn or K % bk declines
    assert not kernel.supported(4, 64, 100)
    assert kernel.supported(16, 4096, 2048)
    assert not kernel.supported(16, 4096, 2048, Config(16, 16, 64, 1, 3, 1))  # 64-byte steps: not built
    assert kernel.supported(16, 4096, 2048, Config(16, 16, 256, 8, 3, 1))     # through LDS, 1 step
    assert kernel.supported(16, 4096, 2048, Config(16, 16, 128, 4, 3, 1))     # 4 steps a wave
    assert kernel.supported(16, 4096, 2048, Config(16, 32, 128, 16, 3, 1))    # 32 columns, 1 step
    assert kernel.supported(16, 4096, 2048, Config(16, 32, 128, 8, 3, 1))     # ... or 2 steps
    assert kernel.supported(16, 4096, 2048, Config(16, 64, 128, 8, 3, 1))      # 64 columns
    assert not kernel.supported(16, 4096, 2048, Config(16, 128, 128, 8, 3, 1))  # 128: not built
    assert not kernel.supported(16, 4096, 2048, Config(32, 64, 128, 16, 3, 1))  # would spill
    assert not kernel.supported(16, 4096, 2048, Config(16, 16, 384, 4, 3, 1))  # K % (bk*warps)
    assert not kernel.supported(16, 4096, 2048, Config(16, 16, 512, 16, 3, 1))  # LDS > 160 KiB
    assert kernel.supported(16, 4096, 2048, Config(16, 16, 64, 1, 1, 1))
    assert kernel.supported(4096, 4096, 4096, Config(256, 256, 64, 8, 2, 8))
    assert not kernel.supported(4096, 4096, 4096, Config(256, 256, 64, 4, 2, 8))  # would spill
    assert kernel.supported(4096, 4096, 4096, Config(256, 256, 64, 8, 12, 8))  # overlapped ring
    assert kernel.supported(4096, 4096, 4096, Config(256, 256, 64, 8, 4, 8))   # DMA ring of 4
    assert not kernel.supported(4096, 4096, 4096, Config(256, 256, 64, 16, 2, 8))


def test_split_of_k_configs_and_their_workspace():
    """stages 5 splits K into group_m parts (2, 4, 8), each a whole number of the tile's
    bk * warps steps; the workspace is one int32 plane [M, N] a part, and only a split
    needs one."""
    L = _lib.lib()
    split = Config(64, 64, 128, 4, 5, 4)
    assert kernel.supported(128, 2048, 6144, split)
    assert L.i8l_w8a8_mm_workspace_bytes(128, 2048, 6144, kernel._cconfig(split)) == 4 * 128 * 2048 * 4
    assert L.i8l_w8a8_mm_workspace_bytes(100, 2048, 6144, kernel._cconfig(split)) == 4 * 100 * 2048 * 4
    assert L.i8l_w8a8_mm_workspace_bytes(0, 2048, 6144, kernel._cconfig(split)) == 0
    assert L.i8l_w8a8_mm_workspace_bytes(128, 2048, 6144, None) == 0          # default: no split
    unsplit = Config(64, 64, 128, 4, 3, 1)
    assert L.i8l_w8a8_mm_workspace_bytes(128, 2048, 6144, kernel._cconfig(unsplit)) == 0
    assert kernel.supported(128, 2048, 6144, Config(64, 64, 128, 6, 5, 8))    # 768 bytes a part
    assert not kernel.supported(128, 2048, 6144, Config(64, 64, 128, 4, 5, 8))  # 768 % 512
    assert not kernel.supported(128, 2048, 6144, Config(64, 64, 128, 4, 5, 3))  # 3 parts
    assert not kernel.supported(128, 2048, 2048, Config(64, 64, 256, 4, 5, 4))  # 512 a part < 1024
    assert not kernel.supported(128, 2048, 6144, Config(64, 128, 128, 4, 5, 4))  # not built
    assert kernel.supported(32, 4096, 14336, Config(32, 64, 128, 4, 5, 4))
    assert L.i8l_w8a8_mm_workspace_bytes(
        32, 4096, 14336, kernel._cconfig(Config(32, 64, 128, 4, 5, 4))) == 4 * 32 * 4096 * 4


def test_supported_reports_the_reason():
    c = _lib.CConfig(16, 16, 64, 1, 1, 1)
    assert _lib.lib().i8l_w8a8_mm_supported(4, 64, 100, ctypes.byref(c)) == _lib.UNSUPPORTED
    assert "must divide" in _lib.last_error()
    with pytest.raises(NotSupported):
        _lib.check(_lib.UNSUPPORTED, NotSupported)
    with pytest.raises(ValueError):
        _lib.check(_lib.INVALID_ARG, NotSupported)
    with pytest.raises(RuntimeError):
        _lib.check(_lib.HIP_ERROR, NotSupported)


def test_invalid_sizes_are_rejected_before_any_launch():
    L = _lib.lib()
    st = L.i8l_w8a8_mm(None, 0, 1, None, 1, 0, None, 3, None, 1, None, 0, None, 0, _lib.BF16,
                       2, 16, 64, None, None)
    assert st == _lib.INVALID_ARG and "scale_a" in _lib.last_error()
    st = L.i8l_add_rmsnorm_quant(None, None, None, 1e-6, None, None, None, 1, 8, 7, 1, 1, None)
    assert st == _lib.UNSUPPORTED
    # M == 0 launches nothing and succeeds without touching any pointer
    assert L.i8l_silu_mul_quant(None, None, None, 0, 64, _lib.BF16, 1, 1, None) == _lib.OK
    assert L.i8l_quant_per_token(None, 64, None, None, 0, 64, _lib.BF16, 1, None) == _lib.OK
    # a row stride below the row length is an error
    assert L.i8l_quant_per_token(None, 32, None, None, 2, 64, _lib.BF16, 1, None) == _lib.INVALID_ARG


def test_config_name_format():
    """The reference's Config fields and name format (int8_linear/kernel.py:49-60)."""
    import dataclasses
    assert Config(16, 64, 64, 4, 1, 1).name == "16x64x64 w4 s1 g1"
    assert Config(256, 256, 64, 4, 2, 8).name == "256x256x64 w4 s2 g8"
    assert [f.name for f in dataclasses.fields(Config)] == ["bm", "bn", "bk", "warps", "stages",
                                                             "group_m"]
    assert [f for f, _ in _lib.CConfig._fields_] == ["bm", "bn", "bk", "warps", "stages",
                                                     "group_m"]


def test_tuned_config_takes_the_largest_bucket_at_or_below_m(monkeypatch):
    table = {"2048x4096": {"1": {"config": {"bm": 16, "bn": 16, "bk": 512, "warps": 8,
                                           "stages": 1, "group_m": 1}},
                           "17": {"config": {"bm": 32, "bn": 16, "bk": 512, "warps": 8,
                                            "stages": 1, "group_m": 1}}}}
    monkeypatch.setattr(kernel.torch.cuda, "current_device", lambda: 0)
    monkeypatch.setattr(kernel, "_device_table", lambda dev: table)
    assert kernel.tuned_config(1, 4096, 2048).bm == 16
    assert kernel.tuned_config(16, 4096, 2048).bm == 16
    assert kernel.tuned_config(17, 4096, 2048).bm == 32
    assert kernel.tuned_config(500, 4096, 2048).bm == 32
    assert kernel.tuned_config(5, 2048, 2048) is None


def test_shipped_tuned_table_is_valid():
    import json
    tables = json.loads(kernel.TUNED_PATH.read_text())
    for device, shapes in tables.items():
        for kn, buckets in shapes.items():
            k, n = map(int, kn.split("x"))
            for m, row in buckets.items():
                cfg = Config(**row["config"])
                assert kernel.supported(int(m), n, k, cfg), (device, kn, m, cfg)


def test_cpu_tensors_are_declined_not_computed():
    import torch
    a = torch.zeros((2, 64), dtype=torch.int8)
    with pytest.raises(NotSupported):
        kernel.w8a8_mm(a, torch.zeros((64, 16), dtype=torch.int8), torch.ones(1), torch.ones(1))


def test_cpp_binding_loads_and_chooses_the_tuned_config():
    """The C++ eager binding chooses the configuration kernel.tuned_config / default_config
    would: the largest tuned bucket at or below M, else the library's default."""
    from int8_linear import kernel as kn
    f = _lib.fast()
    assert f is not None, "the binding is built with the library"
    for name in ("mm", "add_rmsnorm_quant", "silu_mul_quant", "quant_per_token", "set_table"):
        assert hasattr(f, name)
    rows = [[2048, 4096, 1, 16, 16, 512, 8, 1, 1], [2048, 4096, 17, 32, 16, 512, 8, 1, 1]]
    f.set_table(7, rows)
    assert f.has_table(7) and not f.has_table(6)
    assert f.config_for(6, 1, 4096, 2048) is None
    assert f.config_for(7, 1, 4096, 2048)[:2] == (16, 16)
    assert f.config_for(7, 16, 4096, 2048)[:2] == (16, 16)
    assert f.config_for(7, 17, 4096, 2048)[:2] == (32, 16)
    assert f.config_for(7, 500, 4096, 2048)[:2] == (32, 16)
    for m, n, k in ((5, 2048, 2048), (4096, 4096, 4096), (96, 12288, 2048)):
        d = kn.default_config(m, n, k)
        assert f.config_for(7, m, n, k) == (d.bm, d.bn, d.bk, d.warps, d.stages, d.group_m)


def test_cpp_binding_declines_what_the_python_path_must_handle():
    import torch
    f = _lib.fast()
    before = f.launches()
    a = torch.zeros((2, 64), dtype=torch.int8)
    assert f.mm(a, torch.zeros((64, 16), dtype=torch.int8), torch.ones(1), torch.ones(1),
                torch.bfloat16, None) is None                        # host tensors
    x = torch.zeros((2, 64), dtype=torch.bfloat16)
    assert f.add_rmsnorm_quant(x, None, torch.ones(64, dtype=torch.bfloat16), 1e-6, True) is None
    assert f.silu_mul_quant(x, True, False) is None
    assert f.quant_per_token(x, True) is None
    assert f.launches() == before


def test_dynamic_quant_entry_validates_on_the_host():
    L = _lib.lib()
    assert L.i8l_w8a8_mm_dynq_supported(16, 2048, 2048, None) == _lib.OK
    assert L.i8l_w8a8_mm_dynq_supported(1, 4096, 4096, None) == _lib.OK
    assert L.i8l_w8a8_mm_dynq_supported(4, 2048, 6144, None) == _lib.OK      # 12 waves of 512
    assert L.i8l_w8a8_mm_dynq_supported(4, 2048, 3072, None) == _lib.UNSUPPORTED
    assert "one step" in _lib.last_error()
    c = _lib.CConfig(16, 32, 128, 16, 3, 1)
    assert L.i8l_w8a8_mm_dynq_supported(16, 2048, 2048, ctypes.byref(c)) == _lib.OK
    c = _lib.CConfig(16, 32, 128, 8, 3, 1)                     # two steps a wave: not built
    assert L.i8l_w8a8_mm_dynq_supported(16, 2048, 2048, ctypes.byref(c)) == _lib.UNSUPPORTED
    # argument errors come back before anything launches (no pointer is touched)
    args = [None, 2048, _lib.BF16, 1, None, 1, 2048, None, 7, None, 0, None, 2048, _lib.BF16,
            None, 4, 2048, 2048, None, None]
    assert L.i8l_w8a8_mm_dynq(*args) == _lib.INVALID_ARG and "scale_b" in _lib.last_error()
    args[8], args[1] = 2048, 1024                               # row stride below K
    assert L.i8l_w8a8_mm_dynq(*args) == _lib.INVALID_ARG
    args[1], args[2] = 2048, _lib.F32                           # fp32 activations
    assert L.i8l_w8a8_mm_dynq(*args) == _lib.UNSUPPORTED
    args[2], args[15] = _lib.BF16, 0                            # M == 0: nothing to do
    assert L.i8l_w8a8_mm_dynq(*args) == _lib.OK


def test_norm_quant_entry_validates_on_the_host():
    """i8l_add_rmsnorm_quant_mm: its support rule and argument errors, without a launch."""
    L = _lib.lib()
    for m, n, k in ((1, 4096, 2048), (8, 12288, 2048), (8, 6144, 4096), (3, 28672, 4096)):
        assert L.i8l_add_rmsnorm_quant_mm_supported(m, n, k, None) == _lib.OK, (m, n, k)
    assert L.i8l_add_rmsnorm_quant_mm_supported(9, 4096, 2048, None) == _lib.UNSUPPORTED
    assert "up to 8 tokens" in _lib.last_error()
    assert L.i8l_add_rmsnorm_quant_mm_supported(4, 2048, 6144, None) == _lib.UNSUPPORTED
    c = _lib.CConfig(16, 16, 256, 8, 4, 2)
    assert L.i8l_add_rmsnorm_quant_mm_supported(4, 4096, 2048, ctypes.byref(c)) == _lib.OK
    c = _lib.CConfig(16, 16, 256, 8, 4, 2)                     # K must be warps * bk
    assert L.i8l_add_rmsnorm_quant_mm_supported(4, 4096, 4096, ctypes.byref(c)) == _lib.UNSUPPORTED
    c = _lib.CConfig(16, 16, 512, 4, 3, 1)                     # not the persistent form
    assert L.i8l_add_rmsnorm_quant_mm_supported(4, 4096, 2048, ctypes.byref(c)) == _lib.UNSUPPORTED
    c = _lib.CConfig(16, 16, 512, 8, 4, 4)                     # four a CU: beyond the LDS
    assert L.i8l_add_rmsnorm_quant_mm_supported(4, 4096, 4096, ctypes.byref(c)) == _lib.UNSUPPORTED
    # argument errors come back before anything launches (no pointer is touched)
    args = [None, None, None, 1e-6, _lib.BF16, 1, 0, None, None, 1, 2048, None, 7, None, 0,
            None, 4096, _lib.BF16, None, 4, 4096, 2048, None, None]
    assert L.i8l_add_rmsnorm_quant_mm(*args) == _lib.INVALID_ARG and "scale_b" in _lib.last_error()
    args[12] = 4096
    args[4] = _lib.F32                                          # fp32 activations
    assert L.i8l_add_rmsnorm_quant_mm(*args) == _lib.UNSUPPORTED
    args[4], args[7] = _lib.BF16, 1                             # residual_out without residual
    assert L.i8l_add_rmsnorm_quant_mm(*args) == _lib.INVALID_ARG
    args[7] = None
    assert L.i8l_add_rmsnorm_quant_mm(*args) == _lib.INVALID_ARG   # x is NULL
    assert "required" in _lib.last_error()
    args[0], args[2], args[6] = 16, 16, 3                       # an epilogue mode not defined
    assert L.i8l_add_rmsnorm_quant_mm(*args) == _lib.INVALID_ARG
    args[6] = 1                                                 # SiLU epilogue without residual
    assert L.i8l_add_rmsnorm_quant_mm(*args) == _lib.UNSUPPORTED and "SiLU" in _lib.last_error()


def test_silu_epilogue_entry_validates_on_the_host():
    L = _lib.lib()
    assert L.i8l_w8a8_mm_silu_mul_supported(8, 12288, 2048, None) == _lib.OK
    assert L.i8l_w8a8_mm_silu_mul_supported(16, 28672, 4096, None) == _lib.OK
    assert L.i8l_w8a8_mm_silu_mul_supported(17, 12288, 2048, None) == _lib.UNSUPPORTED
    c = _lib.CConfig(16, 32, 128, 16, 4, 1)                      # two fragments: not taken
    assert L.i8l_w8a8_mm_silu_mul_supported(4, 12288, 2048, ctypes.byref(c)) == _lib.UNSUPPORTED
    c = _lib.CConfig(16, 8, 512, 4, 4, 4)
    assert L.i8l_w8a8_mm_silu_mul_supported(4, 12288, 2048, ctypes.byref(c)) == _lib.OK
    # argument errors come back before anything launches (no pointer is touched)
    args = [None, 2048, None, 1, 2048, None, 4, None, 1, None, 0, None, 6144, 0, 4, 12288,
            2048, None, None]                                   # per-tensor scale_b
    assert L.i8l_w8a8_mm_silu_mul(*args) == _lib.INVALID_ARG
    args[8], args[10] = 12288, _lib.F32                         # an fp32 bias
    assert L.i8l_w8a8_mm_silu_mul(*args) == _lib.UNSUPPORTED
    args[10], args[14], args[6] = 0, 0, 1                       # M == 0: nothing to do
    assert L.i8l_w8a8_mm_silu_mul(*args) == _lib.OK


def test_situ_tune_writes_only_kept_sets_as_table_rows():
    """The in-situ tuner's table rows (reference bench/situ_tune.py:241-246): nothing for a
    set that was not kept; for a kept set, one row per linear at the batch, each with its
    configuration and the confirmed stand-in time."""
    from dataclasses import asdict

    from int8_linear import situ_tune
    from int8_linear.standin import SHAPES

    cfg = asdict(Config(16, 16, 256, 8, 4, 2))
    entry = {"batch": 8, "chosen": {name: cfg for name in SHAPES}, "kept": False,
             "confirm_us": {"start": 31.0, "chosen": 30.9}}
    assert situ_tune.table_rows(entry) == {}
    entry["kept"] = True
    rows = situ_tune.table_rows(entry)
    assert set(rows) == {f"{k}x{n}" for k, n in SHAPES.values()}
    for r in rows.values():
        assert r == {"8": {"config": cfg, "stand_in_us": 30.9}}
    assert 0 < situ_tune.ACCEPT < 0.05


def test_situ_tune_tunes_the_kernel_each_linear_runs():
    """The in-situ tuner tunes each linear in the kernel the stand-in runs for it: w8a8_mm,
    the norm-folded projection, gate_up with the SiLU epilogue, or nothing where a folded
    quantizer's own tile runs (DecoderStandIn.forward); and a kept set writes table rows for
    its w8a8_mm linears only."""
    from dataclasses import asdict

    from int8_linear import situ_tune
    from int8_linear.standin import SHAPES

    def kinds(*flags):
        return {name: situ_tune.kernel_of(name, *flags) for name in SHAPES}

    # (fused_norm, fused_silu, fused_down, fused_o, quant_down)
    assert kinds(True, False, True, True, False) == {      # one token
        "qkv_proj": "norm", "o_proj": None, "gate_up_proj": "norm", "down_proj": None}
    assert kinds(True, True, False, True, True) == {       # 2-5 tokens
        "qkv_proj": "norm", "o_proj": None, "gate_up_proj": "norm", "down_proj": None}
    assert kinds(False, True, False, True, True) == {      # 6-8 tokens
        "qkv_proj": "mm", "o_proj": None, "gate_up_proj": "silu", "down_proj": None}
    assert kinds(False, True, False, True, False) == {     # SiLU epilogue, down unfused
        "qkv_proj": "mm", "o_proj": None, "gate_up_proj": "silu", "down_proj": "mm"}
    assert set(kinds(False, False, False, False, False).values()) == {"mm"}
    cfg = asdict(Config(16, 16, 256, 8, 4, 2))
    entry = {"batch": 8, "kernels": kinds(False, True, False, True, True), "kept": True,
             "chosen": {name: cfg for name in SHAPES},
             "confirm_us": {"start": 31.0, "chosen": 30.5}}
    assert set(situ_tune.table_rows(entry)) == {"2048x4096"}


def test_tuner_merge_updates_rows_and_keeps_the_rest(tmp_path):
    """tune.merge writes {"KxN": {M: row}} under the device key, replacing the buckets it is
    given and keeping every other bucket, shape and device (reference merge:
    bench/bench_linear.py:385-389)."""
    import json

    from int8_linear import tune
    path = tmp_path / "table.json"
    row = lambda us: {"config": {"bm": 16, "bn": 16, "bk": 256, "warps": 4, "stages": 3,
                                 "group_m": 1}, "graph_us": us, "default_us": us}
    path.write_text(json.dumps({"gfx950": {"2048x4096": {"1": row(4.0), "16": row(5.0)},
                                           "6144x2048": {"1": row(6.0)}},
                                "other": {"2048x4096": {"1": row(9.0)}}}))
    tune.merge({"2048x4096": {"16": row(4.5), "32": row(5.5)}, "4096x4096": {"1": row(7.0)}},
               "gfx950", path=path)
    t = json.loads(path.read_text())
    assert path.read_text().endswith("\n")
    dev = t["gfx950"]
    assert dev["2048x4096"]["1"]["graph_us"] == 4.0          # untouched bucket
    assert dev["2048x4096"]["16"]["graph_us"] == 4.5         # replaced
    assert dev["2048x4096"]["32"]["graph_us"] == 5.5         # added
    assert dev["6144x2048"] == {"1": row(6.0)} and dev["4096x4096"] == {"1": row(7.0)}
    assert t["other"] == {"2048x4096": {"1": row(9.0)}}     # another device untouched


def test_tuner_candidate_sets(monkeypatch):
    """Refine times the current table entry first, then only stage-3 and split tiles, all of
    them built for the shape; the split is offered only where the unsplit tiles are few;
    `capture` is vLLM's graph batch sizes."""
    import json

    from int8_linear import tune
    from int8_linear.kernel import tuned_config
    shipped = json.loads(kernel.TUNED_PATH.read_text())["gfx950"]
    monkeypatch.setattr(kernel.torch.cuda, "current_device", lambda: 0)
    monkeypatch.setattr(kernel, "_device_table", lambda dev: shipped)
    m, k, n = 64, 14336, 4096                                # Llama-3-8B down_proj
    assert tuned_config(m, n, k) is not None
    ref = tune.refine_candidates(m, k, n)
    assert ref[0] == (tuned_config(m, n, k) or default_config(m, n, k))
    assert len(set(ref)) == len(ref)
    split = lambda c: c.stages == 5 and c.bn <= 64          # wider stage-5 tiles: prefill rings
    assert all(c.stages in (3, 5) and c.bn <= 64 for c in ref[1:]) and any(map(split, ref))
    assert all(kernel.supported(m, n, k, c) for c in ref)
    full = tune.candidate_configs(m, k, n)
    assert set(ref[1:]) <= set(full) and len(full) > len(ref)
    for mm, kk, nn in ((m, k, n), (16, 4096, 28672), (1, 2048, 12288), (128, 4096, 28672)):
        for c in filter(split, tune.candidate_configs(mm, kk, nn)):
            tiles = -(-mm // c.bm) * (nn // c.bn)
            assert tiles < 512 and tiles * c.group_m <= 1024, (mm, c.name)
    # 128 tokens on Llama-3-8B gate_up: every split tile already has 512 or more tiles
    assert not any(map(split, tune.candidate_configs(128, 4096, 28672)))
    assert tune.parse_ms("capture") == list(tune.CAPTURE_SIZES)
    assert tune.parse_ms("1,2,17") == [1, 2, 17]
