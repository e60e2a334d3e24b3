"""Build the gfx950 C-ABI library libint8_linear_amd.so from csrc/*.hip, in-tree, the
host-only C++ binding _i8l_fast over it (csrc/i8l_torch.cpp), and the measurement probes
bench.py times beside it (probes/i8l_floors.hip -> probes/libi8l_floors.so, not part of the
W8A8 C ABI).

    python int8-linear_amd/build_lib.py

Each HIP source is compiled by hipcc for gfx950 only, in parallel, into _build/, then linked
into int8_linear/libint8_linear_amd.so next to the Python package that loads it.  The binding
is compiled by g++ against torch's headers and links the library through $ORIGIN.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "int8_linear" / "libint8_linear_amd.so"
PROBES_SRC = HERE / "probes" / "i8l_floors.hip"
PROBES_LIB = HERE / "probes" / "libi8l_floors.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")

# -ffp-contract=off: the epilogue and quantizer arithmetic is the sequence of IEEE ops
#   written, which the CPU oracle reproduces bit for bit.
# -packed-fp32-ops off: packed fp32 VALU forms are not generated.
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every csrc/*.hip for gfx950 and link the shared library, then the binding;
    returns the library's path."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    with ThreadPoolExecutor(max_workers=min(8, len(sources) + 2)) as ex:
        binding = ex.submit(_compile_binding)
        probes = ex.submit(_build_probes)
        objs = list(ex.map(_compile, sources))
        binding_obj = binding.result()
        probes.result()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    fast = _link_binding(binding_obj)
    if verbose:
        print(f"built {fast}", file=sys.stderr)
    return LIB


def _build_probes() -> Path:
    """The floor probes (empty launch, cold reads, MFMA loops) as their own library."""
    tmp = PROBES_LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, *FLAGS, "-shared", str(PROBES_SRC), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {PROBES_SRC.name}:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, PROBES_LIB)
    return PROBES_LIB


def _compile_binding() -> Path:
    """Compile the C++ eager binding (host code only, against torch's headers)."""
    import sysconfig

    import torch
    from torch.utils.cpp_extension import include_paths

    obj = BUILD / "i8l_torch.o"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [CXX, "-O2", "-std=c++17", "-fPIC", "-D__HIP_PLATFORM_AMD__",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_EXTENSION_NAME=_i8l_fast",
           "-DTORCH_API_INCLUDE_EXTENSION_H", *[f"-I{p}" for p in include_paths()],
           "-I/opt/rocm/include", f"-I{sysconfig.get_paths()['include']}",
           "-c", str(CSRC / "i8l_torch.cpp"), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"g++ failed on i8l_torch.cpp:\n{r.stdout}\n{r.stderr}")
    return obj


def _link_binding(obj: Path) -> Path:
    """Link the binding against torch and the library (found through $ORIGIN at run time)."""
    import sysconfig

    from torch.utils.cpp_extension import library_paths

    out = LIB.with_name("_i8l_fast" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out.with_suffix(".tmp")
    cmd = [CXX, "-shared", str(obj), *[f"-L{p}" for p in library_paths()], "-lc10",
           "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python", f"-L{LIB.parent}",
           "-lint8_linear_amd", "-Wl,-rpath,$ORIGIN", "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"binding link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    build(verbose=True)
