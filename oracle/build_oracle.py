"""Build recipe of the CPU oracle (test infrastructure): oracle/_build/liboracle.so.

    python oracle/build_oracle.py

gcc, -ffp-contract=off and no fast-math, so the oracle's float arithmetic is exactly the
IEEE operations written in i8l_oracle.c.  The reference (AshrithaG/int8-linear) is Python
and Triton only, so there is no reference C source to build into oracle/_ref.
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "i8l_oracle.c"
OUT = HERE / "_build" / "liboracle.so"
FLAGS = ["-O3", "-march=x86-64-v3", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
         "-fno-fast-math", "-std=c11", "-Wall"]


def build(verbose: bool = False) -> Path:
    OUT.parent.mkdir(exist_ok=True)
    tmp = OUT.with_suffix(".so.tmp")
    r = subprocess.run(["gcc", *FLAGS, str(SRC), "-o", str(tmp), "-lm"],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stdout}\n{r.stderr}")
    tmp.replace(OUT)
    if verbose:
        print(f"built {OUT}", file=sys.stderr)
    return OUT


if __name__ == "__main__":
    build(verbose=True)
