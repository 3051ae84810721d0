"""Build the C oracle ``oracle/liboracle_combine.so`` with gcc (test infrastructure only).

The reference itself is Python + Triton (no C/C++ sources), so there is no ``oracle/_ref`` build;
this compiles the oracle's own C restatement.  ``-ffp-contract=off``: products are rounded to fp32
before they are added, like torch's CPU ``t * w`` followed by ``index_add_``.
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "combine_ref.c"
LIB = HERE / "liboracle_combine.so"


def build() -> Path:
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("oracle: no C compiler found")
    tmp = LIB.with_suffix(".so.tmp")
    subprocess.run(
        [cc, "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
         "-Wall", str(SRC), "-o", str(tmp), "-lm"],
        check=True,
    )
    tmp.replace(LIB)
    return LIB


if __name__ == "__main__":
    print(build())
