"""Build the C restatement ``pa_oracle.c`` into ``oracle/_build/libpa_oracle.so``.

Test infrastructure only (see ``oracle/__init__.py``). The reference's own
kernels cannot be compiled here (they need the un-vendored pto-isa headers and
g++-15), so there is no ``oracle/_ref`` build.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT_DIR = HERE / "_build"
LIB = OUT_DIR / "libpa_oracle.so"


def build(verbose: bool = False) -> Path:
    OUT_DIR.mkdir(exist_ok=True)
    cc = os.environ.get("CC") or shutil.which("gcc") or "cc"
    tmp = LIB.with_suffix(".so.tmp")
    # x86-64-v3 (AVX2/FMA) so the library built here also runs on the GPU hosts' CPUs.
    cmd = [cc, "-O3", "-march=x86-64-v3", "-fPIC", "-shared", "-pthread", "-std=c11",
           str(HERE / "pa_oracle.c"), "-o", str(tmp), "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
