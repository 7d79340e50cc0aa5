"""Build libsimpler_hip.so (gfx950) in-tree with hipcc.

``python -m simpler_amd.build`` or ``simpler_amd.build.build()``. The library is
written to ``simpler_amd/lib/libsimpler_hip.so`` so that it travels with the
source tree; nothing is installed.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB_DIR = PKG / "lib"
LIB_PATH = LIB_DIR / "libsimpler_hip.so"
SOURCES = [
    CSRC / "pa_decode.hip",
    CSRC / "pa_kernels_gqa_bf16.hip",
    CSRC / "pa_kernels_gqa_f16.hip",
    CSRC / "pa_kernels_gqa_bf16_append.hip",
    CSRC / "pa_kernels_gqa_f16_append.hip",
    CSRC / "pa_kernels_fp8.hip",
    CSRC / "pa_kernels_mla.hip",
    CSRC / "pa_kernels_merge.hip",
    CSRC / "kv_cache.hip",
    CSRC / "incore_kernels.hip",
    CSRC / "task_graph.cpp",
    CSRC / "orchestrations.cpp",
    CSRC / "host_runtime.cpp",
]
ARCH = os.environ.get("SIMPLER_HIP_ARCH", "gfx950")
BUILD_DIR = ROOT / "_build"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def compile_flags(extra_flags: list[str] | None = None) -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-fvisibility=hidden",
        # packed fp32 ops (v_pk_*_f32) are disabled for all device code
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # MFMA accumulators in VGPRs: the kernels rescale them with VALU ops
        # every KV block, which AGPR accumulators would route through
        # v_accvgpr moves (measured 10% on the MLA kernel, neutral elsewhere)
        "-mllvm", "-amdgpu-mfma-vgpr-form=1",
        f"-I{ROOT / 'include'}",
        "-Wno-unused-command-line-argument",
        *(extra_flags or []),
    ]


_NOISE = "is not a recognized feature for this target"


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in res.stderr.splitlines() if _NOISE not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False, extra_flags: list[str] | None = None, jobs: int | None = None) -> Path:
    """Compile every source to an object in _build/ (in parallel), then link
    simpler_amd/lib/libsimpler_hip.so."""
    LIB_DIR.mkdir(exist_ok=True)
    BUILD_DIR.mkdir(exist_ok=True)
    flags = compile_flags(extra_flags)
    objs = [BUILD_DIR / (src.name + ".o") for src in SOURCES]
    jobs = jobs or min(len(SOURCES), max(1, (os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        futs = [pool.submit(_run, [hipcc(), *flags, "-c", str(src), "-o", str(obj)], verbose)
                for src, obj in zip(SOURCES, objs)]
        for f in futs:
            f.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *[str(o) for o in objs], "-o", str(tmp)], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def build_code_object(src: Path | str, out: Path | str, verbose: bool = False,
                      extra_flags: list[str] | None = None) -> Path:
    """Compile one ``.hip`` file to a gfx950 code object (``hipcc --genco``) for
    ``simpler_hip_tg_register_kernel``: kernels declared ``extern "C"
    __global__`` taking one ``SimplerHipKernelArgs``."""
    src, out = Path(src), Path(out)
    out.parent.mkdir(parents=True, exist_ok=True)
    tmp = out.with_name(out.name + ".tmp")
    _run([hipcc(), "--genco", f"--offload-arch={ARCH}", "-O3", "-std=c++17",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", f"-I{ROOT / 'include'}",
          "-Wno-unused-command-line-argument", *(extra_flags or []), str(src), "-o", str(tmp)], verbose)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
