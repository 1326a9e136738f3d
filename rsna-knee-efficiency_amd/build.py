"""Builds libd8s_hip.so for gfx950 with hipcc (no JIT, no torch extension: a plain C-ABI library).

    python -c "import __graft_entry__ as g; g.build()"

The source hash (kernel source + header) is compiled into the library (`d8s_version()`), the role of
the reference's `kernels_sha` (`src/knee/dense8s.py:781-783`).
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

from . import hip

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-shared", "-fPIC",
    # no contraction into fused operations other than the explicit fma of the kernels
    "-ffp-contract=off",
    # no packed fp32 arithmetic
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # `#pragma unroll` loops unrolled in full also when large (the fused kernels' interleaved K loops:
    # a partly unrolled one computes its LDS addresses at run time)
    "-mllvm", "-pragma-unroll-threshold=100000",
]


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise FileNotFoundError("hipcc not found")


def build_library(out: Path | None = None, verbose: bool = False) -> Path:
    out = Path(out or hip.LIB_PATH)
    tmp = out.with_suffix(f".so.tmp{os.getpid()}")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{hip.HEADER.parent}", f'-DD8S_SRC_HASH="{hip.source_sha()}"',
           *(str(f) for f in hip.SOURCES if f.suffix == ".hip"), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-4000:]}")
    if verbose and res.stderr:
        print(res.stderr[-2000:])
    os.replace(tmp, out)
    return out
