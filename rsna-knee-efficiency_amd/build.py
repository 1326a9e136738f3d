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
    """Compiles every `.hip` source of the library to an object in parallel (one hipcc per file), then
    links them into `out` (default: the package's libd8s_hip.so), replacing it atomically."""
    out = Path(out or hip.LIB_PATH)
    tag = f"{os.getpid()}"
    common = [*HIPCC_FLAGS, f"-I{hip.HEADER.parent}", f'-DD8S_SRC_HASH="{hip.source_sha()}"']
    srcs = [f for f in hip.SOURCES if f.suffix == ".hip"]
    objs = [out.with_name(f"{f.stem}.{tag}.o") for f in srcs]
    procs = [subprocess.Popen([hipcc(), *common, "-c", str(f), "-o", str(o)], stdout=subprocess.PIPE,
                              stderr=subprocess.PIPE, text=True) for f, o in zip(srcs, objs)]
    errs = []
    for f, pr in zip(srcs, procs):
        _, err = pr.communicate()
        if pr.returncode != 0:
            errs.append(f"{f.name}: hipcc failed ({pr.returncode}):\n{err[-4000:]}")
        elif verbose and err:
            print(err[-2000:])
    try:
        if errs:
            raise RuntimeError("\n".join(errs))
        tmp = out.with_suffix(f".so.tmp{tag}")
        res = subprocess.run([hipcc(), *HIPCC_FLAGS, *(str(o) for o in objs), "-o", str(tmp)],
                             capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link failed ({res.returncode}):\n{res.stderr[-4000:]}")
        os.replace(tmp, out)
    finally:
        for o in objs:
            o.unlink(missing_ok=True)
    return out
