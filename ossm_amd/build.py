"""Build libossm_scan.so (gfx950) in-tree with hipcc.

    python -m ossm_amd.build          # from the repository root

Every source is compiled for gfx950 only.  Packed-FP32 instruction selection
is disabled (-target-feature -packed-fp32-ops): the scans are memory-bound and
packed FP32 forms are not trusted on this pool.
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
LIBDIR = PKG / "_lib"
OBJDIR = PKG / "_build"
LIB = LIBDIR / "libossm_scan.so"

SOURCES = ["runtime.cpp", "oscillator_scan.hip", "selective_scan.hip", "sdlinoss_scan.hip",
           "diag_scan.hip", "dlinoss_layer.hip", "mamba_conv.hip", "scan_f64.hip",
           "shard_scan.hip"]
# standalone measurement program (not linked into the library)
ISSUE_RATE_SRC = "valu_issue_rate.hip"
ISSUE_RATE = LIBDIR / "valu_issue_rate"
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; set HIPCC")


def _flags() -> list[str]:
    return [
        "-O3",
        "-std=c++17",
        "-fPIC",
        f"--offload-arch={ARCH}",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-result",
        f"-I{ROOT / 'include'}",
    ]


def _compile(src: str) -> Path:
    OBJDIR.mkdir(parents=True, exist_ok=True)
    obj = OBJDIR / (Path(src).stem + ".o")
    cmd = [hipcc(), *_flags(), "-x", "hip", "-c", str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    if res.stderr.strip():
        sys.stderr.write(res.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every source and link the shared library; returns its path."""
    sources = [s for s in SOURCES if (CSRC / s).exists()]
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        objs = list(pool.map(_compile, sources))
    LIBDIR.mkdir(parents=True, exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    cmd = [hipcc(), *_flags(), "-x", "hip", str(CSRC / ISSUE_RATE_SRC), "-o", str(ISSUE_RATE)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {ISSUE_RATE_SRC}:\n{res.stderr}")
    if verbose:
        print(f"built {LIB.relative_to(ROOT)}, {ISSUE_RATE.relative_to(ROOT)}")
    return LIB


if __name__ == "__main__":
    build()
