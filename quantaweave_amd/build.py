"""Build the gfx950 C-ABI library ``libqwmoe.so`` in-tree with hipcc.

Every ``csrc/*.hip`` file is compiled for gfx950 only and linked into one
shared library next to this file.  Object files go to ``_build/``.  The build
always recompiles (it is the "does it build" check); loading code never builds.

    python -m quantaweave_amd.build
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libqwmoe.so"
ARCH = "gfx950"

# Files whose arithmetic must be the plain IEEE sequence written in the source.
NO_CONTRACT = {"qw_route.hip"}
# Files whose matrix-core results feed VALU work right away: keep them in
# VGPRs (the AGPR form costs a copy per result register).
MFMA_VGPR = {"qw_ffn_gemv.hip"}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the gfx950 library cannot be built")


def compile_flags(name: str) -> list[str]:
    flags = [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
        "-I", str(ROOT / "include"), "-I", str(CSRC),
        # no packed fp32 instructions in any kernel
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall", "-Wno-unused-function", "-Wno-unknown-pragmas",
    ]
    if name in NO_CONTRACT:
        flags.append("-ffp-contract=off")
    if name in MFMA_VGPR:
        flags += ["-mllvm", "-amdgpu-mfma-vgpr-form"]
    return flags


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *compile_flags(src.name), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources")
    return LIB


if __name__ == "__main__":
    build()
