"""Build libdsa_mli.so (the HIP kernels + C ABI) for gfx950, in-tree.

Run as ``python -m lagged_indexer_dsa_amd._build`` or call :func:`build`.
hipcc cross-compiles without a GPU; the library lands next to this file in
``_lib/`` so it travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT_DIR = PKG_DIR.parent            # dsa-multi-layer-indexer_amd/
REPO_DIR = ROOT_DIR.parent
CSRC = ROOT_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
LIB_DIR = PKG_DIR / "_lib"
LIB_PATH = LIB_DIR / "libdsa_mli.so"
SOURCES = ["libdsa_mli.hip"]
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the DSA HIP library cannot be built")


def build(verbose: bool = False, out: Path | None = None, phase_stamps: bool = False) -> Path:
    """Compile every HIP source into LIB_PATH, or `out` (always recompiles).
    phase_stamps: compile in the per-phase timestamps (profiling builds only;
    they cost a memory round trip per phase)."""
    target = Path(out) if out else LIB_PATH
    target.parent.mkdir(parents=True, exist_ok=True)
    tmp = target.with_suffix(".so.tmp")
    cmd = [
        hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
        # packed fp32 VALU ops are disabled on purpose (they have produced
        # silent wrong results on this hardware pool)
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{INCLUDE}", f"-I{CSRC}",
        *(["-DDSA_PHASE_STAMPS"] if phase_stamps else []),
        *[str(CSRC / s) for s in SOURCES],
        "-o", str(tmp),
    ]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-4000:]}")
    if verbose and res.stderr:
        print(res.stderr, file=sys.stderr)
    os.replace(tmp, target)
    return target


if __name__ == "__main__":
    print(build(verbose=True))
