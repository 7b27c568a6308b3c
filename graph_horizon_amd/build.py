"""In-tree build: gfx950 code objects + libgh_hip.so (graph_horizon_amd/csrc/Makefile)."""
from __future__ import annotations

import os
import subprocess

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)


def build_backend(jobs: int = 8, force: bool = True) -> None:
    """Compile every HIP kernel for gfx950 and the host library (always recompiles when
    force=True, so a stale artifact never passes for a fresh build)."""
    csrc = os.path.join(PKG, "csrc")
    args = ["make", "-C", csrc, f"-j{jobs}"]
    if force:
        args.append("-B")
    subprocess.run(args, check=True)


def build_oracle(jobs: int = 8, force: bool = True) -> bool:
    """Compile the CPU oracle (test infrastructure) when its sources are present."""
    odir = os.path.join(ROOT, "oracle")
    if not os.path.exists(os.path.join(odir, "Makefile")):
        return False
    args = ["make", "-C", odir, f"-j{jobs}"]
    if force:
        args.append("-B")
    subprocess.run(args, check=True)
    return True
