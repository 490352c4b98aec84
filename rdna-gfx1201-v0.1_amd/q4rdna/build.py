"""In-tree build of libq4rdna_gfx950.so (hipcc, --offload-arch=gfx950)."""
from __future__ import annotations

import os
import subprocess

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def build(force: bool = True, jobs: int = 4) -> str:
    """Compile the HIP kernels and the host runtime; returns the library path."""
    cmd = ["make", "-C", PKG_ROOT, f"-j{jobs}"]
    if force:
        cmd.append("-B")
    subprocess.run(cmd, check=True)
    return os.path.join(PKG_ROOT, "q4rdna", "libq4rdna_gfx950.so")
