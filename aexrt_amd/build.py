"""Builds libaexrt_hip.so in-tree with hipcc for gfx950 (no JIT cache)."""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"


def build(force: bool = True, jobs: int | None = None) -> Path:
    """Compile every HIP/C++ source of the library; returns the .so path."""
    jobs = jobs or min(16, os.cpu_count() or 4)
    cmd = ["make", "-C", str(CSRC), f"-j{jobs}"]
    if force:
        cmd.insert(1, "-B")
    subprocess.run(cmd, check=True)
    return PKG / "libaexrt_hip.so"


if __name__ == "__main__":
    print(build())
