"""Builds the native pieces in-tree.

``build()`` compiles libarthip.so (hipcc, gfx950) into ``arthip_amd/_build``.
The GPU box runs what is built here; nothing compiles at import time.
"""

from __future__ import annotations

import os
import subprocess
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"


def build(jobs: int | None = None, verbose: bool = False, force: bool = False) -> Path:
    """force: recompile every source even when the library is up to date."""
    jobs = jobs or min(8, os.cpu_count() or 4)
    cmd = ["make", "-C", str(CSRC), f"-j{jobs}"] + (["-B"] if force else [])
    if not verbose:
        cmd.append("-s")
    subprocess.run(cmd, check=True)
    lib = PKG_DIR / "_build" / "libarthip.so"
    if not lib.exists():
        raise RuntimeError(f"build finished but {lib} is missing")
    return lib


def clean() -> None:
    subprocess.run(["make", "-C", str(CSRC), "-s", "clean"], check=True)


if __name__ == "__main__":
    print(build(verbose=True))
