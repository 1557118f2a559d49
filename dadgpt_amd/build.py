"""Build step for the HIP library (used by __graft_entry__.build and the tests' setup)."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")


def build(force: bool = True, jobs: int = 8) -> str:
    """Compile every HIP source for gfx950 into lib/libdadgpt_attn.so; returns its path."""
    cmd = ["make", "-C", CSRC, f"-j{jobs}"]
    if force:
        cmd.append("-B")
    subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL)
    path = os.path.join(HERE, "lib", "libdadgpt_attn.so")
    if not os.path.exists(path):
        raise RuntimeError(f"build finished but {path} is missing")
    return path
