"""Builds libdecide_hip.so for gfx950 with the Makefile in csrc/."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))


def build(force: bool = True, jobs: int = 8) -> str:
    cmd = ["make", "-C", os.path.join(HERE, "csrc"), f"-j{jobs}"]
    if force:
        cmd.insert(1, "-B")
    subprocess.run(cmd, check=True)
    return os.path.join(HERE, "libdecide_hip.so")


if __name__ == "__main__":
    print(build())
