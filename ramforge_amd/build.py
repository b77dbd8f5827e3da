"""Build libramforge_hip.so in-tree (hipcc, gfx950) with csrc/Makefile."""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")


def build(jobs: int = 8, arch: str = "gfx950", force: bool = False) -> str:
    env = dict(os.environ)
    env.setdefault("HIPCC", "/opt/rocm/bin/hipcc")
    if force:
        subprocess.run(["make", "-C", CSRC, "clean", "-s"], check=True, env=env)
    subprocess.run(["make", "-C", CSRC, f"-j{jobs}", f"ARCH={arch}"], check=True, env=env)
    return os.path.join(HERE, "libramforge_hip.so")


if __name__ == "__main__":
    print(build(force="--force" in sys.argv))
