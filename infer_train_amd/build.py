"""Builds libit_kv.so for gfx950 with make (infer_train_amd/csrc/Makefile)."""
from __future__ import annotations

import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))


def build_library(jobs: int = 8) -> str:
    subprocess.run(["make", "-s", "-C", os.path.join(PKG, "csrc"), f"-j{jobs}"], check=True, stdout=sys.stdout,
                   stderr=sys.stderr)
    return os.path.join(PKG, "libit_kv.so")


if __name__ == "__main__":
    build_library()
