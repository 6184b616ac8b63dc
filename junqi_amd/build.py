"""Compile the HIP library junqi_amd/_build/libjunqi_amd.so for gfx950 (hipcc)."""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SOURCES = ["csrc/jq_lib.hip", "csrc/jq_topology.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    # packed fp32 forms stay off: every float here is plain scalar arithmetic
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def build(verbose: bool = False, extra: list[str] | None = None) -> Path:
    out = HERE / "_build"
    out.mkdir(exist_ok=True)
    so = out / "libjunqi_amd.so"
    tmp = out / "libjunqi_amd.so.tmp"
    cmd = [HIPCC, *FLAGS, *(extra or []), "-I", str(HERE.parent / "include"),
           *[str(HERE / s) for s in SOURCES], "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, so)
    return so


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
