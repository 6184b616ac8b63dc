"""Compile the C oracle (test infrastructure) into oracle/_build/libjq_oracle.so."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent


def build(verbose: bool = False) -> Path:
    out = HERE / "_build"
    out.mkdir(exist_ok=True)
    so = out / "libjq_oracle.so"
    cmd = ["gcc", "-O2", "-fPIC", "-std=gnu11", "-fopenmp", "-shared",
           "-o", str(so), str(HERE / "jq_oracle.c"), "-lm"]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    return so


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
