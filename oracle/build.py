"""Build recipe for the C oracle (oracle/kda_ref.c -> oracle/_lib/liboracle_kda.so).

Test infrastructure only.  Plain gcc with OpenMP; no reference sources are
compiled (the reference is Python and its CPU path is restated, not built).
"""

from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "_lib")
LIB_PATH = os.path.join(LIB_DIR, "liboracle_kda.so")


def build(verbose: bool = False) -> str:
    os.makedirs(LIB_DIR, exist_ok=True)
    src = os.path.join(HERE, "kda_ref.c")
    tmp = LIB_PATH + ".tmp"
    cmd = ["gcc", "-O3", "-march=x86-64-v2", "-fopenmp", "-fPIC", "-shared", "-std=c11",
           src, "-o", tmp, "-lm"]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
