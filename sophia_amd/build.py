"""Build recipe of the HIP library: sophia_amd/csrc/* -> sophia_amd/_lib/libsophia_kda.so.

hipcc for gfx950 only; each translation unit is compiled to an object in
sophia_amd/_build/ and linked into one shared library exporting the C ABI of
include/sophia_kda.h and include/sophia_decoder.h.  Run ``python -m sophia_amd.build``.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC_DIR = os.path.join(HERE, "csrc")
BUILD_DIR = os.path.join(HERE, "_build")
LIB_DIR = os.path.join(HERE, "_lib")
LIB_NAME = "libsophia_kda.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)
ARCH = "gfx950"
SOURCES = ("errors.cpp", "short_conv.hip", "kda_decode.hip", "kda_chunk.hip", "decoder_ops.hip", "kda_bwd.hip")

# Packed-fp32 VALU ops are switched off for all device code.
COMMON_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm toolchain required to build sophia_amd)")
    return path


def _compile(src: str, extra: list[str], verbose: bool) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *extra, "-c", os.path.join(SRC_DIR, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
    noise = "'-packed-fp32-ops' is not a recognized feature"
    msgs = [ln for ln in (res.stderr or "").splitlines() if ln.strip() and noise not in ln]
    if msgs and verbose:
        print("\n".join(msgs), file=sys.stderr)
    return obj


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    extra = list(extra_flags or [])
    with cf.ThreadPoolExecutor(max_workers=min(4, len(SOURCES))) as ex:
        objs = list(ex.map(lambda s: _compile(s, extra, verbose), SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
