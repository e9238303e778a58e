"""A build of libsophia_kda.so with AddressSanitizer and UndefinedBehaviorSanitizer
on the host code only (the entry points' argument checks, workspace carving
and launch planning); the device code is compiled as usual (-Xarch_host).  The
library links the clang sanitizer runtime dynamically: load it with that
runtime preloaded, in a process that launches no kernel.  CPU test
infrastructure (tests/test_abi_sanitized.py); never used on a GPU.
"""

from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess

from sophia_amd.build import ARCH, COMMON_FLAGS, SOURCES, SRC_DIR, hipcc

HOST_SANITIZE = ["-O1", "-g", "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                 "-Xarch_host", "-fno-omit-frame-pointer"]


def sanitizer_runtime() -> str:
    """Path of the clang AddressSanitizer runtime that a host-sanitized build needs preloaded."""
    hits = sorted(glob.glob(os.path.join(os.path.dirname(os.path.dirname(hipcc())), "llvm", "lib", "clang", "*",
                                         "lib", "linux", "libclang_rt.asan-x86_64.so")))
    if not hits:
        raise RuntimeError("clang AddressSanitizer runtime not found under the ROCm llvm")
    return hits[-1]


def build_host_sanitized(out_dir: str, verbose: bool = False) -> str:
    """The same library with the host code under ASan/UBSan, in ``out_dir``."""
    os.makedirs(out_dir, exist_ok=True)
    flags = [f for f in COMMON_FLAGS if f != "-O3"] + HOST_SANITIZE

    def one(src: str) -> str:
        obj = os.path.join(out_dir, os.path.basename(src) + ".o")
        cmd = [hipcc(), *flags, "-c", os.path.join(SRC_DIR, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
        return obj

    with cf.ThreadPoolExecutor(max_workers=min(4, len(SOURCES))) as ex:
        objs = list(ex.map(one, SOURCES))
    out = os.path.join(out_dir, "libsophia_kda_host_sanitized.so")
    subprocess.run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Xarch_host",
                    "-fsanitize=address,undefined", "-shared-libasan", *objs, "-o", out], check=True)
    return out


