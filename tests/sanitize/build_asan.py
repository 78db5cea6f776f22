"""Builds libmoeinfra_hip_asan.so: the same HIP sources as the product library, with the
host code instrumented by AddressSanitizer and UndefinedBehaviorSanitizer (the device code
is built as usual; GPU sanitizers are not used).  CPU tests load it in a subprocess with the
clang ASan runtime preloaded and drive the C ABI's argument checking through it.

Usage: python tests/sanitize/build_asan.py [OUT_DIR]   (default: _build/asan)
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
CSRC = os.path.join(REPO, "moeinfra_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"
SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
       "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer"]
FLAGS = ["--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fPIC", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-unused-function"]


def asan_runtime() -> str:
    """The clang ASan runtime matching hipcc's host compiler."""
    hits = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not hits:
        raise RuntimeError("clang ASan runtime not found under /opt/rocm/llvm")
    return hits[-1]


def build(out_dir: str | None = None) -> str:
    out_dir = out_dir or os.path.join(REPO, "_build", "asan")
    os.makedirs(out_dir, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))

    def compile_one(src):
        obj = os.path.join(out_dir, os.path.basename(src) + ".o")
        cmd = [HIPCC, *FLAGS, *SAN, "-c", src, "-o", obj]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src}:\n{proc.stderr}")
        return obj

    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        objs = list(pool.map(compile_one, sources))
    lib = os.path.join(out_dir, "libmoeinfra_hip_asan.so")
    proc = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", lib, *objs],
                          capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    return lib


if __name__ == "__main__":
    print(build(sys.argv[1] if len(sys.argv) > 1 else None))
