"""Compile ``libkivi_hip.so`` (all HIP sources under csrc/) for gfx950.

Run as ``python -m intel_kivi_hybrid_amd.build`` or via
``__graft_entry__.build()``.  The library is written next to this file so that
it ships with the source tree.
"""

from __future__ import annotations

import glob
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libkivi_hip.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
ARCH = os.environ.get("KIVI_OFFLOAD_ARCH", "gfx950")

# IEEE fp32 semantics are part of the parity contract: no contraction of
# q*scale+zero, correctly rounded division, fp32 denormals kept.  Packed-FP32
# instructions are disabled for the whole library.
HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC",
    f"--offload-arch={ARCH}",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


def sources() -> list:
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def _run(cmd: list, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in proc.stdout.splitlines()
                    if "packed-fp32-ops" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out)


def build(verbose: bool = False, jobs: int = 0) -> str:
    """Always recompiles; returns the library path.  Each source compiles to
    an object in parallel (the attention kernel is split into one translation
    unit per Hq/Hkv ratio), then the objects link into the shared library."""
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    srcs = sources()
    objs = [os.path.join(objdir, os.path.basename(s)[:-4] + ".o") for s in srcs]
    jobs = jobs or max(1, min(len(srcs), os.cpu_count() or 4, 16))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        for f in [pool.submit(_run, [hipcc()] + HIPCC_FLAGS + ["-c", s, "-o", o], verbose)
                  for s, o in zip(srcs, objs)]:
            f.result()
    tmp = LIB_PATH + ".tmp"
    _run([hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}"] + objs + ["-o", tmp], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
