"""Build libsas.so (HIP kernels + C++ scheduler) for gfx950, in-tree.

    python -m dsv4_amd.build

The library lands next to this file (dsv4_amd/libsas.so) so it travels with
the source tree; nothing is installed elsewhere.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libsas.so")
ARCH = os.environ.get("SAS_OFFLOAD_ARCH", "gfx950")

HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # packed fp32 VALU forms are kept out of generated code on this pool
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result", "-Wno-inline-asm",
]
# keep MFMA accumulators in arch VGPRs: with AGPR accumulators the register
# allocator inserts AGPR<->VGPR copies on every loop back-edge
VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
SOURCES = [("sas_fwd.hip", VGPR_FORM), ("sas_bwd.hip", []), ("sas_cache.hip", []), ("sas_sched.hip", []), ("sas_metadata.cpp", []), ("sas_error.cpp", []), ("sas_bench.hip", [])]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libsas.so)")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"libsas build failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False) -> str:
    """Compile every source into dsv4_amd/libsas.so; returns the path."""
    from concurrent.futures import ThreadPoolExecutor
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    objs, cmds = [], []
    for src, extra in SOURCES:
        obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
        cmds.append([hipcc(), *HIP_FLAGS, *extra, "-c", "-o", obj, os.path.join(CSRC, src)])
        objs.append(obj)
    with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        for f in [ex.submit(_run, c, verbose) for c in cmds]:
            f.result()
    tmp = LIB + ".tmp"
    _run([hipcc(), *HIP_FLAGS, "-shared", "-o", tmp, *objs], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
