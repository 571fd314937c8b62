"""Build the gfx950 HIP library (in-tree) with hipcc.

    python -m polar_pack_amd.build

Produces ``polar_pack_amd/lib/libpolar_pack.so``.  No torch extension
machinery: the library is a plain C-ABI shared object loaded with ctypes.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
LIB_DIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIB_DIR, "libpolar_pack.so")
OBJ_DIR = os.path.join(LIB_DIR, "obj")
SOURCES = ["capi.hip", "quad.hip", "quad_rows.hip", "quad_mfma.hip", "quad_big.hip", "quad_kn.hip", "dual.hip", "dual_rows.hip", "dual_kn.hip", "dual_mfma.hip", "noalloc.hip"]
ARCH = "gfx950"

# Packed FP32 instructions are disabled for all device code (their results have been
# unreliable on these boards); hipcc's host pass ignores the feature with a warning.
HIPCC_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-Wall", "-Wno-unused-function", "-Wno-unused-parameter"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build polar_pack_amd)")


def _run(cmd, verbose):
    proc = subprocess.run(cmd, cwd=CSRC, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (proc.stderr or "").splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False, jobs: int = 0) -> str:
    """Compile every source to an object (in parallel), then link the shared library."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    objs = [os.path.join(OBJ_DIR, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    cmds = [[hipcc(), *compile_flags, "-c", os.path.join(CSRC, s), "-o", o] for s, o in zip(SOURCES, objs)]
    jobs = jobs or min(len(cmds), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        list(pool.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB + ".tmp"
    _run([hipcc(), *HIPCC_FLAGS, "-o", tmp, *objs], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
