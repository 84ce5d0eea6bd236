"""Build libsaga_amd.so (HIP kernels + C ABI) for gfx950 with hipcc.

Usage: python -m saga_amd.build   (or __graft_entry__.build())
Every csrc/*.hip is compiled to its own object in saga_amd/_build/ (in
parallel), then the objects are linked into libsaga_amd.so next to this
file; saga_amd._lib loads it.  Each call recompiles every source.
"""
from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libsaga_amd.so")

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # selection is defined on the rounded fp32 products of separate
    # multiply and add steps, as in the reference's scale-then-mask
    "-ffp-contract=off",
    # packed fp32 VALU ops stay off (v_pk_* fp32 forms)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]

# hipcc's host pass does not know the packed-fp32 target feature: harmless
_NOISE = "is not a recognized feature for this target"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libsaga_amd.so)")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if _NOISE not in l)
    return res.returncode, err


def build(verbose: bool = False, jobs: int | None = None) -> str:
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    os.makedirs(OBJ_DIR, exist_ok=True)
    cc = hipcc()
    inc = ["-I", os.path.join(HERE, "..", "include")]

    def compile_one(src):
        obj = os.path.join(OBJ_DIR, os.path.splitext(os.path.basename(src))[0] + ".o")
        rc, err = _run([cc, *HIPCC_FLAGS, *inc, "-c", src, "-o", obj], verbose)
        return src, obj, rc, err

    jobs = jobs or min(len(srcs), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        results = list(pool.map(compile_one, srcs))
    failed = [(s, rc, err) for s, _, rc, err in results if rc != 0]
    if failed:
        msg = "\n".join(f"{os.path.basename(s)} ({rc}):\n{err}" for s, rc, err in failed)
        raise RuntimeError(f"hipcc failed:\n{msg}")
    if verbose:
        for _, _, _, err in results:
            if err.strip():
                print(err)
    tmp = LIB + ".tmp"
    rc, err = _run([cc, "--offload-arch=gfx950", "-shared", "-fPIC", *[o for _, o, _, _ in results], "-o", tmp],
                   verbose)
    if rc != 0:
        raise RuntimeError(f"link failed ({rc}):\n{err}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
