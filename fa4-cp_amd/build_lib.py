"""Builds libfa4cp.so (the gfx950 HIP kernels and their C ABI) in-tree with hipcc.

    python fa4-cp_amd/build_lib.py            # compile every csrc/*.hip and link

Objects go to fa4-cp_amd/_build/, the library to fa4-cp_amd/fa4_ring/libfa4cp.so.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "fa4_ring", "libfa4cp.so")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")

ARCH = "gfx950"
# -packed-fp32-ops: keep the compiler from forming v_pk_{add,mul,fma}_f32
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", f"-I{INCLUDE}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Per-file additions.  The attention kernels take finite inputs (as the reference's): without
# NaN semantics the compiler drops the canonicalising moves of every row-max step.
FILE_FLAGS = {"attn_fwd.hip": ["-fno-honor-nans"]}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libfa4cp.so)")


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; drop that noise
    out = "\n".join(l for l in p.stdout.splitlines() if "not a recognized feature" not in l)
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{out}")
    return out


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def check_resolved(path: str) -> None:
    """Fails the build when the library references one of its own symbols it does not
    define (clang can drop a kernel's host stub without a diagnostic)."""
    out = subprocess.run(["nm", "-D", "--undefined-only", path], stdout=subprocess.PIPE,
                         stderr=subprocess.STDOUT, text=True).stdout
    missing = [l.split()[-1] for l in out.splitlines() if "fa4cp" in l]
    if missing:
        raise RuntimeError(f"{path}: unresolved internal symbols: {missing[:4]}")


def build_library(verbose: bool = False, jobs: int = 8) -> str:
    """Compiles every csrc/*.hip for gfx950 and links libfa4cp.so; returns its path."""
    cc = hipcc()
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    objs = [os.path.join(BUILD, os.path.basename(s)[:-4] + ".o") for s in srcs]
    cmds = [[cc, *HIPCC_FLAGS, *FILE_FLAGS.get(os.path.basename(s), []), "-c", s, "-o", o]
            for s, o in zip(srcs, objs)]
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(cmds)))) as ex:
        for cmd, out in zip(cmds, ex.map(_run, cmds)):
            if verbose:
                print(" ".join(cmd))
                if out.strip():
                    print(out)
    tmp = LIB + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    check_resolved(tmp)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build_library(verbose="-q" not in sys.argv)
