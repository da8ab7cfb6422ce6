"""Builds libmuon_sr_amd.so (the gfx950 HIP kernels + C ABI) in-tree.

The library depends only on the HIP runtime; it is loaded with ctypes.
"""
from __future__ import annotations

import glob
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libmuon_sr_amd.so")
ARCH = os.environ.get("MSR_OFFLOAD_ARCH", "gfx950")

# IEEE fp32 without contraction (the kernels restate the reference's expression
# order), no packed-fp32 instructions, correctly rounded / and sqrt (HIP default).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = os.path.join(rocm, "bin", "hipcc")
    return cand if os.path.exists(cand) else "hipcc"


# Per-source extra flags (none at present; kept so a source can get its own).
EXTRA_FLAGS = {}

_NOISE = "is not a recognized feature for this target"  # hipcc host pass; harmless


def _finish(cmd, res, verbose):
    err = "\n".join(line for line in res.stderr.splitlines() if _NOISE not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err)


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    _finish(cmd, subprocess.run(cmd, capture_output=True, text=True), verbose)


def build(verbose: bool = False) -> str:
    """Compile every HIP source (each with its own flags, all at once) and link one
    shared library.  Always recompiles; objects go to muon_sr_amd/_build/."""
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    objs, jobs = [], []
    for src in sources():
        obj = os.path.join(objdir, os.path.basename(src) + ".o")
        flags = [f for f in HIPCC_FLAGS if f != "-shared"]
        cmd = [hipcc(), *flags, *EXTRA_FLAGS.get(os.path.basename(src), []), "-c", "-o", obj, src]
        if verbose:
            print(" ".join(cmd), flush=True)
        jobs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
        objs.append(obj)
    for cmd, proc in jobs:
        out, err = proc.communicate()
        _finish(cmd, subprocess.CompletedProcess(cmd, proc.returncode, out, err), verbose)
    tmp = LIB + ".tmp"
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
