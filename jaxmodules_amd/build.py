"""Builds ``libmattn.so`` (the gfx950 kernels + C ABI) in-tree with hipcc.

Usage: ``python -m jaxmodules_amd.build`` (or ``__graft_entry__.build()``).
Every call recompiles; objects go to ``jaxmodules_amd/_build/`` and the library
to ``jaxmodules_amd/libmattn.so``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD_DIR = os.path.join(PKG, "_build")
LIB_PATH = os.path.join(PKG, "libmattn.so")
SOURCES = ["fwd.hip", "bwd_pre.hip", "bwd_dq.hip", "bwd_dkdv.hip", "simt.hip", "tilemap.hip", "capi.hip"]
# machine-scheduler strategy per source: the ILP-oriented ones hoist LDS operand
# reads ahead of the MFMA chains; each file uses the one measured fastest
# without register spills for its kernels (bwd_dkdv.hip orders its operand reads
# by hand and takes LLVM's default)
SCHED = {"fwd.hip": "iterative-ilp", "bwd_dq.hip": "iterative-ilp"}
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libmattn.so)")


def common_flags(extra=()):
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-I", INCLUDE,
        "-I", CSRC,
        # packed fp32 VALU ops are kept out of the generated code
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-result",
        *extra,
    ]


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass does not know the GPU target feature above; that warning is noise
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    return err


def build(verbose: bool = False, extra_flags=(), sched_override=None, lib_path=None) -> str:
    """sched_override: a scheduler strategy for every MFMA source ("" = LLVM's
    default); lib_path: where to write the library (default: in-tree)."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    cc = hipcc()
    flags = common_flags(extra_flags)

    def compile_one(src):
        obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
        sched = ["-mllvm", f"-amdgpu-sched-strategy={SCHED[src]}"] if src in SCHED else []
        if sched_override is not None and src in SCHED:
            sched = ["-mllvm", f"-amdgpu-sched-strategy={sched_override}"] if sched_override else []
        err = _run([cc, *flags, *sched, "-c", os.path.join(CSRC, src), "-o", obj])
        if verbose and err.strip():
            print(err, file=sys.stderr)
        return obj

    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    out = lib_path or LIB_PATH
    tmp = out + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build(verbose=True)
