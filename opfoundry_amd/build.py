"""Build libdsa_mla.so (gfx950) in-tree with hipcc, and beside it the
measurement probes libdsa_gather_floor.so (bench.py --gather-floor) and
libdsa_issue_probe.so (bench.py --issue-probe).

    python -m opfoundry_amd.build [--verbose]

The shared objects land in opfoundry_amd/_build/ so they travel with the
source tree; nothing is installed.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

from .abi import LIB_PATH, PKG_DIR

SRC = os.path.join(PKG_DIR, "csrc", "dsa_mla.hip")
SRCS = [SRC, os.path.join(PKG_DIR, "csrc", "dsa_topk.hip"), os.path.join(PKG_DIR, "csrc", "dsa_indexer.hip")]
PROBE_SRC = os.path.join(PKG_DIR, "csrc", "dsa_gather_floor.hip")
PROBE_LIB_PATH = os.path.join(os.path.dirname(LIB_PATH), "libdsa_gather_floor.so")
ISSUE_PROBE_SRC = os.path.join(PKG_DIR, "csrc", "dsa_issue_probe.hip")
ISSUE_PROBE_LIB_PATH = os.path.join(os.path.dirname(LIB_PATH), "libdsa_issue_probe.so")
INCLUDE = os.path.normpath(os.path.join(PKG_DIR, "..", "include"))

# Packed-fp32 VALU ops are disabled for all device code: only ordinary
# scalar / float2 code is written and the compiler may not fuse it into
# v_pk_*_f32.  The host pass warns that it does not know the feature.
# MFMAs the compiler emits take their accumulators in VGPRs
# (amdgpu-mfma-vgpr-form): the AGPR file holds the O accumulators, which the
# kernel binds there itself.
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libdsa_mla.so)")


def _compile(srcs: list[str], lib: str, verbose: bool, extra_flags: list[str] | None) -> str:
    os.makedirs(os.path.dirname(lib), exist_ok=True)
    tmp = lib + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, *(extra_flags or []), f"-I{INCLUDE}", *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(line for line in (res.stdout + res.stderr).splitlines()
                    if "packed-fp32-ops" not in line and "unknown target feature" not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{out}")
    if verbose and out.strip():
        print(out)
    os.replace(tmp, lib)
    return lib


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> str:
    """Compile libdsa_mla.so and the two measurement probes; return the library's path."""
    _compile([PROBE_SRC], PROBE_LIB_PATH, verbose, extra_flags)
    _compile([ISSUE_PROBE_SRC], ISSUE_PROBE_LIB_PATH, verbose, extra_flags)
    return _compile(SRCS, LIB_PATH, verbose, extra_flags)


if __name__ == "__main__":
    print(build(verbose="--verbose" in sys.argv))
