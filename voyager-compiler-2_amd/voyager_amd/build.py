"""Build ``_lib/libvoyager_hip.so`` from ``csrc/*.hip`` with hipcc for gfx950.

Usage: ``python -m voyager_amd.build`` (from ``voyager-compiler-2_amd/``) or
``__graft_entry__.build()``.
"""

import glob
import os
import subprocess
import sys

from .paths import CSRC_DIR, INCLUDE_DIR, PKG_DIR

ARCH = "gfx950"
OUT = os.path.join(PKG_DIR, "_lib", "libvoyager_hip.so")

# Packed-fp32 instructions are disabled: some of their forms have given wrong
# results on these machines.  No fast-math: the ops must keep denormals and
# correctly rounded division to match the reference's eager numerics.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def sources():
    return sorted(glob.glob(os.path.join(CSRC_DIR, "*.hip")))


def build(verbose: bool = False) -> str:
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    cmd = [hipcc, *HIPCC_FLAGS, f"-I{INCLUDE_DIR}", *sources(), "-o", OUT + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (res.stderr or "").splitlines() if noise not in l and "ignoring feature" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(OUT + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
