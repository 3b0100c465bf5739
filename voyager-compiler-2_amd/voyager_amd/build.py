"""Build ``_lib/libvoyager_hip.so`` from ``csrc/*.hip`` with hipcc for gfx950.

Each source compiles to its own object in parallel (``_build/``), then one
link step makes the shared library.  ``build()`` recompiles every source;
``build(incremental=True)`` (``python -m voyager_amd.build --incremental``)
recompiles only sources older than their object or than a header.

Usage: ``python -m voyager_amd.build`` (from ``voyager-compiler-2_amd/``) or
``__graft_entry__.build()``.
"""

import glob
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

from .paths import CSRC_DIR, INCLUDE_DIR, PKG_DIR, SRC_ROOT

ARCH = "gfx950"
OUT = os.path.join(PKG_DIR, "_lib", "libvoyager_hip.so")
OBJ_DIR = os.path.join(SRC_ROOT, "_build")

# Packed-fp32 instructions are disabled: some of their forms have given wrong
# results on these machines.  No fast-math: the ops must keep denormals and
# correctly rounded division to match the reference's eager numerics.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

_NOISE = ("is not a recognized feature for this target", "ignoring feature")


def sources():
    return sorted(glob.glob(os.path.join(CSRC_DIR, "*.hip")))


def _headers():
    return glob.glob(os.path.join(CSRC_DIR, "*.h")) + glob.glob(os.path.join(INCLUDE_DIR, "*.h"))


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in (res.stderr or "").splitlines() if not any(n in l for n in _NOISE))
    return res.returncode, err


def _jobs():
    n = os.cpu_count() or 4
    return max(1, min(n, int(os.environ.get("MAX_JOBS", n)), 16))


def build(verbose: bool = False, incremental: bool = False) -> str:
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    os.makedirs(OBJ_DIR, exist_ok=True)
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    newest_header = max((os.path.getmtime(h) for h in _headers()), default=0.0)
    objs, todo = [], []
    for src in sources():
        obj = os.path.join(OBJ_DIR, os.path.basename(src)[:-4] + ".o")
        objs.append(obj)
        fresh = (incremental and os.path.exists(obj)
                 and os.path.getmtime(obj) >= max(os.path.getmtime(src), newest_header))
        if not fresh:
            todo.append((src, obj))

    def compile_one(item):
        src, obj = item
        cmd = [hipcc, *HIPCC_FLAGS, f"-I{INCLUDE_DIR}", "-c", src, "-o", obj + ".tmp"]
        if verbose:
            print(" ".join(cmd), flush=True)
        rc, err = _run(cmd)
        if rc == 0:
            os.replace(obj + ".tmp", obj)
        return src, rc, err

    with ThreadPoolExecutor(_jobs()) as pool:
        results = list(pool.map(compile_one, todo))
    failed = [(s, e) for s, rc, e in results if rc != 0]
    if failed:
        raise RuntimeError("hipcc failed:\n" + "\n".join(f"{s}:\n{e}" for s, e in failed))
    for s, rc, e in results:
        if verbose and e.strip():
            print(e, file=sys.stderr)
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", OUT + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    rc, err = _run(cmd)
    if rc != 0:
        raise RuntimeError(f"hipcc link failed ({rc}):\n{err}")
    os.replace(OUT + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True, incremental="--incremental" in sys.argv))
