"""Build libforge_mi355x.so in-tree with hipcc for gfx950 (no JIT cache: the .so travels with the source tree).

Recipe (also what ``python -m forge_amd.build`` runs)::

    hipcc --offload-arch=gfx950 -O3 -std=c++17 -fPIC -ffp-contract=off \
          -Xclang -target-feature -Xclang -packed-fp32-ops -c csrc/<file>.hip -o _build/<file>.o   (each file, in parallel)
    hipcc --offload-arch=gfx950 -shared -o forge_amd/libforge_mi355x.so _build/*.o

``-ffp-contract=off`` keeps every fp32 multiply and add separately rounded unless the source asks for an fma, so
epilogues such as ``(float(acc) * sa) * sb + bias`` round exactly like the CPU oracle.  Packed fp32 instructions are
disabled for the whole library.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)  # forge-llm_amd/
CSRC = os.path.join(ROOT, "csrc")
BUILD = os.path.join(ROOT, "_build")
LIB = os.path.join(PKG, "libforge_mi355x.so")
ARCH = os.environ.get("FORGE_AMD_ARCH", "gfx950")

CFLAGS = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Wall", "-Wno-unused-function",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
# every kernel is this library's own: the HIP runtime is the only dependency hipcc links by default
LINK: list[str] = []


def _hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if c and (os.path.sep not in c or os.path.exists(c)):
            return c
    raise RuntimeError("hipcc not found")


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(BUILD, os.path.basename(src).replace(".hip", ".o"))
    cmd = [_hipcc(), f"--offload-arch={ARCH}", *CFLAGS, "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(ln for ln in (r.stderr or "").splitlines() if noise not in ln)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    if err.strip() and verbose:
        print(err)
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile every ``csrc/*.hip`` and link ``libforge_mi355x.so`` next to this file; returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB + f".tmp{os.getpid()}"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-o", tmp, *objs, *LINK]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True, capture_output=not verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
