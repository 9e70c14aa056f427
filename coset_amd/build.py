"""Compile libcoset_amd.so in-tree for gfx950 with hipcc.

    python -m coset_amd.build          # or coset_amd.build.build()

The library is plain HIP with an extern "C" surface (include/coset_amd.h); no
torch headers are involved, so it builds without a GPU.  Each source is
compiled to its own object in parallel (no device symbol crosses a
translation unit, so no relocatable device code is needed), then the objects
are linked into the shared library.
"""
from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libcoset_amd.so")
OBJ_DIR = os.path.join(PKG, "_build")

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # reference arithmetic is op-by-op IEEE; never contract to FMA
    "-ffp-contract=off",
    # keep the compiler from emitting packed fp32 ALU ops
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


# per-source extra flags: the TN GEMM keeps its staging registers in
# registers (at one wave per SIMD the compiler would otherwise move them to
# LDS, beside the kernel's own 96 KiB of stage buffers)
EXTRA_FLAGS = {
    "gemm_tn.hip": ["-mllvm", "-disable-promote-alloca-to-lds"],
}


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found: install ROCm or set HIPCC")


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
    return r.returncode


def build(verbose: bool = False, jobs: int = 0) -> str:
    """Compile every HIP source into libcoset_amd.so (always recompiles)."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    cc = hipcc()
    inc = ["-I", os.path.join(ROOT, "include")]
    srcs = sources()
    objs = [os.path.join(OBJ_DIR, os.path.basename(s)[:-4] + ".o") for s in srcs]
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)), 16)
    with ThreadPoolExecutor(jobs) as ex:
        rcs = list(ex.map(lambda so: _run([cc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(os.path.basename(so[0]), []), *inc,
                                           "-c", "-o", so[1], so[0]], verbose),
                          zip(srcs, objs)))
    bad = [s for s, rc in zip(srcs, rcs) if rc != 0]
    if bad:
        raise RuntimeError("hipcc failed on " + ", ".join(os.path.basename(b) for b in bad))
    tmp = LIB + ".tmp"
    if _run([cc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs], verbose) != 0:
        raise RuntimeError("hipcc failed linking libcoset_amd.so")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
