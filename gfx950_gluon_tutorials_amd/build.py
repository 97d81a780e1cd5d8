"""Builds the gfx950 GEMM library (``libg9gemm.so``) in-tree with hipcc.

The library is plain HIP C++ behind the C ABI of ``include/gfx950_gemm.h``;
Python loads it with ctypes (no torch extension, no JIT cache), so the built
file travels with the source tree.

Usage: ``python -m gfx950_gluon_tutorials_amd.build`` (or ``build()``).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_NAME = "libg9gemm.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
# The same kernels with per-workgroup phase stamps (-DG9_TIMING), for
# profiling.py; never loaded by the wrappers unless G9_LIBRARY points at it.
LIB_TIMING_PATH = os.path.join(PKG_DIR, "libg9gemm_timing.so")
SOURCES = ["g9_capi.hip"]
HEADERS = ["g9_common.hpp", "g9_gemm.hpp"]

# -packed-fp32-ops: keep the compiler from forming v_pk_*_f32, whose results
# have been unreliable on the target machines.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-shared",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def build(verbose: bool = False, timing: bool = False) -> str:
    """Compiles the library for gfx950, checks its device assembly for MFMA
    hazards (isa_check) and returns its path.  The library is only replaced
    when both steps pass; the kernels' register and scratch use is written
    next to it (``<lib>.resources.json``).  ``timing`` builds the stamped
    variant instead."""
    import json

    from . import isa_check

    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    lib_path = LIB_TIMING_PATH if timing else LIB_PATH
    flags = HIPCC_FLAGS + (["-DG9_TIMING"] if timing else [])
    tmp = lib_path + ".tmp"
    with tempfile.TemporaryDirectory(prefix="g9build") as work:
        # -save-temps keeps the device assembly (in the scratch directory)
        # without a second compilation.
        cmd = [hipcc_path(), *flags, "-save-temps", "-I", os.path.join(REPO_DIR, "include"), *srcs, "-o", tmp]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True, cwd=work)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
        asm = [f for f in os.listdir(work) if f.endswith("gfx950.s")]
        if len(asm) != len(SOURCES):
            raise RuntimeError(f"expected {len(SOURCES)} device assembly file(s), found {asm}")
        bad, resources = [], []
        for f in asm:
            with open(os.path.join(work, f)) as fh:
                text = fh.read()
            bad += isa_check.check_text(text)
            resources += isa_check.resource_table(text)
        if bad:
            os.unlink(tmp)
            raise RuntimeError("MFMA hazards in the device code:\n" + "\n".join(bad[:20]))
    os.replace(tmp, lib_path)
    with open(lib_path + ".resources.json", "w") as fh:
        json.dump(resources, fh, indent=1)
    return lib_path


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv, timing="--timing" in sys.argv))
