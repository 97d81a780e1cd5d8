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
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_NAME = "libg9gemm.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
# The same kernels with per-workgroup phase stamps (-DG9_TIMING), for
# profiling.py; never loaded by the wrappers unless G9_LIBRARY points at it.
LIB_TIMING_PATH = os.path.join(PKG_DIR, "libg9gemm_timing.so")
SOURCES = ["g9_capi.hip", "g9_fmha.hip"]  # GEMM + MoE + C ABI; flash-attention forward
# Per-source flags.  g9_fmha.hip: without NaN-preserving semantics for fmax
# the row-max reduction is one v_max3 per two scores instead of also
# canonicalizing every MFMA result first (NaN inputs still give NaN rows:
# their exponentials are NaN).
SOURCE_FLAGS = {"g9_fmha.hip": ["-fno-honor-nans"]}
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

    lib_path = LIB_TIMING_PATH if timing else LIB_PATH
    flags = HIPCC_FLAGS + (["-DG9_TIMING"] if timing else [])
    tmp = lib_path + ".tmp"
    with tempfile.TemporaryDirectory(prefix="g9build") as work:
        # Each source compiles to an object in a directory of its own, in
        # parallel; -save-temps keeps its device assembly there without a
        # second compilation.
        def compile_one(src: str) -> tuple[str, str]:
            d = os.path.join(work, os.path.splitext(src)[0])
            os.makedirs(d)
            obj = os.path.join(d, src + ".o")
            cmd = [hipcc_path(), *[f for f in flags if f != "-shared"], *SOURCE_FLAGS.get(src, []), "-c", "-save-temps", "-I",
                   os.path.join(REPO_DIR, "include"), os.path.join(CSRC, src), "-o", obj]
            if verbose:
                print(" ".join(cmd), flush=True)
            res = subprocess.run(cmd, capture_output=True, text=True, cwd=d)
            if res.returncode != 0:
                raise RuntimeError(f"hipcc failed on {src} ({res.returncode}):\n{res.stdout}\n{res.stderr}")
            asm = [os.path.join(d, f) for f in os.listdir(d) if f.endswith("gfx950.s")]
            if len(asm) != 1:
                raise RuntimeError(f"expected one device assembly file for {src}, found {asm}")
            return obj, asm[0]

        with ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
            built = list(pool.map(compile_one, SOURCES))
        cmd = [hipcc_path(), *flags, *[o for o, _ in built], "-o", tmp]
        res = subprocess.run(cmd, capture_output=True, text=True, cwd=work)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc link failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
        asm = [a for _, a in built]
        bad, resources = [], []
        for f in asm:
            with open(f) as fh:
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


def resource_table_text(lib_path: str = LIB_PATH) -> str:
    """The per-kernel register, scratch and LDS table of a built library (from
    the ``<lib>.resources.json`` build() writes next to it)."""
    import json

    with open(lib_path + ".resources.json") as fh:
        rows = json.load(fh)
    cols = ["agpr", "vgpr_total", "sgpr", "vgpr_spill", "sgpr_spill", "scratch_bytes", "lds_bytes"]
    heads = ["agpr", "vgpr_total", "sgpr", "vgpr_spill", "sgpr_spill", "scratch_B", "lds_B"]
    width = max(len(r["kernel"]) for r in rows) + 2
    out = [f"{'kernel':{width}s}" + " ".join(f"{h:>10s}" for h in heads)]
    for r in rows:
        out.append(f"{r['kernel']:{width}s}" + " ".join(f"{r[c]:>10d}" for c in cols))
    return "\n".join(out)


if __name__ == "__main__":
    if "--table" in sys.argv:
        print(resource_table_text(LIB_TIMING_PATH if "--timing" in sys.argv else LIB_PATH))
    else:
        print(build(verbose="-v" in sys.argv, timing="--timing" in sys.argv))
