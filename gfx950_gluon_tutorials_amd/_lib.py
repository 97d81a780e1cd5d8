"""ctypes binding of the C ABI in ``include/gfx950_gemm.h`` and
``include/gfx950_fmha.h``.

The library is loaded from this package directory (built by ``build.py``).
There is no fallback: if it is missing the import of a wrapper succeeds but
the first call raises, so a GPU run can never silently fall back to torch.
"""

from __future__ import annotations

import ctypes
import os
import threading

from . import build as _build

# G9_LIBRARY overrides the path (e.g. to compare two builds); default: the
# library built in this package directory.
LIB_PATH = os.environ.get("G9_LIBRARY") or _build.LIB_PATH

# Status codes (gfx950_gemm.h).
G9_OK = 0
G9_ERR_SHAPE = 1
G9_ERR_LAYOUT = 2
G9_ERR_DTYPE = 3
G9_ERR_SCHEDULE = 4
G9_ERR_WORKSPACE = 5
G9_ERR_HIP = 6
G9_ERR_SCRATCH = 7
G9_ERR_PLAN = 8

# Size of a g9_plan (G9_PLAN_BYTES in gfx950_gemm.h).
G9_PLAN_BYTES = 512

# Element types.
G9_F16 = 0
G9_BF16 = 1
G9_BF8 = 2
G9_FP4 = 3
G9_FP4P = 4  # MXFP4 with preshuffled scales (g9_gemm_a4w4_preshuffled)
G9_FP4K = 5  # MXFP4 with K-major scales (g9_gemm_a4w4 given K-major scale views)

# Schedules.
G9_SCHED_DP = 0
G9_SCHED_SK = 1
G9_SCHED_SPLITK = 2
G9_SCHED_SK_HALF = 3  # stream-K over 256x128 tiles (a16w16, 4 waves)

SCHEDULES = {"dp": G9_SCHED_DP, "data_parallel": G9_SCHED_DP, "sk": G9_SCHED_SK, "streamk": G9_SCHED_SK,
             "splitk": G9_SCHED_SPLITK, "split_k": G9_SCHED_SPLITK, "streamk_half": G9_SCHED_SK_HALF,
             "sk_half": G9_SCHED_SK_HALF}

# Exported symbols and their signatures; the CPU test checks the library
# exports exactly these.
_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_int = ctypes.c_int
_sz = ctypes.c_size_t
SIGNATURES = {
    "g9_gemm_a16w16": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                              _int, _int, _int, _vp, _sz, _vp]),
    "g9_gemm_a16w16_noalloc": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                      _int, _int, _int, _vp]),
    "g9_gemm_a8w8": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                            _vp, _vp, _int, _int, _int, _vp, _sz, _vp]),
    "g9_gemm_a4w4": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                            _i64, _i64, _i64, _i64, _i64, _int, _int, _int, _vp, _sz, _vp]),
    "g9_gemm_a4w4_preshuffled": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                        _i64, _i64, _i64, _int, _int, _int, _vp, _sz, _vp]),
    "g9_moe_a16w16": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _vp]),
    "g9_moe_a8w8": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int,
                           _vp]),
    "g9_moe_a4w4": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                           _i64, _i64, _int, _vp]),
    "g9_moe_kernel_name": (ctypes.c_char_p, [_int, _int]),
    "g9_fmha_fwd": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp,
                           ctypes.c_float, _int, _int, _int, _vp]),
    "g9_workspace_size": (_sz, [_int, _i64, _i64, _i64, _int, _int]),
    "g9_workspace_init": (_int, [_vp, _sz, _vp]),
    "g9_workspace_error": (_int, [_vp, _sz, _vp, ctypes.POINTER(_int)]),
    "g9_workspace_watch": (_int, [_vp, _sz, _vp, _vp]),
    "g9_set_streamk_spin_limit": (ctypes.c_uint32, [ctypes.c_uint32]),
    "g9_transpose_u8": (_int, [_vp, _i64, _i64, _i64, _vp, _i64, _vp]),
    "g9_noalloc_error": (_int, [_vp, ctypes.POINTER(_int)]),
    "g9_plan_a16w16": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                              _int, _int, _int, _vp, _sz]),
    "g9_plan_a8w8": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                            _vp, _vp, _int, _int, _int, _vp, _sz]),
    "g9_plan_a4w4": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                            _i64, _i64, _i64, _i64, _i64, _int, _int, _int, _vp, _sz]),
    "g9_plan_a4w4_preshuffled": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                        _i64, _i64, _i64, _i64, _int, _int, _int, _vp, _sz]),
    "g9_plan_launch": (_int, [_vp, _vp]),
    "g9_kernel_name": (ctypes.c_char_p, [_int, _int, _int, _int]),
    "g9_status_string": (ctypes.c_char_p, [_int]),
    "g9_streamk_workgroups": (_int, []),
    "g9_splitk_factor": (_int, [ctypes.c_int64, _int, _int]),
    "g9_version": (_int, []),
}

_lock = threading.Lock()
_lib = None


class LibraryMissing(RuntimeError):
    pass


def load():
    """Returns the loaded library, raising if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise LibraryMissing(
                    f"{LIB_PATH} is not built; run `python -m gfx950_gluon_tutorials_amd.build`"
                )
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def status_text(code: int) -> str:
    return load().g9_status_string(code).decode()


def check(code: int, what: str) -> None:
    """Maps a C status code to the Python exception a caller expects."""
    if code == G9_OK:
        return
    msg = f"{what}: {status_text(code)} (status {code})"
    if code in (G9_ERR_SHAPE, G9_ERR_LAYOUT, G9_ERR_DTYPE, G9_ERR_SCHEDULE, G9_ERR_PLAN):
        raise ValueError(msg)
    raise RuntimeError(msg)


def kernel_name(dtype: int, out_dtype: int, schedule: int, waves: int) -> str | None:
    name = load().g9_kernel_name(dtype, out_dtype, schedule, waves)
    return name.decode() if name else None


def moe_kernel_name(dtype: int, out_dtype: int) -> str | None:
    name = load().g9_moe_kernel_name(dtype, out_dtype)
    return name.decode() if name else None
