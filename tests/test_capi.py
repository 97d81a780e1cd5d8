"""CPU checks of the C ABI: the built library loads, exports exactly the
entry points include/gfx950_gemm.h and include/gfx950_fmha.h declare, and rejects bad arguments with
the documented status codes before touching the GPU (no launches here)."""

import ctypes
import os
import re

import pytest

from gfx950_gluon_tutorials_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "gfx950_gemm.h")
FMHA_HEADER = os.path.join(os.path.dirname(HEADER), "gfx950_fmha.h")
FAKE = 0x10000  # 16-byte aligned non-null address; never dereferenced on these paths


def declared_functions():
    text = open(HEADER).read() + open(FMHA_HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(g9_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_function():
    lib = _lib.load()
    names = declared_functions()
    assert names == sorted(_lib.SIGNATURES), "binding table out of sync with the header"
    for n in names:
        assert hasattr(lib, n), f"{n} declared in a header but not exported"


TIMING_HEADER = os.path.join(os.path.dirname(HEADER), "gfx950_gemm_timing.h")


def test_timing_build_exports_its_header_and_the_regular_one_does_not():
    from gfx950_gluon_tutorials_amd import build as _b

    text = open(TIMING_HEADER).read()
    names = sorted(set(re.findall(r"^\s*\w+\s*\*?\s*(g9_\w+)\s*\(", text, flags=re.M)))
    assert names == ["g9_fmha_timing_read", "g9_timing_capacity", "g9_timing_read"]
    regular = _lib.load()
    for n in names:
        assert not hasattr(regular, n), f"{n} leaked into the regular library"
    if not os.path.exists(_b.LIB_TIMING_PATH):
        pytest.skip("timing library not built")
    timing = ctypes.CDLL(_b.LIB_TIMING_PATH)
    for n in names + declared_functions():
        assert hasattr(timing, n), f"{n} missing from the timing library"
    timing.g9_timing_capacity.restype = ctypes.c_int
    assert timing.g9_timing_capacity() >= 256


def test_version_and_status_strings():
    lib = _lib.load()
    assert lib.g9_version() >= 100
    for code in range(9):
        assert _lib.status_text(code) != "unknown status"
    assert _lib.status_text(0) == "ok"
    assert "scratch" in _lib.status_text(_lib.G9_ERR_SCRATCH)


def test_plan_constants_match_the_header():
    text = open(HEADER).read()
    assert re.search(r"#define G9_PLAN_BYTES (\d+)", text).group(1) == str(_lib.G9_PLAN_BYTES)
    assert re.search(r"G9_ERR_PLAN = (\d+)", text).group(1) == str(_lib.G9_ERR_PLAN)
    assert "device" in _lib.status_text(_lib.G9_ERR_PLAN)


def test_plan_launch_refuses_a_plan_no_g9_plan_call_made():
    lib = _lib.load()
    zero = (ctypes.c_uint64 * (_lib.G9_PLAN_BYTES // 8))()
    assert lib.g9_plan_launch(ctypes.addressof(zero), None) == _lib.G9_ERR_PLAN
    assert lib.g9_plan_launch(None, None) == _lib.G9_ERR_PLAN


@pytest.mark.parametrize("kw,code", [
    (dict(M=0), _lib.G9_ERR_SHAPE),
    (dict(K=100), _lib.G9_ERR_SHAPE),
    (dict(sak=2), _lib.G9_ERR_LAYOUT),
    (dict(dtype=_lib.G9_BF8), _lib.G9_ERR_DTYPE),
    (dict(plan=False), _lib.G9_ERR_PLAN),
])
def test_plan_validates_like_the_launching_entry_point(kw, code):
    """g9_plan_a16w16 returns g9_gemm_a16w16's status for the same bad
    arguments, and leaves the plan unusable (nothing reaches the device)."""
    args = dict(M=512, N=512, K=1024, sak=1, dtype=_lib.G9_F16, plan=True)
    args.update(kw)
    M, N, K = args["M"], args["N"], args["K"]
    lib = _lib.load()
    plan = (ctypes.c_uint64 * (_lib.G9_PLAN_BYTES // 8))()
    rest = (FAKE, FAKE, FAKE, M, N, K, K, args["sak"], 1, K, N, 1, args["dtype"], _lib.G9_SCHED_DP, 4, None, 0)
    assert lib.g9_plan_a16w16(ctypes.addressof(plan) if args["plan"] else None, *rest) == code
    if args["plan"]:
        assert lib.g9_gemm_a16w16(*rest, None) == code
        assert lib.g9_plan_launch(ctypes.addressof(plan), None) == _lib.G9_ERR_PLAN


@pytest.mark.parametrize("kw,code", [
    (dict(M=0), _lib.G9_ERR_SHAPE),
    (dict(K=100), _lib.G9_ERR_SHAPE),
    (dict(sak=2), _lib.G9_ERR_LAYOUT),
    (dict(dtype=_lib.G9_BF8), _lib.G9_ERR_DTYPE),
])
def test_noalloc_argument_validation(kw, code):
    """The allocation-free entry validates exactly like g9_gemm_a16w16 (bad
    arguments only: nothing reaches the device)."""
    args = dict(M=512, N=512, K=1024, sak=1, dtype=_lib.G9_F16)
    args.update(kw)
    M, N, K = args["M"], args["N"], args["K"]
    lib = _lib.load()
    assert lib.g9_gemm_a16w16_noalloc(FAKE, FAKE, FAKE, M, N, K, K, args["sak"], 1, K, N, 1, args["dtype"],
                                      _lib.G9_SCHED_SK, 4, None) == code


def test_kernel_names_are_stable_and_unique():
    names = set()
    for dt, out in [(_lib.G9_F16, _lib.G9_F16), (_lib.G9_BF16, _lib.G9_BF16), (_lib.G9_BF8, _lib.G9_F16),
                    (_lib.G9_BF8, _lib.G9_BF16), (_lib.G9_FP4, _lib.G9_BF16), (_lib.G9_FP4, _lib.G9_F16)]:
        for sched in (_lib.G9_SCHED_DP, _lib.G9_SCHED_SK):
            for waves in (4, 8):
                n = _lib.kernel_name(dt, out, sched, waves)
                assert n and n.startswith("g9_a") and n.endswith(f"_{waves}w") and n not in names
                names.add(n)
    assert _lib.kernel_name(_lib.G9_F16, _lib.G9_BF16, 0, 4) is None


def test_splitk_kernel_names():
    # One segment kernel per operand type and wave count (its output is fp32
    # partials, so both output types of BF8 / MXFP4 share it).
    for dt, out, stem in [(_lib.G9_F16, _lib.G9_F16, "g9_a16w16_f16"), (_lib.G9_BF16, _lib.G9_BF16, "g9_a16w16_bf16"),
                          (_lib.G9_BF8, _lib.G9_F16, "g9_a8w8"), (_lib.G9_BF8, _lib.G9_BF16, "g9_a8w8"),
                          (_lib.G9_FP4, _lib.G9_BF16, "g9_a4w4"), (_lib.G9_FP4, _lib.G9_F16, "g9_a4w4")]:
        for waves in (4, 8):
            assert _lib.kernel_name(dt, out, _lib.G9_SCHED_SPLITK, waves) == f"{stem}_splitk_{waves}w"


@pytest.mark.parametrize("tiles,stages,cus,want", [
    (32, 128, 256, 8),    # one GPU's shard of a 4096-row GEMM over 8 GPUs: 512 x 4096, K = 8192 fp16
    (2, 64, 256, 16),     # a few-row GEMM: capped at 16 segments
    (128, 128, 256, 2),   # half the CUs: two segments per tile still fill the chip
    (129, 128, 256, 1),   # more than half the CUs busy already: data-parallel
    (160, 128, 256, 1),
    (4, 1, 256, 1),       # one K stage cannot be split
    (4, 3, 256, 1),       # too few stages to pay for a segment's prologue and partial store
    (4, 40, 256, 14),     # 14 segments of <= 3 stages cost less than 16 (still 3 stages, more partials)
    (0, 64, 256, 1),
])
def test_splitk_factor_known_answers(tiles, stages, cus, want):
    assert _lib.load().g9_splitk_factor(tiles, stages, cus) == want


def test_splitk_factor_invariants():
    lib = _lib.load()
    for cus in (80, 256, 304):
        for tiles in (1, 2, 3, 7, 16, 31, 64, 100, 151, 200, 1000):
            for stages in (1, 2, 5, 16, 32, 128, 512):
                s = lib.g9_splitk_factor(tiles, stages, cus)
                assert 1 <= s <= 16 and s <= max(stages, 1)
                assert s == 1 or tiles * s <= cus
                if 2 * tiles > cus:
                    assert s == 1
                # The model never picks a split that costs more than data-parallel.
                if s > 1:
                    assert 100 * (-(-stages // s)) + 700 + 4 * s * tiles < 100 * stages + 400


def _flags_base(ws_bytes):
    """Start of the partials in a workspace of ws_bytes: behind the header and
    the flag words g9_workspace_init clears for that size (one per 256x128
    partial that fits, plus one, rounded up to 256 bytes)."""
    unit = 256 * 128 * 4
    max_units = (ws_bytes - 256) // unit + 1
    return 256 + -(-max_units * 4 // 256) * 256


def test_workspace_size():
    lib = _lib.load()
    assert lib.g9_workspace_size(_lib.G9_F16, 4096, 4096, 8192, _lib.G9_SCHED_DP, 4) == 0
    sk = lib.g9_workspace_size(_lib.G9_F16, 3840, 3840, 16384, _lib.G9_SCHED_SK, 4)
    assert sk >= 225 * 256 * 256 * 4 + 225 * 4
    # An exact-size workspace holds every tile's partial behind the flag
    # region its own size implies (tile counts up to and past the point where
    # the flags outgrow one 256 KiB partial).
    for M, N in ((256, 256), (3840, 3840), (5120, 5120), (65536, 65536), (65536 + 256, 65536 + 512)):
        tiles = -(-M // 256) * -(-N // 256)
        ws = lib.g9_workspace_size(_lib.G9_F16, M, N, 1024, _lib.G9_SCHED_SK, 4)
        assert _flags_base(ws) + tiles * 256 * 256 * 4 <= ws, (M, N)
        assert _flags_base(ws) >= 256 + 4 * (tiles + 1)
        # 256x128 tiles: twice as many flags, each partial half the size.
        tiles_h = -(-M // 256) * -(-N // 128)
        wh = lib.g9_workspace_size(_lib.G9_F16, M, N, 1024, _lib.G9_SCHED_SK_HALF, 4)
        assert _flags_base(wh) + tiles_h * 256 * 128 * 4 <= wh, (M, N)
        assert _flags_base(wh) >= 256 + 4 * (tiles_h + 1)
    # Only FP16/BF16 with 4 waves run 256x128 tiles.
    assert lib.g9_workspace_size(_lib.G9_BF16, 3840, 3840, 1024, _lib.G9_SCHED_SK_HALF, 4) > 0
    assert lib.g9_workspace_size(_lib.G9_F16, 3840, 3840, 1024, _lib.G9_SCHED_SK_HALF, 8) == 0
    assert lib.g9_workspace_size(_lib.G9_BF8, 3840, 3840, 1024, _lib.G9_SCHED_SK_HALF, 4) == 0


def test_streamk_rejects_a_workspace_256_bytes_short():
    """Validation only: the call fails before launching (no GPU work)."""
    lib = _lib.load()
    M, N, K = 3840, 3840, 1024
    ws = lib.g9_workspace_size(_lib.G9_F16, M, N, K, _lib.G9_SCHED_SK, 4)
    short = lib.g9_gemm_a16w16(FAKE, FAKE, FAKE, M, N, K, K, 1, 1, K, N, 1, _lib.G9_F16, _lib.G9_SCHED_SK, 4,
                               FAKE, ws - 256, None)
    assert short == _lib.G9_ERR_WORKSPACE


def test_streamk_half_validation():
    """Validation only: rejected before any launch (no GPU work)."""
    lib = _lib.load()
    M, N, K = 3840, 3840, 1024
    ws = lib.g9_workspace_size(_lib.G9_F16, M, N, K, _lib.G9_SCHED_SK_HALF, 4)
    args = (FAKE, FAKE, FAKE, M, N, K, K, 1, 1, K, N, 1, _lib.G9_F16, _lib.G9_SCHED_SK_HALF)
    assert lib.g9_gemm_a16w16(*args, 8, FAKE, ws, None) == _lib.G9_ERR_SCHEDULE
    assert lib.g9_gemm_a16w16(*args, 4, FAKE, ws - 256, None) == _lib.G9_ERR_WORKSPACE
    assert lib.g9_gemm_a16w16_noalloc(*args, 8, None) == _lib.G9_ERR_SCHEDULE


def test_b_operand_rows_not_16_byte_aligned_are_repacked():
    import torch

    from gfx950_gluon_tutorials_amd.gemm import _launch

    buf = torch.zeros(384, 1024 + 4, dtype=torch.float16)
    for off in (0, 4):
        b_kn = buf[:, off:off + 1024].T  # (K, N) view with unit K stride
        got = _launch._k_major(b_kn)
        assert got.stride(0) == 1 and got.data_ptr() % 16 == 0 and (got.stride(1) * 2) % 16 == 0
        assert torch.equal(got, b_kn)
    # Unit K stride but a 1028-element (2056-byte) row pitch: repacked.
    assert _launch._k_major(buf[:, :1024].T).data_ptr() != buf.data_ptr()
    aligned = torch.zeros(384, 1024, dtype=torch.float16)
    assert _launch._k_major(aligned.T).data_ptr() == aligned.data_ptr()  # used in place


def _a16w16(M=512, N=512, K=1024, sam=None, sak=1, sbk=1, sbn=None, scm=None, scn=1, dtype=0, sched=0,
            waves=4, ws=None, ws_bytes=0):
    lib = _lib.load()
    return lib.g9_gemm_a16w16(FAKE, FAKE, FAKE, M, N, K, K if sam is None else sam, sak, sbk,
                              K if sbn is None else sbn, N if scm is None else scm, scn, dtype, sched, waves,
                              ws, ws_bytes, None)


@pytest.mark.parametrize("kw,code", [
    (dict(M=0), _lib.G9_ERR_SHAPE),
    (dict(N=-5), _lib.G9_ERR_SHAPE),
    (dict(K=100), _lib.G9_ERR_SHAPE),
    (dict(K=0), _lib.G9_ERR_SHAPE),
    (dict(M=(1 << 30) + 1), _lib.G9_ERR_SHAPE),
    (dict(M=1 << 30, N=1 << 30), _lib.G9_ERR_SHAPE),  # 2^44 tiles: tile ids are 32-bit
    (dict(sak=2), _lib.G9_ERR_LAYOUT),
    (dict(sbk=1024, sbn=1), _lib.G9_ERR_LAYOUT),
    (dict(scn=2), _lib.G9_ERR_LAYOUT),
    (dict(sam=1000), _lib.G9_ERR_LAYOUT),
    (dict(dtype=_lib.G9_BF8), _lib.G9_ERR_DTYPE),
    (dict(dtype=9), _lib.G9_ERR_DTYPE),
    (dict(waves=3), _lib.G9_ERR_SCHEDULE),
    (dict(sched=7), _lib.G9_ERR_SCHEDULE),
    (dict(sched=_lib.G9_SCHED_SK), _lib.G9_ERR_WORKSPACE),
    (dict(sched=_lib.G9_SCHED_SK, ws=FAKE, ws_bytes=1024), _lib.G9_ERR_WORKSPACE),
])
def test_a16w16_argument_validation(kw, code):
    assert _a16w16(**kw) == code


def test_a8w8_and_a4w4_argument_validation():
    lib = _lib.load()
    # a8w8: K must be a multiple of 16 (whole 16-byte chunks); output dtype fp16/bf16 only.
    assert lib.g9_gemm_a8w8(FAKE, FAKE, FAKE, 256, 256, 200, 208, 1, 1, 208, 256, 1, None, None,
                            _lib.G9_F16, 0, 4, None, 0, None) == _lib.G9_ERR_SHAPE
    assert lib.g9_gemm_a8w8(FAKE, FAKE, FAKE, 256, 256, 256, 256, 1, 1, 256, 256, 1, None, None,
                            _lib.G9_BF8, 0, 4, None, 0, None) == _lib.G9_ERR_DTYPE
    # a4w4: scales must be row-major-ish and wide enough.
    assert lib.g9_gemm_a4w4(FAKE, FAKE, FAKE, FAKE, FAKE, 256, 256, 512, 256, 1, 256, 1, 256, 1,
                            1, 256, 16, 1, _lib.G9_BF16, 0, 4, None, 0, None) == _lib.G9_ERR_LAYOUT
    assert lib.g9_gemm_a4w4(FAKE, FAKE, FAKE, None, FAKE, 256, 256, 512, 256, 1, 256, 1, 256, 1,
                            16, 1, 16, 1, _lib.G9_BF16, 0, 4, None, 0, None) == _lib.G9_ERR_LAYOUT
    assert lib.g9_gemm_a4w4(FAKE, FAKE, FAKE, FAKE, FAKE, 256, 256, 384, 192, 1, 192, 1, 256, 1,
                            12, 1, 12, 1, _lib.G9_BF16, 0, 4, None, 0, None) == _lib.G9_ERR_SHAPE


def test_status_maps_to_python_exceptions():
    with pytest.raises(ValueError):
        _lib.check(_lib.G9_ERR_SHAPE, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.G9_ERR_HIP, "x")
    _lib.check(_lib.G9_OK, "x")


def test_auto_schedule_rule():
    from gfx950_gluon_tutorials_amd.gemm import _launch

    dp, sk = _lib.G9_SCHED_DP, _lib.G9_SCHED_SK
    cases = {(3840, 3840): dp, (8192, 1280): dp, (4096, 4096): dp, (4352, 4096): sk, (4096, 5120): sk,
             (4352, 4864): dp, (5120, 5120): dp, (4097, 4096): sk}
    for (M, N), want in cases.items():
        assert _launch.auto_schedule(M, N, cus=256) == want, (M, N)
    assert _launch.auto_schedule(4352, 4096, cus=0) == dp  # no device: never stream-K
    assert _launch.auto_schedule(4352, 4096, cus=256, dtype=_lib.G9_BF16) == sk
    for dt in (_lib.G9_BF8, _lib.G9_FP4):  # fewer K stages per tile: stream-K measured slower
        assert _launch.auto_schedule(4352, 4096, cus=256, dtype=dt) == dp


def test_headers_compile_as_c_and_cpp(tmp_path):
    """The headers are plain C (C99 and C++17), and a C caller can size a
    g9_plan on its stack and pass it to the plan entry points."""
    import shutil
    import subprocess

    src = tmp_path / "use.c"
    src.write_text(
        '#include "gfx950_gemm.h"\n#include "gfx950_fmha.h"\n'
        "int use(const void* a, const void* b, void* c, void* stream) {\n"
        "  g9_plan plan;\n"
        "  int rc = g9_plan_a16w16(&plan, a, b, c, 256, 256, 512, 512, 1, 1, 512, 256, 1, G9_F16, G9_SCHED_DP, 4,\n"
        "                          0, 0);\n"
        "  return rc ? rc : g9_plan_launch(&plan, stream);\n"
        "}\n"
        "typedef char plan_size_ok[sizeof(g9_plan) == G9_PLAN_BYTES ? 1 : -1];\n")
    inc = os.path.dirname(HEADER)
    for compiler, std in (("gcc", "-std=c99"), ("g++", "-std=c++17")):
        if not shutil.which(compiler):
            pytest.skip(f"{compiler} not found")
        lang = ["-x", "c++"] if compiler == "g++" else []
        r = subprocess.run([compiler, std, "-Wall", "-Werror", "-fsyntax-only", "-I", inc, *lang, str(src)],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr
