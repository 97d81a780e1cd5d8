"""Tensor-level launch helpers shared by the per-dtype ``matmul`` wrappers.

Every wrapper ends here: tensors are checked (device, dtype, layout), turned
into raw pointers/strides and passed to the C ABI on the current HIP stream of
the operands' device.  The launch is asynchronous, as in the reference.

Layout handling mirrors the reference's contract: the kernels want both
operands K-contiguous ("NT").  A B operand given as a (K, N) view of an (N, K)
buffer (the reference benches' ``b = randn(N, K).T``) is used in place; any
other layout is first repacked to (N, K) contiguous on the device, which is
what ``kernels/gemm/inter_wave/a8w8/matmul_kernel.py:385`` does unconditionally.
"""

from __future__ import annotations

import os
import threading
from typing import NamedTuple

import torch

from .. import _lib

_DTYPE_CODE = {torch.float16: _lib.G9_F16, torch.bfloat16: _lib.G9_BF16}
_OUT_CODE = {torch.float16: _lib.G9_F16, torch.bfloat16: _lib.G9_BF16}

# Stage depth in K elements per operand type (K must be a multiple).
STAGE_K = {_lib.G9_F16: 64, _lib.G9_BF16: 64, _lib.G9_BF8: 128, _lib.G9_FP4: 256}


# schedule="auto": stream-K where it measured faster than data-parallel (one
# MI355X at steady state, K = 8192): FP16/BF16 outputs of more 256x256 tiles
# than CUs but at most 1.25 waves of them (272 tiles: +25% 4-wave, +13%
# 8-wave; 320 tiles: +9% / +1%).  Data-parallel otherwise: with fewer tiles
# than CUs the K-ordered stream-K chains cannot shorten a tile (3840^2: -11%),
# from ~1.3 waves the workgroups' misaligned K offsets cost more L2 traffic
# than the balance gains (400 tiles: -18%), and BF8 and MXFP4, with 2-4x
# fewer K stages per tile to amortise a partial-tile handoff, lose at 272
# tiles already (BF8 -2%, MXFP4 -21%).
AUTO_SK_MAX_WAVES = 1.25


def auto_schedule(M: int, N: int, cus: int | None = None, dtype: int = _lib.G9_F16) -> int:
    """The schedule code schedule="auto" picks for an M x N output of operand
    type `dtype` on a device with `cus` compute units (queried when None)."""
    if dtype not in (_lib.G9_F16, _lib.G9_BF16):
        return _lib.G9_SCHED_DP
    tiles = -(-M // 256) * -(-N // 256)
    if cus is None:
        cus = _lib.load().g9_streamk_workgroups()
    return _lib.G9_SCHED_SK if 0 < cus < tiles <= AUTO_SK_MAX_WAVES * cus else _lib.G9_SCHED_DP


def _schedule_code(schedule, M: int, N: int, dtype: int) -> int:
    if isinstance(schedule, int):
        return schedule
    name = str(schedule).lower()
    if name == "auto":
        return auto_schedule(M, N, dtype=dtype)
    try:
        return _lib.SCHEDULES[name]
    except KeyError:
        raise ValueError(f"unknown schedule {schedule!r} (expected 'dp', 'streamk', 'streamk_half', 'splitk' or "
                         "'auto')") from None


def _require_device(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    for t in tensors:
        if t.device.type != "cuda":
            raise ValueError(f"gfx950 GEMM operands must be GPU tensors, got one on {t.device}")
        if t.device != dev:
            raise ValueError(f"operands on different devices: {dev} and {t.device}")
    return dev


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _k_major_ok(b_kn: torch.Tensor) -> bool:
    """A (K, N) view whose K stride is 1 and whose N rows start on 16-byte
    boundaries (an (N, K) row-major buffer, as the kernels' LDS-DMA needs)."""
    es = b_kn.element_size()
    return (b_kn.stride(0) == 1 and b_kn.stride(1) >= b_kn.shape[0] and b_kn.data_ptr() % 16 == 0
            and (b_kn.stride(1) * es) % 16 == 0)


def _k_major(b_kn: torch.Tensor) -> torch.Tensor:
    """`b_kn` if _k_major_ok, else an (N, K) contiguous copy viewed as (K, N)."""
    return b_kn if _k_major_ok(b_kn) else b_kn.t().contiguous().t()


def _rows_ok(t: torch.Tensor) -> bool:
    """Row-major with unit inner stride and 16-byte aligned rows."""
    es = t.element_size()
    return (
        t.dim() == 2
        and t.stride(1) == 1
        and t.data_ptr() % 16 == 0
        and (t.stride(0) * es) % 16 == 0
        and t.stride(0) >= t.shape[1]
    )


def _dev_index(dev: torch.device) -> int:
    return dev.index if dev.index is not None else torch.cuda.current_device()


class _Workspaces:
    """Stream-K / split-K workspaces (fp32 partial tiles + flags), one per
    (device, stream), grown on demand and zeroed when (re)allocated.

    A workspace is only ever used by launches on its own stream, which the
    stream orders, so launches on different streams never share partials or
    flags.  Each workspace is allocated while its stream is current, so the
    caching allocator ties the memory to that stream as well.

    Each workspace has a pinned host int registered with g9_workspace_watch:
    a launch whose flag wait times out sets it, and the next stream-K launch
    on that stream (or ``poll``) raises, with no synchronisation."""

    def __init__(self):
        self._lock = threading.Lock()
        self._ws: dict[tuple[int, int], torch.Tensor] = {}
        self._flag: dict[tuple[int, int], torch.Tensor] = {}

    def _init(self, ws: torch.Tensor, key, stream: int) -> None:
        lib = _lib.load()
        _lib.check(lib.g9_workspace_init(ws.data_ptr(), ws.numel(), stream), "workspace init")
        flag = self._flag.get(key)
        if flag is None:
            flag = torch.zeros(1, dtype=torch.int32, pin_memory=True)
            self._flag[key] = flag
        flag.zero_()
        _lib.check(lib.g9_workspace_watch(ws.data_ptr(), ws.numel(), flag.data_ptr(), stream), "workspace watch")

    def get(self, dev: torch.device, nbytes: int, stream: int) -> tuple[int, int]:
        if nbytes == 0:
            return 0, 0
        key = (_dev_index(dev), int(stream))
        with self._lock:
            ws = self._ws.get(key)
            if ws is None or ws.numel() < nbytes:
                ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
                self._init(ws, key, stream)
                self._ws[key] = ws
        return ws.data_ptr(), ws.numel()

    def poll(self, dev: torch.device, stream: int | None = None) -> None:
        """Raises RuntimeError if a stream-K launch on `stream` has timed out
        in a flag wait since the last check (without synchronising: launches
        still running are seen by a later poll), after clearing the
        workspace so later launches start clean."""
        s = _stream(dev) if stream is None else int(stream)
        key = (_dev_index(dev), s)
        flag = self._flag.get(key)
        if flag is None or int(flag[0]) == 0:
            return
        with self._lock:
            self._init(self._ws[key], key, s)
        raise RuntimeError(f"a stream-K flag wait timed out on {dev} (stream {s:#x}) since the last check; "
                           "that launch's output is wrong")

    def error(self, dev: torch.device, stream: int | None = None) -> int:
        """Synchronises `stream` (default: the device's current stream) and
        returns its workspace's error word (1 = a stream-K flag wait timed
        out; the output of that launch is wrong)."""
        s = _stream(dev) if stream is None else int(stream)
        ws = self._ws.get((_dev_index(dev), s))
        if ws is None:
            return 0
        out = _lib.ctypes.c_int(0)
        _lib.check(_lib.load().g9_workspace_error(ws.data_ptr(), ws.numel(), s, _lib.ctypes.byref(out)),
                   "workspace error query")
        return out.value

    def check(self, dev: torch.device, stream: int | None = None) -> None:
        """Raises RuntimeError if a stream-K launch on `stream` timed out in a
        flag wait, after clearing the workspace so later launches start
        clean."""
        err = self.error(dev, stream)
        if err:
            s = _stream(dev) if stream is None else int(stream)
            key = (_dev_index(dev), s)
            with self._lock:
                self._init(self._ws[key], key, s)
            raise RuntimeError(f"stream-K flag wait timed out on {dev} (error word {err}); that output is wrong")

    def release(self) -> None:
        """Drops every cached workspace (their memory returns to torch's
        caching allocator once the streams that used it are done)."""
        with self._lock:
            self._ws.clear()
            self._flag.clear()


WORKSPACES = _Workspaces()

# Every stream-K launch first polls its workspace's host flag, so a timed-out
# flag wait of an earlier launch on the stream raises at the next one.
# G9_CHECK=1 also synchronises after every stream-K launch and raises for that
# launch itself (a debugging aid: it serialises the host with the GPU).
CHECK_STREAMK = os.environ.get("G9_CHECK", "0") not in ("", "0")


_STREAMK = (_lib.G9_SCHED_SK, _lib.G9_SCHED_SK_HALF)


def _workspace(lib, dt: int, M: int, N: int, K: int, sched: int, waves: int, dev, stream) -> tuple[int, int]:
    if sched == _lib.G9_SCHED_DP:
        return 0, 0  # data-parallel launches take no workspace
    if sched in _STREAMK:
        WORKSPACES.poll(dev, stream)
    need = lib.g9_workspace_size(dt, M, N, K, sched, waves)
    return WORKSPACES.get(dev, need, stream)


def _after_launch(sched: int, dev, stream: int) -> None:
    if CHECK_STREAMK and sched in _STREAMK:
        WORKSPACES.check(dev, stream)


class _Call(NamedTuple):
    """One resolved GEMM launch: the C entry point, its arguments up to (not
    including) the workspace, and what the workspace size depends on."""
    entry: str          # g9_gemm_*; the matching plan entry is g9_plan_*
    args: tuple
    dtype: int          # operand type code (g9_workspace_size's first argument)
    M: int
    N: int
    K: int
    schedule: int
    waves: int
    keep: tuple         # the tensors whose pointers are in args (repacked copies included)


def _repack(strict: bool, what: str, make):
    """A copy of an operand in a layout the kernels read (make()), or, for a
    prepared launch (strict), a ValueError: a prepared launch binds the
    caller's tensors themselves, so a hidden copy would go stale."""
    if strict:
        raise ValueError(f"{what} is not in a layout the kernels read in place; a prepared launch binds the "
                         "tensors themselves, so pass it in that layout (see the matmul wrappers' docstrings)")
    return make()


def _run(call: _Call, dev: torch.device) -> None:
    lib = _lib.load()
    stream = _stream(dev)
    ws, ws_bytes = _workspace(lib, call.dtype, call.M, call.N, call.K, call.schedule, call.waves, dev, stream)
    _lib.check(getattr(lib, call.entry)(*call.args, ws, ws_bytes, stream), call.entry)
    _after_launch(call.schedule, dev, stream)


def _a16w16_call(a, b_kn, c, schedule, waves, strict=False) -> _Call:
    _require_device(a, b_kn, c)
    if a.dtype not in _DTYPE_CODE or b_kn.dtype != a.dtype or c.dtype != a.dtype:
        raise ValueError(f"a16w16 needs matching fp16/bf16 a, b, c; got {a.dtype}, {b_kn.dtype}, {c.dtype}")
    M, K = a.shape
    N = b_kn.shape[1]
    if c.shape != (M, N):
        raise ValueError(f"c must be ({M}, {N}), got {tuple(c.shape)}")
    if not _rows_ok(a):
        a = _repack(strict, "a", a.contiguous)
    if not _k_major_ok(b_kn):
        b_kn = _repack(strict, "b", lambda: _k_major(b_kn))
    dt = _DTYPE_CODE[a.dtype]
    sched = _schedule_code(schedule, M, N, dt)
    args = (a.data_ptr(), b_kn.data_ptr(), c.data_ptr(), M, N, K, a.stride(0), a.stride(1), b_kn.stride(0),
            b_kn.stride(1), c.stride(0), c.stride(1), dt, sched, waves)
    return _Call("g9_gemm_a16w16", args, dt, M, N, K, sched, waves, (a, b_kn, c))


def gemm_a16w16(a: torch.Tensor, b_kn: torch.Tensor, c: torch.Tensor, *, schedule="dp", waves: int = 4):
    """C = A @ B with A (M, K), B a (K, N) view, C (M, N); fp16 or bf16."""
    _run(_a16w16_call(a, b_kn, c, schedule, waves), c.device)
    return c


def _scale_tensor(s, dev) -> torch.Tensor | None:
    if s is None:
        return None
    if not isinstance(s, torch.Tensor):
        return torch.tensor([float(s)], dtype=torch.float32, device=dev)
    if s.numel() != 1:
        raise ValueError("a8w8 scales are per-tensor: one fp32 value each")
    return s.detach().reshape(1).to(device=dev, dtype=torch.float32)


def _a8w8_call(a, b_kn, c, a_scale, b_scale, schedule, waves, strict=False) -> _Call:
    dev = _require_device(a, b_kn, c)
    if a.dtype != torch.float8_e5m2 or b_kn.dtype != torch.float8_e5m2:
        raise ValueError(f"a8w8 needs float8_e5m2 operands; got {a.dtype}, {b_kn.dtype}")
    if c.dtype not in _OUT_CODE:
        raise ValueError(f"a8w8 output must be fp16 or bf16, got {c.dtype}")
    M, K = a.shape
    N = b_kn.shape[1]
    if c.shape != (M, N):
        raise ValueError(f"c must be ({M}, {N}), got {tuple(c.shape)}")
    if not _rows_ok(a):
        a = _repack(strict, "a", a.contiguous)
    if not _k_major_ok(b_kn):
        b_kn = _repack(strict, "b", lambda: _k_major(b_kn))
    scales = []
    for name, s in (("a_scale", a_scale), ("b_scale", b_scale)):
        if strict and s is not None and not (isinstance(s, torch.Tensor) and s.dtype == torch.float32
                                             and s.numel() == 1 and s.device == dev):
            raise ValueError(f"a prepared a8w8 launch takes {name} as a one-element fp32 tensor on {dev} (or None)")
        scales.append(_scale_tensor(s, dev))
    sa, sb = scales
    sched = _schedule_code(schedule, M, N, _lib.G9_BF8)
    args = (a.data_ptr(), b_kn.data_ptr(), c.data_ptr(), M, N, K, a.stride(0), a.stride(1), b_kn.stride(0),
            b_kn.stride(1), c.stride(0), c.stride(1), sa.data_ptr() if sa is not None else None,
            sb.data_ptr() if sb is not None else None, _OUT_CODE[c.dtype], sched, waves)
    return _Call("g9_gemm_a8w8", args, _lib.G9_BF8, M, N, K, sched, waves, (a, b_kn, c, sa, sb))


def gemm_a8w8(a: torch.Tensor, b_kn: torch.Tensor, c: torch.Tensor, *, a_scale=None, b_scale=None,
              schedule="dp", waves: int = 4):
    """C = (A @ B) * a_scale * b_scale with BF8 (e5m2) A (M, K), B a (K, N) view."""
    _run(_a8w8_call(a, b_kn, c, a_scale, b_scale, schedule, waves), c.device)
    return c


def _scales_ok(s: torch.Tensor) -> bool:
    return s.stride(1) == 1 and s.stride(0) % 4 == 0 and s.stride(0) >= s.shape[1] and s.data_ptr() % 4 == 0


def _kmajor_scales_ok(s: torch.Tensor) -> bool:
    """A K-major (rows contiguous, one group after another) scale view, as the
    reference bench's ``randint((K // 32, M)).T`` produces."""
    return (s.shape[1] > 1 and s.stride(0) == 1 and s.stride(1) % 4 == 0 and s.stride(1) >= s.shape[0]
            and s.data_ptr() % 4 == 0)


def _row_major_scales(lib, s: torch.Tensor, dev) -> torch.Tensor:
    """A row-major copy of scales `s`: K-major views (rows contiguous, groups
    s.stride(1) apart) with the library's byte transpose on the current
    stream (measured inside 8-wave 4096 x 4096 x 8192 calls: 6.5 us for both
    operands' scales, against 11.5 us with torch's strided copy), anything
    else with torch."""
    rows, groups = s.shape
    if s.stride(0) != 1 or s.stride(1) < rows or rows == 0 or groups == 0:
        return s.contiguous()
    out = torch.empty((rows, groups), dtype=torch.uint8, device=dev)
    rc = lib.g9_transpose_u8(s.data_ptr(), groups, rows, s.stride(1), out.data_ptr(), groups, _stream(dev))
    _lib.check(rc, "g9_transpose_u8")
    return out


def _ps_scales_ok(s: torch.Tensor) -> bool:
    return s.stride(2) == 1 and s.stride(1) == 32 and s.stride(0) % 16 == 0 and s.data_ptr() % 16 == 0


def _a4w4_preshuffled_call(a, b, a_scales, b_scales, c, M, N, K, schedule, waves, strict) -> _Call:
    chunks = -(-K // 1024)
    if a_scales.shape != (chunks, M, 32) or b_scales.shape != (chunks, N, 32):
        raise ValueError(f"preshuffled scales must be ({chunks}, {M}, 32) and ({chunks}, {N}, 32); got "
                         f"{tuple(a_scales.shape)}, {tuple(b_scales.shape)}")
    if not _ps_scales_ok(a_scales):
        a_scales = _repack(strict, "a_scales", a_scales.contiguous)
    if not _ps_scales_ok(b_scales):
        b_scales = _repack(strict, "b_scales", b_scales.contiguous)
    sched = _schedule_code(schedule, M, N, _lib.G9_FP4)
    if sched != _lib.G9_SCHED_DP or waves != 4:
        raise ValueError("preshuffled MXFP4 scales run on the 4-wave data-parallel kernel only")
    args = (a.data_ptr(), b.data_ptr(), c.data_ptr(), a_scales.data_ptr(), b_scales.data_ptr(), M, N, K,
            a.stride(0), a.stride(1), b.stride(0), b.stride(1), c.stride(0), c.stride(1), a_scales.stride(0),
            b_scales.stride(0), _OUT_CODE[c.dtype], sched, waves)
    return _Call("g9_gemm_a4w4_preshuffled", args, _lib.G9_FP4P, M, N, K, sched, waves, (a, b, c, a_scales, b_scales))


def _a4w4_call(a, b, a_scales, b_scales, c, schedule, waves, strict=False) -> _Call:
    lib = _lib.load()
    dev = _require_device(a, b, a_scales, b_scales, c)
    preshuffled = a_scales.dim() == 3
    for name, t in (("a", a), ("b", b), ("a_scales", a_scales), ("b_scales", b_scales)):
        want = 3 if preshuffled and name.endswith("scales") else 2
        if t.dtype != torch.uint8 or t.dim() != want:
            raise ValueError(f"a4w4 {name} must be a {want}-D uint8 tensor, got {t.dtype} {tuple(t.shape)}")
    M, Kp = a.shape
    N = b.shape[0]
    K = 2 * Kp
    if b.shape[1] != Kp:
        raise ValueError(f"a and b packed K differ: {Kp} vs {b.shape[1]}")
    if c.dtype not in _OUT_CODE:
        raise ValueError(f"a4w4 output must be bf16 or fp16, got {c.dtype}")
    if c.shape != (M, N):
        raise ValueError(f"c must be ({M}, {N}), got {tuple(c.shape)}")
    if not _rows_ok(a):
        a = _repack(strict, "a", a.contiguous)
    if not _rows_ok(b):
        b = _repack(strict, "b", b.contiguous)
    if preshuffled:
        return _a4w4_preshuffled_call(a, b, a_scales, b_scales, c, M, N, K, schedule, waves, strict)
    if a_scales.shape != (M, K // 32) or b_scales.shape != (N, K // 32):
        raise ValueError(f"scales must be ({M}, {K // 32}) and ({N}, {K // 32}); got "
                         f"{tuple(a_scales.shape)}, {tuple(b_scales.shape)}")
    # K-major scale views (both operands) go to the 4-wave kernels as they
    # are; anything else is read row-major, repacked if need be.
    kmajor = waves == 4 and _kmajor_scales_ok(a_scales) and _kmajor_scales_ok(b_scales)
    if not kmajor:
        if not _scales_ok(a_scales):
            a_scales = _repack(strict, "a_scales", lambda: _row_major_scales(lib, a_scales, dev))
        if not _scales_ok(b_scales):
            b_scales = _repack(strict, "b_scales", lambda: _row_major_scales(lib, b_scales, dev))
    dt = _lib.G9_FP4K if kmajor else _lib.G9_FP4
    sched = _schedule_code(schedule, M, N, _lib.G9_FP4)
    args = (a.data_ptr(), b.data_ptr(), c.data_ptr(), a_scales.data_ptr(), b_scales.data_ptr(), M, N, K,
            a.stride(0), a.stride(1), b.stride(0), b.stride(1), c.stride(0), c.stride(1), a_scales.stride(0),
            a_scales.stride(1), b_scales.stride(0), b_scales.stride(1), _OUT_CODE[c.dtype], sched, waves)
    return _Call("g9_gemm_a4w4", args, dt, M, N, K, sched, waves, (a, b, c, a_scales, b_scales))


def gemm_a4w4(a: torch.Tensor, b: torch.Tensor, a_scales: torch.Tensor, b_scales: torch.Tensor, c: torch.Tensor,
              *, schedule="dp", waves: int = 4):
    """C = dequant(A) @ dequant(B)^T with packed MXFP4 A (M, K/2), B (N, K/2)
    and E8M0 scales (M, K/32), (N, K/32), or both in the preshuffled layout
    of quant.preshuffle_e8m0 ((ceil(K/1024), M, 32), (ceil(K/1024), N, 32);
    4-wave data-parallel kernel)."""
    _run(_a4w4_call(a, b, a_scales, b_scales, c, schedule, waves), c.device)
    return c
