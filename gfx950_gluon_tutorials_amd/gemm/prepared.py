"""Prepared GEMM launches: each rotating argument set is validated and bound
once, and a launch is a single C call that only enqueues.

Replaces the reference's ``PreparedKernel`` (scripts/prepared_kernel.py:53-138),
which binds a compiled Gluon kernel to each rotating tensor set so that the
profiler timing loop of scripts/benchmark_prepared.py:135-271 enters the
compiled launcher directly: ``PreparedGemm.<op>(sets, ...)`` plays the part of
``PreparedKernel.create`` and ``prepared(slot)`` of ``prepared(slot)``.

Here the host work of a ``matmul`` call (tensor checks, pointers and strides,
the schedule, and a C call of ~20 arguments that validates them again and
resolves the kernel, grid and parameter block) is done once per set by the
``g9_plan_*`` entry points of the C ABI; ``prepared(slot)`` is one
``g9_plan_launch(plan, stream)`` call.  Each launch is the launch the wrapper
makes for the same arguments: same kernels, bit-identical results.

Differences from the wrappers, all by design:

* no hidden copies: every operand must already be in a layout the kernels
  read in place (A rows K-contiguous and 16-byte aligned, B the (K, N) view of
  an (N, K) buffer with aligned rows, MXFP4 scales row-major, K-major or
  preshuffled as the wrappers describe); anything else raises ValueError,
  because a copy made here would go stale when the caller updates the
  original;
* the stream is the current stream of the operands' device at creation, as
  the reference's ``PreparedKernel.create`` takes it;
* a stream-K or split-K object owns its workspace (sized for its largest set
  and shared by its slots, which its stream orders), so cached workspaces of
  the wrappers can grow or be released without affecting it; ``error()``
  reports a timed-out stream-K flag wait.
"""

from __future__ import annotations

import ctypes

import torch

from .. import _lib
from . import _launch


def _set_list(sets) -> list[tuple]:
    sets = [tuple(s) for s in sets]
    if not sets:
        raise ValueError("at least one argument set is required")
    return sets


class PreparedGemm:
    """Launches of one GEMM over one or more rotating argument sets."""

    def __init__(self, calls: list, dev: torch.device):
        lib = _lib.load()
        devs = {t.device for call in calls for t in call.keep if isinstance(t, torch.Tensor)}
        if len(devs) != 1:
            raise ValueError(f"all argument sets must be on one device, got {sorted(map(str, devs))}")
        self.device = dev
        self.stream = _launch._stream(dev)
        self.schedule = calls[0].schedule
        need = max(lib.g9_workspace_size(c.dtype, c.M, c.N, c.K, c.schedule, c.waves) for c in calls)
        self._ws = None
        if need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=dev)
            _lib.check(lib.g9_workspace_init(self._ws.data_ptr(), need, self.stream), "g9_workspace_init")
        ws = self._ws.data_ptr() if self._ws is not None else None
        self._plans = []
        for call in calls:
            plan = (ctypes.c_uint64 * (_lib.G9_PLAN_BYTES // 8))()
            entry = call.entry.replace("g9_gemm_", "g9_plan_", 1)
            _lib.check(getattr(lib, entry)(ctypes.addressof(plan), *call.args, ws, need), entry)
            self._plans.append(plan)
        # The plans hold raw pointers into these tensors: keep them alive.
        self._keep = tuple(call.keep for call in calls)
        self._addr = tuple(ctypes.addressof(p) for p in self._plans)
        self._launch = lib.g9_plan_launch

    @classmethod
    def a16w16(cls, sets, *, schedule="dp", waves: int = 4) -> "PreparedGemm":
        """`sets`: (a, b, c) per slot, as the a16w16 ``matmul(a, b, c)`` takes
        them (b the (K, N) operand)."""
        sets = _set_list(sets)
        calls = [_launch._a16w16_call(a, b, c, schedule, waves, strict=True) for a, b, c in sets]
        return cls(calls, sets[0][2].device)

    @classmethod
    def a8w8(cls, sets, *, schedule="dp", waves: int = 4) -> "PreparedGemm":
        """`sets`: (a, b, c, a_scale, b_scale) per slot: e5m2 a (M, K), b the
        (K, N) operand, c (M, N) fp16 or bf16, scales one-element fp32 device
        tensors or None."""
        sets = _set_list(sets)
        calls = [_launch._a8w8_call(a, b, c, sa, sb, schedule, waves, strict=True) for a, b, c, sa, sb in sets]
        return cls(calls, sets[0][2].device)

    @classmethod
    def a4w4(cls, sets, *, schedule="dp", waves: int = 4) -> "PreparedGemm":
        """`sets`: (a, b, a_scales, b_scales, c) per slot, as the a4w4
        ``matmul`` takes them (scales row-major, K-major views or
        preshuffled)."""
        sets = _set_list(sets)
        calls = [_launch._a4w4_call(a, b, sa, sb, c, schedule, waves, strict=True) for a, b, sa, sb, c in sets]
        return cls(calls, sets[0][4].device)

    @property
    def slots(self) -> int:
        return len(self._addr)

    def __call__(self, slot: int = 0) -> None:
        rc = self._launch(self._addr[slot % len(self._addr)], self.stream)
        if rc:
            _lib.check(rc, "g9_plan_launch")

    def error(self) -> int:
        """Synchronises the stream and returns 1 if a stream-K flag wait of a
        launch since the last call timed out (that launch's output is wrong),
        else 0; the workspace is cleared again after a timeout."""
        if self._ws is None:
            return 0
        lib = _lib.load()
        out = ctypes.c_int(0)
        _lib.check(lib.g9_workspace_error(self._ws.data_ptr(), self._ws.numel(), self.stream, ctypes.byref(out)),
                   "g9_workspace_error")
        if out.value:
            _lib.check(lib.g9_workspace_init(self._ws.data_ptr(), self._ws.numel(), self.stream), "g9_workspace_init")
        return out.value
