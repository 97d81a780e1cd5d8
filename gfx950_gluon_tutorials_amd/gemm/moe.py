"""Grouped ("MoE") GEMMs: tokens sorted by expert times per-expert weights.

No counterpart in the reference: its roadmap plans an MXFP4 MoE kernel
("4-bit + Scales" in its ROADMAP.md).  The operands follow the dense wrappers'
layouts, with an expert dimension in front of B:

* ``a``: (T, K) tokens (fp16/bf16 or BF8 e5m2), or (T, K/2) packed MXFP4
  bytes, rows sorted by expert;
* ``b``: (E, N, K) expert weights, or (E, N, K/2) packed MXFP4 bytes, each
  expert's N rows K-contiguous; BF8 takes one fp32 scale per expert;
* ``a_scales`` (T, K/32) and ``b_scales`` (E, N, K/32) E8M0 bytes for MXFP4;
* ``expert_offsets``: (E + 1,) int32 on the device, prefix sums of the tokens
  per expert (offsets[0] = 0, offsets[E] <= T): expert e owns rows
  [offsets[e], offsets[e + 1]) of A and C.

C[t] = A[t] . B_e^T for every row t of expert e, computed by the same
data-parallel tile as the dense kernels (one 256x256 tile per workgroup, 4
waves), so each expert's rows are bit-identical to a dense ``matmul`` of that
expert's slice.  Rows no expert owns are not written (with ``c=None`` they are
left as ``torch.empty`` leaves them).  The launch is asynchronous on the
current stream; the offsets are read on the device (no synchronisation).
"""

from __future__ import annotations

import torch

from .. import _lib
from ._launch import _DTYPE_CODE, _OUT_CODE, _require_device, _stream

KERNEL_NAME = "_moe_4w"


def _offsets(expert_offsets: torch.Tensor, dev, E: int) -> torch.Tensor:
    if expert_offsets.dtype != torch.int32 or expert_offsets.dim() != 1 or expert_offsets.numel() != E + 1:
        raise ValueError(f"expert_offsets must be an int32 vector of E + 1 = {E + 1} prefix sums, got "
                         f"{expert_offsets.dtype} {tuple(expert_offsets.shape)}")
    if expert_offsets.device != dev:
        raise ValueError(f"expert_offsets on {expert_offsets.device}, operands on {dev}")
    return expert_offsets.contiguous()


def _rows(t: torch.Tensor) -> torch.Tensor:
    return t if (t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and (t.stride(-2) * t.element_size()) % 16 == 0) \
        else t.contiguous()


def moe_matmul(a: torch.Tensor, b: torch.Tensor, expert_offsets: torch.Tensor, c: torch.Tensor | None = None):
    """FP16/BF16 grouped GEMM: a (T, K), b (E, N, K), c (T, N) in a.dtype."""
    assert a.dim() == 2 and b.dim() == 3 and a.shape[1] == b.shape[2], "Incompatible dimensions"
    T, K = a.shape
    E, N = b.shape[0], b.shape[1]
    if c is None:
        c = torch.empty((T, N), device=a.device, dtype=a.dtype)
    dev = _require_device(a, b, c)
    if a.dtype not in _DTYPE_CODE or b.dtype != a.dtype or c.dtype != a.dtype:
        raise ValueError(f"moe_matmul needs matching fp16/bf16 a, b, c; got {a.dtype}, {b.dtype}, {c.dtype}")
    if c.shape != (T, N) or c.stride(1) != 1:
        raise ValueError(f"c must be a ({T}, {N}) row-major view, got {tuple(c.shape)} strides {c.stride()}")
    off = _offsets(expert_offsets, dev, E)
    a, b = _rows(a), _rows(b)
    es = a.element_size()
    rc = _lib.load().g9_moe_a16w16(a.data_ptr(), b.data_ptr(), c.data_ptr(), off.data_ptr(), T, N, K, E,
                                   a.stride(0), b.stride(1), b.stride(0) * es, c.stride(0), _DTYPE_CODE[a.dtype],
                                   _stream(dev))
    _lib.check(rc, "g9_moe_a16w16")
    return c


def moe_matmul_a8w8(a: torch.Tensor, b: torch.Tensor, expert_offsets: torch.Tensor, c: torch.Tensor | None = None,
                    *, a_scale=None, b_scales=None, out_dtype=torch.bfloat16):
    """BF8 (fp8 e5m2) grouped GEMM: a (T, K), b (E, N, K); C rows of expert e =
    (A . B_e^T) * a_scale * b_scales[e] in out_dtype.  a_scale: one fp32 value
    (tensor or float), b_scales: E fp32 values; None = 1."""
    assert a.dim() == 2 and b.dim() == 3 and a.shape[1] == b.shape[2], "Incompatible dimensions"
    T, K = a.shape
    E, N = b.shape[0], b.shape[1]
    if c is None:
        c = torch.empty((T, N), device=a.device, dtype=out_dtype)
    dev = _require_device(a, b, c)
    if a.dtype != torch.float8_e5m2 or b.dtype != torch.float8_e5m2:
        raise ValueError(f"moe a8w8 needs float8_e5m2 operands; got {a.dtype}, {b.dtype}")
    if c.dtype not in _OUT_CODE:
        raise ValueError(f"moe a8w8 output must be bf16 or fp16, got {c.dtype}")
    if c.shape != (T, N) or c.stride(1) != 1:
        raise ValueError(f"c must be a ({T}, {N}) row-major view, got {tuple(c.shape)} strides {c.stride()}")
    off = _offsets(expert_offsets, dev, E)
    a, b = _rows(a), _rows(b)
    sa = None
    if a_scale is not None:
        sa = a_scale if isinstance(a_scale, torch.Tensor) else torch.tensor([float(a_scale)])
        if sa.numel() != 1:
            raise ValueError("a_scale is per tensor: one fp32 value")
        sa = sa.detach().reshape(1).to(device=dev, dtype=torch.float32)
    sb = None
    if b_scales is not None:
        if not isinstance(b_scales, torch.Tensor) or b_scales.numel() != E:
            raise ValueError(f"b_scales must be a tensor of E = {E} fp32 values")
        sb = b_scales.detach().reshape(E).to(device=dev, dtype=torch.float32).contiguous()
    rc = _lib.load().g9_moe_a8w8(a.data_ptr(), b.data_ptr(), c.data_ptr(), off.data_ptr(),
                                 sa.data_ptr() if sa is not None else None, sb.data_ptr() if sb is not None else None,
                                 T, N, K, E, a.stride(0), b.stride(1), b.stride(0), c.stride(0), _OUT_CODE[c.dtype],
                                 _stream(dev))
    _lib.check(rc, "g9_moe_a8w8")
    return c


def moe_matmul_a4w4(a: torch.Tensor, b: torch.Tensor, a_scales: torch.Tensor, b_scales: torch.Tensor,
                    expert_offsets: torch.Tensor, c: torch.Tensor | None = None, *, out_dtype=torch.bfloat16):
    """MXFP4 grouped GEMM: a (T, K/2), b (E, N, K/2), a_scales (T, K/32), b_scales (E, N, K/32) uint8;
    c (T, N) in out_dtype (bf16 by default, as the dense a4w4 wrapper)."""
    assert a.dim() == 2 and b.dim() == 3 and a.shape[1] == b.shape[2], "Incompatible dimensions"
    T, Kp = a.shape
    E, N = b.shape[0], b.shape[1]
    K = 2 * Kp
    if c is None:
        c = torch.empty((T, N), device=a.device, dtype=out_dtype)
    dev = _require_device(a, b, a_scales, b_scales, c)
    for name, t in (("a", a), ("b", b), ("a_scales", a_scales), ("b_scales", b_scales)):
        if t.dtype != torch.uint8:
            raise ValueError(f"moe a4w4 {name} must be uint8, got {t.dtype}")
    if c.dtype not in _OUT_CODE:
        raise ValueError(f"moe a4w4 output must be bf16 or fp16, got {c.dtype}")
    if a_scales.shape != (T, K // 32) or b_scales.shape != (E, N, K // 32):
        raise ValueError(f"scales must be ({T}, {K // 32}) and ({E}, {N}, {K // 32}); got "
                         f"{tuple(a_scales.shape)}, {tuple(b_scales.shape)}")
    if c.shape != (T, N) or c.stride(1) != 1:
        raise ValueError(f"c must be a ({T}, {N}) row-major view, got {tuple(c.shape)} strides {c.stride()}")
    off = _offsets(expert_offsets, dev, E)
    a, b = _rows(a), _rows(b)
    if a_scales.stride(1) != 1 or a_scales.stride(0) % 4 or a_scales.data_ptr() % 4:
        a_scales = a_scales.contiguous()
    if b_scales.stride(2) != 1 or b_scales.stride(1) % 4 or b_scales.stride(0) % 4 or b_scales.data_ptr() % 4:
        b_scales = b_scales.contiguous()
    rc = _lib.load().g9_moe_a4w4(a.data_ptr(), b.data_ptr(), c.data_ptr(), a_scales.data_ptr(), b_scales.data_ptr(),
                                 off.data_ptr(), T, N, K, E, a.stride(0), b.stride(1), b.stride(0),
                                 a_scales.stride(0), b_scales.stride(1), b_scales.stride(0), c.stride(0),
                                 _OUT_CODE[c.dtype], _stream(dev))
    _lib.check(rc, "g9_moe_a4w4")
    return c
