"""Operand quantizers for the BF8 and MXFP4 GEMMs (torch, any device).

The reference has no quantizers (its benches cast fp16 straight to e5m2 and
draw random MXFP4 nibbles/scales, kernels/gemm/intra_wave/a8w8/bench.py:133-136,
kernels/gemm/intra_wave/a4w4/bench.py:115-146); these produce the operands of
the BF8 and MXFP4 benchmark configurations:

* ``quantize_e5m2(x)``: one fp32 scale per tensor, ``scale = absmax / 57344``
  so the largest magnitude lands on the largest finite e5m2 value, codes
  ``RNE(x / scale)``.
* ``quantize_mxfp4(x)``: OCP Microscaling v1.0 MXFP4 along the last axis,
  one E8M0 scale per 32 values: ``E = floor(log2(absmax)) - 2`` (2 is the
  largest e2m1 exponent), code ``E + 127`` (0 for an all-zero group),
  elements ``RNE(x / 2^E)`` to e2m1 saturated at +-6 with the sign kept,
  packed two per byte with the even k in the low nibble.
* ``preshuffle_e8m0(scales)``: the MXFP4 scales in the read order of the
  preshuffled-scale kernel (``g9_gemm_a4w4_preshuffled``): chunk-major, 32
  bytes per row per chunk of 32 K groups (1024 K values), byte 8j + 2s + h of
  chunk row r holding group 8s + 4h + g with g = j ^ ((r >> 2) & 3).
"""

from __future__ import annotations

import torch

E5M2_MAX = 57344.0
SCALE_GROUP = 32

# Boundaries between consecutive e2m1 magnitudes 0, .5, 1, 1.5, 2, 3, 4, 6.
_E2M1_MIDS = (0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0)


def quantize_e5m2(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Returns (codes as torch.float8_e5m2, fp32 scale tensor of shape (1,))."""
    x = x.float()
    amax = x.abs().amax()
    scale = torch.where(amax > 0, amax / E5M2_MAX, torch.ones_like(amax))
    q = (x / scale).clamp_(-E5M2_MAX, E5M2_MAX).to(torch.float8_e5m2)
    return q, scale.reshape(1).to(torch.float32)


def _e2m1_code(m: torch.Tensor) -> torch.Tensor:
    """Magnitude (after the block scale) -> e2m1 magnitude code, RNE, saturating."""
    code = torch.zeros_like(m, dtype=torch.uint8)
    for i, mid in enumerate(_E2M1_MIDS):
        above = m > mid
        # Exactly on a midpoint between codes i and i+1: round to the even code.
        tie_up = (m == mid) & (i % 2 == 1)
        code = torch.where(above | tie_up, torch.full_like(code, i + 1), code)
    return code


def quantize_mxfp4(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(R, K) float -> (packed (R, K/2) uint8, scales (R, K/32) uint8)."""
    if x.dim() != 2 or x.shape[1] % SCALE_GROUP:
        raise ValueError(f"quantize_mxfp4 needs (R, K) with K % 32 == 0, got {tuple(x.shape)}")
    R, K = x.shape
    g = x.float().reshape(R, K // SCALE_GROUP, SCALE_GROUP)
    amax = g.abs().amax(dim=-1)
    _, ex = torch.frexp(amax)  # amax = m * 2^ex, m in [0.5, 1)
    E = ex.to(torch.int32) - 3
    E = torch.where(amax > 0, E, torch.full_like(E, -127)).clamp_(-127, 127)
    scales = (E + 127).to(torch.uint8)
    y = g.double() * torch.pow(2.0, -E.double()).unsqueeze(-1)
    code = _e2m1_code(y.abs()) | torch.where(y < 0, 8, 0).to(torch.uint8)
    code = code.reshape(R, K)
    packed = (code[:, 0::2] & 0xF) | ((code[:, 1::2] & 0xF) << 4)
    return packed.contiguous(), scales.contiguous()


def dequantize_mxfp4(packed: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """Inverse view used by callers that want the fp32 operand (not by the GEMM)."""
    table = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
                         dtype=torch.float32, device=packed.device)
    codes = torch.stack([packed & 0xF, packed >> 4], dim=-1).reshape(packed.shape[0], -1)
    vals = table[codes.long()]
    s = torch.pow(2.0, scales.float() - 127.0)
    s = torch.where(scales == 255, torch.full_like(s, float("nan")), s)
    return vals * s.repeat_interleave(SCALE_GROUP, dim=1)


# Chunks of the preshuffled scale layout: 32 K groups (4 K stages of 256 values).
PS_CHUNK_GROUPS = 32


def _ps_group_order(rows: int, device=None) -> torch.Tensor:
    """(rows, 32): position 8j + 2s + h of preshuffled chunk row r holds group
    8s + 4h + g of the chunk, g = j ^ ((r >> 2) & 3).  The row-dependent XOR
    puts the 16 rows one LDS read serves on distinct bank pairs."""
    p = torch.arange(PS_CHUNK_GROUPS, device=device)
    j, s, h = p // 8, (p % 8) // 2, p % 2
    r = torch.arange(rows, device=device).unsqueeze(1)
    g = j ^ ((r >> 2) & 3)
    return 8 * s + 4 * h + g


def preshuffle_e8m0(scales: torch.Tensor) -> torch.Tensor:
    """(R, K/32) uint8 E8M0 scales -> (ceil(K/1024), R, 32) uint8 in the read
    order of g9_gemm_a4w4_preshuffled (chunk stride 32 * R bytes).  Groups
    past K/32 in the last chunk are filled with 127 (scale 1.0); the kernel
    never uses them."""
    if scales.dim() != 2 or scales.dtype != torch.uint8:
        raise ValueError(f"preshuffle_e8m0 needs a 2-D uint8 tensor, got {scales.dtype} {tuple(scales.shape)}")
    R, G = scales.shape
    chunks = -(-G // PS_CHUNK_GROUPS)
    padded = torch.full((R, chunks * PS_CHUNK_GROUPS), 127, dtype=torch.uint8, device=scales.device)
    padded[:, :G] = scales
    grouped = padded.reshape(R, chunks, PS_CHUNK_GROUPS)
    order = _ps_group_order(R, scales.device).unsqueeze(1).expand(R, chunks, PS_CHUNK_GROUPS)
    return torch.gather(grouped, 2, order).permute(1, 0, 2).contiguous()


def unshuffle_e8m0(ps: torch.Tensor, groups: int) -> torch.Tensor:
    """Inverse of preshuffle_e8m0: (chunks, R, 32) -> (R, groups)."""
    chunks, R, w = ps.shape
    if w != PS_CHUNK_GROUPS or groups > chunks * PS_CHUNK_GROUPS:
        raise ValueError(f"not a preshuffled scale tensor for {groups} groups: {tuple(ps.shape)}")
    out = torch.empty(R, chunks, PS_CHUNK_GROUPS, dtype=ps.dtype, device=ps.device)
    order = _ps_group_order(R, ps.device).unsqueeze(1).expand(R, chunks, PS_CHUNK_GROUPS)
    out.scatter_(2, order, ps.permute(1, 0, 2))
    return out.reshape(R, chunks * PS_CHUNK_GROUPS)[:, :groups].contiguous()
