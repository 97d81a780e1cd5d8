"""4-wave MXFP4 GEMM: drop-in for the reference's a4w4 kernel.

Replaces ``matmul(a, b, a_scales, b_scales)`` of
kernels/gemm/intra_wave/a4w4/v1_sliceMN/matmul_kernel.py:696-742:
``a`` (M, K/2) and ``b`` (N, K/2) uint8 with two e2m1 values per byte (low
nibble = even k), ``a_scales`` (M, K/32) and ``b_scales`` (N, K/32) uint8 E8M0
(any strides; non-row-major views are repacked), bf16 output.  Scales already
in the preshuffled layout of ``quant.preshuffle_e8m0`` (3-D tensors) run the
preshuffled-scale kernel; its results are bit-identical.
"""

import torch

from ..._launch import gemm_a4w4

BLOCK_M, BLOCK_N, BLOCK_K = 256, 256, 256
NUM_WARPS = 4
NUM_XCDS = 8
GROUP_SIZE_M = 4
SCALE_GROUP_SIZE = 32
MIN_K = BLOCK_K
KERNEL_NAME = "g9_a4w4"


def matmul(a, b, a_scales, b_scales, *, out_dtype=torch.bfloat16, schedule="dp"):
    M = a.shape[0]
    N = b.shape[0]
    c = torch.empty((M, N), device=a.device, dtype=out_dtype)
    return gemm_a4w4(a, b, a_scales, b_scales, c, schedule=schedule, waves=NUM_WARPS)
