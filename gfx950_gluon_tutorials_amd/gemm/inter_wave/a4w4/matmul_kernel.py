"""8-wave (two waves per SIMD, ping-pong) MXFP4 GEMM.

Drop-in for kernels/gemm/inter_wave/a4w4/v2_mfma32x32x64/matmul_kernel.py:614-668:
``matmul_kernel_only(a, b, a_scales, b_scales, c)`` and
``matmul(a, b, a_scales, b_scales, c=None)``; bf16 output by default.
"""

import torch

from ..._launch import gemm_a4w4

BLOCK_M, BLOCK_N, BLOCK_K = 256, 256, 256
NUM_WARPS = 8
WARPS_M, WARPS_N = 2, 4
NUM_XCDS = 8
GROUP_SIZE_M = 4
SCALE_GROUP_SIZE = 32
MIN_K = 4 * BLOCK_K
KERNEL_NAME = "g9_a4w4"


def matmul_kernel_only(a, b, a_scales, b_scales, c, *, schedule="dp"):
    return gemm_a4w4(a, b, a_scales, b_scales, c, schedule=schedule, waves=NUM_WARPS)


def matmul(a, b, a_scales, b_scales, c=None, *, out_dtype=torch.bfloat16, schedule="dp"):
    M = a.shape[0]
    N = b.shape[0]
    if c is None:
        c = torch.empty((M, N), device=a.device, dtype=out_dtype)
    return gemm_a4w4(a, b, a_scales, b_scales, c, schedule=schedule, waves=NUM_WARPS)
