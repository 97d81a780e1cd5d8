"""4-wave BF8 (fp8 e5m2) GEMM: drop-in for the reference's a8w8 kernel.

Replaces ``matmul(a, b)`` of kernels/gemm/intra_wave/a8w8/matmul_kernel.py:437-470:
same positional signature, ``b`` a (K, N) view, fp16 output by default.  The
keyword-only extras carry the per-tensor fp32 scales and the output dtype of
the BF8 configuration (C = (A @ B) * a_scale * b_scale, written as bf16 or
fp16); with their defaults the result is exactly the reference's unscaled
fp16 product.
"""

import torch

from ..._launch import gemm_a8w8

BLOCK_M, BLOCK_N, BLOCK_K = 256, 256, 128
NUM_WARPS = 4
NUM_XCDS = 8
GROUP_SIZE_M = 4
MIN_K = BLOCK_K
KERNEL_NAME = "g9_a8w8"


def matmul(a, b, *, a_scale=None, b_scale=None, out_dtype=torch.float16, schedule="dp"):
    assert a.shape[1] == b.shape[0], "Incompatible dimensions"
    assert a.is_contiguous(), "Matrix A must be contiguous"
    M, K = a.shape
    K, N = b.shape
    c = torch.empty((M, N), device=a.device, dtype=out_dtype)
    return gemm_a8w8(a, b, c, a_scale=a_scale, b_scale=b_scale, schedule=schedule, waves=NUM_WARPS)
