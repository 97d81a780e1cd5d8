"""8-wave (two waves per SIMD, ping-pong) BF8 (fp8 e5m2) GEMM.

Drop-in for kernels/gemm/inter_wave/a8w8/matmul_kernel.py:343-388:
``matmul_kernel_only(a, b_t, c)`` (B pre-transposed to (N, K), C
pre-allocated, fp16 by default) and ``matmul(a, b, c=None)`` with the (K, N)
operand.  Unlike the reference, ``matmul`` does not copy a B that is already a
K-contiguous view.  Keyword-only extras: per-tensor fp32 scales and, for
``matmul``, the output dtype.
"""

import torch

from ..._launch import gemm_a8w8

BLOCK_M, BLOCK_N, BLOCK_K = 256, 256, 128
NUM_WARPS = 8
WARPS_M, WARPS_N = 2, 4
NUM_XCDS = 8
GROUP_SIZE_M = 4
MIN_K = 4 * BLOCK_K
KERNEL_NAME = "g9_a8w8"


def matmul_kernel_only(a, b_t, c, *, a_scale=None, b_scale=None, schedule="dp"):
    """C = (A @ B_t^T) * a_scale * b_scale; b_t (N, K) contiguous, c pre-allocated."""
    return gemm_a8w8(a, b_t.t(), c, a_scale=a_scale, b_scale=b_scale, schedule=schedule, waves=NUM_WARPS)


def matmul(a, b, c=None, *, a_scale=None, b_scale=None, out_dtype=torch.float16, schedule="dp"):
    assert a.shape[1] == b.shape[0], "Incompatible dimensions"
    M, K = a.shape
    N = b.shape[1]
    if c is None:
        c = torch.empty((M, N), device=a.device, dtype=out_dtype)
    return gemm_a8w8(a, b, c, a_scale=a_scale, b_scale=b_scale, schedule=schedule, waves=NUM_WARPS)
