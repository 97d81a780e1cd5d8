"""8-wave (two waves per SIMD, ping-pong) FP16/BF16 GEMM.

Provides the interface the reference's 8-wave bench binds
(kernels/gemm/inter_wave/a16w16/bench.py:48: ``KERNEL_NAME, MIN_K,
matmul_kernel_only``), whose kernel source is absent from the reference.
``matmul_kernel_only(a, b_t, c)`` takes B pre-transposed to (N, K) contiguous
and a pre-allocated C; ``matmul(a, b, c=None)`` takes the (K, N) operand.
"""

import torch

from ..._launch import gemm_a16w16

BLOCK_M, BLOCK_N, BLOCK_K = 256, 256, 64
NUM_WARPS = 8
WARPS_M, WARPS_N = 2, 4
NUM_XCDS = 8
GROUP_SIZE_M = 4
MIN_K = BLOCK_K
KERNEL_NAME = "g9_a16w16"


def matmul_kernel_only(a, b_t, c, *, schedule="dp"):
    """C = A @ B_t^T; b_t is (N, K) K-contiguous, c pre-allocated (M, N) a.dtype."""
    return gemm_a16w16(a, b_t.t(), c, schedule=schedule, waves=NUM_WARPS)


def matmul(a, b, c=None, *, schedule="dp"):
    assert a.shape[1] == b.shape[0], "Incompatible dimensions"
    M, K = a.shape
    N = b.shape[1]
    if c is None:
        c = torch.empty((M, N), device=a.device, dtype=a.dtype)
    return gemm_a16w16(a, b, c, schedule=schedule, waves=NUM_WARPS)
