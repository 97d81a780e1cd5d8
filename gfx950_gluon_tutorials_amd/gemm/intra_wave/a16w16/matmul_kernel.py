"""4-wave FP16/BF16 GEMM: drop-in for the reference's final a16w16 kernel.

Replaces ``matmul`` of kernels/gemm/intra_wave/a16w16/v9_beyond_hotloop/matmul_kernel.py:390-424
(same signature, argument order, layouts and output dtype).  ``b`` is the
(K, N) operand, normally the ``.T`` view of an (N, K) buffer as the reference
bench passes it (kernels/gemm/intra_wave/a16w16/bench.py:208); the output has
``a.dtype``.  The launch is asynchronous on the current stream.

``schedule`` (keyword-only, an addition) selects the data-parallel grid
("dp", the reference's only schedule), persistent stream-K ("streamk"),
split-K ("splitk": for outputs of at most half a wave of 256x256 tiles, K cut
into segments whose fp32 partials a second kernel sums in a fixed order;
deterministic, within rounding of "dp", which it runs on fuller grids), or
"auto": stream-K for outputs of more than one and at most 1.25 waves of
256x256 tiles per CU, where it measured faster, data-parallel otherwise.
"""

import torch

from ..._launch import gemm_a16w16

BLOCK_M, BLOCK_N, BLOCK_K = 256, 256, 64
NUM_WARPS = 4
NUM_XCDS = 8
GROUP_SIZE_M = 4
MIN_K = BLOCK_K
KERNEL_NAME = "g9_a16w16"


def matmul(a, b, c=None, *, schedule="dp"):
    assert a.shape[1] == b.shape[0], "Incompatible dimensions"
    assert a.is_contiguous(), "Matrix A must be contiguous"
    M, K = a.shape
    K, N = b.shape
    if c is None:
        c = torch.empty((M, N), device=a.device, dtype=a.dtype)
    return gemm_a16w16(a, b, c, schedule=schedule, waves=NUM_WARPS)
