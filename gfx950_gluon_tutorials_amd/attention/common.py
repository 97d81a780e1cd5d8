"""Host-side helpers of the attention drop-in, with the reference's names and
meaning (kernels/attention/common.py:56-112, 177-184): the problem descriptor,
the shape / stride readers for the ``bhsd`` and ``bshd`` layouts, the input
generator and the FLOP model.  The correctness reference lives with the test
oracle, not here.
"""

from __future__ import annotations

import torch

LAYOUTS = ("bhsd", "bshd")


class MetaData:
    """Descriptor of one attention problem (kernels/attention/common.py:56-69).

    Non-causal self-attention in the ``bhsd`` or ``bshd`` layout; the fields
    are the ones the launchers read."""

    causal = False
    layout = None
    max_seqlens_q = 0
    max_seqlens_k = 0

    def __init__(self, sm_scale=1.0):
        self.sm_scale = sm_scale


def get_shape_from_layout(q, k, metadata):
    """(batch, query heads, key/value heads, head dim) of a problem
    (kernels/attention/common.py:72-81)."""
    if metadata.layout == "bhsd":
        batch, nheads_q, _, head_size = q.shape
        nheads_k = k.shape[1]
    elif metadata.layout == "bshd":
        batch, _, nheads_q, head_size = q.shape
        nheads_k = k.shape[2]
    else:
        raise ValueError(f"Unsupported layout: {metadata.layout}")
    return batch, nheads_q, nheads_k, head_size


def _axis_order(layout):
    if layout == "bhsd":
        return (0, 1, 2, 3)
    if layout == "bshd":
        return (0, 2, 1, 3)
    raise ValueError(f"Unsupported layout: {layout}")


def get_strides_from_layout(q, k, v, o, metadata):
    """Element strides of q, k, v, o in (batch, head, seq, dim) order
    (kernels/attention/common.py:84-92)."""
    order = _axis_order(metadata.layout)
    return tuple(tuple(t.stride(i) for i in order) for t in (q, k, v, o))


def input_helper(Z, HQ, HK, N_CTX_Q, N_CTX_K, D_HEAD, dtype, layout, requires_grad=False, device="cuda"):
    """Seeded standard-normal q, k, v in ``layout`` and their MetaData
    (kernels/attention/common.py:95-112; ``device`` added so the same inputs
    can be drawn on the CPU)."""
    torch.manual_seed(20)

    def rand(heads, n_ctx):
        shape = (Z, heads, n_ctx, D_HEAD) if layout == "bhsd" else (Z, n_ctx, heads, D_HEAD)
        return torch.randn(shape, dtype=dtype, device=device, requires_grad=requires_grad)

    if layout not in LAYOUTS:
        raise ValueError(f"Unsupported layout: {layout}")
    q = rand(HQ, N_CTX_Q)
    k = rand(HK, N_CTX_K)
    v = rand(HK, N_CTX_K)
    md = MetaData(sm_scale=D_HEAD**-0.5)
    md.max_seqlens_q = N_CTX_Q
    md.max_seqlens_k = N_CTX_K
    md.layout = layout
    return q, k, v, md


def compute_flops(B, HQ, M, N, D, causal):
    """FLOPs of the forward pass, two B*HQ*M*N*D matmuls
    (kernels/attention/common.py:177-184)."""
    if causal:
        valid = ((N**2 + N) / 2) if M > N else (M * N - ((M**2 - M) / 2))
        flops_per_matmul = 2.0 * B * HQ * valid * D
    else:
        flops_per_matmul = 2.0 * B * HQ * M * N * D
    return 2 * flops_per_matmul
