"""Launch of the gfx950 flash-attention kernel (``g9_fmha_fwd``) from torch
tensors: the argument checks of the reference launchers, then one call
through the C ABI on the current stream.  No fallback: without the built
library the call raises."""

from __future__ import annotations

import torch

from .. import _lib
from .common import get_shape_from_layout, get_strides_from_layout

BLOCK_N = 64  # keys per tile: the sequence length must be a multiple of it
HEAD_DIMS = (64, 128)
_DTYPES = {torch.float16: _lib.G9_F16, torch.bfloat16: _lib.G9_BF16}


def fmha_forward(q, k, v, o, metadata, scale_on_q: bool, variant: int, lse=None) -> None:
    """Writes softmax(q k^T * sm_scale) v into ``o``.

    The checks follow run_gluon_attention (kernels/attention/fmha_v4.py:761-775):
    non-causal only, K sequence length a multiple of 64, Q and K sequence
    lengths equal (assertions there and here); beyond those this kernel needs
    head dim 64 or 128 and 16-bit tensors on one GPU (ValueError).  ``lse``, if
    given, is a contiguous fp32 (batch, query heads, seq) tensor that receives
    each query's natural-log log-sum-exp of its scaled scores."""
    assert not metadata.causal, "the gfx950 FMHA kernel supports non-causal attention only"
    assert metadata.max_seqlens_k % BLOCK_N == 0, "K seqlen must be a multiple of BLOCK_N (64)"
    assert metadata.max_seqlens_q == metadata.max_seqlens_k, "combined N_CTX requires Q seqlen == K seqlen"
    batch, nheads_q, nheads_k, head_size = get_shape_from_layout(q, k, metadata)
    assert head_size & (head_size - 1) == 0, "head dim must be a power of two"
    if head_size not in HEAD_DIMS:
        raise ValueError(f"head dim {head_size} unsupported: the gfx950 kernels are built for {HEAD_DIMS}")
    if q.dtype not in _DTYPES or any(t.dtype != q.dtype for t in (k, v, o)):
        raise ValueError(f"q, k, v, o must share one of {list(_DTYPES)}; got {[t.dtype for t in (q, k, v, o)]}")
    dev = q.device
    if dev.type != "cuda" or any(t.device != dev for t in (k, v, o)):
        raise ValueError("q, k, v, o must be on one GPU")
    S = metadata.max_seqlens_q
    order = (0, 1, 2, 3) if metadata.layout == "bhsd" else (0, 2, 1, 3)
    want_q = (batch, nheads_q, S, head_size)
    want_k = (batch, nheads_k, S, head_size)
    for name, t, want in (("q", q, want_q), ("k", k, want_k), ("v", v, want_k), ("o", o, want_q)):
        got = tuple(t.shape[i] for i in order)
        if got != want:
            raise ValueError(f"{name} has (batch, head, seq, dim) {got}, expected {want}")
    if nheads_q % nheads_k != 0:
        raise ValueError(f"query heads {nheads_q} not a multiple of key/value heads {nheads_k}")
    if lse is not None:
        if (lse.dtype != torch.float32 or not lse.is_contiguous() or tuple(lse.shape) != (batch, nheads_q, S)
                or lse.device != dev):
            raise ValueError("lse must be a contiguous fp32 (batch, query heads, seq) tensor on the same GPU")
    strides = get_strides_from_layout(q, k, v, o, metadata)
    arr = [(_lib.ctypes.c_int64 * 4)(*st) for st in strides]
    lib = _lib.load()
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        rc = lib.g9_fmha_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                             lse.data_ptr() if lse is not None else None, batch, nheads_q, nheads_k, S, head_size,
                             arr[0], arr[1], arr[2], arr[3], float(metadata.sm_scale), _DTYPES[q.dtype],
                             1 if scale_on_q else 0, variant, stream)
    _lib.check(rc, "g9_fmha_fwd")
