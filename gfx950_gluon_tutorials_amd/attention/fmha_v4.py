"""Drop-in for kernels/attention/fmha_v4.py: ``run_gluon_attention`` with the
lazy softmax rescale (a row's running max advances only when a tile exceeds it
by more than 8 in log2 units; the accumulator rescale is skipped for waves
whose rows did not move)."""

from __future__ import annotations

from ._launch import fmha_forward
from .common import MetaData


def run_gluon_attention(q, k, v, o, metadata: MetaData, scale_on_q: bool = True, *, lse=None):
    """Runs the gfx950 flash-attention forward on q, k, v and writes the output
    into ``o`` (kernels/attention/fmha_v4.py:761-790).

    Non-causal self-attention, Q and K sequence lengths equal and a multiple
    of 64, head dim 128 or 64, fp16 or bf16, ``bhsd`` or ``bshd`` layout, grouped
    K/V heads allowed.  ``scale_on_q`` folds sm_scale * log2(e) into Q before
    the loop, as the reference's SCALE_ON_Q.  ``lse`` (keyword, optional)
    receives the per-query log-sum-exp."""
    fmha_forward(q, k, v, o, metadata, scale_on_q, 4, lse=lse)
