"""Drop-in for kernels/attention/fmha_v3.py: ``run_gluon_attention`` with the
eager softmax rescale (the accumulator is rescaled whenever a row's running
max grows)."""

from __future__ import annotations

from ._launch import fmha_forward
from .common import MetaData


def run_gluon_attention(q, k, v, o, metadata: MetaData, scale_on_q: bool = True, *, lse=None):
    """Runs the gfx950 flash-attention forward on q, k, v and writes the output
    into ``o`` (kernels/attention/fmha_v3.py:522-549); arguments as
    fmha_v4.run_gluon_attention."""
    fmha_forward(q, k, v, o, metadata, scale_on_q, 3, lse=lse)
