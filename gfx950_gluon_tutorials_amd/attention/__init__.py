"""Flash-attention forward for gfx950: the drop-in for the reference's
``kernels/attention`` launchers (``fmha_v3.run_gluon_attention``,
``fmha_v4.run_gluon_attention``) and their host-side helpers (``common``).

The kernel is hand-written HIP behind ``g9_fmha_fwd`` (include/gfx950_fmha.h).
"""

from .common import MetaData, compute_flops, get_shape_from_layout, get_strides_from_layout, input_helper
from .fmha_v4 import run_gluon_attention

__all__ = [
    "MetaData",
    "compute_flops",
    "get_shape_from_layout",
    "get_strides_from_layout",
    "input_helper",
    "run_gluon_attention",
]
