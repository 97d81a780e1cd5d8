"""Bench of the 4-wave FP16/BF16 GEMM with the command line of the reference's
kernels/gemm/intra_wave/a16w16/bench.py: correctness against torch on the
reference's inputs, then TFLOPS over its K list, or --rocprof launches for an
external rocprofv3 kernel trace (gemm/utils/family_bench.py)::

    python -m gfx950_gluon_tutorials_amd.gemm.intra_wave.a16w16.bench [--K 8192] [--rocprof]
"""

import sys

from ...utils.family_bench import main
from .matmul_kernel import NUM_WARPS, matmul

if __name__ == "__main__":
    sys.exit(main("a16w16", matmul, NUM_WARPS))
