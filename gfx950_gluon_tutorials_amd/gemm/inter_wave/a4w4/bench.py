"""Bench of the 8-wave MXFP4 GEMM with the command line of the reference's
kernels/gemm/inter_wave/a4w4/bench.py: correctness against torch on the
reference's inputs, then TFLOPS over its K list, or --rocprof launches for an
external rocprofv3 kernel trace (gemm/utils/family_bench.py)::

    python -m gfx950_gluon_tutorials_amd.gemm.inter_wave.a4w4.bench [--K 8192] [--rocprof]
"""

import sys

from ...utils.family_bench import main
from .matmul_kernel import NUM_WARPS, matmul

if __name__ == "__main__":
    sys.exit(main("a4w4", matmul, NUM_WARPS))
