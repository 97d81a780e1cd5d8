"""MI355X (gfx950) NT GEMM library: FP16/BF16, BF8 and MXFP4 GEMMs with
data-parallel and stream-K tile schedules, hand-written HIP behind a C ABI
(include/gfx950_gemm.h), with the reference tutorials' Python ``matmul`` call
surface under ``gemm.{intra_wave,inter_wave}.{a16w16,a8w8,a4w4}``.
"""

__version__ = "0.1.0"
