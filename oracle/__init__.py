"""CPU oracle of the gfx950 GEMM path.  TEST INFRASTRUCTURE ONLY: imported by
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
checker / CPU baseline, never by the product package."""
