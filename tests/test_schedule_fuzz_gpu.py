"""Seeded random shapes through every schedule and scale layout (GPU, C ABI).

Each case draws M, N (any size, 1 .. 2000), K (a multiple of 8 for the 16-bit
types, of 256 for MXFP4) from a fixed seed and checks the invariants the
schedules promise on the same inputs:

* FP16: stream-K with 256x256 and with 256x128 tiles bit-identical to
  data-parallel, split-K within the FP16 tolerance of it, 8 waves
  bit-identical to 4 waves;
* MXFP4: K-major and preshuffled scale layouts bit-identical to row-major,
  stream-K bit-identical to data-parallel.

The sizes stay small enough that the whole file runs in seconds.
"""

import numpy as np
import pytest
import torch

from gfx950_gluon_tutorials_amd import quant
from gfx950_gluon_tutorials_amd.gemm import _launch

pytestmark = pytest.mark.gpu

_RNG = np.random.default_rng(20261202)
_F16_CASES = [(int(_RNG.integers(1, 2000)), int(_RNG.integers(1, 2000)), 8 * int(_RNG.integers(1, 400)))
              for _ in range(12)]
# Every other MXFP4 case has M and N multiples of 4, so its K-major views are
# read in place (the others are repacked row-major by the wrapper).
_FP4_CASES = [((4 if i % 2 == 0 else 1) * int(_RNG.integers(1, 375 if i % 2 == 0 else 1500)),
               (4 if i % 2 == 0 else 1) * int(_RNG.integers(1, 375 if i % 2 == 0 else 1500)),
               256 * int(_RNG.integers(1, 12))) for i in range(8)]


def _say(msg):
    print(f"\n[case] {msg}", flush=True)


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy()


def _clean(dev):
    assert _launch.WORKSPACES.error(dev) == 0, "a stream-K flag wait timed out"


@pytest.mark.parametrize("M,N,K", _F16_CASES)
def test_fp16_schedules_agree(gpu, M, N, K):
    _say(f"fuzz fp16 {M}x{N}x{K}")
    gen = torch.Generator().manual_seed(M * 7919 + N * 31 + K)
    a = (torch.randn(M, K, generator=gen) * 0.3).half().to(gpu)
    b = (torch.randn(N, K, generator=gen) * 0.3).half().to(gpu)

    def run(schedule, waves=4):
        c = torch.empty(M, N, dtype=torch.float16, device=gpu)
        return _launch.gemm_a16w16(a, b.T, c, schedule=schedule, waves=waves)

    dp = run("dp")
    outs = {s: run(s) for s in ("streamk", "streamk_half")}
    dp8 = run("dp", waves=8)
    sp = run("splitk")
    torch.cuda.synchronize()
    _clean(gpu)
    for s, c in outs.items():
        np.testing.assert_array_equal(_bits(c), _bits(dp), err_msg=s)
    np.testing.assert_array_equal(_bits(dp8), _bits(dp))
    # Split-K sums fp32 partials in another order: within the FP16 tolerance.
    tol = 1e-2 * np.sqrt(K) * 0.3 * 0.3
    np.testing.assert_allclose(sp.float().cpu().numpy(), dp.float().cpu().numpy(), rtol=1e-2, atol=tol)


@pytest.mark.parametrize("M,N,K", _FP4_CASES)
def test_mxfp4_layouts_and_schedules_agree(gpu, M, N, K):
    _say(f"fuzz mxfp4 {M}x{N}x{K}")
    gen = torch.Generator().manual_seed(M * 104729 + N * 13 + K)
    pa, sa = quant.quantize_mxfp4(torch.randn(M, K, generator=gen))
    pb, sb = quant.quantize_mxfp4(torch.randn(N, K, generator=gen))
    a, b, sa, sb = pa.to(gpu), pb.to(gpu), sa.to(gpu), sb.to(gpu)

    def run(xa, xb, schedule="dp"):
        c = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
        return _launch.gemm_a4w4(a, b, xa, xb, c, schedule=schedule, waves=4)

    rm = run(sa, sb)
    km = run(sa.t().contiguous().t(), sb.t().contiguous().t())
    ps = run(quant.preshuffle_e8m0(sa), quant.preshuffle_e8m0(sb))
    sk = run(sa, sb, "streamk")
    sk_km = run(sa.t().contiguous().t(), sb.t().contiguous().t(), "streamk")
    torch.cuda.synchronize()
    _clean(gpu)
    for name, c in (("k-major", km), ("preshuffled", ps), ("stream-K", sk), ("stream-K k-major", sk_km)):
        np.testing.assert_array_equal(_bits(c), _bits(rm), err_msg=name)
