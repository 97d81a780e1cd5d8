"""Stream-K over 256x128 tiles (schedule="streamk_half", G9_SCHED_SK_HALF) on the GPU.

The two quadrants of a 256x128 tile are computed exactly as the matching
quadrants of a 256x256 tile, so every output element sees the data-parallel
kernel's MFMA sequence: the output must equal the data-parallel kernel's bit
for bit, at the BASELINE stream-K shapes (configs[4], randn(seed=4)*0.1,
450 and 320 tiles: every workgroup owns more than a tile), at ragged edges
(M, N not multiples of the tile), at every stage count of a partial six-stage
loop body, with a K tail, and against the oracle on sampled rows.
"""

import numpy as np
import pytest
import torch

from gfx950_gluon_tutorials_amd import _lib
from gfx950_gluon_tutorials_amd.gemm import _launch
from gfx950_gluon_tutorials_amd.gemm.intra_wave.a16w16 import matmul as a16w16_matmul
from oracle import gemm_ref as R

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"\n[case] {msg}", flush=True)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _clean(dev):
    assert _launch.WORKSPACES.error(dev) == 0, "a stream-K flag wait timed out"


def _randn(gen, shape, scale=1.0):
    return torch.randn(*shape, generator=gen) * scale


def test_kernel_names_and_rejections():
    lib = _lib.load()
    assert lib.g9_kernel_name(_lib.G9_F16, _lib.G9_F16, _lib.G9_SCHED_SK_HALF, 4) == b"g9_a16w16_f16_skh_4w"
    assert lib.g9_kernel_name(_lib.G9_BF16, _lib.G9_BF16, _lib.G9_SCHED_SK_HALF, 4) == b"g9_a16w16_bf16_skh_4w"
    assert lib.g9_kernel_name(_lib.G9_F16, _lib.G9_F16, _lib.G9_SCHED_SK_HALF, 8) is None
    assert lib.g9_kernel_name(_lib.G9_BF8, _lib.G9_BF16, _lib.G9_SCHED_SK_HALF, 4) is None


@pytest.mark.parametrize("M,N,K", [(3840, 3840, 16384), (8192, 1280, 8192)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_baseline_shapes_bit_identical_to_dp(gpu, M, N, K, dtype):
    _say(f"stream-K 256x128 vs DP {M}x{N}x{K} {dtype}")
    gen = torch.Generator().manual_seed(4)
    a = _randn(gen, (M, K), 0.1).to(dtype).to(gpu)
    b = _randn(gen, (N, K), 0.1).to(dtype).to(gpu)
    dp = a16w16_matmul(a, b.T, schedule="dp")
    skh = a16w16_matmul(a, b.T, schedule="streamk_half")
    torch.cuda.synchronize()
    _clean(gpu)
    np.testing.assert_array_equal(_bits(skh), _bits(dp))
    if dtype == torch.float16:
        rows = torch.from_numpy(np.unique(np.r_[0, M - 1, np.random.default_rng(M).integers(0, M, 48)]))
        ref = R.a16w16_ref(a[rows].cpu().numpy(), b.cpu().numpy())
        got = skh[rows].float().cpu().numpy()
        np.testing.assert_allclose(got, ref, rtol=1e-2, atol=1e-2 * np.sqrt(K) * 0.01)


@pytest.mark.parametrize("ns", [1, 2, 3, 4, 5, 6, 7, 8, 11, 12, 13, 17])
def test_stage_counts_and_ragged_edges(gpu, ns):
    # 300 x 200: a partial 256-row tile and a partial 128-column tile; the
    # stage counts cover every partial loop body (six stages per body).
    M, N, K = 300, 200, 64 * ns
    _say(f"stream-K 256x128 {M}x{N}x{K}")
    gen = torch.Generator().manual_seed(100 + ns)
    a = _randn(gen, (M, K), 0.5).half().to(gpu)
    b = _randn(gen, (N, K), 0.5).half().to(gpu)
    dp = a16w16_matmul(a, b.T, schedule="dp")
    skh = a16w16_matmul(a, b.T, schedule="streamk_half")
    torch.cuda.synchronize()
    _clean(gpu)
    np.testing.assert_array_equal(_bits(skh), _bits(dp))


@pytest.mark.parametrize("M,N,K", [(1024, 1000, 3000), (2560, 2304, 4104), (512, 384, 8)])
def test_k_tails_and_many_segments(gpu, M, N, K):
    # K not a multiple of 64 (a partial first stage), and tile counts from a
    # handful to several per workgroup.
    _say(f"stream-K 256x128 K tail {M}x{N}x{K}")
    gen = torch.Generator().manual_seed(M + N + K)
    a = _randn(gen, (M, K), 0.5).half().to(gpu)
    b = _randn(gen, (N, K), 0.5).half().to(gpu)
    dp = a16w16_matmul(a, b.T, schedule="dp")
    skh = a16w16_matmul(a, b.T, schedule="streamk_half")
    torch.cuda.synchronize()
    _clean(gpu)
    np.testing.assert_array_equal(_bits(skh), _bits(dp))


def test_small_integer_operands_match_the_oracle_exactly(gpu):
    # Every partial sum is an exact small integer in fp32, so the result is
    # the oracle's bit for bit whatever the accumulation order.
    M, N, K = 640, 384, 2048
    _say(f"stream-K 256x128 exact {M}x{N}x{K}")
    rng = np.random.default_rng(9)
    a = rng.integers(-3, 4, (M, K)).astype(np.float16)
    b = rng.integers(-3, 4, (N, K)).astype(np.float16)
    skh = a16w16_matmul(torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu).T, schedule="streamk_half")
    torch.cuda.synchronize()
    _clean(gpu)
    ref = R.a16w16_ref(a, b)
    np.testing.assert_array_equal(skh.float().cpu().numpy(), ref)


def test_repeated_launches_share_a_workspace(gpu):
    # Epochs keep stale flags from matching: back-to-back launches on one
    # workspace (with a 256x256 stream-K launch between them) stay identical.
    M, N, K = 1536, 1152, 4096
    _say(f"stream-K 256x128 repeated {M}x{N}x{K}")
    gen = torch.Generator().manual_seed(11)
    a = _randn(gen, (M, K), 0.1).half().to(gpu)
    b = _randn(gen, (N, K), 0.1).half().to(gpu)
    first = a16w16_matmul(a, b.T, schedule="streamk_half")
    sk = a16w16_matmul(a, b.T, schedule="streamk")
    again = [a16w16_matmul(a, b.T, schedule="streamk_half") for _ in range(3)]
    torch.cuda.synchronize()
    _clean(gpu)
    for c in again + [sk]:
        np.testing.assert_array_equal(_bits(c), _bits(first))
