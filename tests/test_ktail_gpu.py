"""K tails: K not a multiple of the 64-element (FP16/BF16) or 128-element
(BF8) stage.  The first stage is then partial: the kernels start it before
k = 0 and load zeros for the missing leading chunks.

The operands are views into larger buffers whose other elements (each row's
padding after K and the 16 bytes before each row) are NaN, so any load of a
chunk outside [0, K) would poison the output.  Small-integer operands make
every fp32 sum exact, so the outputs must equal the oracle's bit for bit, for
every schedule and both wave counts; random operands at a larger K are checked
against the oracle's tolerance, and stream-K against data-parallel bitwise.
"""

import numpy as np
import pytest
import torch

from gfx950_gluon_tutorials_amd.gemm import _launch
from oracle import gemm_ref as R

pytestmark = pytest.mark.gpu

PAD_BYTES = 16  # NaN bytes before each row's first element (and 32 after its last)


def _say(msg):
    print(f"\n[case] {msg}", flush=True)


def _poisoned(vals: np.ndarray, dtype, dev, nan_code=None):
    """A (rows, K) view into a NaN-filled buffer: 16 bytes of NaN before each
    row and 32 after it.  ``vals`` are float values, or uint8 codes when
    dtype is float8_e5m2 (nan_code fills the rest)."""
    rows, K = vals.shape
    esize = 1 if dtype == torch.float8_e5m2 else 2
    PAD = PAD_BYTES // esize
    width = PAD + K + 32 // esize
    if dtype == torch.float8_e5m2:
        big = torch.full((rows, width), nan_code, dtype=torch.uint8)
        big[:, PAD:PAD + K] = torch.from_numpy(vals)
        big = big.view(torch.float8_e5m2).to(dev)
    else:
        big = torch.full((rows, width), float("nan"), dtype=dtype)
        big[:, PAD:PAD + K] = torch.from_numpy(vals).to(dtype)
        big = big.to(dev)
    view = big[:, PAD:PAD + K]
    assert view.data_ptr() % 16 == 0 and (view.stride(0) * view.element_size()) % 16 == 0
    return view


def _small_ints(g, shape):
    return g.integers(-1, 2, size=shape).astype(np.float32)


@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("schedule", ["dp", "streamk", "splitk"])
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_a16w16_k_tails_exact(gpu, dtype, schedule, waves):
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    g = np.random.default_rng(3)
    M, N = 300, 520
    for K in (8, 40, 72, 136, 1000, 2056):
        _say(f"a16w16 {dtype} K={K} {schedule} {waves}w")
        a = _small_ints(g, (M, K))
        b = _small_ints(g, (N, K))
        av, bv = _poisoned(a, tdt, gpu), _poisoned(b, tdt, gpu)
        c = torch.empty(M, N, dtype=tdt, device=gpu)
        _launch.gemm_a16w16(av, bv.T, c, schedule=schedule, waves=waves)
        torch.cuda.synchronize()
        want = R.a16w16_ref(a, b, dtype)
        got = c.float().cpu().numpy()
        assert np.isfinite(got).all(), f"K={K}: a masked chunk was loaded"
        np.testing.assert_array_equal(got, want.astype(np.float32), err_msg=f"K={K}")


@pytest.mark.parametrize("schedule", ["dp", "streamk", "splitk"])
@pytest.mark.parametrize("waves", [4, 8])
def test_a8w8_k_tails_exact(gpu, schedule, waves):
    g = np.random.default_rng(4)
    M, N = 260, 300
    codes = {-1: 0xBC, 0: 0x00, 1: 0x3C}  # e5m2 -1.0, 0, 1.0
    for K in (16, 144, 1040):
        _say(f"a8w8 K={K} {schedule} {waves}w")
        a = np.vectorize(codes.get)(g.integers(-1, 2, size=(M, K))).astype(np.uint8)
        b = np.vectorize(codes.get)(g.integers(-1, 2, size=(N, K))).astype(np.uint8)
        av = _poisoned(a, torch.float8_e5m2, gpu, nan_code=0x7F)
        bv = _poisoned(b, torch.float8_e5m2, gpu, nan_code=0x7F)
        c = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
        _launch.gemm_a8w8(av, bv.T, c, schedule=schedule, waves=waves)
        torch.cuda.synchronize()
        want = R.a8w8_ref(a, b, out_dtype="bf16")
        got = c.float().cpu().numpy()
        assert np.isfinite(got).all(), f"K={K}: a masked chunk was loaded"
        np.testing.assert_array_equal(got, want.astype(np.float32), err_msg=f"K={K}")


@pytest.mark.parametrize("waves", [4, 8])
def test_a16w16_k_tail_random_and_streamk_bitwise(gpu, waves):
    # Random operands at K = 4104 (64 stages + 8): within the FP16 tolerance of
    # the oracle on sampled rows; stream-K on 289 tiles bit-identical to DP.
    _say(f"a16w16 random K tail {waves}w")
    gen = torch.Generator().manual_seed(5)
    M = N = 4352
    K = 4104
    a = (torch.randn(M, K, generator=gen) * 0.1).half()
    b = (torch.randn(N, K, generator=gen) * 0.1).half()
    ad, bd = a.to(gpu), b.to(gpu)
    c_dp = torch.empty(M, N, dtype=torch.float16, device=gpu)
    c_sk = torch.empty_like(c_dp)
    _launch.gemm_a16w16(ad, bd.T, c_dp, schedule="dp", waves=waves)
    _launch.gemm_a16w16(ad, bd.T, c_sk, schedule="streamk", waves=waves)
    torch.cuda.synchronize()
    assert torch.equal(c_dp, c_sk)
    rows = np.random.default_rng(6).choice(M, 64, replace=False)
    want = R.gemm_f32(a.float().numpy()[rows], b.float().numpy())
    got = c_dp.float().cpu().numpy()[rows]
    atol = 1e-2 * np.sqrt(K) * 0.01
    assert np.allclose(got, want, rtol=1e-2, atol=atol), np.abs(got - want).max()


def test_k_granularity_is_still_enforced(gpu):
    with pytest.raises(ValueError):  # FP16: K a multiple of 8
        _launch.gemm_a16w16(torch.zeros(256, 100, dtype=torch.float16, device=gpu)[:, :100],
                            torch.zeros(256, 104, dtype=torch.float16, device=gpu)[:, :100].T,
                            torch.empty(256, 256, dtype=torch.float16, device=gpu))
    with pytest.raises(ValueError):  # BF8: K a multiple of 16
        z = torch.zeros(256, 208, dtype=torch.uint8, device=gpu).view(torch.float8_e5m2)[:, :200]
        _launch.gemm_a8w8(z, z.T, torch.empty(256, 256, dtype=torch.float16, device=gpu))
