"""GPU parity on special values: infinities and NaNs in the operands, an E8M0
scale of 255 (NaN, kernels/gemm/intra_wave/a4w4/bench.py:110-111) and fp16
overflow in the epilogue.  The oracle's fp32 result decides where the output
is +inf, -inf or NaN (an inf meeting an inf of the other sign, or a zero, is
NaN in any summation order, so the positions do not depend on the order of
the products); every finite output stays within the dtype's tolerance."""

import numpy as np
import pytest
import torch

from gfx950_gluon_tutorials_amd import quant
from gfx950_gluon_tutorials_amd.gemm import _launch
from oracle import gemm_ref as R

pytestmark = pytest.mark.gpu

SCHEDULES = ["dp", "streamk"]


def _say(msg):
    print(f"\n[case] {msg}", flush=True)


def _check_special(out: torch.Tensor, ref: np.ndarray, frob: float | None = None, rtol=1e-2, atol=0.0):
    o = out.float().cpu().numpy()
    np.testing.assert_array_equal(np.isnan(o), np.isnan(ref), err_msg="NaN positions differ")
    np.testing.assert_array_equal(np.isposinf(o), np.isposinf(ref), err_msg="+inf positions differ")
    np.testing.assert_array_equal(np.isneginf(o), np.isneginf(ref), err_msg="-inf positions differ")
    fin = np.isfinite(ref)
    assert fin.sum() > ref.size // 2, "the case must keep most outputs finite"
    if frob is not None:
        err = R.rel_frobenius(o[fin], ref[fin])
        assert err <= frob, f"relative Frobenius error {err:.3g} on the finite outputs"
    else:
        np.testing.assert_allclose(o[fin], ref[fin], rtol=rtol, atol=atol)


@pytest.mark.parametrize("schedule", SCHEDULES)
@pytest.mark.parametrize("waves", [4, 8])
def test_a16w16_inf_nan_and_overflow(gpu, schedule, waves):
    M, N, K = 300, 264, 512
    _say(f"a16w16 special values {M}x{N}x{K} {schedule} waves={waves}")
    g = torch.Generator().manual_seed(31)
    a = (torch.randn(M, K, generator=g) * 0.1).half()
    b = (torch.randn(N, K, generator=g) * 0.1).half()
    a[3, 10] = float("inf")
    a[5, 20] = float("nan")
    a[270, 40] = float("-inf")
    b[7, 30] = float("-inf")
    b[260, 50] = float("inf")
    # Row 9 x column 11: a dot product of 512 * 120 * 120 = 7.4e6, finite in
    # fp32, +inf after the round to fp16 (max 65504).
    a[9] = 120.0
    b[11] = 120.0
    with np.errstate(over="ignore", invalid="ignore"):
        ref = R.a16w16_ref(a.numpy(), b.numpy(), "f16")
    assert np.isposinf(ref[9, 11]) and np.isnan(ref[5]).all()
    c = torch.empty(M, N, dtype=torch.float16, device=gpu)
    _launch.gemm_a16w16(a.to(gpu), b.to(gpu).T, c, schedule=schedule, waves=waves)
    torch.cuda.synchronize()
    _check_special(c, ref, atol=1e-2 * np.sqrt(K) * 0.01)


@pytest.mark.parametrize("schedule", SCHEDULES)
@pytest.mark.parametrize("waves", [4, 8])
def test_a8w8_inf_nan_codes(gpu, schedule, waves):
    M, N, K = 260, 300, 512
    _say(f"a8w8 special codes {M}x{N}x{K} {schedule} waves={waves}")
    g = torch.Generator().manual_seed(32)
    qa, sa = quant.quantize_e5m2(torch.randn(M, K, generator=g))
    qb, sb = quant.quantize_e5m2(torch.randn(N, K, generator=g))
    ca, cb = qa.view(torch.uint8).clone(), qb.view(torch.uint8).clone()
    ca[3, 10] = 0x7C   # +inf
    ca[5, 20] = 0x7F   # NaN
    cb[7, 30] = 0xFC   # -inf
    cb[290, 64] = 0x7D  # NaN
    with np.errstate(over="ignore", invalid="ignore"):
        ref = R.a8w8_ref(ca.numpy(), cb.numpy(), float(sa), float(sb), "bf16")
    assert np.isnan(ref[5]).all() and np.isnan(ref[:, 290]).all() and np.isinf(ref[3, 0])
    a = ca.view(torch.float8_e5m2).to(gpu)
    b = cb.view(torch.float8_e5m2).to(gpu)
    c = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
    _launch.gemm_a8w8(a, b.T, c, a_scale=sa.to(gpu), b_scale=sb.to(gpu), schedule=schedule, waves=waves)
    torch.cuda.synchronize()
    _check_special(c, ref, frob=1e-3)


@pytest.mark.parametrize("schedule", SCHEDULES)
@pytest.mark.parametrize("waves", [4, 8])
def test_a4w4_nan_scale(gpu, schedule, waves):
    M, N, K = 300, 264, 1024
    _say(f"a4w4 E8M0 255 {M}x{N}x{K} {schedule} waves={waves}")
    g = torch.Generator().manual_seed(33)
    pa, sa = quant.quantize_mxfp4(torch.randn(M, K, generator=g))
    pb, sb = quant.quantize_mxfp4(torch.randn(N, K, generator=g))
    sa[3, 5] = 255
    sa[299, 31] = 255
    sb[7, 0] = 255
    with np.errstate(over="ignore", invalid="ignore"):
        ref = R.a4w4_ref(pa.numpy(), pb.numpy(), sa.numpy(), sb.numpy(), "bf16")
    assert np.isnan(ref[3]).all() and np.isnan(ref[299]).all() and np.isnan(ref[:, 7]).all()
    c = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
    _launch.gemm_a4w4(pa.to(gpu), pb.to(gpu), sa.to(gpu), sb.to(gpu), c, schedule=schedule, waves=waves)
    torch.cuda.synchronize()
    _check_special(c, ref, frob=1e-3)
