"""MXFP4 scale handling on the GPU, through the C ABI.

* Preshuffled scales (g9_gemm_a4w4_preshuffled): bit-identical to the
  row-major-scale kernel on the same values (same data, MFMAs and order), at
  the BASELINE MXFP4 configuration and on ragged shapes of 1-17 stages (chunks
  cut short by K), and within the oracle's tolerance.
* Extreme E8M0 codes (0-8 and 246-254: operands that are fp32 subnormals or
  near fp32's top when dequantized): with one operand's scales small and the
  other's large every product is a normal fp32 value and the oracle's result is
  exact, so both MXFP4 kernels must match it to the output rounding; with both
  small every product underflows fp32 and the output is zero.
* e5m2 subnormal operands (codes 1-3 and 0x81-0x83) in the BF8 kernel.
* The error against the fp32 product of the dequantized operands (the bound
  BASELINE states): with an fp16 output it is within 1e-3; with bf16 (the
  reference's output type) the bf16 rounding alone is ~1.1e-3, so there the
  bound is checked against the oracle rounded to bf16 and the fp32 error is
  bounded by 2e-3.
"""

import numpy as np
import pytest
import torch

from gfx950_gluon_tutorials_amd import quant
from gfx950_gluon_tutorials_amd.gemm import _launch
from gfx950_gluon_tutorials_amd.gemm.intra_wave.a4w4 import matmul as a4w4_matmul
from oracle import gemm_ref as R

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"\n[case] {msg}", flush=True)


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy()


def _f32(t):
    return t.float().cpu().numpy()


def _row_sample(M, n=192, seed=0):
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(seed).integers(0, M, n)]))
    return torch.from_numpy(rows)


def _both(gpu, pa, pb, sa, sb, out=torch.bfloat16):
    """(row-major-scale output, preshuffled-scale output), 4-wave data-parallel."""
    a, b = pa.to(gpu), pb.to(gpu)
    M, N = a.shape[0], b.shape[0]
    c_rm = _launch.gemm_a4w4(a, b, sa.to(gpu), sb.to(gpu), torch.empty(M, N, dtype=out, device=gpu))
    c_ps = _launch.gemm_a4w4(a, b, quant.preshuffle_e8m0(sa).to(gpu), quant.preshuffle_e8m0(sb).to(gpu),
                             torch.empty(M, N, dtype=out, device=gpu))
    torch.cuda.synchronize()
    return c_rm, c_ps


def test_preshuffled_baseline_config(gpu):
    """configs[3] (MXFP4 4096x4096x8192, seed 3) with preshuffled scales."""
    _say("a4w4 preshuffled 4096x4096x8192 seed3")
    gen = torch.Generator().manual_seed(3)
    pa, sa = quant.quantize_mxfp4(torch.randn(4096, 8192, generator=gen))
    pb, sb = quant.quantize_mxfp4(torch.randn(4096, 8192, generator=gen))
    c_rm, c_ps = _both(gpu, pa, pb, sa, sb)
    np.testing.assert_array_equal(_bits(c_ps), _bits(c_rm))
    rows = _row_sample(4096)
    ref = R.a4w4_ref(pa[rows].numpy(), pb.numpy(), sa[rows].numpy(), sb.numpy(), "bf16")
    assert R.rel_frobenius(_f32(c_ps[rows]), ref) <= 1e-3
    # Through the drop-in wrapper as well (3-D scales select the kernel).
    c = a4w4_matmul(pa.to(gpu), pb.to(gpu), quant.preshuffle_e8m0(sa).to(gpu), quant.preshuffle_e8m0(sb).to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(c, c_ps)


@pytest.mark.parametrize("ns", [1, 2, 3, 4, 5, 7, 8, 9, 12, 17])
def test_preshuffled_stage_counts_and_ragged_edges(gpu, ns):
    M, N, K = 300, 264, 256 * ns
    _say(f"a4w4 preshuffled {M}x{N}x{K}")
    gen = torch.Generator().manual_seed(300 + ns)
    pa, sa = quant.quantize_mxfp4(torch.randn(M, K, generator=gen))
    pb, sb = quant.quantize_mxfp4(torch.randn(N, K, generator=gen))
    c_rm, c_ps = _both(gpu, pa, pb, sa, sb)
    np.testing.assert_array_equal(_bits(c_ps), _bits(c_rm))
    ref = R.a4w4_ref(pa.numpy(), pb.numpy(), sa.numpy(), sb.numpy(), "bf16")
    assert R.rel_frobenius(_f32(c_ps), ref) <= 1e-3


def test_preshuffled_scales_with_padded_chunk_stride(gpu):
    """Chunks further apart than 32 * rows bytes (a strided view) and an fp16 output."""
    M, N, K = 512, 384, 2048
    _say(f"a4w4 preshuffled strided chunks {M}x{N}x{K}")
    gen = torch.Generator().manual_seed(31)
    pa, sa = quant.quantize_mxfp4(torch.randn(M, K, generator=gen))
    pb, sb = quant.quantize_mxfp4(torch.randn(N, K, generator=gen))
    psa, psb = quant.preshuffle_e8m0(sa), quant.preshuffle_e8m0(sb)
    big_a = torch.zeros(psa.shape[0], M + 8, 32, dtype=torch.uint8)
    big_a[:, :M] = psa
    big_b = torch.full((psb.shape[0], N + 24, 32), 255, dtype=torch.uint8)  # NaN scales outside the view
    big_b[:, :N] = psb
    a, b = pa.to(gpu), pb.to(gpu)
    va, vb = big_a.to(gpu)[:, :M], big_b.to(gpu)[:, :N]
    assert va.stride(0) == (M + 8) * 32
    c = _launch.gemm_a4w4(a, b, va, vb, torch.empty(M, N, dtype=torch.float16, device=gpu))
    want = _launch.gemm_a4w4(a, b, sa.to(gpu), sb.to(gpu), torch.empty(M, N, dtype=torch.float16, device=gpu))
    torch.cuda.synchronize()
    assert torch.equal(c, want)


def _extreme_case(gen, M, N, K, a_codes, b_codes):
    pa, _ = quant.quantize_mxfp4(torch.randn(M, K, generator=gen))
    pb, _ = quant.quantize_mxfp4(torch.randn(N, K, generator=gen))
    lo_a, hi_a = a_codes
    lo_b, hi_b = b_codes
    sa = torch.randint(lo_a, hi_a + 1, (M, K // 32), generator=gen, dtype=torch.int32).to(torch.uint8)
    sb = torch.randint(lo_b, hi_b + 1, (N, K // 32), generator=gen, dtype=torch.int32).to(torch.uint8)
    return pa, pb, sa, sb


def _dequant64(packed, scales):
    """The dequantized operand in float64, where 6 * 2^127 is still finite."""
    return R.mxfp4_to_f32(packed.numpy()).astype(np.float64) * np.repeat(
        np.ldexp(1.0, scales.numpy().astype(np.int64) - 127), 32, axis=1)


@pytest.mark.parametrize("a_codes,b_codes", [((0, 8), (246, 254)), ((246, 254), (0, 8))])
@pytest.mark.parametrize("waves", [4, 8])
def test_extreme_e8m0_scales_small_times_large(gpu, a_codes, b_codes, waves):
    """The kernels apply the scales inside the MFMA, so a product of a small
    and a large scale is exact even where the large one's dequantized operand
    (6 * 2^127 for code 254) is past fp32's range: the result matches the exact
    (float64) product.  The reference's formula, which dequantizes to fp32
    first, gives inf there; where it stays finite it agrees."""
    M, N, K = 320, 288, 1024
    _say(f"a4w4 extreme E8M0 A{a_codes} B{b_codes} waves={waves}")
    gen = torch.Generator().manual_seed(41 + a_codes[0])
    pa, pb, sa, sb = _extreme_case(gen, M, N, K, a_codes, b_codes)
    exact = _dequant64(pa, sa) @ _dequant64(pb, sb).T
    assert np.abs(exact).max() > 1.0 and np.abs(exact).max() < 1e30
    want = R.round_to(exact.astype(np.float32), "bf16")
    c = _launch.gemm_a4w4(pa.to(gpu), pb.to(gpu), sa.to(gpu), sb.to(gpu),
                          torch.empty(M, N, dtype=torch.bfloat16, device=gpu), waves=waves)
    torch.cuda.synchronize()
    assert R.rel_frobenius(_f32(c), want) <= 1e-3
    ref32 = R.a4w4_ref(pa.numpy(), pb.numpy(), sa.numpy(), sb.numpy(), "bf16")
    fin = np.isfinite(ref32)
    assert R.rel_frobenius(_f32(c)[fin], ref32[fin]) <= 1e-3
    if waves == 4:
        _, c_ps = _both(gpu, pa, pb, sa, sb)
        assert torch.equal(c_ps, c)


def test_extreme_e8m0_scales_both_small_underflow_to_zero(gpu):
    M, N, K = 256, 256, 512
    _say("a4w4 extreme E8M0 both 0-8")
    gen = torch.Generator().manual_seed(43)
    pa, pb, sa, sb = _extreme_case(gen, M, N, K, (0, 8), (0, 8))
    ref = R.a4w4_ref(pa.numpy(), pb.numpy(), sa.numpy(), sb.numpy(), "bf16")
    assert not ref.any()  # every product is below fp32's smallest subnormal
    c_rm, c_ps = _both(gpu, pa, pb, sa, sb)
    assert not c_rm.float().any() and not c_ps.float().any()


@pytest.mark.parametrize("waves", [4, 8])
def test_e5m2_subnormal_operands(gpu, waves):
    M, N, K = 272, 320, 512
    _say(f"a8w8 e5m2 subnormals waves={waves}")
    g = torch.Generator().manual_seed(47)
    # Codes 0x01-0x03 / 0x81-0x83 are the e5m2 subnormals (1-3 x 2^-16); mix in
    # the smallest normals (0x04-0x07) and zero.
    pool = torch.tensor([0x00, 0x01, 0x02, 0x03, 0x81, 0x82, 0x83, 0x04, 0x85, 0x06, 0x87], dtype=torch.uint8)
    ca = pool[torch.randint(0, len(pool), (M, K), generator=g)]
    cb = pool[torch.randint(0, len(pool), (N, K), generator=g)]
    a = ca.view(torch.float8_e5m2).to(gpu)
    b = cb.view(torch.float8_e5m2).to(gpu)
    c = _launch.gemm_a8w8(a, b.T, torch.empty(M, N, dtype=torch.float16, device=gpu), a_scale=2.0 ** 14,
                          b_scale=2.0 ** 14, waves=waves)
    torch.cuda.synchronize()
    ref32 = R.a8w8_ref_f32(ca.numpy(), cb.numpy(), 2.0 ** 14, 2.0 ** 14)
    assert np.abs(ref32).max() > 0
    assert R.rel_frobenius(_f32(c), ref32) <= 1e-3


def test_error_against_the_fp32_product(gpu):
    """BASELINE's bound is relative Frobenius <= 1e-3 against the fp32 product of the dequantized
    operands.  fp16 output: met directly.  bf16 output: met against the bf16-rounded product; against
    the fp32 product the bf16 rounding alone costs ~1.1e-3."""
    M, N, K = 1024, 1024, 4096
    _say(f"a4w4 and a8w8 error vs the fp32 product {M}x{N}x{K}")
    gen = torch.Generator().manual_seed(3)
    pa, sa = quant.quantize_mxfp4(torch.randn(M, K, generator=gen))
    pb, sb = quant.quantize_mxfp4(torch.randn(N, K, generator=gen))
    ref32 = R.a4w4_ref_f32(pa.numpy(), pb.numpy(), sa.numpy(), sb.numpy())
    errs = {}
    for out in (torch.float16, torch.bfloat16):
        c_rm, c_ps = _both(gpu, pa, pb, sa, sb, out=out)
        errs[out] = R.rel_frobenius(_f32(c_ps), ref32)
        assert torch.equal(c_rm, c_ps)
    print(f"\nmxfp4 rel. Frobenius vs fp32 product: fp16 out {errs[torch.float16]:.3g}, "
          f"bf16 out {errs[torch.bfloat16]:.3g}", flush=True)
    assert errs[torch.float16] <= 1e-3
    assert errs[torch.bfloat16] <= 2e-3
    qa, xa = quant.quantize_e5m2(torch.randn(M, K, generator=gen))
    qb, xb = quant.quantize_e5m2(torch.randn(N, K, generator=gen))
    c = _launch.gemm_a8w8(qa.to(gpu), qb.to(gpu).T, torch.empty(M, N, dtype=torch.float16, device=gpu),
                          a_scale=xa.to(gpu), b_scale=xb.to(gpu))
    torch.cuda.synchronize()
    ref8 = R.a8w8_ref_f32(qa.view(torch.uint8).numpy(), qb.view(torch.uint8).numpy(), float(xa), float(xb))
    e8 = R.rel_frobenius(_f32(c), ref8)
    print(f"bf8 rel. Frobenius vs fp32 product, fp16 out: {e8:.3g}", flush=True)
    assert e8 <= 1e-3
