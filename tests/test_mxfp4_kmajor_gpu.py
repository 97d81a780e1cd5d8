"""MXFP4 with K-major E8M0 scales on the GPU, through the C ABI.

The reference bench builds its scales as ``randint(124, 128, (K // 32, M_pad)).T[:M]``
(kernels/gemm/intra_wave/a4w4/bench.py:137-146): (M, K/32) views whose rows are
contiguous and whose groups are M_pad bytes apart.  The 4-wave kernels read
such views as they are (G9_FP4K: the chunk DMA writes the transposed LDS
layout that the row-major kernel builds with its in-place transpose), so:

* the output is bit-identical to the row-major-scale kernel on the same
  values (same data, MFMAs and order) and to the preshuffled-scale kernel, on
  the reference bench's own inputs at its 4096 x 4096 x 8192 point, on the
  BASELINE MXFP4 configuration and on ragged shapes of 1-17 stages;
* the padding rows M..M_pad of the storage (set to the NaN code 255 here) only
  meet rows that are not stored;
* stream-K stays bit-identical to data-parallel, split-K within the oracle's
  tolerance, and the 8-wave kernels (which read row-major chunks) take the
  same views through a repack.
"""

import numpy as np
import pytest
import torch

from gfx950_gluon_tutorials_amd import _lib, quant
from gfx950_gluon_tutorials_amd.gemm import _launch
from gfx950_gluon_tutorials_amd.gemm.intra_wave.a4w4 import matmul as a4w4_matmul
from oracle import gemm_ref as R

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"\n[case] {msg}", flush=True)


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy()


def _kmajor(s: torch.Tensor, pad_rows: int = 0, fill: int = 255) -> torch.Tensor:
    """The (M, G) scales as a K-major view of (G, M + pad_rows) storage whose
    padding rows hold `fill`."""
    M, G = s.shape
    store = torch.full((G, M + pad_rows), fill, dtype=torch.uint8, device=s.device)
    store[:, :M] = s.t()
    v = store.t()[:M]
    assert v.stride() == (1, M + pad_rows)
    return v


def _run(gpu, a, b, sa, sb, out=torch.bfloat16, schedule="dp", waves=4):
    M, N = a.shape[0], b.shape[0]
    c = torch.empty(M, N, dtype=out, device=gpu)
    return _launch.gemm_a4w4(a, b, sa, sb, c, schedule=schedule, waves=waves)


def _reference_bench_inputs(M, N, K, gpu):
    """kernels/gemm/intra_wave/a4w4/bench.py:115-146, on the CPU generator."""
    g = torch.Generator().manual_seed(42)
    a_lo = torch.randint(0, 16, (M, K // 2), dtype=torch.uint8, generator=g)
    a_hi = torch.randint(0, 16, (M, K // 2), dtype=torch.uint8, generator=g)
    b_lo = torch.randint(0, 16, (N, K // 2), dtype=torch.uint8, generator=g)
    b_hi = torch.randint(0, 16, (N, K // 2), dtype=torch.uint8, generator=g)
    M_pad = (M + 255) // 256 * 256
    sa = torch.randint(124, 128, (K // 32, M_pad), dtype=torch.uint8, generator=g).to(gpu).T[:M]
    sb = torch.randint(124, 128, (K // 32, N), dtype=torch.uint8, generator=g).to(gpu).T
    return (a_hi << 4 | a_lo).to(gpu), (b_lo | b_hi << 4).to(gpu), sa, sb


def test_kernel_is_selected_for_kmajor_views():
    lib = _lib.load()
    assert lib.g9_kernel_name(_lib.G9_FP4K, _lib.G9_BF16, _lib.G9_SCHED_DP, 4) == b"g9_a4w4km_bf16out_dp_4w"
    assert lib.g9_kernel_name(_lib.G9_FP4K, _lib.G9_BF16, _lib.G9_SCHED_DP, 8) is None


def test_reference_bench_inputs(gpu):
    M = N = 4096
    K = 8192
    _say(f"a4w4 K-major reference-bench inputs {M}x{N}x{K}")
    a, b, sa, sb = _reference_bench_inputs(M, N, K, gpu)
    assert sa.stride(0) == 1 and sb.stride(0) == 1
    c_km = a4w4_matmul(a, b, sa, sb)
    c_rm = _run(gpu, a, b, sa.contiguous(), sb.contiguous())
    c_ps = _run(gpu, a, b, quant.preshuffle_e8m0(sa.contiguous()), quant.preshuffle_e8m0(sb.contiguous()))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(c_km), _bits(c_rm))
    np.testing.assert_array_equal(_bits(c_km), _bits(c_ps))
    rows = torch.from_numpy(np.unique(np.r_[0, M - 1, np.random.default_rng(7).integers(0, M, 128)]))
    ref = R.a4w4_ref(a[rows].cpu().numpy(), b.cpu().numpy(), sa[rows].cpu().numpy(), sb.cpu().numpy(), "bf16")
    assert R.rel_frobenius(c_km[rows].float().cpu().numpy(), ref) <= 1e-3


def test_baseline_config(gpu):
    """configs[3] (MXFP4 4096x4096x8192, seed 3), scales passed K-major."""
    _say("a4w4 K-major 4096x4096x8192 seed3")
    gen = torch.Generator().manual_seed(3)
    pa, sa = quant.quantize_mxfp4(torch.randn(4096, 8192, generator=gen))
    pb, sb = quant.quantize_mxfp4(torch.randn(4096, 8192, generator=gen))
    a, b = pa.to(gpu), pb.to(gpu)
    c_km = _run(gpu, a, b, _kmajor(sa.to(gpu)), _kmajor(sb.to(gpu), pad_rows=16))
    c_rm = _run(gpu, a, b, sa.to(gpu), sb.to(gpu))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(c_km), _bits(c_rm))


@pytest.mark.parametrize("ns", [1, 2, 3, 4, 5, 7, 8, 9, 12, 17])
def test_stage_counts_and_ragged_edges(gpu, ns):
    M, N, K = 300, 264, 256 * ns
    _say(f"a4w4 K-major {M}x{N}x{K}")
    gen = torch.Generator().manual_seed(500 + ns)
    pa, sa = quant.quantize_mxfp4(torch.randn(M, K, generator=gen))
    pb, sb = quant.quantize_mxfp4(torch.randn(N, K, generator=gen))
    a, b = pa.to(gpu), pb.to(gpu)
    # Padding rows with the NaN code: they only meet A or B rows past the
    # edge, whose outputs are not stored.
    ka, kb = _kmajor(sa.to(gpu), pad_rows=20), _kmajor(sb.to(gpu), pad_rows=8)
    for out in (torch.bfloat16, torch.float16):
        c_km = _run(gpu, a, b, ka, kb, out=out)
        c_rm = _run(gpu, a, b, sa.to(gpu), sb.to(gpu), out=out)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_bits(c_km), _bits(c_rm))
    ref = R.a4w4_ref(pa.numpy(), pb.numpy(), sa.numpy(), sb.numpy(), "f16")
    assert R.rel_frobenius(c_km.float().cpu().numpy(), ref) <= 1e-3


@pytest.mark.parametrize("M,N,K", [(3840, 3840, 4096), (1280, 2304, 2560)])
def test_streamk_and_splitk(gpu, M, N, K):
    _say(f"a4w4 K-major stream-K / split-K {M}x{N}x{K}")
    gen = torch.Generator().manual_seed(M + K)
    pa, sa = quant.quantize_mxfp4(torch.randn(M, K, generator=gen))
    pb, sb = quant.quantize_mxfp4(torch.randn(N, K, generator=gen))
    a, b = pa.to(gpu), pb.to(gpu)
    ka, kb = _kmajor(sa.to(gpu), pad_rows=4), _kmajor(sb.to(gpu))
    dp = _run(gpu, a, b, ka, kb)
    sk = _run(gpu, a, b, ka, kb, schedule="streamk")
    sp = _run(gpu, a, b, ka, kb, schedule="splitk")
    rm_sp = _run(gpu, a, b, sa.to(gpu), sb.to(gpu), schedule="splitk")
    torch.cuda.synchronize()
    assert torch.equal(sk, dp)
    assert torch.equal(sp, rm_sp)
    rows = torch.from_numpy(np.unique(np.r_[0, M - 1, np.random.default_rng(3).integers(0, M, 64)]))
    ref = R.a4w4_ref(pa[rows].numpy(), pb.numpy(), sa[rows].numpy(), sb.numpy(), "bf16")
    assert R.rel_frobenius(sp[rows].float().cpu().numpy(), ref) <= 1e-3


def test_eight_waves_take_the_views_through_a_repack(gpu):
    M, N, K = 512, 512, 2048
    _say(f"a4w4 K-major views, 8 waves {M}x{N}x{K}")
    gen = torch.Generator().manual_seed(77)
    pa, sa = quant.quantize_mxfp4(torch.randn(M, K, generator=gen))
    pb, sb = quant.quantize_mxfp4(torch.randn(N, K, generator=gen))
    a, b = pa.to(gpu), pb.to(gpu)
    c8 = _run(gpu, a, b, _kmajor(sa.to(gpu)), _kmajor(sb.to(gpu)), waves=8)
    want = _run(gpu, a, b, sa.to(gpu), sb.to(gpu), waves=8)
    torch.cuda.synchronize()
    assert torch.equal(c8, want)


def test_mixed_layouts_are_repacked(gpu):
    M, N, K = 256, 384, 1024
    _say(f"a4w4 mixed scale layouts {M}x{N}x{K}")
    gen = torch.Generator().manual_seed(78)
    pa, sa = quant.quantize_mxfp4(torch.randn(M, K, generator=gen))
    pb, sb = quant.quantize_mxfp4(torch.randn(N, K, generator=gen))
    a, b = pa.to(gpu), pb.to(gpu)
    c = _run(gpu, a, b, _kmajor(sa.to(gpu)), sb.to(gpu))
    want = _run(gpu, a, b, sa.to(gpu), sb.to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(c, want)


@pytest.mark.parametrize("rows,groups,pad", [(1, 8, 0), (100, 8, 28), (4096, 256, 0), (300, 257, 212), (65, 64, 3)])
def test_byte_transpose_matches_torch(gpu, rows, groups, pad):
    # g9_transpose_u8 on a (groups, rows + pad) buffer seen as a (rows, groups)
    # view: the row-major copy equals torch's, byte for byte, at ragged tile
    # edges and with storage padding, and nothing outside the output changes.
    _say(f"byte transpose {rows}x{groups} pad {pad}")
    lib = _lib.load()
    gen = torch.Generator().manual_seed(rows + groups)
    store = torch.randint(0, 256, (groups, rows + pad), generator=gen, dtype=torch.uint8).to(gpu)
    view = store.T[:rows]
    out = torch.full((rows + 1, groups), 7, dtype=torch.uint8, device=gpu)
    rc = lib.g9_transpose_u8(view.data_ptr(), groups, rows, view.stride(1), out.data_ptr(), groups,
                             torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.G9_OK
    torch.cuda.synchronize()
    assert torch.equal(out[:rows], view.contiguous())
    assert (out[rows:] == 7).all()


def test_eight_waves_with_padded_reference_views(gpu):
    # The reference bench's A scales: randint((K // 32, M_pad)).T[:M], M_pad a
    # multiple of 256 (kernels/gemm/inter_wave/a4w4/bench.py:110-115).
    M, N, K = 300, 256, 1024
    _say(f"a4w4 8 waves, padded K-major views {M}x{N}x{K}")
    gen = torch.Generator().manual_seed(79)
    pa, sa = quant.quantize_mxfp4(torch.randn(M, K, generator=gen))
    pb, sb = quant.quantize_mxfp4(torch.randn(N, K, generator=gen))
    a, b = pa.to(gpu), pb.to(gpu)
    # Padding rows of NaN scales (255): the repack must not read them.
    c8 = _run(gpu, a, b, _kmajor(sa.to(gpu), pad_rows=512 - M), _kmajor(sb.to(gpu)), waves=8)
    want = _run(gpu, a, b, sa.to(gpu), sb.to(gpu), waves=8)
    torch.cuda.synchronize()
    assert torch.equal(c8, want)
