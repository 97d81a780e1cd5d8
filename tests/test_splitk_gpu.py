"""GPU parity of the split-K schedule (through the C ABI): within the dtype's
tolerance of the CPU oracle and of the data-parallel kernel, deterministic
(bit-identical over repeated launches), correct on ragged M/N and on stage
counts the split factor does not divide, run as data-parallel when the grid
already fills half the chip, and sharing one workspace with stream-K without
disturbing stream-K's flags."""

import numpy as np
import pytest
import torch

from gfx950_gluon_tutorials_amd import _lib, quant
from gfx950_gluon_tutorials_amd.gemm import _launch
from oracle import gemm_ref as R

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"\n[case] {msg}", flush=True)


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _factor(M, N, K, dtype):
    lib = _lib.load()
    tiles = -(-M // 256) * -(-N // 256)
    return lib.g9_splitk_factor(tiles, K // _launch.STAGE_K[dtype], lib.g9_streamk_workgroups())


def _check_f16(out, ref, K, sigma):
    o = out.float().cpu().numpy()
    atol = 1e-2 * np.sqrt(K) * sigma
    bad = ~np.isclose(o, ref, rtol=1e-2, atol=atol)
    assert not bad.any(), f"{int(bad.sum())} outputs outside rtol 1e-2 / atol {atol:.3g}"


@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,N,K", [(300, 264, 4096), (512, 4096, 2048), (77, 1000, 64 * 37)])
def test_a16w16_splitk(gpu, M, N, K, dtype, waves):
    code = _launch._DTYPE_CODE[dtype]
    S = _factor(M, N, K, code)
    _say(f"a16w16 split-K {M}x{N}x{K} {dtype} waves={waves} split={S}")
    assert S > 1
    g = torch.Generator().manual_seed(40)
    a = (torch.randn(M, K, generator=g) * 0.1).to(dtype)
    b = (torch.randn(N, K, generator=g) * 0.1).to(dtype)
    ad, bd = a.to(gpu), b.to(gpu)
    outs = {}
    for sched in ("dp", "splitk", "splitk2"):
        c = torch.full((M, N), float("nan"), dtype=dtype, device=gpu)
        outs[sched] = _launch.gemm_a16w16(ad, bd.T, c, schedule=sched.rstrip("2"), waves=waves)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(outs["splitk"]), _bits(outs["splitk2"]))
    ref = R.a16w16_ref(a.float().numpy(), b.float().numpy(), "f16" if dtype == torch.float16 else "bf16")
    _check_f16(outs["splitk"], ref, K, 0.01)
    _check_f16(outs["splitk"], outs["dp"].float().cpu().numpy(), K, 0.01)


@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_a8w8_splitk(gpu, out_dtype, waves):
    M, N, K = 260, 300, 128 * 40
    S = _factor(M, N, K, _lib.G9_BF8)
    _say(f"a8w8 split-K {M}x{N}x{K} out={out_dtype} waves={waves} split={S}")
    assert S > 1
    g = torch.Generator().manual_seed(41)
    qa, sa = quant.quantize_e5m2(torch.randn(M, K, generator=g))
    qb, sb = quant.quantize_e5m2(torch.randn(N, K, generator=g))
    a, b = qa.to(gpu), qb.to(gpu)
    c = torch.empty(M, N, dtype=out_dtype, device=gpu)
    _launch.gemm_a8w8(a, b.T, c, a_scale=sa.to(gpu), b_scale=sb.to(gpu), schedule="splitk", waves=waves)
    c2 = torch.empty_like(c)
    _launch.gemm_a8w8(a, b.T, c2, a_scale=sa.to(gpu), b_scale=sb.to(gpu), schedule="splitk", waves=waves)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(c), _bits(c2))
    ref = R.a8w8_ref(qa.view(torch.uint8).numpy(), qb.view(torch.uint8).numpy(), float(sa), float(sb),
                     "bf16" if out_dtype == torch.bfloat16 else "f16")
    err = R.rel_frobenius(c.float().cpu().numpy(), ref)
    assert err <= 1e-3, f"relative Frobenius error {err:.3g}"


@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("ns", [9, 32])
def test_a4w4_splitk(gpu, ns, waves):
    M, N, K = 300, 264, 256 * ns
    S = _factor(M, N, K, _lib.G9_FP4)
    _say(f"a4w4 split-K {M}x{N}x{K} waves={waves} split={S}")
    assert S > 1
    g = torch.Generator().manual_seed(42 + ns)
    pa, sa = quant.quantize_mxfp4(torch.randn(M, K, generator=g))
    pb, sb = quant.quantize_mxfp4(torch.randn(N, K, generator=g))
    args = [t.to(gpu) for t in (pa, pb, sa, sb)]
    c = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
    _launch.gemm_a4w4(*args, c, schedule="splitk", waves=waves)
    c2 = torch.empty_like(c)
    _launch.gemm_a4w4(*args, c2, schedule="splitk", waves=waves)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(c), _bits(c2))
    ref = R.a4w4_ref(pa.numpy(), pb.numpy(), sa.numpy(), sb.numpy(), "bf16")
    err = R.rel_frobenius(c.float().cpu().numpy(), ref)
    assert err <= 1e-3, f"relative Frobenius error {err:.3g}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_splitk_exact_integers(gpu, dtype):
    """Small-integer operands: every partial sum is an integer below 2^24, exact in
    fp32 in any order, so split-K must reproduce the oracle bit for bit whatever
    its segment boundaries (13 segments of 2-3 stages here)."""
    M, N, K = 300, 264, 64 * 37
    _say(f"a16w16 split-K exact integers {M}x{N}x{K} {dtype} split={_factor(M, N, K, _launch._DTYPE_CODE[dtype])}")
    g = torch.Generator().manual_seed(45)
    a = torch.randint(-2, 3, (M, K), generator=g).to(dtype)
    b = torch.randint(-2, 3, (N, K), generator=g).to(dtype)
    c = torch.empty(M, N, dtype=dtype, device=gpu)
    _launch.gemm_a16w16(a.to(gpu), b.to(gpu).T, c, schedule="splitk")
    torch.cuda.synchronize()
    ref = R.a16w16_ref(a.float().numpy(), b.float().numpy(), "f16" if dtype == torch.float16 else "bf16")
    want = torch.from_numpy(ref).to(dtype)
    np.testing.assert_array_equal(_bits(c), _bits(want))


def test_splitk_on_a_full_grid_runs_data_parallel(gpu):
    M, N, K = 4096, 4096, 1024
    lib = _lib.load()
    assert _factor(M, N, K, _lib.G9_F16) == 1
    assert lib.g9_workspace_size(_lib.G9_F16, M, N, K, _lib.G9_SCHED_SPLITK, 4) == 0
    _say(f"split-K on a full grid {M}x{N}x{K}")
    g = torch.Generator().manual_seed(43)
    a = (torch.randn(M, K, generator=g) * 0.1).half().to(gpu)
    b = (torch.randn(N, K, generator=g) * 0.1).half().to(gpu)
    c1 = torch.empty(M, N, dtype=torch.float16, device=gpu)
    c2 = torch.empty_like(c1)
    _launch.gemm_a16w16(a, b.T, c1, schedule="dp")
    _launch.gemm_a16w16(a, b.T, c2, schedule="splitk")
    torch.cuda.synchronize()
    assert torch.equal(c1, c2)


def test_splitk_workspace_size_and_sharing_with_streamk(gpu):
    lib = _lib.load()
    M, N, K = 512, 4096, 2048
    S = _factor(M, N, K, _lib.G9_F16)
    need = lib.g9_workspace_size(_lib.G9_F16, M, N, K, _lib.G9_SCHED_SPLITK, 4)
    assert S > 1 and need >= S * 32 * 256 * 256 * 4
    _say("stream-K, then split-K, then stream-K again on one workspace")
    g = torch.Generator().manual_seed(44)
    # 272 tiles: stream-K workgroups hand partial tiles along K chains (flags in use).
    Ms, Ns, Ks = 4352, 4096, 1024
    a = (torch.randn(Ms, Ks, generator=g) * 0.1).half().to(gpu)
    b = (torch.randn(Ns, Ks, generator=g) * 0.1).half().to(gpu)
    dp = torch.empty(Ms, Ns, dtype=torch.float16, device=gpu)
    _launch.gemm_a16w16(a, b.T, dp, schedule="dp")
    x = (torch.randn(M, K, generator=g) * 0.1).half().to(gpu)
    y = (torch.randn(N, K, generator=g) * 0.1).half().to(gpu)
    for _ in range(2):
        sk = torch.empty_like(dp)
        _launch.gemm_a16w16(a, b.T, sk, schedule="streamk")
        out = torch.empty(M, N, dtype=torch.float16, device=gpu)
        _launch.gemm_a16w16(x, y.T, out, schedule="splitk")
        torch.cuda.synchronize()
        assert _launch.WORKSPACES.error(gpu) == 0
        assert torch.equal(sk, dp)


def _random_shapes(n=12, seed=7):
    """Seeded shapes of 1-128 tiles with ragged M/N and K of 2-80 stages."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        M, N = int(rng.integers(1, 3000)), int(rng.integers(8, 3000))
        if -(-M // 256) * -(-N // 256) > 128:
            continue
        out.append((M, N, int(rng.integers(2, 81)), int(rng.choice([4, 8])), str(rng.choice(["fp16", "bf16", "bf8", "mxfp4"]))))
    return out


@pytest.mark.parametrize("M,N,stages,waves,kind", _random_shapes())
def test_splitk_random_shapes_match_dp(gpu, M, N, stages, waves, kind):
    """Split-K against data-parallel (the FP16 tolerance; BF8 / MXFP4: relative
    Frobenius 1e-3 of DP's own output) on seeded ragged shapes."""
    N = (N + 7) // 8 * 8 if kind == "mxfp4" else N
    code = {"fp16": _lib.G9_F16, "bf16": _lib.G9_BF16, "bf8": _lib.G9_BF8, "mxfp4": _lib.G9_FP4}[kind]
    K = stages * _launch.STAGE_K[code]
    _say(f"split-K random {kind} {M}x{N}x{K} waves={waves} split={_factor(M, N, K, code)}")
    g = torch.Generator().manual_seed(M * 7919 + N)
    outs = {}
    if kind in ("fp16", "bf16"):
        dt = torch.float16 if kind == "fp16" else torch.bfloat16
        a = (torch.randn(M, K, generator=g) * 0.1).to(dt).to(gpu)
        b = (torch.randn(N, K, generator=g) * 0.1).to(dt).to(gpu)
        for sched in ("dp", "splitk"):
            outs[sched] = _launch.gemm_a16w16(a, b.T, torch.empty(M, N, dtype=dt, device=gpu), schedule=sched,
                                              waves=waves)
    elif kind == "bf8":
        qa, sa = quant.quantize_e5m2(torch.randn(M, K, generator=g))
        qb, sb = quant.quantize_e5m2(torch.randn(N, K, generator=g))
        for sched in ("dp", "splitk"):
            outs[sched] = _launch.gemm_a8w8(qa.to(gpu), qb.to(gpu).T, torch.empty(M, N, dtype=torch.bfloat16, device=gpu),
                                            a_scale=sa.to(gpu), b_scale=sb.to(gpu), schedule=sched, waves=waves)
    else:
        pa, sa = quant.quantize_mxfp4(torch.randn(M, K, generator=g))
        pb, sb = quant.quantize_mxfp4(torch.randn(N, K, generator=g))
        args = [t.to(gpu) for t in (pa, pb, sa, sb)]
        for sched in ("dp", "splitk"):
            outs[sched] = _launch.gemm_a4w4(*args, torch.empty(M, N, dtype=torch.bfloat16, device=gpu),
                                            schedule=sched, waves=waves)
    torch.cuda.synchronize()
    dp = outs["dp"].float().cpu().numpy()
    if kind in ("fp16", "bf16"):
        _check_f16(outs["splitk"], dp, K, 0.01)
    else:
        err = R.rel_frobenius(outs["splitk"].float().cpu().numpy(), dp)
        assert err <= 1e-3, f"relative Frobenius error {err:.3g} against data-parallel"


def test_splitk_through_the_drop_in_wrappers(gpu):
    """schedule="splitk" on the reference-shaped wrappers (4-wave a16w16 `matmul`,
    8-wave a4w4 `matmul_kernel_only`)."""
    from gfx950_gluon_tutorials_amd.gemm.inter_wave.a4w4 import matmul_kernel_only as a4w4_8w
    from gfx950_gluon_tutorials_amd.gemm.intra_wave.a16w16 import matmul as a16w16_4w

    _say("split-K through the wrappers")
    g = torch.Generator().manual_seed(46)
    a = (torch.randn(512, 4096, generator=g) * 0.1).half().to(gpu)
    b = (torch.randn(1024, 4096, generator=g) * 0.1).half().to(gpu)
    c_sk = a16w16_4w(a, b.T, schedule="splitk")
    c_dp = a16w16_4w(a, b.T)
    pa, sa = quant.quantize_mxfp4(torch.randn(300, 2048, generator=g))
    pb, sb = quant.quantize_mxfp4(torch.randn(520, 2048, generator=g))
    args = [t.to(gpu) for t in (pa, pb, sa, sb)]
    f_sk = a4w4_8w(*args, torch.empty(300, 520, dtype=torch.bfloat16, device=gpu), schedule="splitk")
    torch.cuda.synchronize()
    _check_f16(c_sk, c_dp.float().cpu().numpy(), 4096, 0.01)
    ref = R.a4w4_ref(pa.numpy(), pb.numpy(), sa.numpy(), sb.numpy(), "bf16")
    err = R.rel_frobenius(f_sk.float().cpu().numpy(), ref)
    assert err <= 1e-3, f"relative Frobenius error {err:.3g}"


@pytest.mark.parametrize("pad", [24, 5])
def test_splitk_strided_c_leaves_the_padding_alone(gpu, pad):
    """C as a column slice of a wider buffer (row stride N + pad; pad 5 makes rows
    misaligned for 16-byte stores): split-K writes exactly the M x N window."""
    M, N, K = 300, 520, 2048
    _say(f"split-K strided C {M}x{N}x{K} pad={pad}")
    g = torch.Generator().manual_seed(47)
    a = (torch.randn(M, K, generator=g) * 0.1).half().to(gpu)
    b = (torch.randn(N, K, generator=g) * 0.1).half().to(gpu)
    buf = torch.full((M, N + pad), 7.0, dtype=torch.float16, device=gpu)
    c = buf[:, :N]
    _launch.gemm_a16w16(a, b.T, c, schedule="splitk")
    want = torch.empty(M, N, dtype=torch.float16, device=gpu)
    _launch.gemm_a16w16(a, b.T, want, schedule="dp")
    torch.cuda.synchronize()
    assert torch.all(buf[:, N:] == 7.0)
    _check_f16(c, want.float().cpu().numpy(), K, 0.01)
