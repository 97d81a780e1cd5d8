"""GPU parity of the HIP GEMMs against the CPU oracle (oracle/gemm_ref.py).

* Exact fixtures (tests/golden, built with integer arithmetic): every kernel
  and schedule must reproduce them bit for bit.
* Seeded BASELINE configurations: FP16 within rtol 1e-2 / atol 1e-2*sqrt(K)*sigma,
  BF8 / MXFP4 within relative Frobenius error 1e-3 of the oracle's result in
  the output dtype.  Full-size outputs are checked on a sample of rows (the
  oracle computes those rows in full).
* Stream-K is bit-identical to data-parallel (size-independent property, run
  at the full BASELINE stream-K shapes).
Inputs are drawn on the CPU generator, so every machine sees the same values.
"""

import os

import numpy as np
import pytest
import torch

from gfx950_gluon_tutorials_amd import _lib, quant
from gfx950_gluon_tutorials_amd.gemm import _launch
from gfx950_gluon_tutorials_amd.gemm.inter_wave.a4w4 import matmul as a4w4_matmul_8w_mod  # noqa: F401
from gfx950_gluon_tutorials_amd.gemm.intra_wave.a4w4 import matmul as a4w4_matmul
from gfx950_gluon_tutorials_amd.gemm.intra_wave.a8w8 import matmul as a8w8_matmul
from gfx950_gluon_tutorials_amd.gemm.intra_wave.a16w16 import matmul as a16w16_matmul
from oracle import gemm_ref as R

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
SCHEDULES = ["dp", "streamk"]


def _say(msg):
    print(f"\n[case] {msg}", flush=True)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _f32(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


def _check_streamk_clean(dev):
    assert _launch.WORKSPACES.error(dev) == 0, "a stream-K flag wait timed out"


# ---------------------------------------------------------------------------
# Exact fixtures
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("schedule", SCHEDULES)
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_a16w16_exact_fixture(gpu, dtype, schedule):
    _say(f"a16w16 exact {dtype} {schedule}")
    g = np.load(os.path.join(GOLDEN, "a16w16_exact.npz"))
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    a = torch.from_numpy(g["a"].astype(np.float32)).to(tdt).to(gpu)
    b_nk = torch.from_numpy(g["b_nk"].astype(np.float32)).to(tdt).to(gpu)
    c = a16w16_matmul(a, b_nk.T, schedule=schedule)
    torch.cuda.synchronize()
    key = "c_f16_bits" if dtype == "f16" else "c_bf16_bits"
    np.testing.assert_array_equal(_bits(c), g[key])
    if schedule == "streamk":
        _check_streamk_clean(gpu)


@pytest.mark.parametrize("schedule", SCHEDULES)
def test_a8w8_exact_fixture(gpu, schedule):
    _say(f"a8w8 exact {schedule}")
    g = np.load(os.path.join(GOLDEN, "a8w8_exact.npz"))
    a = torch.from_numpy(g["a_codes"]).view(torch.float8_e5m2).to(gpu)
    b_nk = torch.from_numpy(g["b_codes"]).view(torch.float8_e5m2).to(gpu)
    c = a8w8_matmul(a, b_nk.T, schedule=schedule)  # reference defaults: no scales, fp16 out
    assert c.dtype == torch.float16
    c2 = a8w8_matmul(a, b_nk.T, a_scale=float(g["a_scale"]), b_scale=torch.tensor(float(g["b_scale"])),
                     out_dtype=torch.bfloat16, schedule=schedule)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(c), g["c_f16_bits"])
    np.testing.assert_array_equal(_bits(c2), g["c_bf16_scaled_bits"])


@pytest.mark.parametrize("schedule", SCHEDULES)
@pytest.mark.parametrize("scale_layout", ["row_major", "m_contiguous"])
def test_a4w4_exact_fixture(gpu, schedule, scale_layout):
    _say(f"a4w4 exact {schedule} {scale_layout}")
    g = np.load(os.path.join(GOLDEN, "a4w4_exact.npz"))
    a = torch.from_numpy(g["a"]).to(gpu)
    b = torch.from_numpy(g["b"]).to(gpu)
    sa = torch.from_numpy(g["a_scales"]).to(gpu)
    sb = torch.from_numpy(g["b_scales"]).to(gpu)
    if scale_layout == "m_contiguous":
        # The reference's generator hands the kernel transposed scale views
        # (kernels/gemm/intra_wave/a4w4/bench.py:138-144).
        sa = sa.T.contiguous().T
        sb = sb.T.contiguous().T
    c = a4w4_matmul(a, b, sa, sb, schedule=schedule)
    torch.cuda.synchronize()
    assert c.dtype == torch.bfloat16
    np.testing.assert_array_equal(_bits(c), g["c_bf16_bits"])


# ---------------------------------------------------------------------------
# Seeded configurations
# ---------------------------------------------------------------------------


def _randn(gen, shape, scale=1.0):
    return torch.randn(shape, generator=gen) * scale


def _check_f16(out: torch.Tensor, ref: np.ndarray, K: int, sigma: float, rows=None):
    o = _f32(out if rows is None else out[rows])
    atol = 1e-2 * np.sqrt(K) * sigma
    bad = ~np.isclose(o, ref, rtol=1e-2, atol=atol)
    assert not bad.any(), f"{int(bad.sum())} outputs outside rtol 1e-2 / atol {atol:.3g}; max |err| {np.abs(o - ref).max():.3g}"


def _row_sample(M, n=192, seed=0):
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(seed).integers(0, M, n)]))
    return torch.from_numpy(rows)


@pytest.mark.parametrize("schedule", SCHEDULES)
def test_a16w16_cpu_plumbing_config(gpu, schedule):
    """512x512x1024 fp16, randn(seed=0), C = A.B^T."""
    _say(f"a16w16 512x512x1024 seed0 {schedule}")
    gen = torch.Generator().manual_seed(0)
    a = _randn(gen, (512, 1024)).half()
    b = _randn(gen, (512, 1024)).half()
    c = a16w16_matmul(a.to(gpu), b.to(gpu).T, schedule=schedule)
    torch.cuda.synchronize()
    _check_f16(c, R.a16w16_ref(a.numpy(), b.numpy()), K=1024, sigma=1.0)


@pytest.mark.parametrize("M,N", [(1, 1), (129, 127), (130, 129), (255, 136), (256, 257), (300, 390)])
@pytest.mark.parametrize("pad", [0, 3, 8])
@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("schedule", SCHEDULES)
def test_a16w16_epilogue_edges_exact(gpu, M, N, pad, waves, schedule):
    # Small-integer operands make every output exact in fp32 and fp16, so the
    # kernel must match the oracle bit for bit.  M and N fall on both sides of
    # the 128-row / 128-column quadrant boundaries of a 256x256 tile (the
    # 4-wave epilogue stores quadrant by quadrant), and C is a view of a wider
    # NaN-filled buffer (row stride N + pad; pad 3 misaligns the 16-byte
    # stores): nothing outside the view may change.
    K = 64
    _say(f"a16w16 epilogue edges {M}x{N}x{K} pad {pad} {waves}w {schedule}")
    rng = np.random.default_rng(M * 1000 + N + pad)
    a = rng.integers(-3, 4, (M, K)).astype(np.float16)
    b = rng.integers(-3, 4, (N, K)).astype(np.float16)
    full = torch.full((M, N + pad), float("nan"), dtype=torch.float16, device=gpu)
    c = full[:, :N]
    _launch.gemm_a16w16(torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu).T, c, schedule=schedule,
                        waves=waves)
    torch.cuda.synchronize()
    _check_streamk_clean(gpu)
    np.testing.assert_array_equal(_f32(c), R.a16w16_ref(a, b))
    if pad:
        assert torch.isnan(full[:, N:]).all()


@pytest.mark.parametrize("M,N,K", [(300, 200, 512), (257, 129, 64), (64, 1000, 192), (1, 8, 128), (513, 77, 320)])
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_a16w16_ragged_shapes(gpu, M, N, K, dtype):
    _say(f"a16w16 ragged {M}x{N}x{K} {dtype}")
    gen = torch.Generator().manual_seed(M * 7 + N)
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    a = _randn(gen, (M, K)).to(tdt)
    b = _randn(gen, (N, K)).to(tdt)
    c = a16w16_matmul(a.to(gpu), b.to(gpu).T)
    torch.cuda.synchronize()
    ref = R.a16w16_ref(a.float().numpy(), b.float().numpy(), dtype)
    _check_f16(c, ref, K=K, sigma=1.0)


def test_a16w16_b_as_contiguous_kn(gpu):
    """A (K, N) row-major B (not a transposed view) is repacked, same result."""
    _say("a16w16 contiguous (K,N) b")
    gen = torch.Generator().manual_seed(11)
    a = _randn(gen, (256, 512)).half()
    b_kn = _randn(gen, (512, 384)).half()
    c = a16w16_matmul(a.to(gpu), b_kn.to(gpu))
    torch.cuda.synchronize()
    _check_f16(c, R.a16w16_ref(a.numpy(), b_kn.T.contiguous().numpy()), K=512, sigma=1.0)


def test_a16w16_baseline_config(gpu):
    """4096x4096x8192 fp16, randn(seed=1)*0.1, 256x256x64 tiles, DP."""
    _say("a16w16 4096x4096x8192 seed1")
    gen = torch.Generator().manual_seed(1)
    a = (_randn(gen, (4096, 8192), 0.1)).half()
    b = (_randn(gen, (4096, 8192), 0.1)).half()
    c = a16w16_matmul(a.to(gpu), b.to(gpu).T)
    torch.cuda.synchronize()
    rows = _row_sample(4096)
    ref = R.a16w16_ref(a[rows].numpy(), b.numpy())
    _check_f16(c, ref, K=8192, sigma=0.01, rows=rows)


def test_a8w8_baseline_config(gpu):
    """BF8 4096x4096x8192, randn(seed=2) with per-tensor scales, bf16 out."""
    _say("a8w8 4096x4096x8192 seed2")
    gen = torch.Generator().manual_seed(2)
    a = _randn(gen, (4096, 8192))
    b = _randn(gen, (4096, 8192))
    qa, sa = quant.quantize_e5m2(a)
    qb, sb = quant.quantize_e5m2(b)
    c = a8w8_matmul(qa.to(gpu), qb.to(gpu).T, a_scale=sa.to(gpu), b_scale=sb.to(gpu), out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    rows = _row_sample(4096)
    ref = R.a8w8_ref(qa.view(torch.uint8)[rows].numpy(), qb.view(torch.uint8).numpy(), float(sa), float(sb), "bf16")
    err = R.rel_frobenius(_f32(c[rows]), ref)
    assert err <= 1e-3, f"relative Frobenius error {err:.3g}"


def test_a4w4_baseline_config(gpu):
    """MXFP4 4096x4096x8192 quantized from randn(seed=3), bf16 out."""
    _say("a4w4 4096x4096x8192 seed3")
    gen = torch.Generator().manual_seed(3)
    a = _randn(gen, (4096, 8192))
    b = _randn(gen, (4096, 8192))
    pa, sa = quant.quantize_mxfp4(a)
    pb, sb = quant.quantize_mxfp4(b)
    c = a4w4_matmul(pa.to(gpu), pb.to(gpu), sa.to(gpu), sb.to(gpu))
    torch.cuda.synchronize()
    rows = _row_sample(4096)
    ref = R.a4w4_ref(pa[rows].numpy(), pb.numpy(), sa[rows].numpy(), sb.numpy(), "bf16")
    err = R.rel_frobenius(_f32(c[rows]), ref)
    assert err <= 1e-3, f"relative Frobenius error {err:.3g}"


# Stage counts around the loop structure: the MXFP4 loop body is 8 stages (two
# 4-stage scale chunks), the others 2; shorter counts run only the tail, and
# the last stages' DMAs fall past the end of K.  Ragged M/N add edge tiles.
# Stream-K splits these into segments that start at any stage.
@pytest.mark.parametrize("ns", [1, 2, 3, 4, 5, 7, 8, 9, 10, 17])
@pytest.mark.parametrize("waves", [4, 8])
def test_a4w4_stage_counts(gpu, ns, waves):
    M, N, K = 300, 264, 256 * ns
    _say(f"a4w4 {M}x{N}x{K} waves={waves}")
    gen = torch.Generator().manual_seed(100 + ns)
    pa, sa = quant.quantize_mxfp4(_randn(gen, (M, K)))
    pb, sb = quant.quantize_mxfp4(_randn(gen, (N, K)))
    args = [t.to(gpu) for t in (pa, pb, sa, sb)]
    outs = {}
    for sched in SCHEDULES:
        c = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
        outs[sched] = _launch.gemm_a4w4(*args, c, schedule=sched, waves=waves)
    torch.cuda.synchronize()
    _check_streamk_clean(gpu)
    ref = R.a4w4_ref(pa.numpy(), pb.numpy(), sa.numpy(), sb.numpy(), "bf16")
    err = R.rel_frobenius(_f32(outs["dp"]), ref)
    assert err <= 1e-3, f"relative Frobenius error {err:.3g}"
    np.testing.assert_array_equal(_bits(outs["streamk"]), _bits(outs["dp"]))


@pytest.mark.parametrize("ns", [1, 2, 3, 5, 9])
@pytest.mark.parametrize("waves", [4, 8])
def test_a8w8_stage_counts(gpu, ns, waves):
    M, N, K = 260, 300, 128 * ns
    _say(f"a8w8 {M}x{N}x{K} waves={waves}")
    gen = torch.Generator().manual_seed(200 + ns)
    qa, sa = quant.quantize_e5m2(_randn(gen, (M, K)))
    qb, sb = quant.quantize_e5m2(_randn(gen, (N, K)))
    a, b = qa.to(gpu), qb.to(gpu)
    outs = {}
    for sched in SCHEDULES:
        c = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
        outs[sched] = _launch.gemm_a8w8(a, b.T, c, a_scale=sa.to(gpu), b_scale=sb.to(gpu), schedule=sched,
                                        waves=waves)
    torch.cuda.synchronize()
    _check_streamk_clean(gpu)
    ref = R.a8w8_ref(qa.view(torch.uint8).numpy(), qb.view(torch.uint8).numpy(), float(sa), float(sb), "bf16")
    err = R.rel_frobenius(_f32(outs["dp"]), ref)
    assert err <= 1e-3, f"relative Frobenius error {err:.3g}"
    np.testing.assert_array_equal(_bits(outs["streamk"]), _bits(outs["dp"]))


@pytest.mark.parametrize("M,N,K", [(3840, 3840, 16384), (8192, 1280, 8192), (4352, 4096, 1024), (5120, 5120, 2048)])
def test_streamk_bit_identical_to_dp(gpu, M, N, K):
    """fp16 randn(seed=4)*0.1; stream-K output == data-parallel output, bit for bit.  The
    last two shapes have more tiles than workgroups (272 and 400 tiles), so workgroups own a tile's
    suffix, whole tiles and the next tile's prefix."""
    _say(f"stream-K vs DP {M}x{N}x{K} seed4")
    gen = torch.Generator().manual_seed(4)
    a = _randn(gen, (M, K), 0.1).half().to(gpu)
    b = _randn(gen, (N, K), 0.1).half().to(gpu)
    dp = a16w16_matmul(a, b.T, schedule="dp")
    sk = a16w16_matmul(a, b.T, schedule="streamk")
    torch.cuda.synchronize()
    _check_streamk_clean(gpu)
    np.testing.assert_array_equal(_bits(sk), _bits(dp))
    rows = _row_sample(M, n=64)
    _check_f16(dp, R.a16w16_ref(a[rows].cpu().numpy(), b.cpu().numpy()), K=K, sigma=0.01, rows=rows)


def test_auto_schedule_picks_streamk_at_272_tiles(gpu):
    _say("schedule=auto 4352x4096x1024")
    gen = torch.Generator().manual_seed(6)
    M, N, K = 4352, 4096, 1024
    a = _randn(gen, (M, K), 0.1).half().to(gpu)
    b = _randn(gen, (N, K), 0.1).half().to(gpu)
    if _lib.load().g9_streamk_workgroups() == 256:
        assert _launch.auto_schedule(M, N) == _lib.G9_SCHED_SK
    dp = a16w16_matmul(a, b.T, schedule="dp")
    auto = a16w16_matmul(a, b.T, schedule="auto")
    torch.cuda.synchronize()
    _check_streamk_clean(gpu)
    np.testing.assert_array_equal(_bits(auto), _bits(dp))


@pytest.mark.parametrize("kind", ["a8w8", "a4w4", "bf16"])
def test_streamk_bit_identical_other_dtypes(gpu, kind):
    _say(f"stream-K vs DP {kind}")
    gen = torch.Generator().manual_seed(5)
    M, N, K = 1280, 768, 4096
    x = _randn(gen, (M, K))
    y = _randn(gen, (N, K))
    if kind == "a8w8":
        qa, sa = quant.quantize_e5m2(x)
        qb, sb = quant.quantize_e5m2(y)
        args = (qa.to(gpu), qb.to(gpu).T)
        run = lambda s: a8w8_matmul(*args, a_scale=sa.to(gpu), b_scale=sb.to(gpu), out_dtype=torch.bfloat16,
                                    schedule=s)
    elif kind == "a4w4":
        pa, sa = quant.quantize_mxfp4(x)
        pb, sb = quant.quantize_mxfp4(y)
        args = (pa.to(gpu), pb.to(gpu), sa.to(gpu), sb.to(gpu))
        run = lambda s: a4w4_matmul(*args, schedule=s)
    else:
        args = (x.bfloat16().to(gpu), y.bfloat16().to(gpu).T)
        run = lambda s: a16w16_matmul(*args, schedule=s)
    dp = run("dp")
    sk = run("streamk")
    torch.cuda.synchronize()
    _check_streamk_clean(gpu)
    np.testing.assert_array_equal(_bits(sk), _bits(dp))


# ---------------------------------------------------------------------------
# Call-surface behaviour
# ---------------------------------------------------------------------------


def test_reference_assertions_and_errors(gpu):
    _say("errors")
    a = torch.zeros(256, 512, dtype=torch.float16, device=gpu)
    b = torch.zeros(384, 256, dtype=torch.float16, device=gpu)
    with pytest.raises(AssertionError):
        a16w16_matmul(a, b.T)  # (256, 512) x (256, 384): incompatible
    with pytest.raises(AssertionError):
        a16w16_matmul(a.T, b.T)  # A not contiguous
    with pytest.raises(ValueError):
        a16w16_matmul(torch.zeros(256, 100, dtype=torch.float16, device=gpu),
                      torch.zeros(256, 100, dtype=torch.float16, device=gpu).T)  # K % 8
    with pytest.raises(ValueError):
        a16w16_matmul(torch.zeros(256, 512, dtype=torch.float16), torch.zeros(256, 512, dtype=torch.float16).T)
    with pytest.raises(ValueError):
        a16w16_matmul(a, torch.zeros(256, 512, dtype=torch.float16, device=gpu).T, schedule="bogus")


def test_launch_on_side_stream_and_preallocated_c(gpu):
    _say("side stream")
    gen = torch.Generator().manual_seed(12)
    a = _randn(gen, (512, 256)).half().to(gpu)
    b = _randn(gen, (256, 256)).half().to(gpu)
    c = torch.full((512, 256), 7.0, dtype=torch.float16, device=gpu)
    s = torch.cuda.Stream(gpu)
    s.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(s):
        out = a16w16_matmul(a, b.T, c)
    s.synchronize()
    assert out.data_ptr() == c.data_ptr()
    _check_f16(c, R.a16w16_ref(a.cpu().numpy(), b.cpu().numpy()), K=256, sigma=1.0)


# ---------------------------------------------------------------------------
# 8-wave (inter_wave) kernels: same per-element MFMA sequence as the 4-wave
# kernels for FP16/BF16/BF8, so their outputs must be bitwise equal.  The
# 8-wave MXFP4 kernel uses 32x32x64 MFMAs (4-wave: 16x16x128): the same exact
# products, summed in another order inside the MFMA, so it matches the exact
# fixtures bit for bit and the 4-wave kernel to fp32 rounding.
# ---------------------------------------------------------------------------
from gfx950_gluon_tutorials_amd.gemm.inter_wave import a4w4 as iw_a4w4  # noqa: E402
from gfx950_gluon_tutorials_amd.gemm.inter_wave import a8w8 as iw_a8w8  # noqa: E402
from gfx950_gluon_tutorials_amd.gemm.inter_wave import a16w16 as iw_a16w16  # noqa: E402


@pytest.mark.parametrize("schedule", SCHEDULES)
def test_inter_wave_exact_fixtures(gpu, schedule):
    _say(f"8-wave exact fixtures {schedule}")
    g = np.load(os.path.join(GOLDEN, "a16w16_exact.npz"))
    a = torch.from_numpy(g["a"]).to(gpu)
    b_nk = torch.from_numpy(g["b_nk"]).to(gpu)
    c = torch.empty(a.shape[0], b_nk.shape[0], dtype=torch.float16, device=gpu)
    iw_a16w16.matmul_kernel_only(a, b_nk, c, schedule=schedule)
    c2 = iw_a16w16.matmul(a, b_nk.T, schedule=schedule)
    g8 = np.load(os.path.join(GOLDEN, "a8w8_exact.npz"))
    a8 = torch.from_numpy(g8["a_codes"]).view(torch.float8_e5m2).to(gpu)
    b8 = torch.from_numpy(g8["b_codes"]).view(torch.float8_e5m2).to(gpu)
    c8 = iw_a8w8.matmul(a8, b8.T, schedule=schedule)
    c8s = torch.empty(a8.shape[0], b8.shape[0], dtype=torch.bfloat16, device=gpu)
    iw_a8w8.matmul_kernel_only(a8, b8, c8s, a_scale=float(g8["a_scale"]), b_scale=float(g8["b_scale"]),
                               schedule=schedule)
    g4 = np.load(os.path.join(GOLDEN, "a4w4_exact.npz"))
    args4 = [torch.from_numpy(g4[k]).to(gpu) for k in ("a", "b", "a_scales", "b_scales")]
    c4 = iw_a4w4.matmul(*args4, schedule=schedule)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(c), g["c_f16_bits"])
    np.testing.assert_array_equal(_bits(c2), g["c_f16_bits"])
    assert c8.dtype == torch.float16
    np.testing.assert_array_equal(_bits(c8), g8["c_f16_bits"])
    np.testing.assert_array_equal(_bits(c8s), g8["c_bf16_scaled_bits"])
    assert c4.dtype == torch.bfloat16
    np.testing.assert_array_equal(_bits(c4), g4["c_bf16_bits"])


@pytest.mark.parametrize("kind", ["fp16", "bf16", "bf8", "mxfp4"])
def test_8wave_matches_4wave_at_baseline_size(gpu, kind):
    _say(f"8-wave vs 4-wave {kind} 4096x4096x8192")
    gen = torch.Generator().manual_seed({"fp16": 1, "bf16": 1, "bf8": 2, "mxfp4": 3}[kind])
    x = _randn(gen, (4096, 8192))
    y = _randn(gen, (4096, 8192))
    if kind in ("fp16", "bf16"):
        tdt = torch.float16 if kind == "fp16" else torch.bfloat16
        a, b = (x * 0.1).to(tdt).to(gpu), (y * 0.1).to(tdt).to(gpu)
        run = lambda w, s: _launch.gemm_a16w16(a, b.T, torch.empty(4096, 4096, dtype=tdt, device=gpu),
                                               schedule=s, waves=w)
    elif kind == "bf8":
        qa, sa = quant.quantize_e5m2(x)
        qb, sb = quant.quantize_e5m2(y)
        qa, qb, sa, sb = qa.to(gpu), qb.to(gpu), sa.to(gpu), sb.to(gpu)
        run = lambda w, s: _launch.gemm_a8w8(qa, qb.T, torch.empty(4096, 4096, dtype=torch.bfloat16, device=gpu),
                                             a_scale=sa, b_scale=sb, schedule=s, waves=w)
    else:
        pa, sa = quant.quantize_mxfp4(x)
        pb, sb = quant.quantize_mxfp4(y)
        args = [t.to(gpu) for t in (pa, pb, sa, sb)]
        run = lambda w, s: _launch.gemm_a4w4(*args, torch.empty(4096, 4096, dtype=torch.bfloat16, device=gpu),
                                             schedule=s, waves=w)
    c4 = run(4, "dp")
    c8 = run(8, "dp")
    c8sk = run(8, "streamk")
    torch.cuda.synchronize()
    _check_streamk_clean(gpu)
    if kind == "mxfp4":
        # bf16 outputs of fp32 sums that differ in the last bits: a few
        # elements land one bf16 step apart.
        assert R.rel_frobenius(_f32(c8), _f32(c4)) < 2e-4
    else:
        np.testing.assert_array_equal(_bits(c8), _bits(c4))
    np.testing.assert_array_equal(_bits(c8sk), _bits(c8))
