"""Prepared launches (g9_plan_* / g9_plan_launch, PreparedGemm) on the GPU.

A prepared launch must be the launch the matmul wrappers make for the same
arguments: every slot of a PreparedGemm, launched any number of times and in
any order, gives the wrapper's output bit for bit, for every operand type,
schedule (data-parallel, stream-K on 256x256 and 256x128 tiles, split-K),
wave count and MXFP4 scale layout.  Operands the kernels cannot read in place
are refused instead of copied, and a plan is plain data: a byte copy of it
launches the same GEMM.
"""

import ctypes

import numpy as np
import pytest
import torch

from gfx950_gluon_tutorials_amd import _lib, quant
from gfx950_gluon_tutorials_amd.gemm import _launch
from gfx950_gluon_tutorials_amd.gemm.prepared import PreparedGemm

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"\n[case] {msg}", flush=True)


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy()


def _f16_sets(gpu, M, N, K, dtype, n, seed):
    gen = torch.Generator().manual_seed(seed)
    sets = []
    for _ in range(n):
        a = (torch.randn(M, K, generator=gen) * 0.2).to(dtype).to(gpu)
        b = (torch.randn(N, K, generator=gen) * 0.2).to(dtype).to(gpu)
        sets.append((a, b.T, torch.empty(M, N, dtype=dtype, device=gpu)))
    return sets


@pytest.mark.parametrize("schedule,waves,M,N,K", [
    ("dp", 4, 1000, 700, 1032), ("dp", 8, 600, 520, 2048), ("streamk", 4, 1300, 1100, 2048),
    ("streamk", 8, 1024, 768, 4096), ("streamk_half", 4, 600, 900, 1536), ("splitk", 4, 512, 1024, 4096),
    ("splitk", 8, 256, 512, 2048)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_a16w16_slots_match_the_wrapper(gpu, schedule, waves, M, N, K, dtype):
    _say(f"prepared a16w16 {schedule} {waves}w {M}x{N}x{K} {dtype}")
    sets = _f16_sets(gpu, M, N, K, dtype, 3, M + N + K)
    prep = PreparedGemm.a16w16(sets, schedule=schedule, waves=waves)
    assert prep.slots == 3
    ref = [_launch.gemm_a16w16(a, b, torch.empty_like(c), schedule=schedule, waves=waves) for a, b, c in sets]
    for slot in (2, 0, 1, 2, 4):  # any order, any number of times; slot 4 is slot 1
        prep(slot)
    torch.cuda.synchronize()
    assert prep.error() == 0
    for (_, _, c), r in zip(sets, ref):
        np.testing.assert_array_equal(_bits(c), _bits(r))


@pytest.mark.parametrize("schedule,waves", [("dp", 4), ("dp", 8), ("streamk", 4), ("splitk", 4)])
def test_a8w8_slots_match_the_wrapper(gpu, schedule, waves):
    M, N, K = (512, 1024, 4096) if schedule == "splitk" else (900, 1300, 2048)
    _say(f"prepared a8w8 {schedule} {waves}w {M}x{N}x{K}")
    gen = torch.Generator().manual_seed(7)
    sets = []
    for _ in range(2):
        qa, sa = quant.quantize_e5m2(torch.randn(M, K, generator=gen).to(gpu))
        qb, sb = quant.quantize_e5m2(torch.randn(N, K, generator=gen).to(gpu))
        sets.append((qa, qb.T, torch.empty(M, N, dtype=torch.bfloat16, device=gpu), sa, sb))
    prep = PreparedGemm.a8w8(sets, schedule=schedule, waves=waves)
    ref = [_launch.gemm_a8w8(a, b, torch.empty_like(c), a_scale=sa, b_scale=sb, schedule=schedule, waves=waves)
           for a, b, c, sa, sb in sets]
    prep(1)
    prep(0)
    torch.cuda.synchronize()
    assert prep.error() == 0
    for s, r in zip(sets, ref):
        np.testing.assert_array_equal(_bits(s[2]), _bits(r))


@pytest.mark.parametrize("layout,schedule,waves", [
    ("row", "dp", 4), ("row", "dp", 8), ("row", "streamk", 4), ("row", "splitk", 4), ("kmajor", "dp", 4),
    ("kmajor", "streamk", 4), ("preshuffled", "dp", 4)])
def test_a4w4_slots_match_the_wrapper(gpu, layout, schedule, waves):
    M, N, K = (512, 1024, 4096) if schedule == "splitk" else (1024, 768, 2048)
    _say(f"prepared a4w4 {layout} {schedule} {waves}w {M}x{N}x{K}")
    gen = torch.Generator().manual_seed(11)
    sets = []
    for _ in range(2):
        pa, sa = quant.quantize_mxfp4(torch.randn(M, K, generator=gen))
        pb, sb = quant.quantize_mxfp4(torch.randn(N, K, generator=gen))
        if layout == "kmajor":
            sa, sb = sa.t().contiguous().t(), sb.t().contiguous().t()
        elif layout == "preshuffled":
            sa, sb = quant.preshuffle_e8m0(sa), quant.preshuffle_e8m0(sb)
        sets.append((pa.to(gpu), pb.to(gpu), sa.to(gpu), sb.to(gpu),
                     torch.empty(M, N, dtype=torch.bfloat16, device=gpu)))
    if layout == "kmajor":
        assert sets[0][2].stride(0) == 1  # the views survived the copy to the device
    prep = PreparedGemm.a4w4(sets, schedule=schedule, waves=waves)
    ref = [_launch.gemm_a4w4(a, b, sa, sb, torch.empty_like(c), schedule=schedule, waves=waves)
           for a, b, sa, sb, c in sets]
    prep(0)
    prep(1)
    prep(0)
    torch.cuda.synchronize()
    assert prep.error() == 0
    for s, r in zip(sets, ref):
        np.testing.assert_array_equal(_bits(s[4]), _bits(r))


def test_operands_needing_a_copy_are_refused(gpu):
    _say("prepared launches refuse repacks")
    M, N, K = 256, 256, 512
    a = torch.randn(M, K, device=gpu).half()
    b = torch.randn(N, K, device=gpu).half()
    c = torch.empty(M, N, dtype=torch.half, device=gpu)
    with pytest.raises(ValueError, match="b is not in a layout"):
        PreparedGemm.a16w16([(a, b.T.contiguous(), c)])  # (K, N) row-major: the wrapper would repack it
    with pytest.raises(ValueError, match="a is not in a layout"):
        PreparedGemm.a16w16([(a.T.contiguous().T, b.T, c)])
    qa, sa = quant.quantize_e5m2(torch.randn(M, K, device=gpu))
    qb, sb = quant.quantize_e5m2(torch.randn(N, K, device=gpu))
    with pytest.raises(ValueError, match="a_scale"):
        PreparedGemm.a8w8([(qa, qb.T, c, 2.0, sb)])  # a Python float would need a device copy
    pa, psa = quant.quantize_mxfp4(torch.randn(M, K))
    pb, psb = quant.quantize_mxfp4(torch.randn(N, K))
    pa, pb = pa.to(gpu), pb.to(gpu)
    km_a, km_b = psa.t().contiguous().t().to(gpu), psb.t().contiguous().t().to(gpu)
    c16 = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError, match="a_scales is not in a layout"):
        PreparedGemm.a4w4([(pa, pb, km_a, km_b, c16)], waves=8)  # 8 waves read row-major scales only
    # The same operands in the kernels' layouts are accepted and computed.
    PreparedGemm.a4w4([(pa, pb, km_a, km_b, c16)])()
    torch.cuda.synchronize()


def test_own_workspace_survives_a_release_of_the_cached_ones(gpu):
    _say("prepared stream-K after WORKSPACES.release")
    sets = _f16_sets(gpu, 1536, 1280, 4096, torch.float16, 2, 5)
    prep = PreparedGemm.a16w16(sets, schedule="streamk")
    ref = [_launch.gemm_a16w16(a, b, torch.empty_like(c), schedule="streamk") for a, b, c in sets]
    torch.cuda.synchronize()
    _launch.WORKSPACES.release()
    for i in range(6):
        prep(i)
    torch.cuda.synchronize()
    assert prep.error() == 0
    for (_, _, c), r in zip(sets, ref):
        np.testing.assert_array_equal(_bits(c), _bits(r))


def test_c_abi_plan_is_plain_data(gpu):
    """A plan made through the C ABI directly, and a byte copy of it, launch
    the GEMM g9_gemm_a16w16 launches; a zeroed plan is refused."""
    _say("C ABI plan byte copy")
    lib = _lib.load()
    M, N, K = 768, 512, 1024
    a = torch.randn(M, K, device=gpu).half()
    b = torch.randn(N, K, device=gpu).half()
    c_ref = torch.empty(M, N, dtype=torch.half, device=gpu)
    c = torch.empty(M, N, dtype=torch.half, device=gpu)
    stream = torch.cuda.current_stream(gpu).cuda_stream
    args = (M, N, K, K, 1, 1, K, N, 1, _lib.G9_F16, _lib.G9_SCHED_DP, 4)
    assert lib.g9_gemm_a16w16(a.data_ptr(), b.data_ptr(), c_ref.data_ptr(), *args, None, 0, stream) == 0
    plan = (ctypes.c_uint64 * (_lib.G9_PLAN_BYTES // 8))()
    assert lib.g9_plan_a16w16(ctypes.addressof(plan), a.data_ptr(), b.data_ptr(), c.data_ptr(), *args, None, 0) == 0
    copy = (ctypes.c_uint64 * (_lib.G9_PLAN_BYTES // 8))()
    ctypes.memmove(copy, plan, ctypes.sizeof(plan))
    del plan
    assert lib.g9_plan_launch(ctypes.addressof(copy), stream) == 0
    zero = (ctypes.c_uint64 * (_lib.G9_PLAN_BYTES // 8))()
    assert lib.g9_plan_launch(ctypes.addressof(zero), stream) == _lib.G9_ERR_PLAN
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(c), _bits(c_ref))


@pytest.mark.parametrize("schedule,M,N,K", [("dp", 1000, 700, 2048), ("splitk", 512, 1024, 4096),
                                            ("streamk", 1300, 1100, 2048), ("streamk_half", 600, 900, 1536)])
def test_prepared_launches_replay_in_a_graph(gpu, schedule, M, N, K):
    """Two slots' launches captured in one HIP graph (a plan launch is a bare
    hipLaunchKernel, split-K's two kernels included) and replayed three
    times with eager work and synchronisations in between: every replay
    matches the wrappers' eager output bit for bit.  A captured stream-K
    launch keeps the flag epoch it was captured with; every tile's last
    owner clears its flag, so each replay starts from clear flags."""
    _say(f"prepared {schedule} {M}x{N}x{K} captured in a graph")
    sets = _f16_sets(gpu, M, N, K, torch.float16, 2, 99)
    want = [_launch.gemm_a16w16(a, b, torch.empty_like(c), schedule=schedule) for a, b, c in sets]
    torch.cuda.synchronize()
    side = torch.cuda.Stream(device=gpu)
    with torch.cuda.stream(side):
        prep = PreparedGemm.a16w16(sets, schedule=schedule)  # bound to `side`
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        prep(0)
        prep(1)
    for r in range(3):
        for _, _, c in sets:
            c.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for (_, _, c), w in zip(sets, want):
            assert torch.equal(c, w), r
    assert prep.error() == 0
