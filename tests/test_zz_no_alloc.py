"""The allocation-free a16w16 entry point (g9_gemm_a16w16_noalloc) against
g9_gemm_a16w16 with a caller-owned workspace, through the C ABI.

Both launch the same kernels, so for every schedule the outputs must be
bit-identical.  Each schedule runs two calls in a row on the library's static
scratch array, the second on a smaller problem (the array keeps the first
call's contents), and a call needing more than the array's
G9_NOALLOC_MAX_TILES partial tiles is rejected with G9_ERR_SCRATCH before any
launch.
"""

import pytest
import torch

from gfx950_gluon_tutorials_amd import _lib

pytestmark = pytest.mark.gpu

MAX_TILES = 256  # G9_NOALLOC_MAX_TILES in include/gfx950_gemm.h


def _say(msg):
    print(f"\n[case] {msg}", flush=True)


def _call(fn, a, b_nk, c, dtype, sched, waves, ws=None):
    lib = _lib.load()
    M, K = a.shape
    N = b_nk.shape[0]
    stream = torch.cuda.current_stream(a.device).cuda_stream
    args = [a.data_ptr(), b_nk.data_ptr(), c.data_ptr(), M, N, K, a.stride(0), 1, 1, b_nk.stride(0),
            c.stride(0), 1, dtype, sched, waves]
    if fn == "noalloc":
        return lib.g9_gemm_a16w16_noalloc(*args, stream)
    ws_ptr, ws_bytes = (ws.data_ptr(), ws.numel()) if ws is not None else (None, 0)
    return lib.g9_gemm_a16w16(*args, ws_ptr, ws_bytes, stream)


def _with_workspace(a, b_nk, dtype, sched, waves):
    """Output of g9_gemm_a16w16 with a fresh caller-owned workspace."""
    lib = _lib.load()
    M, K = a.shape
    N = b_nk.shape[0]
    need = lib.g9_workspace_size(dtype, M, N, K, sched, waves)
    ws = None
    if need:
        ws = torch.empty(need, dtype=torch.uint8, device=a.device)
        assert lib.g9_workspace_init(ws.data_ptr(), ws.numel(), torch.cuda.current_stream(a.device).cuda_stream) == 0
    c = torch.empty(M, N, dtype=a.dtype, device=a.device)
    assert _call("ws", a, b_nk, c, dtype, sched, waves, ws) == 0
    torch.cuda.synchronize()
    return c


def _operands(gen, M, N, K, dt, dev):
    a = (torch.randn(M, K, generator=gen) * 0.1).to(dt).to(dev)
    b = (torch.randn(N, K, generator=gen) * 0.1).to(dt).to(dev)
    return a, b


# (schedule, [(M, N, K), smaller (M, N, K)]): stream-K at 225 tiles (the BASELINE
# shape's tile count) then 60; split-K at 32 tiles x 8 segments then 8 tiles.
CASES = [
    (_lib.G9_SCHED_SK, [(3840, 3840, 2048), (1920, 2048, 1024)]),
    (_lib.G9_SCHED_SPLITK, [(512, 4096, 8192), (256, 2048, 4096)]),
    (_lib.G9_SCHED_DP, [(1024, 1024, 1024), (512, 256, 512)]),
]


@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("sched,shapes", CASES)
def test_noalloc_matches_workspace_entry_point(gpu, sched, shapes, waves):
    g = torch.Generator().manual_seed(71 + sched)
    dt, code = torch.float16, _lib.G9_F16
    lib = _lib.load()
    for M, N, K in shapes:
        need = lib.g9_workspace_size(code, M, N, K, sched, waves)
        _say(f"noalloc schedule={sched} waves={waves} {M}x{N}x{K} workspace={need}")
        a, b = _operands(g, M, N, K, dt, gpu)
        want = _with_workspace(a, b, code, sched, waves)
        got = torch.full((M, N), float("nan"), dtype=dt, device=gpu)
        assert _call("noalloc", a, b, got, code, sched, waves) == 0
        torch.cuda.synchronize()
        assert torch.equal(got, want), (M, N, K)


def test_noalloc_bf16_streamk_twice(gpu):
    g = torch.Generator().manual_seed(79)
    dt, code = torch.bfloat16, _lib.G9_BF16
    for M, N, K in [(4352, 3840, 1024), (2304, 2560, 512)]:
        _say(f"noalloc bf16 stream-K {M}x{N}x{K}")
        a, b = _operands(g, M, N, K, dt, gpu)
        want = _with_workspace(a, b, code, _lib.G9_SCHED_SK, 4)
        got = torch.empty(M, N, dtype=dt, device=gpu)
        assert _call("noalloc", a, b, got, code, _lib.G9_SCHED_SK, 4) == 0
        torch.cuda.synchronize()
        assert torch.equal(got, want), (M, N, K)


def test_noalloc_streamk_half_tiles_twice(gpu):
    # 256x128 stream-K tiles (4 waves only): 450 tiles, then 60, in the same
    # scratch array.
    g = torch.Generator().manual_seed(83)
    dt, code, sched = torch.float16, _lib.G9_F16, _lib.G9_SCHED_SK_HALF
    for M, N, K in [(3840, 3840, 2048), (1920, 1024, 1024)]:
        _say(f"noalloc stream-K 256x128 {M}x{N}x{K}")
        a, b = _operands(g, M, N, K, dt, gpu)
        want = _with_workspace(a, b, code, sched, 4)
        got = torch.full((M, N), float("nan"), dtype=dt, device=gpu)
        assert _call("noalloc", a, b, got, code, sched, 4) == 0
        torch.cuda.synchronize()
        assert torch.equal(got, want), (M, N, K)
    c = torch.empty(64, 64, dtype=dt, device=gpu)
    assert _call("noalloc", a[:64], b[:64], c, code, sched, 8) == _lib.G9_ERR_SCHEDULE


def test_noalloc_rejects_more_than_the_scratch_holds(gpu):
    g = torch.Generator().manual_seed(80)
    M, N, K = 5120, 3328, 512  # 20 x 13 = 260 tiles > 256 partials
    assert -(-M // 256) * -(-N // 256) > MAX_TILES
    a, b = _operands(g, M, N, K, torch.float16, gpu)
    c = torch.zeros(M, N, dtype=torch.float16, device=gpu)
    _say("noalloc stream-K beyond the scratch array: rejected, nothing launched")
    assert _call("noalloc", a, b, c, _lib.G9_F16, _lib.G9_SCHED_SK, 4) == _lib.G9_ERR_SCRATCH
    torch.cuda.synchronize()
    assert not c.any()  # nothing was written
    # Data-parallel on the same shape needs no scratch.
    assert _call("noalloc", a, b, c, _lib.G9_F16, _lib.G9_SCHED_DP, 4) == 0
    torch.cuda.synchronize()
    assert torch.equal(c, _with_workspace(a, b, _lib.G9_F16, _lib.G9_SCHED_DP, 4))


def _noalloc_error(dev):
    out = _lib.ctypes.c_int(-1)
    assert _lib.load().g9_noalloc_error(torch.cuda.current_stream(dev).cuda_stream, _lib.ctypes.byref(out)) == 0
    return out.value


def test_noalloc_reports_a_timed_out_flag_wait(gpu):
    """g9_noalloc_error reads the static array's error word.  A spin limit of
    one poll (set from the host) makes the chained waits of a stream-K call
    time out while every workgroup still exits; the call's output is then
    wrong and the word reads 1.  With the default limit the next call clears
    it, reads 0 and matches the workspace entry point again."""
    g = torch.Generator().manual_seed(83)
    M, N, K = 2048, 2048, 8192  # 64 tiles x 128 stages over 256 workgroups: 4 per tile, chained
    a, b = _operands(g, M, N, K, torch.float16, gpu)
    want = _with_workspace(a, b, _lib.G9_F16, _lib.G9_SCHED_SK, 4)
    c = torch.empty(M, N, dtype=torch.float16, device=gpu)
    lib = _lib.load()
    _say("noalloc stream-K, default spin limit: error word 0")
    assert _call("noalloc", a, b, c, _lib.G9_F16, _lib.G9_SCHED_SK, 4) == 0
    assert _noalloc_error(gpu) == 0
    assert torch.equal(c, want)
    _say("noalloc stream-K, spin limit 1: error word 1")
    prev = lib.g9_set_streamk_spin_limit(1)
    try:
        assert _call("noalloc", a, b, c, _lib.G9_F16, _lib.G9_SCHED_SK, 4) == 0
        assert _noalloc_error(gpu) == 1
    finally:
        lib.g9_set_streamk_spin_limit(prev)
    _say("noalloc stream-K, default spin limit again: error word 0, output right")
    assert _call("noalloc", a, b, c, _lib.G9_F16, _lib.G9_SCHED_SK, 4) == 0
    assert _noalloc_error(gpu) == 0
    assert torch.equal(c, want)


@pytest.mark.parametrize("sched,shape", [(_lib.G9_SCHED_SK, (3840, 3840, 2048)),
                                         (_lib.G9_SCHED_SPLITK, (512, 4096, 8192))])
def test_noalloc_under_graph_capture(gpu, sched, shape):
    """One call captured in a HIP graph (its stream-K flag clearing is a fill
    kernel, not a memset) and replayed three times with eager work and
    synchronisations in between: every replay is bit-equal to the workspace
    entry point."""
    g = torch.Generator().manual_seed(90 + sched)
    M, N, K = shape
    a, b = _operands(g, M, N, K, torch.float16, gpu)
    want = _with_workspace(a, b, _lib.G9_F16, sched, 4)
    c = torch.empty(M, N, dtype=torch.float16, device=gpu)
    _say(f"noalloc schedule={sched} {M}x{N}x{K}: eager call, then capture")
    assert _call("noalloc", a, b, c, _lib.G9_F16, sched, 4) == 0  # looks up the array outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = _call("noalloc", a, b, c, _lib.G9_F16, sched, 4)
    assert rc == 0
    for r in range(3):
        _say(f"noalloc schedule={sched}: replay {r}")
        c.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(c, want), r
