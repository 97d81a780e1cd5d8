"""Concurrent launches on several streams, and one workspace reused by
stream-K launches of different tile counts.

* Every (device, stream) pair has its own workspace, so stream-K and split-K
  launches running at the same time on two streams never share partials or
  flags: each result equals what the same launch gives alone (stream-K:
  bit-identical to data-parallel; split-K: bit-identical to its own
  single-stream result, which is deterministic).
* A 272-tile stream-K launch between two 400-tile ones on one workspace
  leaves the larger launch's flags intact (the partials sit behind the whole
  flag region), so all three stay bit-identical to data-parallel.
"""

import pytest
import torch

from gfx950_gluon_tutorials_amd.gemm import _launch

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"\n[case] {msg}", flush=True)


def _operands(gen, M, N, K, dev):
    a = (torch.randn(M, K, generator=gen) * 0.1).half().to(dev)
    b = (torch.randn(N, K, generator=gen) * 0.1).half().to(dev)
    return a, b


def test_streamk_and_splitk_on_two_streams_at_once(gpu):
    g = torch.Generator().manual_seed(61)
    # 272 tiles: stream-K hands partial tiles along K chains (flags in use);
    # 512 x 4096: split-K runs 8 segments per tile (partials in use).
    sk_shape = (4352, 4096, 2048)
    sp_shape = (512, 4096, 8192)
    sk_in = [_operands(g, *sk_shape, gpu) for _ in range(2)]
    sp_in = [_operands(g, *sp_shape, gpu) for _ in range(2)]
    _say("single-stream references: data-parallel for stream-K, split-K alone")
    want_sk, want_sp = [], []
    for (a, b), (x, y) in zip(sk_in, sp_in):
        want_sk.append(_launch.gemm_a16w16(a, b.T, torch.empty(sk_shape[0], sk_shape[1], dtype=torch.float16,
                                                                 device=gpu), schedule="dp"))
        want_sp.append(_launch.gemm_a16w16(x, y.T, torch.empty(sp_shape[0], sp_shape[1], dtype=torch.float16,
                                                                 device=gpu), schedule="splitk"))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(gpu), torch.cuda.Stream(gpu)]
    reps = 3
    outs_sk = [[torch.empty(sk_shape[0], sk_shape[1], dtype=torch.float16, device=gpu) for _ in range(reps)]
               for _ in range(2)]
    outs_sp = [[torch.empty(sp_shape[0], sp_shape[1], dtype=torch.float16, device=gpu) for _ in range(reps)]
               for _ in range(2)]
    torch.cuda.synchronize()
    _say("stream-K and split-K interleaved on two streams")
    for r in range(reps):
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                a, b = sk_in[i]
                _launch.gemm_a16w16(a, b.T, outs_sk[i][r], schedule="streamk")
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                x, y = sp_in[i]
                _launch.gemm_a16w16(x, y.T, outs_sp[i][r], schedule="splitk")
    torch.cuda.synchronize()
    for i, s in enumerate(streams):
        assert _launch.WORKSPACES.error(gpu, s.cuda_stream) == 0, "a stream-K flag wait timed out"
        for r in range(reps):
            assert torch.equal(outs_sk[i][r], want_sk[i]), (i, r)
            assert torch.equal(outs_sp[i][r], want_sp[i]), (i, r)


def test_streamk_smaller_launch_between_larger_ones(gpu):
    g = torch.Generator().manual_seed(62)
    K = 1024
    big = _operands(g, 5120, 5120, K, gpu)      # 400 tiles
    small = _operands(g, 4352, 4096, K, gpu)    # 272 tiles
    want = {}
    for name, (a, b) in (("big", big), ("small", small)):
        want[name] = _launch.gemm_a16w16(a, b.T, torch.empty(a.shape[0], b.shape[0], dtype=torch.float16,
                                                             device=gpu), schedule="dp")
    torch.cuda.synchronize()
    _say("stream-K 400 -> 272 -> 400 tiles on one workspace")
    for name in ("big", "small", "big", "small"):
        a, b = big if name == "big" else small
        out = _launch.gemm_a16w16(a, b.T, torch.empty(a.shape[0], b.shape[0], dtype=torch.float16, device=gpu),
                                  schedule="streamk")
        torch.cuda.synchronize()
        _launch.WORKSPACES.check(gpu)
        assert torch.equal(out, want[name]), name


def test_misaligned_b_view_is_repacked(gpu):
    g = torch.Generator().manual_seed(63)
    M, N, K = 512, 384, 1024
    a = (torch.randn(M, K, generator=g) * 0.1).half().to(gpu)
    buf = (torch.randn(N, K + 4, generator=g) * 0.1).half().to(gpu)
    b_nk = buf[:, 4:]  # rows start 8 bytes past a 16-byte boundary
    assert b_nk.data_ptr() % 16 == 8
    _say("a16w16 with a B view whose rows are not 16-byte aligned")
    got = _launch.gemm_a16w16(a, b_nk.T, torch.empty(M, N, dtype=torch.float16, device=gpu))
    want = _launch.gemm_a16w16(a, b_nk.contiguous().T, torch.empty(M, N, dtype=torch.float16, device=gpu))
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_timed_out_flag_wait_raises_at_the_next_launch(gpu):
    """A stream-K flag wait that gives up (forced from the host with a spin
    limit of one poll; every workgroup still exits) sets the workspace's
    pinned host flag, and the next stream-K launch on that stream raises
    without any synchronisation of its own.  The workspace is cleared, so the
    launch after that is bit-identical to data-parallel again."""
    from gfx950_gluon_tutorials_amd import _lib

    g = torch.Generator().manual_seed(67)
    M, N, K = 2048, 2048, 8192  # 64 tiles x 128 stages over 256 workgroups: chained waits
    a, b = _operands(g, M, N, K, gpu)
    dp = _launch.gemm_a16w16(a, b.T, torch.empty(M, N, dtype=torch.float16, device=gpu))
    lib = _lib.load()
    _say("stream-K with a spin limit of one poll")
    prev = lib.g9_set_streamk_spin_limit(1)
    try:
        _launch.gemm_a16w16(a, b.T, torch.empty(M, N, dtype=torch.float16, device=gpu), schedule="streamk")
        torch.cuda.synchronize()
    finally:
        lib.g9_set_streamk_spin_limit(prev)
    _say("next stream-K launch raises")
    with pytest.raises(RuntimeError, match="timed out"):
        _launch.gemm_a16w16(a, b.T, torch.empty(M, N, dtype=torch.float16, device=gpu), schedule="streamk")
    _say("and the one after is right")
    c = _launch.gemm_a16w16(a, b.T, torch.empty(M, N, dtype=torch.float16, device=gpu), schedule="streamk")
    torch.cuda.synchronize()
    assert torch.equal(c, dp)
    _launch.WORKSPACES.poll(gpu)  # nothing pending
