"""GPU parity of the grouped (MoE) GEMM, through the C ABI (ctypes wrappers):
each expert's rows are bit-identical to the dense data-parallel kernel on that
expert's slice, within tolerance of the CPU oracle, rows no expert owns are
left untouched, and out-of-range offsets are clamped (the lookup that keeps
every access in bounds is restated and checked on the CPU in test_moe.py)."""

import numpy as np
import pytest
import torch

from gfx950_gluon_tutorials_amd import quant
from gfx950_gluon_tutorials_amd.gemm.intra_wave.a4w4 import matmul as a4w4_matmul
from gfx950_gluon_tutorials_amd.gemm.intra_wave.a8w8 import matmul as a8w8_matmul
from gfx950_gluon_tutorials_amd.gemm.intra_wave.a16w16 import matmul as a16w16_matmul
from gfx950_gluon_tutorials_amd.gemm.moe import moe_matmul, moe_matmul_a4w4, moe_matmul_a8w8
from oracle import gemm_ref as R

pytestmark = pytest.mark.gpu

COUNTS = [300, 0, 17, 512, 289, 1]  # tokens per expert: empty, tiny, exact and ragged tiles


def _say(msg):
    print(f"\n[case] {msg}", flush=True)


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _offsets(counts, dev, start=0):
    return torch.tensor(np.concatenate([[start], start + np.cumsum(counts)]), dtype=torch.int32, device=dev)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_moe_a16w16_matches_dense_per_expert(gpu, dtype):
    _say(f"moe a16w16 {dtype} counts {COUNTS}")
    g = torch.Generator().manual_seed(11)
    E, N, K = len(COUNTS), 320, 256
    T = sum(COUNTS)
    a = (torch.randn(T, K, generator=g) * 0.1).to(dtype).to(gpu)
    b = (torch.randn(E, N, K, generator=g) * 0.1).to(dtype).to(gpu)
    off = _offsets(COUNTS, gpu)
    c = moe_matmul(a, b, off)
    torch.cuda.synchronize()
    o = off.cpu().numpy()
    for e in range(E):
        lo, hi = int(o[e]), int(o[e + 1])
        if hi > lo:
            dense = a16w16_matmul(a[lo:hi].contiguous(), b[e].T)
            np.testing.assert_array_equal(_bits(c[lo:hi]), _bits(dense), err_msg=f"expert {e}")
    if dtype == torch.float16:
        ref = R.moe_ref(R.a16w16_ref, a.cpu().numpy(), b.cpu().numpy(), o)
        assert np.allclose(c.float().cpu().numpy(), ref, rtol=1e-2, atol=1e-2 * np.sqrt(K) * 0.01)


def test_moe_a4w4_matches_dense_per_expert(gpu):
    _say(f"moe a4w4 counts {COUNTS}")
    g = torch.Generator().manual_seed(12)
    E, N, K = len(COUNTS), 264, 512
    T = sum(COUNTS)
    pa, sa = quant.quantize_mxfp4(torch.randn(T, K, generator=g))
    pbs, sbs = zip(*[quant.quantize_mxfp4(torch.randn(N, K, generator=g)) for _ in range(E)])
    pb, sb = torch.stack(pbs), torch.stack(sbs)
    pa, sa, pb, sb = (t.to(gpu) for t in (pa, sa, pb, sb))
    off = _offsets(COUNTS, gpu)
    c = moe_matmul_a4w4(pa, pb, sa, sb, off)
    torch.cuda.synchronize()
    o = off.cpu().numpy()
    for e in range(E):
        lo, hi = int(o[e]), int(o[e + 1])
        if hi > lo:
            dense = a4w4_matmul(pa[lo:hi].contiguous(), pb[e], sa[lo:hi].contiguous(), sb[e])
            np.testing.assert_array_equal(_bits(c[lo:hi]), _bits(dense), err_msg=f"expert {e}")
    # The reference's torch_reference rounds to bf16 like the kernel's output.
    ref = R.moe_ref(R.a4w4_ref, pa.cpu().numpy(), pb.cpu().numpy(), o, sa.cpu().numpy(),
                    expert_args=(sb.cpu().numpy(),))
    assert R.rel_frobenius(c.float().cpu().numpy(), ref) <= 1e-3


def test_moe_leaves_rows_no_expert_owns(gpu):
    _say("moe rows outside the offsets")
    g = torch.Generator().manual_seed(13)
    T, N, K = 400, 256, 128
    a = (torch.randn(T, K, generator=g) * 0.1).half().to(gpu)
    b = (torch.randn(3, N, K, generator=g) * 0.1).half().to(gpu)
    off = _offsets([84, 0, 200], gpu, start=16)  # experts own rows [16, 300)
    c = torch.full((T, N), 7.0, dtype=torch.float16, device=gpu)
    moe_matmul(a, b, off, c)
    torch.cuda.synchronize()
    assert torch.all(c[:16] == 7.0) and torch.all(c[300:] == 7.0)
    np.testing.assert_array_equal(_bits(c[16:100]), _bits(a16w16_matmul(a[16:100].contiguous(), b[0].T)))
    np.testing.assert_array_equal(_bits(c[100:300]), _bits(a16w16_matmul(a[100:300].contiguous(), b[2].T)))


def test_moe_clamps_out_of_range_offsets(gpu):
    _say("moe offsets past T and decreasing")
    g = torch.Generator().manual_seed(14)
    T, N, K = 600, 256, 128
    a = (torch.randn(T, K, generator=g) * 0.1).half().to(gpu)
    b = (torch.randn(3, N, K, generator=g) * 0.1).half().to(gpu)
    # expert 0: [0, 250); expert 1: [250, 100) -> empty; expert 2: [100, 10^6) -> [100, 600)
    off = torch.tensor([0, 250, 100, 1_000_000], dtype=torch.int32, device=gpu)
    c = torch.zeros((T, N), dtype=torch.float16, device=gpu)
    moe_matmul(a, b, off, c)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(c[:100]), _bits(a16w16_matmul(a[:100].contiguous(), b[0].T)))
    np.testing.assert_array_equal(_bits(c[250:]), _bits(a16w16_matmul(a[100:].contiguous(), b[2].T)[150:]))


def test_moe_many_experts_multi_pass_lookup(gpu):
    # 130 experts: the lookup walks the offsets 64 experts per pass (three passes); most experts are small
    # or empty, a few span several m-tiles.
    _say("moe a16w16 130 experts")
    rng = np.random.default_rng(15)
    E, N, K = 130, 256, 128
    counts = rng.integers(0, 40, E)
    counts[rng.random(E) < 0.3] = 0
    counts[[5, 70, 129]] = [300, 513, 257]
    T = int(counts.sum())
    g = torch.Generator().manual_seed(15)
    a = (torch.randn(T, K, generator=g) * 0.1).half().to(gpu)
    b = (torch.randn(E, N, K, generator=g) * 0.1).half().to(gpu)
    off = _offsets(counts, gpu)
    c = moe_matmul(a, b, off)
    torch.cuda.synchronize()
    o = off.cpu().numpy()
    ref = R.moe_ref(R.a16w16_ref, a.cpu().numpy(), b.cpu().numpy(), o)
    assert np.allclose(c.float().cpu().numpy(), ref, rtol=1e-2, atol=1e-2 * np.sqrt(K) * 0.01)
    for e in (5, 70, 129):
        lo, hi = int(o[e]), int(o[e + 1])
        np.testing.assert_array_equal(_bits(c[lo:hi]), _bits(a16w16_matmul(a[lo:hi].contiguous(), b[e].T)))


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_moe_a8w8_matches_dense_per_expert(gpu, out_dtype):
    _say(f"moe a8w8 {out_dtype} counts {COUNTS}")
    g = torch.Generator().manual_seed(16)
    E, N, K = len(COUNTS), 384, 512
    T = sum(COUNTS)
    qa, sa = quant.quantize_e5m2(torch.randn(T, K, generator=g))
    qbs, sbs = zip(*[quant.quantize_e5m2(torch.randn(N, K, generator=g) * (1 + e)) for e in range(E)])
    qb, sb = torch.stack(qbs).to(gpu), torch.stack([s.reshape(()) for s in sbs]).float().to(gpu)
    qa, sa = qa.to(gpu), sa.to(gpu)
    off = _offsets(COUNTS, gpu)
    c = moe_matmul_a8w8(qa, qb, off, a_scale=sa, b_scales=sb, out_dtype=out_dtype)
    torch.cuda.synchronize()
    o = off.cpu().numpy()
    for e in range(E):
        lo, hi = int(o[e]), int(o[e + 1])
        if hi > lo:
            dense = a8w8_matmul(qa[lo:hi].contiguous(), qb[e].T, a_scale=sa, b_scale=sb[e], out_dtype=out_dtype)
            np.testing.assert_array_equal(_bits(c[lo:hi]), _bits(dense), err_msg=f"expert {e}")
    codes = lambda t: t.view(torch.uint8).cpu().numpy()
    out = "bf16" if out_dtype == torch.bfloat16 else "f16"
    ref = R.moe_ref(lambda x, y, s: R.a8w8_ref(x, y, float(sa.cpu()), s, out), codes(qa), codes(qb), o,
                    expert_args=(sb.cpu().numpy(),))
    assert R.rel_frobenius(c.float().cpu().numpy(), ref) <= 1e-3
