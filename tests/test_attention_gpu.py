"""GPU parity of the gfx950 flash-attention forward (g9_fmha_fwd through the
drop-in run_gluon_attention) against the float64 oracle, under the
reference's acceptance rule (kernels/attention/common.py:142-171):
|o - o_ref| <= atol + 1e-3 |o_ref| with atol = max(1e-3, 2 eps(out) max|o_ref|).

Cases: both input types, both layouts, both rescale variants, scale on Q or
on the scores, head dims 128 and 64, grouped K/V heads (MHA, GQA, MQA),
sequence lengths that leave a partial 256-query block, strided views, extreme
score ranges, the log-sum-exp output, determinism, and the benchmark shape
checked on sampled rows.
"""

import math

import numpy as np
import pytest
import torch

from gfx950_gluon_tutorials_amd.attention import MetaData, fmha_v3, fmha_v4, input_helper
from oracle import attention_ref as A

pytestmark = pytest.mark.gpu

DT = {"fp16": torch.float16, "bf16": torch.bfloat16}
DT_NAME = {torch.float16: "float16", torch.bfloat16: "bfloat16"}
RUN = {3: fmha_v3.run_gluon_attention, 4: fmha_v4.run_gluon_attention}


def _inputs(B, HQ, HK, S, dtype, layout, seed, scale=1.0, D=128):
    g = torch.Generator().manual_seed(seed)
    shp = (lambda h: (B, h, S, D)) if layout == "bhsd" else (lambda h: (B, S, h, D))
    q, k, v = (torch.randn(shp(h), generator=g) * sc for h, sc in ((HQ, scale), (HK, 1.0), (HK, 1.0)))
    q, k, v = (t.to(dtype) for t in (q, k, v))
    md = MetaData(sm_scale=D**-0.5)
    md.max_seqlens_q = md.max_seqlens_k = S
    md.layout = layout
    return q, k, v, md


def _run(q, k, v, md, dev, variant=4, scale_on_q=True, lse=True):
    qd, kd, vd = (t.to(dev) for t in (q, k, v))
    o = torch.full_like(qd, float("nan"))
    B, HQ = (q.shape[0], q.shape[1]) if md.layout == "bhsd" else (q.shape[0], q.shape[2])
    L = torch.full((B, HQ, md.max_seqlens_q), float("nan"), device=dev) if lse else None
    RUN[variant](qd, kd, vd, o, md, scale_on_q, lse=L)
    torch.cuda.synchronize()
    return o.cpu(), (L.cpu() if lse else None)


def _check(o, L, q, k, v, md):
    ref, ref_lse = A.sdpa_reference(q.float().numpy(), k.float().numpy(), v.float().numpy(), md.sm_scale, md.layout)
    got = A.to_bhsd(o.float().numpy(), md.layout)
    ok, mx, mean = A.within_tolerance(got, ref, DT_NAME[o.dtype])
    assert ok, f"max |diff| {mx:.3g}, mean {mean:.3g}, tolerance {A.check_tolerance(DT_NAME[o.dtype], ref)}"
    if L is not None:
        # Scores are exact fp32 sums of 16-bit products up to accumulation order,
        # except that scale_on_q rounds Q * scale to the input type: allow that
        # rounding of the largest score magnitude.
        qf, kf = (A.to_bhsd(t.float().numpy().astype(np.float64), md.layout) for t in (q, k))
        bound = np.abs(qf).sum(-1).max() * np.abs(kf).max() * md.sm_scale
        tol = 2 * A.FINFO_EPS[DT_NAME[o.dtype]] * bound + 1e-4
        np.testing.assert_allclose(L.numpy(), ref_lse, rtol=0, atol=tol)
    return mx


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("layout", ["bhsd", "bshd"])
@pytest.mark.parametrize("variant", [3, 4])
@pytest.mark.parametrize("scale_on_q", [True, False])
def test_small_problems(gpu, dtype, layout, variant, scale_on_q):
    q, k, v, md = _inputs(2, 4, 2, 320, DT[dtype], layout, seed=1)
    o, L = _run(q, k, v, md, gpu, variant, scale_on_q)
    _check(o, L, q, k, v, md)


@pytest.mark.parametrize("B,HQ,HK,S", [(1, 8, 8, 1024), (1, 4, 1, 2048), (3, 2, 2, 64), (1, 1, 1, 256),
                                       (2, 6, 3, 576), (1, 2, 1, 128), (1, 2, 2, 192)])
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_head_groupings_and_lengths(gpu, B, HQ, HK, S, dtype):
    q, k, v, md = _inputs(B, HQ, HK, S, DT[dtype], "bhsd", seed=S + HQ)
    o, L = _run(q, k, v, md, gpu)
    _check(o, L, q, k, v, md)


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("layout", ["bhsd", "bshd"])
@pytest.mark.parametrize("variant", [3, 4])
@pytest.mark.parametrize("scale_on_q", [True, False])
def test_head_dim_64(gpu, dtype, layout, variant, scale_on_q):
    # Head dim 64: half the MFMAs per tile, one DMA per operand per wave.
    q, k, v, md = _inputs(2, 4, 2, 320, DT[dtype], layout, seed=21, D=64)
    o, L = _run(q, k, v, md, gpu, variant, scale_on_q)
    _check(o, L, q, k, v, md)


@pytest.mark.parametrize("B,HQ,HK,S,qscale", [(1, 8, 1, 1024, 1.0), (2, 3, 3, 576, 1.0), (1, 2, 2, 512, 16.0),
                                              (1, 1, 1, 64, 1.0), (1, 2, 1, 128, 1.0), (1, 2, 2, 192, 4.0)])
def test_head_dim_64_groupings_lengths_and_ranges(gpu, B, HQ, HK, S, qscale):
    q, k, v, md = _inputs(B, HQ, HK, S, torch.bfloat16, "bhsd", seed=S + 7 * HQ, scale=qscale, D=64)
    for variant in (3, 4):
        o, L = _run(q, k, v, md, gpu, variant, scale_on_q=False)
        _check(o, L, q, k, v, md)


def test_head_dim_64_strided_views(gpu):
    # bshd views of one packed (B, S, 3, H, 64) buffer; the output a view with a
    # padded head stride whose padding must stay untouched.
    B, S, H = 2, 448, 3
    g = torch.Generator().manual_seed(22)
    qkv = torch.randn(B, S, 3, H, 64, generator=g).to(torch.float16)
    q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
    md = MetaData(sm_scale=64**-0.5)
    md.max_seqlens_q = md.max_seqlens_k = S
    md.layout = "bshd"
    big = torch.full((B, S, H, 72), float("nan"), dtype=torch.float16, device=gpu)
    o = big[..., :64]
    qkv_d = qkv.to(gpu)
    fmha_v4.run_gluon_attention(qkv_d[:, :, 0], qkv_d[:, :, 1], qkv_d[:, :, 2], o, md)
    torch.cuda.synchronize()
    _check(o.cpu(), None, q, k, v, md)
    assert torch.isnan(big[..., 64:].cpu().float()).all(), "wrote past the output view"


@pytest.mark.parametrize("variant", [3, 4])
def test_strided_packed_qkv_views(gpu, variant):
    # One (B, S, 3, H, D) buffer, q/k/v as bshd views of it, and an output view
    # with a padded head stride.
    B, S, H = 2, 384, 4
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(B, S, 3, H, 128, generator=g).to(torch.bfloat16)
    q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
    md = MetaData(sm_scale=128**-0.5)
    md.max_seqlens_q = md.max_seqlens_k = S
    md.layout = "bshd"
    big = torch.full((B, S, H, 136), float("nan"), dtype=torch.bfloat16, device=gpu)
    o = big[..., :128]
    qkv_d = qkv.to(gpu)
    RUN[variant](qkv_d[:, :, 0], qkv_d[:, :, 1], qkv_d[:, :, 2], o, md)
    torch.cuda.synchronize()
    _check(o.cpu(), None, q, k, v, md)
    assert torch.isnan(big[..., 128:].cpu().float()).all(), "wrote past the output view"


@pytest.mark.parametrize("variant", [3, 4])
@pytest.mark.parametrize("qscale", [0.0, 4.0, 16.0])
def test_score_ranges(gpu, variant, qscale):
    # qscale 0: every score equal (o = mean of V); 4 and 16: score ranges of
    # tens to hundreds of log2 units, so the running max moves and the lazy
    # variant rescales many times.
    q, k, v, md = _inputs(1, 2, 2, 512, torch.bfloat16, "bhsd", seed=7, scale=qscale)
    o, L = _run(q, k, v, md, gpu, variant, scale_on_q=False)
    _check(o, L, q, k, v, md)
    if qscale == 0.0:
        mean = v.float().mean(dim=2, keepdim=True).expand_as(o)
        assert (o.float() - mean).abs().max() <= 2 * 2**-7 * mean.abs().max() + 1e-3
        np.testing.assert_allclose(L.numpy(), math.log(512), rtol=1e-6)


def test_rising_scores_force_rescales(gpu):
    # Keys grow along the sequence, so every tile raises the row max.
    q, k, v, md = _inputs(1, 2, 1, 1024, torch.float16, "bhsd", seed=8)
    k = (k.float() * torch.linspace(0.1, 6.0, 1024)[None, None, :, None]).half()
    for variant in (3, 4):
        o, L = _run(q, k, v, md, gpu, variant, scale_on_q=False)
        _check(o, L, q, k, v, md)


def test_variants_and_lse_option_agree(gpu):
    q, k, v, md = _inputs(1, 4, 4, 512, torch.bfloat16, "bhsd", seed=9)
    o3, _ = _run(q, k, v, md, gpu, 3, lse=False)
    o4, L4 = _run(q, k, v, md, gpu, 4)
    o4b, _ = _run(q, k, v, md, gpu, 4, lse=False)
    assert torch.equal(o4, o4b), "the lse output changed o"
    assert (o3.float() - o4.float()).abs().max() <= 2 * 2**-7 * o4.float().abs().max()
    o4c, L4c = _run(q, k, v, md, gpu, 4)
    assert torch.equal(o4, o4c) and torch.equal(L4, L4c), "not deterministic"


def test_input_helper_case_of_the_reference_bench(gpu):
    # The reference bench's correctness step: input_helper's seeded inputs,
    # sm_scale = D^-0.5, both layouts (kernels/attention/bench.py:157-184).
    for layout in ("bhsd", "bshd"):
        q, k, v, md = input_helper(1, 4, 4, 1024, 1024, 128, torch.bfloat16, layout, device="cpu")
        o, L = _run(q, k, v, md, gpu)
        _check(o, L, q, k, v, md)


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_benchmark_shape_on_sampled_rows(gpu, dtype):
    # B=32, H=8, S=8192, D=128 (the reference's tuned shape): the whole output
    # is computed on the GPU, 96 of its rows are checked against the oracle,
    # and every row must be finite.
    B, H, S = 32, 8, 8192
    torch.manual_seed(11)
    q, k, v = (torch.randn(B, H, S, 128, device=gpu, dtype=DT[dtype]) for _ in range(3))
    md = MetaData(sm_scale=128**-0.5)
    md.max_seqlens_q = md.max_seqlens_k = S
    md.layout = "bhsd"
    o = torch.empty_like(q)
    L = torch.empty(B, H, S, device=gpu)
    fmha_v4.run_gluon_attention(q, k, v, o, md, lse=L)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all() and torch.isfinite(L).all()
    rng = np.random.default_rng(12)
    rows = [(int(rng.integers(B)), int(rng.integers(H)), int(rng.integers(S))) for _ in range(90)]
    rows += [(0, 0, 0), (B - 1, H - 1, S - 1), (5, 3, 255), (5, 3, 256), (7, 1, 4095), (31, 0, 8191)]
    heads = sorted({(b, h) for b, h, _ in rows})
    cpu = {(b, h): [t[b, h].float().cpu().numpy() for t in (q, k, v)] for b, h in heads}
    got_o = o.float().cpu().numpy()
    got_l = L.cpu().numpy()
    for b, h, s in rows:
        qq, kk, vv = cpu[(b, h)]
        ref, ref_l = A.sdpa_rows(qq[None, None], kk[None, None], vv[None, None], [(0, 0, s)], md.sm_scale)
        ok, mx, _ = A.within_tolerance(got_o[b, h, s][None], ref, DT_NAME[DT[dtype]])
        assert ok, f"row {(b, h, s)}: max |diff| {mx:.3g}"
        bound = np.abs(qq[s]).sum() * np.abs(kk).max() * md.sm_scale
        assert abs(got_l[b, h, s] - ref_l[0]) <= 2 * A.FINFO_EPS[DT_NAME[DT[dtype]]] * bound + 1e-4


@pytest.mark.parametrize("D,variant", [(128, 4), (64, 3)])
def test_longest_sweep_shape_on_sampled_rows(gpu, D, variant):
    # The longest point of the reference bench's sweep (B=1, HQ=HK=64,
    # S=16384, kernels/attention/bench.py:100,107-113): 256 key tiles at head
    # dim 128, 128 at 64; 40 sampled rows against the oracle.
    B, H, S = 1, 64, 16384
    torch.manual_seed(17 + D)
    q, k, v = (torch.randn(B, H, S, D, device=gpu, dtype=torch.bfloat16) for _ in range(3))
    md = MetaData(sm_scale=D**-0.5)
    md.max_seqlens_q = md.max_seqlens_k = S
    md.layout = "bhsd"
    o = torch.empty_like(q)
    (fmha_v4 if variant == 4 else fmha_v3).run_gluon_attention(q, k, v, o, md)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all()
    rng = np.random.default_rng(18 + D)
    rows = [(0, int(rng.integers(H)), int(rng.integers(S))) for _ in range(36)]
    rows += [(0, 0, 0), (0, H - 1, S - 1), (0, 7, 8191), (0, 7, 8192)]
    heads = sorted({(b, h) for b, h, _ in rows})
    cpu = {(b, h): [t[b, h].float().cpu().numpy() for t in (q, k, v)] for b, h in heads}
    got = o.float().cpu().numpy()
    for b, h, s in rows:
        qq, kk, vv = cpu[(b, h)]
        ref, _ = A.sdpa_rows(qq[None, None], kk[None, None], vv[None, None], [(0, 0, s)], md.sm_scale)
        ok, mx, _ = A.within_tolerance(got[b, h, s][None], ref, "bfloat16")
        assert ok, f"row {(b, h, s)}: max |diff| {mx:.3g}"


@pytest.mark.parametrize("variant", [3, 4])
def test_nan_inputs_give_nan_rows(gpu, variant):
    # As the reference's fp32 SDPA: a NaN in a query row makes that row NaN; a
    # NaN in a key row makes every row of the heads reading that K head NaN.
    # Everything else is unaffected.
    q, k, v, md = _inputs(1, 4, 2, 256, torch.bfloat16, "bhsd", seed=13)
    q[0, 1, 5, 3] = float("nan")
    k[0, 1, 100, 7] = float("nan")  # K head 1 = query heads 2, 3
    o, _ = _run(q, k, v, md, gpu, variant, lse=False)
    o = o.float()
    assert torch.isnan(o[0, 1, 5]).all()
    assert torch.isnan(o[0, 2:]).all()
    keep = torch.ones(4, 256, dtype=torch.bool)
    keep[1, 5] = False
    keep[2:] = False
    got = o[0][keep]
    assert torch.isfinite(got).all()
    ref, _ = A.sdpa_reference(q.float().numpy(), k.float().numpy(), v.float().numpy(), md.sm_scale)
    ok, mx, _ = A.within_tolerance(got.numpy(), ref[0][keep.numpy()], "bfloat16")
    assert ok, mx
