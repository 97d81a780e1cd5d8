"""Pins of the attention oracle (oracle/attention_ref.py) and the host side of
the attention drop-in, on the CPU.

The reference's only check of its FMHA kernels is a comparison with torch's
scaled_dot_product_attention in fp32 under _check_output's tolerance
(kernels/attention/common.py:115-171); it holds no golden vectors.  The
oracle is pinned here by closed forms (uniform scores give the mean of V and
lse = ln S; one dominant key gives that key's value row), by torch's own
CPU scaled_dot_product_attention (with its enable_gqa head mapping), by a
known-answer GQA head map that a modulo mapping fails, and by the equality
of the streaming (tiled, lazily rescaled) form with the direct one on inputs
whose row max grows tile by tile.
"""

import math

import numpy as np
import pytest
import torch

from gfx950_gluon_tutorials_amd import _lib
from gfx950_gluon_tutorials_amd.attention import (
    MetaData,
    compute_flops,
    get_shape_from_layout,
    get_strides_from_layout,
    input_helper,
    run_gluon_attention,
)
from gfx950_gluon_tutorials_amd.attention import fmha_v3
from oracle import attention_ref as A


def _rand(shape, seed, scale=1.0):
    return np.random.default_rng(seed).standard_normal(shape) * scale


def test_uniform_scores_give_the_mean_of_v_and_log_s():
    B, H, S, D = 2, 3, 96, 128
    q = np.zeros((B, H, S, D))
    k = _rand((B, H, S, D), 1)
    v = _rand((B, H, S, D), 2)
    o, lse = A.sdpa_reference(q, k, v)
    np.testing.assert_allclose(o, np.broadcast_to(v.mean(axis=2, keepdims=True), o.shape), rtol=0, atol=1e-12)
    np.testing.assert_allclose(lse, np.full((B, H, S), math.log(S)), rtol=0, atol=1e-12)


def test_one_dominant_key_selects_its_value_row():
    S, D = 128, 128
    q = np.zeros((1, 1, S, D))
    k = np.zeros((1, 1, S, D))
    q[..., 0] = 40.0
    j0 = 77
    k[0, 0, j0, 0] = 40.0  # score 1600 / sqrt(128) = 141 nats above the rest
    v = _rand((1, 1, S, D), 3)
    o, lse = A.sdpa_reference(q, k, v)
    np.testing.assert_allclose(o[0, 0], np.broadcast_to(v[0, 0, j0], (S, D)), rtol=0, atol=1e-12)
    np.testing.assert_allclose(lse, 1600 / math.sqrt(D), rtol=1e-12)


@pytest.mark.parametrize("HQ,HK", [(4, 4), (4, 2), (8, 1)])
def test_matches_torch_sdpa_on_cpu(HQ, HK):
    B, S, D = 2, 80, 128
    q, k, v = _rand((B, HQ, S, D), 4), _rand((B, HK, S, D), 5), _rand((B, HK, S, D), 6)
    o, lse = A.sdpa_reference(q, k, v, sm_scale=0.1)
    t = [torch.from_numpy(x) for x in (q, k, v)]
    want = torch.nn.functional.scaled_dot_product_attention(*t, scale=0.1, enable_gqa=HQ != HK).numpy()
    np.testing.assert_allclose(o, want, rtol=1e-10, atol=1e-12)
    kk = torch.from_numpy(k).repeat_interleave(HQ // HK, dim=1)
    want_lse = torch.logsumexp(torch.from_numpy(q) @ kk.transpose(-1, -2) * 0.1, dim=-1).numpy()
    np.testing.assert_allclose(lse, want_lse, rtol=1e-12)


def test_gqa_head_map_is_contiguous_groups():
    # Query heads 0,1 read K/V head 0 and heads 2,3 read head 1; a modulo map
    # (h % HK) would give 1,2,1,2 instead of 1,1,2,2.
    B, S, D = 1, 64, 128
    q, k = _rand((B, 4, S, D), 7), _rand((B, 2, S, D), 8)
    v = np.stack([np.ones((S, D)), 2 * np.ones((S, D))])[None]
    o, _ = A.sdpa_reference(q, k, v)
    np.testing.assert_allclose(o[0, :, 0, 0], [1, 1, 2, 2], rtol=1e-12)
    assert [A.kv_head(h, 4, 2) for h in range(4)] == [0, 0, 1, 1]
    assert [A.kv_head(h, 8, 2) for h in range(8)] == [h * 2 // 8 for h in range(8)]


def test_bshd_is_the_transposed_bhsd_problem():
    B, H, S, D = 2, 2, 64, 128
    q, k, v = _rand((B, S, H, D), 9), _rand((B, S, H, D), 10), _rand((B, S, H, D), 11)
    o1, l1 = A.sdpa_reference(q, k, v, layout="bshd")
    tr = [x.transpose(0, 2, 1, 3) for x in (q, k, v)]
    o2, l2 = A.sdpa_reference(*tr, layout="bhsd")
    np.testing.assert_array_equal(o1, o2)
    np.testing.assert_array_equal(l1, l2)


@pytest.mark.parametrize("lazy", [True, False])
@pytest.mark.parametrize("growth", ["rising", "falling", "flat"])
def test_streaming_form_equals_direct_softmax(lazy, growth):
    B, HQ, HK, S, D = 1, 4, 2, 320, 128
    q, k, v = _rand((B, HQ, S, D), 12), _rand((B, HK, S, D), 13), _rand((B, HK, S, D), 14)
    ramp = {"rising": np.linspace(0.2, 4.0, S), "falling": np.linspace(4.0, 0.2, S), "flat": np.ones(S)}[growth]
    k = k * ramp[None, None, :, None]  # the row max moves tile by tile (or not at all)
    o1, l1 = A.flash_forward(q, k, v, lazy=lazy)
    o2, l2 = A.sdpa_reference(q, k, v)
    np.testing.assert_allclose(o1, o2, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(l1, l2, rtol=1e-12, atol=1e-12)


def test_sampled_rows_match_the_full_reference():
    B, HQ, HK, S, D = 2, 4, 2, 128, 128
    q, k, v = _rand((B, S, HQ, D), 15), _rand((B, S, HK, D), 16), _rand((B, S, HK, D), 17)
    o, lse = A.sdpa_reference(q, k, v, layout="bshd")
    rows = [(0, 0, 0), (1, 3, 127), (0, 2, 64), (1, 1, 5)]
    ro, rl = A.sdpa_rows(q, k, v, rows, layout="bshd")
    for i, (b, h, s) in enumerate(rows):
        np.testing.assert_allclose(ro[i], o[b, h, s], rtol=1e-12, atol=1e-14)
        np.testing.assert_allclose(rl[i], lse[b, h, s], rtol=1e-12)


def test_tolerance_is_two_ulps_of_the_output_format():
    assert A.FINFO_EPS["bfloat16"] == torch.finfo(torch.bfloat16).eps
    assert A.FINFO_EPS["float16"] == torch.finfo(torch.float16).eps
    assert A.check_tolerance("bfloat16", np.array([1.0, -0.5])) == (2 * 2.0**-7, 1e-3)
    assert A.check_tolerance("float16", np.array([0.1])) == (1e-3, 1e-3)  # floor wins
    ok, mx, _ = A.within_tolerance(np.array([1.0 + 2**-7]), np.array([1.0]), "bfloat16")
    assert ok and mx == 2**-7
    ok, _, _ = A.within_tolerance(np.array([1.05]), np.array([1.0]), "bfloat16")
    assert not ok
    ok, _, _ = A.within_tolerance(np.array([np.nan]), np.array([1.0]), "bfloat16")
    assert not ok


# --- host side of the drop-in -------------------------------------------------


def test_layout_helpers():
    q = torch.empty(2, 16, 4, 128)  # bshd
    k = torch.empty(2, 16, 2, 128)
    md = MetaData(0.5)
    md.layout = "bshd"
    assert get_shape_from_layout(q, k, md) == (2, 4, 2, 128)
    st = get_strides_from_layout(q, k, k, q, md)
    assert st[0] == (16 * 4 * 128, 128, 4 * 128, 1)
    assert st[1] == (16 * 2 * 128, 128, 2 * 128, 1)
    md.layout = "bhsd"
    assert get_shape_from_layout(q, k, md) == (2, 16, 16, 128)
    md.layout = "sbhd"
    with pytest.raises(ValueError):
        get_shape_from_layout(q, k, md)


def test_flops_model_and_input_helper():
    assert compute_flops(32, 8, 8192, 8192, 128, False) == 4 * 32 * 8 * 8192 * 8192 * 128
    assert compute_flops(1, 1, 4, 4, 1, True) == 4 * (4 * 4 - 6)
    q, k, v, md = input_helper(2, 4, 2, 64, 64, 128, torch.float16, "bshd", device="cpu")
    assert q.shape == (2, 64, 4, 128) and k.shape == (2, 64, 2, 128) and md.sm_scale == 128**-0.5
    q2, _, _, _ = input_helper(2, 4, 2, 64, 64, 128, torch.float16, "bshd", device="cpu")
    assert torch.equal(q, q2)


def _case(**kw):
    md = MetaData(128**-0.5)
    md.layout = kw.pop("layout", "bhsd")
    S = kw.pop("S", 128)
    md.max_seqlens_q = md.max_seqlens_k = S
    D = kw.pop("D", 128)
    dt = kw.pop("dtype", torch.float16)
    q = torch.zeros(1, 2, S, D, dtype=dt)
    return q, q.clone(), q.clone(), q.clone(), md


def test_drop_in_rejects_what_the_reference_asserts_and_more():
    q, k, v, o, md = _case()
    md.causal = True
    with pytest.raises(AssertionError):
        run_gluon_attention(q, k, v, o, md)
    q, k, v, o, md = _case(S=100)
    with pytest.raises(AssertionError):
        run_gluon_attention(q, k, v, o, md)
    q, k, v, o, md = _case(D=96)
    with pytest.raises(AssertionError):  # not a power of two
        fmha_v3.run_gluon_attention(q, k, v, o, md)
    q, k, v, o, md = _case(D=32)
    with pytest.raises(ValueError, match="head dim"):
        run_gluon_attention(q, k, v, o, md)
    q, k, v, o, md = _case(D=64)
    with pytest.raises(ValueError, match="GPU"):  # head dim 64 is accepted; CPU tensors are not
        run_gluon_attention(q, k, v, o, md)
    q, k, v, o, md = _case(dtype=torch.float32)
    with pytest.raises(ValueError):
        run_gluon_attention(q, k, v, o, md)
    q, k, v, o, md = _case()
    with pytest.raises(ValueError, match="GPU"):  # CPU tensors never reach the library
        run_gluon_attention(q, k, v, o, md)


# --- C ABI argument checks (every call is rejected before any launch) -----------

FAKE = 0x10000


def _call(**kw):
    a = dict(q=FAKE, k=FAKE, v=FAKE, o=FAKE, lse=None, B=1, HQ=2, HK=2, S=128, D=128,
             qs=(2 * 128 * 128, 128 * 128, 128, 1), ks=None, vs=None, os_=None, scale=0.088,
             dtype=_lib.G9_BF16, soq=1, variant=4)
    a.update(kw)
    for n in ("ks", "vs", "os_"):
        if a[n] is None:
            a[n] = a["qs"]
    arr = [(_lib.ctypes.c_int64 * 4)(*a[n]) for n in ("qs", "ks", "vs", "os_")]
    return _lib.load().g9_fmha_fwd(a["q"], a["k"], a["v"], a["o"], a["lse"], a["B"], a["HQ"], a["HK"], a["S"],
                                   a["D"], *arr, a["scale"], a["dtype"], a["soq"], a["variant"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(dtype=_lib.G9_BF8), _lib.G9_ERR_DTYPE),
    (dict(variant=5), _lib.G9_ERR_SCHEDULE),
    (dict(D=32), _lib.G9_ERR_SHAPE),
    (dict(D=256), _lib.G9_ERR_SHAPE),
    (dict(S=100), _lib.G9_ERR_SHAPE),
    (dict(S=0), _lib.G9_ERR_SHAPE),
    (dict(HQ=3, HK=2), _lib.G9_ERR_SHAPE),
    (dict(scale=0.0), _lib.G9_ERR_SHAPE),
    (dict(scale=float("nan")), _lib.G9_ERR_SHAPE),
    (dict(scale=-float("nan")), _lib.G9_ERR_SHAPE),
    (dict(scale=float("inf")), _lib.G9_ERR_SHAPE),
    (dict(scale=-0.088), _lib.G9_ERR_SHAPE),
    (dict(scale=-0.0), _lib.G9_ERR_SHAPE),
    (dict(q=0), _lib.G9_ERR_LAYOUT),
    (dict(v=FAKE + 2), _lib.G9_ERR_LAYOUT),
    (dict(qs=(2 * 128 * 128, 128 * 128, 128, 2)), _lib.G9_ERR_LAYOUT),
    (dict(ks=(2 * 128 * 128, 128 * 128, 100, 1)), _lib.G9_ERR_LAYOUT),
    (dict(os_=(2 * 128 * 128, 128 * 128, 132, 1)), _lib.G9_ERR_LAYOUT),  # rows not 16-byte aligned
    (dict(vs=(2 * 128 * 128 + 4, 128 * 128, 128, 1)), _lib.G9_ERR_LAYOUT),
    (dict(lse=FAKE + 2), _lib.G9_ERR_LAYOUT),
    (dict(S=1 << 23, qs=(1 << 31, 1 << 30, 128, 1)), _lib.G9_ERR_SHAPE),  # row offsets past 2^31 bytes
])
def test_capi_rejects_bad_arguments(kw, code):
    assert _call(**kw) == code
