"""CPU oracle for the gfx950 flash-attention forward -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this module, and only as the checker (or the timed CPU baseline).
The product (``gfx950_gluon_tutorials_amd``) never imports it.

It restates, in numpy float64, the reference's correctness path for its FMHA
kernels:

* ``sdpa_reference`` -- softmax(q k^T * sm_scale) v with grouped K/V heads
  expanded by ``repeat_interleave`` (query head h reads K/V head
  h // (HQ / HK)), non-causal, on a ``bhsd`` frame
  (kernels/attention/common.py:115-139), plus the per-query log-sum-exp the
  kernels store in their L buffer (kernels/attention/fmha_v4.py:755-758);
* ``flash_forward`` -- the streaming form the kernels compute: 64-key tiles,
  running max m and sum l in log2 units, eager (fmha_v3.py:96-152) or lazy
  (fmha_v4.py:143-210, 247-270, threshold 8) rescale of the accumulator;
* ``check_tolerance`` -- the acceptance test of _check_output
  (kernels/attention/common.py:142-171): assert_close with rtol 1e-3 and
  atol = max(1e-3, 2 ulp(out dtype) * max|o_ref|).

How each function is pinned (closed forms, torch's own scaled_dot_product_attention
on the CPU, brute-force equality of the streaming and direct forms) is listed
in tests/test_attention_oracle.py.
"""

from __future__ import annotations

import math

import numpy as np

LOG2E = 1.4426950408889634
LAZY_THRESHOLD = 8.0  # kernels/attention/fmha_v4.py:143-175 (LAZY_RESCALE_THRESHOLD)


def to_bhsd(x: np.ndarray, layout: str) -> np.ndarray:
    """(batch, head, seq, dim) view of an array in ``layout``."""
    if layout == "bhsd":
        return x
    if layout == "bshd":
        return x.transpose(0, 2, 1, 3)
    raise ValueError(layout)


def kv_head(hq: int, HQ: int, HK: int) -> int:
    """K/V head read by query head hq: repeat_interleave by HQ // HK
    (kernels/attention/common.py:127-130); equal to hq * HK // HQ
    (kernels/attention/fmha_v4.py:359)."""
    return hq // (HQ // HK)


def sdpa_reference(q, k, v, sm_scale=None, layout="bhsd"):
    """(o, lse) in float64 for q (B, HQ, S, D) and k, v (B, HK, S, D) in
    ``layout``; o in bhsd order, lse (B, HQ, S) natural log.
    Restates kernels/attention/common.py:115-139 (non-causal branch)."""
    q, k, v = (to_bhsd(np.asarray(t, dtype=np.float64), layout) for t in (q, k, v))
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[-1])
    HQ, HK = q.shape[1], k.shape[1]
    if HQ != HK:
        r = HQ // HK
        k = np.repeat(k, r, axis=1)
        v = np.repeat(v, r, axis=1)
    s = np.einsum("bhqd,bhkd->bhqk", q, k) * sm_scale
    mx = s.max(axis=-1, keepdims=True)
    e = np.exp(s - mx)
    den = e.sum(axis=-1, keepdims=True)
    o = np.einsum("bhqk,bhkd->bhqd", e / den, v)
    lse = (mx + np.log(den))[..., 0]
    return o, lse


def sdpa_rows(q, k, v, rows, sm_scale=None, layout="bhsd"):
    """(o, lse) of selected query rows only: ``rows`` is a list of
    (batch, query head, position).  Same arithmetic as sdpa_reference, so a
    full-size problem can be checked on a sample of its rows."""
    qb, kb, vb = (to_bhsd(t, layout) for t in (q, k, v))
    HQ, HK = qb.shape[1], kb.shape[1]
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(qb.shape[-1])
    outs, lses = [], []
    for b, h, i in rows:
        hk = kv_head(h, HQ, HK)
        qi = np.asarray(qb[b, h, i], dtype=np.float64)
        kk = np.asarray(kb[b, hk], dtype=np.float64)
        vv = np.asarray(vb[b, hk], dtype=np.float64)
        s = kk @ qi * sm_scale
        mx = s.max()
        e = np.exp(s - mx)
        den = e.sum()
        outs.append(e @ vv / den)
        lses.append(mx + math.log(den))
    return np.array(outs), np.array(lses)


def flash_forward(q, k, v, sm_scale=None, layout="bhsd", block_n=64, lazy=True):
    """(o, lse) by the streaming algorithm of the kernels, in float64: for each
    64-key tile, the tile max t (log2 units), the new running max (lazy: kept
    unless t exceeds it by more than 8; eager: max(m, t)), p = 2^(x - m_new),
    l = l * 2^(m - m_new) + sum p, acc = acc * 2^(m - m_new) + p v; o = acc / l.
    Follows kernels/attention/fmha_v4.py:143-210, 247-310 (lazy) and
    kernels/attention/fmha_v3.py:96-152 (eager)."""
    q, k, v = (to_bhsd(np.asarray(t, dtype=np.float64), layout) for t in (q, k, v))
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[-1])
    B, HQ, S, D = q.shape
    HK, N = k.shape[1], k.shape[2]
    c = sm_scale * LOG2E
    o = np.zeros((B, HQ, S, v.shape[-1]))
    lse = np.zeros((B, HQ, S))
    for b in range(B):
        for h in range(HQ):
            hk = kv_head(h, HQ, HK)
            x_all = q[b, h] @ k[b, hk].T * c  # scores in log2 units
            m = np.full(S, -np.inf)
            l = np.zeros(S)
            acc = np.zeros((S, v.shape[-1]))
            for j0 in range(0, N, block_n):
                x = x_all[:, j0:j0 + block_n]
                t = x.max(axis=1)
                if lazy:
                    m_new = np.where(t - m > LAZY_THRESHOLD, t, m)
                else:
                    m_new = np.maximum(m, t)
                alpha = np.exp2(m - m_new)
                p = np.exp2(x - m_new[:, None])
                l = l * alpha + p.sum(axis=1)
                acc = acc * alpha[:, None] + p @ v[b, hk, j0:j0 + block_n]
                m = m_new
            o[b, h] = acc / l[:, None]
            lse[b, h] = (m + np.log2(l)) / LOG2E
    return o, lse


FINFO_EPS = {"float16": 2.0**-10, "bfloat16": 2.0**-7}


def check_tolerance(out_dtype: str, o_ref: np.ndarray, atol: float = 1e-3, rtol: float = 1e-3):
    """(atol, rtol) of the reference's acceptance test for an output of
    ``out_dtype`` ("float16" / "bfloat16") against the fp32-or-better
    reference o_ref: atol = max(atol, 2 * eps(out_dtype) * max|o_ref|)
    (kernels/attention/common.py:142-171)."""
    scale = float(np.abs(o_ref).max())
    if scale > 0 and math.isfinite(scale):
        atol = max(atol, 2 * FINFO_EPS[out_dtype] * scale)
    return atol, rtol


def within_tolerance(o: np.ndarray, o_ref: np.ndarray, out_dtype: str):
    """(ok, max |diff|, mean |diff|) under check_tolerance, elementwise
    |o - o_ref| <= atol + rtol * |o_ref| (torch.testing.assert_close's rule)."""
    atol, rtol = check_tolerance(out_dtype, o_ref)
    o = np.asarray(o, dtype=np.float64)
    diff = np.abs(o - o_ref)
    ok = bool(np.all(diff <= atol + rtol * np.abs(o_ref))) and not np.isnan(o).any()
    return ok, float(diff.max()), float(diff.mean())
