"""Pins the CPU oracle (oracle/gemm_ref.py) before anything is checked
against it.  Each oracle function is checked against something that does not
restate it: closed forms, torch's own float8/bfloat16 casts, brute force on
tiny inputs, exact-arithmetic golden fixtures, and invariants."""

import os

import numpy as np
import pytest
import torch

from oracle import gemm_ref as R

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_e2m1_table_matches_bit_fields():
    # e2m1: sign | 2-bit exponent (bias 1) | 1-bit mantissa; exponent 0 is subnormal.
    for code in range(16):
        s, e, m = code >> 3, (code >> 1) & 3, code & 1
        mag = (1 + m / 2) * 2.0 ** (e - 1) if e else m * 0.5
        expect = -mag if s else mag
        assert R.E2M1_VALUES[code] == expect
        assert np.signbit(R.E2M1_VALUES[code]) == bool(s)


def test_fp4_nibble_order_low_is_even_k():
    # byte 0x21: low nibble 1 (0.5) is k=0, high nibble 2 (1.0) is k=1.
    packed = np.array([[0x21, 0xF8]], dtype=np.uint8)
    np.testing.assert_array_equal(R.mxfp4_to_f32(packed), [[0.5, 1.0, -0.0, -6.0]])
    codes = np.arange(16, dtype=np.uint8).reshape(1, 16)
    np.testing.assert_array_equal(R.unpack_fp4(R.pack_fp4(codes)), codes)


def test_e8m0_special_values():
    v = R.e8m0_to_f32(np.array([0, 1, 126, 127, 128, 254, 255], dtype=np.uint8))
    assert v[0] == 2.0**-127 and v[1] == 2.0**-126
    assert v[2] == 0.5 and v[3] == 1.0 and v[4] == 2.0 and v[5] == 2.0**127
    assert np.isnan(v[6])


def test_e5m2_decode_matches_torch_for_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e5m2).float().numpy()
    np.testing.assert_array_equal(R.e5m2_to_f32(codes), ref)


def test_e5m2_encode_matches_torch_cast():
    rng = np.random.default_rng(0)
    x = np.concatenate(
        [rng.standard_normal(50000).astype(np.float32) * s for s in (1e-6, 1e-3, 1.0, 1e3, 3e4)]
        + [np.array([0, -0.0, 57344, 61439.99, 61440, 65536, np.inf, -np.inf, np.nan,
                     2**-14, 2**-16, 2**-17, 3 * 2**-18, 1.125, 1.375, -1.625], dtype=np.float32)]
    )
    ref = torch.from_numpy(x).to(torch.float8_e5m2).view(torch.uint8).numpy()
    np.testing.assert_array_equal(R.f32_to_e5m2(x), ref)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10.0**e for e in range(-3, 4)])
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(R.round_to_bf16(x), ref)


def test_e2m1_rounding_brute_force():
    # For every magnitude on a fine grid the chosen code is a nearest one,
    # ties go to the even code, and anything past 6 saturates.
    vals = R.E2M1_VALUES[:8].astype(np.float64)
    m = np.concatenate([np.linspace(0, 7, 28001), np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])])
    codes = R._e2m1_round(m)
    d = np.abs(vals[None, :] - m[:, None])
    best = d.min(axis=1)
    assert np.all(np.abs(vals[codes] - m) == best)
    tie = (d == best[:, None]).sum(axis=1) > 1
    assert np.all(codes[tie] % 2 == 0)
    assert np.all(codes[m > 6] == 7)


def test_mxfp4_quantizer_invariants():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((64, 512)).astype(np.float32)
    x[0, :32] = 0.0
    packed, scales = R.quant_mxfp4(x)
    assert scales[0, 0] == 0 and np.all(R.unpack_fp4(packed)[0, :32] % 8 == 0)
    g = np.abs(x.reshape(64, 16, 32)).max(-1)
    nz = g > 0
    E = scales.astype(np.int64) - 127
    # group absmax / 2^E lands in [4, 8): the top of the e2m1 range.
    r = g[nz] / np.ldexp(1.0, E[nz])
    assert np.all((r >= 4) & (r < 8))
    # Dequantized values are within half an e2m1 step (or saturated at 6 * 2^E).
    deq = R.mxfp4_dequant(packed, scales)
    step = np.repeat(np.ldexp(1.0, E), 32, axis=1)
    err = np.abs(deq - x)
    ok = (err <= 1.0 * step + 1e-30) | (np.abs(deq) == 6 * step)
    assert ok[nz.repeat(32, axis=1)].all()


def test_e5m2_quantizer_maps_absmax_to_max():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((32, 256)).astype(np.float32)
    codes, scale = R.quant_e5m2_per_tensor(x)
    deq = R.e5m2_to_f32(codes)
    assert np.max(np.abs(deq)) == R.E5M2_MAX
    assert np.all(np.isfinite(deq))
    assert np.max(np.abs(deq * scale - x)) <= np.max(np.abs(x)) * 2.0**-2


def _brute_gemm(a, b_nk):
    M, K = a.shape
    N = b_nk.shape[0]
    c = np.zeros((M, N), dtype=np.float64)
    for i in range(M):
        for j in range(N):
            s = 0.0
            for k in range(K):
                s += float(a[i, k]) * float(b_nk[j, k])
            c[i, j] = s
    return c


def test_gemm_refs_against_brute_force():
    # Non-square M != N != K so a transposed operand cannot pass.
    rng = np.random.default_rng(4)
    a = rng.integers(-3, 4, size=(5, 7)).astype(np.float16)
    b = rng.integers(-3, 4, size=(3, 7)).astype(np.float16)
    np.testing.assert_array_equal(R.a16w16_ref(a, b), _brute_gemm(a, b))
    ca = rng.integers(0, 16, size=(4, 64)).astype(np.uint8)
    cb = rng.integers(0, 16, size=(3, 64)).astype(np.uint8)
    sa = rng.integers(120, 130, size=(4, 2)).astype(np.uint8)
    sb = rng.integers(120, 130, size=(3, 2)).astype(np.uint8)
    pa, pb = R.pack_fp4(ca), R.pack_fp4(cb)
    va = np.array([[R.E2M1_VALUES[c] * 2.0 ** (int(sa[i, k // 32]) - 127) for k, c in enumerate(row)]
                   for i, row in enumerate(ca)])
    vb = np.array([[R.E2M1_VALUES[c] * 2.0 ** (int(sb[i, k // 32]) - 127) for k, c in enumerate(row)]
                   for i, row in enumerate(cb)])
    np.testing.assert_array_equal(R.a4w4_ref_f32(pa, pb, sa, sb), _brute_gemm(va, vb))
    e8 = np.array([[0x3C, 0xC0, 0x40, 0x00]], dtype=np.uint8)  # 1, -2, 2, 0
    f8 = np.array([[0x40, 0x3C, 0x44, 0x7B], [0x3C, 0x3C, 0x3C, 0x3C]], dtype=np.uint8)  # 2,1,4,57344 / 1s
    np.testing.assert_array_equal(R.a8w8_ref_f32(e8, f8, 0.5, 2.0), [[2 - 2 + 8 + 0, 1 - 2 + 2 + 0]])


def _bits_to_f32(bits, kind):
    bits = np.asarray(bits, dtype=np.uint16)
    if kind == "f16":
        return bits.view(np.float16).astype(np.float32)
    return (bits.astype(np.uint32) << 16).view(np.float32)


def test_oracle_reproduces_exact_golden_fixtures():
    g = np.load(os.path.join(GOLDEN, "a16w16_exact.npz"))
    np.testing.assert_array_equal(R.a16w16_ref(g["a"], g["b_nk"], "f16"), _bits_to_f32(g["c_f16_bits"], "f16"))
    np.testing.assert_array_equal(R.a16w16_ref(g["a"], g["b_nk"], "bf16"), _bits_to_f32(g["c_bf16_bits"], "bf16"))
    g = np.load(os.path.join(GOLDEN, "a8w8_exact.npz"))
    np.testing.assert_array_equal(R.a8w8_ref(g["a_codes"], g["b_codes"], out_dtype="f16"),
                                  _bits_to_f32(g["c_f16_bits"], "f16"))
    np.testing.assert_array_equal(
        R.a8w8_ref(g["a_codes"], g["b_codes"], g["a_scale"], g["b_scale"], out_dtype="bf16"),
        _bits_to_f32(g["c_bf16_scaled_bits"], "bf16"))
    g = np.load(os.path.join(GOLDEN, "a4w4_exact.npz"))
    np.testing.assert_array_equal(R.a4w4_ref(g["a"], g["b"], g["a_scales"], g["b_scales"]),
                                  _bits_to_f32(g["c_bf16_bits"], "bf16"))


@pytest.mark.parametrize("grid_m,grid_n", [(16, 16), (15, 15), (32, 5), (1, 1), (3, 7), (9, 1), (1, 13), (40, 40)])
@pytest.mark.parametrize("xcds,gm", [(8, 4), (8, 1), (1, 4), (8, 8)])
def test_get_pids_is_a_bijection_with_xcd_locality(grid_m, grid_n, xcds, gm):
    grid = grid_m * grid_n
    M, N = grid_m * 256, grid_n * 256
    seen = set()
    per_xcd = {}
    for pid in range(grid):
        pm, pn = R.get_pids(pid, M, N, 256, 256, grid, xcds, gm)
        assert 0 <= pm < grid_m and 0 <= pn < grid_n
        seen.add((pm, pn))
        per_xcd.setdefault(pid % xcds, []).append((pm, pn))
    assert len(seen) == grid
    if xcds == 8 and gm == 4 and (grid_m, grid_n) == (16, 16):
        # Each XCD owns one 4 x 8 block of tiles (kernels/gemm/intra_wave/a16w16/v9_beyond_hotloop/README.md:92-96).
        for tiles in per_xcd.values():
            ms = {t[0] for t in tiles}
            ns = {t[1] for t in tiles}
            assert len(ms) == 4 and len(ns) == 8 and len(tiles) == 32


@pytest.mark.parametrize("tiles,stages,ctas", [(225, 256, 256), (160, 128, 256), (272, 128, 256), (400, 128, 256),
                                               (4, 7, 3), (3, 5, 16), (10, 2, 7)])
def test_streamk_partition_covers_every_stage_once(tiles, stages, ctas):
    segs = R.streamk_segments(tiles, stages, ctas)
    count = np.zeros((tiles, stages), dtype=np.int64)
    for c in segs:
        for t, sb, se in c:
            assert 0 <= sb < se <= stages
            count[t, sb:se] += 1
    assert np.all(count == 1)
    steps, flags = R.simulate_streamk(tiles, stages, ctas)
    total = tiles * stages
    assert steps >= -(-total // ctas)


@pytest.mark.parametrize("tiles,stages,ctas", [(225, 256, 256), (160, 128, 256), (272, 128, 256), (320, 128, 256),
                                               (400, 128, 256), (512, 128, 256)])
def test_streamk_makespan_is_one_chain_or_the_even_share(tiles, stages, ctas):
    # With K-ordered chains a tile's stages run one after another, so the makespan is at least one tile's
    # chain; with at least a tile per workgroup no workgroup waits and the even share is reached.
    steps, _ = R.simulate_streamk(tiles, stages, ctas)
    assert steps == max(stages, -(-tiles * stages // ctas))


def test_streamk_segments_run_last_tile_first():
    # A CTA owing a prefix to its successor produces it first.
    for c in R.streamk_segments(10, 7, 4):
        tiles = [t for t, _, _ in c]
        assert tiles == sorted(tiles, reverse=True)
        assert all(sb == 0 for t, sb, se in c[:-1])  # only the last segment may inherit a partial


def test_streamk_simulation_catches_a_planted_double_cover(monkeypatch):
    # Plant a mistake in the oracle's partition (two CTAs claim one stage) and
    # check the simulator rejects it.
    good = R.streamk_segments

    def bad(tiles, stages, ctas):
        segs = good(tiles, stages, ctas)
        t, sb, se = segs[1][-1]
        segs[0].append((t, sb, sb + 1))
        return segs

    monkeypatch.setattr(R, "streamk_segments", bad)
    with pytest.raises(AssertionError):
        R.simulate_streamk(10, 7, 4)


@pytest.mark.parametrize("grid_m,grid_n", [(16, 16), (15, 15), (32, 5), (3, 7), (40, 40), (1, 1)])
def test_product_host_get_pids_matches_oracle(grid_m, grid_n):
    from gfx950_gluon_tutorials_amd.gemm.utils.common import get_pids

    grid = grid_m * grid_n
    for pid in range(grid):
        args = (pid, grid_m * 256, grid_n * 256, 256, 256, grid, 8, 4)
        assert get_pids(*args) == R.get_pids(*args)


def test_moe_ref_routes_rows_to_their_expert():
    # A rows of ones; expert e's weights are the constant v_e, so row t of expert e is K * v_e exactly.
    K = 64
    a = np.ones((7, K), np.float16)
    vals = (1.0, 2.0, 0.5, 4.0)
    b = np.stack([np.full((3, K), v, np.float16) for v in vals])
    offsets = [1, 3, 3, 6, 6]  # row 0 and row 6 belong to no expert; experts 1 and 3 are empty
    c = R.moe_ref(R.a16w16_ref, a, b, offsets)
    assert np.all(np.isnan(c[0])) and np.all(np.isnan(c[6]))
    np.testing.assert_array_equal(c[1:3], np.full((2, 3), K * 1.0))
    np.testing.assert_array_equal(c[3:6], np.full((3, 3), K * 0.5))


def test_moe_ref_passes_row_and_expert_operands():
    # MXFP4: A codes 2 (value 1.0) with scale 127 (1.0); expert e's B codes 2 with scale 127 + e, so
    # row t of expert e is K * 2^e.
    K, T, N = 64, 4, 2
    a = R.pack_fp4(np.full((T, K), 2, np.uint8))
    a_sc = np.full((T, K // 32), 127, np.uint8)
    b = np.stack([R.pack_fp4(np.full((N, K), 2, np.uint8)) for _ in range(3)])
    b_sc = np.stack([np.full((N, K // 32), 127 + e, np.uint8) for e in range(3)])
    c = R.moe_ref(R.a4w4_ref_f32, a, b, [0, 1, 1, 4], a_sc, expert_args=(b_sc,))
    np.testing.assert_array_equal(c[0], [K, K])
    np.testing.assert_array_equal(c[1:], np.full((3, N), K * 4.0))


def test_torch_matmul_f32_against_brute_force():
    """The CPU baseline's restatement of the reference's torch.matmul path:
    exact on small integers (every partial sum is exact in fp32) and within
    fp32 rounding of a float64 triple loop on random values."""
    rng = np.random.default_rng(5)
    a = rng.integers(-8, 9, (7, 33)).astype(np.float32)
    b = rng.integers(-8, 9, (5, 33)).astype(np.float32)
    want = [[sum(int(a[i, k]) * int(b[j, k]) for k in range(33)) for j in range(5)] for i in range(7)]
    np.testing.assert_array_equal(R.torch_matmul_f32(a, b).numpy(), np.array(want, dtype=np.float32))
    x = rng.standard_normal((6, 40)).astype(np.float32)
    y = rng.standard_normal((3, 40)).astype(np.float32)
    ref = np.array([[sum(float(x[i, k]) * float(y[j, k]) for k in range(40)) for j in range(3)] for i in range(6)])
    np.testing.assert_allclose(R.torch_matmul_f32(x, y).numpy(), ref, rtol=1e-5, atol=1e-5)


# --- stream-K progress when not every workgroup is resident ------------------
#
# gemm_sk assumes no co-residency.  Workgroup b is dispatched to XCD b % 8
# and each XCD starts its workgroups in increasing b; the XCD remap gives XCD x
# the contiguous ranges 32x .. 32x + 31 in that order.  A range waits only on
# its predecessor, which is either earlier on the same XCD (started before it,
# so resident or finished) or, for XCD x's first range, the last range of XCD
# x - 1.  By induction over the XCDs every range finishes as long as each XCD
# eventually has one free CU; the simulation checks it for the BASELINE
# stream-K shapes and others under many residency limits.

@pytest.mark.parametrize("tiles,stages", [(225, 256), (160, 128), (16, 256), (32, 128), (272, 128), (400, 128),
                                          (450, 256), (320, 128)])
def test_streamk_progress_under_partial_residency(tiles, stages):
    rng = np.random.default_rng(tiles * 1000 + stages)
    limits = [[1] * 8, [2] * 8, [32] * 8, [1, 32] * 4, [32, 1] * 4] + [list(rng.integers(1, 33, 8)) for _ in range(4)]
    for res in limits:
        steps = R.simulate_streamk_dispatch(tiles, stages, 256, res)
        assert steps >= max(stages, -(-tiles * stages // 256))


def test_streamk_cta_of_block_is_the_device_remap():
    # XCD x's blocks (x, x + 8, ...) own the contiguous ranges 32x .. 32x + 31,
    # in dispatch order; uneven grids give the first XCDs one more.
    assert [R.streamk_cta_of_block(b, 256) for b in range(0, 256, 8)] == list(range(32))
    assert [R.streamk_cta_of_block(b, 256) for b in range(3, 256, 8)] == list(range(96, 128))
    got = sorted(R.streamk_cta_of_block(b, 250) for b in range(250))
    assert got == list(range(250))
    assert [R.streamk_cta_of_block(b, 250) for b in range(1, 250, 8)] == list(range(32, 64))


def test_streamk_dispatch_simulation_detects_a_deadlock():
    # Planted mistake: ranges handed out in reverse dispatch order, so a
    # resident workgroup waits on a predecessor queued behind it on its XCD.
    with pytest.raises(AssertionError, match="deadlocked"):
        R.simulate_streamk_dispatch(16, 256, 256, [1] * 8, cta_of_block=lambda b: 255 - b)
