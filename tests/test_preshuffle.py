"""The preshuffled MXFP4 scale layout (quant.preshuffle_e8m0 and its oracle
restatement), checked on the CPU.

The layout is defined by what the preshuffled-scale kernel reads: lane group g
of MFMA step h in stage s of a 4-stage chunk holds K values
[1024c + 256s + 128h + 32g, +32) (16x16x128 fragments, four lane groups of 32
K values per step, two steps per 256-value stage), and reads byte
8j + 2s + h of its row's 32-byte chunk row, j = g ^ ((row >> 2) & 3).  The
checks below derive the expected byte from those K positions, from a
hand-written table, and from a round trip, so a transposed index, a swapped
(s, h) or a missing row XOR fails at least one.
"""

import numpy as np
import pytest
import torch

from gfx950_gluon_tutorials_amd import quant
from oracle import gemm_ref as R


def test_known_answer_rows_of_chunk_zero():
    G = 64  # two chunks
    s = np.tile(np.arange(G, dtype=np.uint8), (13, 1))
    ps = R.preshuffle_e8m0(s)
    assert ps.shape == (2, 13, 32)
    units = [[0, 4, 8, 12, 16, 20, 24, 28], [1, 5, 9, 13, 17, 21, 25, 29],
             [2, 6, 10, 14, 18, 22, 26, 30], [3, 7, 11, 15, 19, 23, 27, 31]]  # lane group g's 8 bytes
    # The lane groups whose units a row stores in unit slots 0..3: rows 0-3 in
    # order, rows 4-7 swap 0<->1 and 2<->3, rows 8-11 swap 0<->2 and 1<->3,
    # rows 12-15 reverse them.
    order = [[0, 1, 2, 3], [1, 0, 3, 2], [2, 3, 0, 1], [3, 2, 1, 0]]
    for r in range(13):
        want = sum((units[g] for g in order[(r // 4) % 4]), [])
        assert ps[0, r].tolist() == want, r
        assert ps[1, r].tolist() == [w + 32 for w in want], r


@pytest.mark.parametrize("R_,G", [(5, 32), (17, 96), (3, 256)])
def test_each_lane_reads_the_scale_of_its_k_values(R_, G):
    rng = np.random.default_rng(R_ * 31 + G)
    s = rng.integers(0, 256, (R_, G), dtype=np.uint8)
    ps = R.preshuffle_e8m0(s)
    for r in range(R_):
        for c in range(ps.shape[0]):
            for g in range(4):
                j = g ^ ((r >> 2) & 3)  # the unit lane group g of this row reads
                for st in range(4):
                    for h in range(2):
                        k0 = 1024 * c + 256 * st + 128 * h + 32 * g  # first K value of the lane group's data
                        assert ps[c, r, 8 * j + 2 * st + h] == s[r, k0 // 32]


def test_groups_past_the_end_are_filled_with_one():
    s = np.full((8, 40), 200, dtype=np.uint8)  # 40 groups: the second chunk holds 8
    ps = R.preshuffle_e8m0(s)
    assert ps.shape == (2, 8, 32)
    for r in range(8):
        for p in range(32):
            grp = 8 * (p % 8 // 2) + 4 * (p % 2) + ((p // 8) ^ ((r >> 2) & 3))
            assert ps[1, r, p] == (200 if grp < 8 else 127), (r, p)


@pytest.mark.parametrize("R_,G", [(1, 32), (300, 64), (257, 40), (64, 1024)])
def test_product_preshuffle_matches_oracle_and_round_trips(R_, G):
    g = torch.Generator().manual_seed(R_ + G)
    s = torch.randint(0, 256, (R_, G), generator=g, dtype=torch.uint8)
    ps = quant.preshuffle_e8m0(s)
    assert ps.is_contiguous() and ps.dtype == torch.uint8
    np.testing.assert_array_equal(ps.numpy(), R.preshuffle_e8m0(s.numpy()))
    assert torch.equal(quant.unshuffle_e8m0(ps, G), s)


def test_preshuffle_rejects_non_2d_or_non_uint8():
    with pytest.raises(ValueError):
        quant.preshuffle_e8m0(torch.zeros(4, 32, dtype=torch.int32))
    with pytest.raises(ValueError):
        quant.preshuffle_e8m0(torch.zeros(2, 4, 32, dtype=torch.uint8))
