"""Byte-level model of the MXFP4 scale chunks of the 4-wave kernels (CPU).

A chunk slot holds four K stages (32 scale groups) of the tile's 512 rows
(A0, A1, B0, B1 half tiles of 128).  The kernels read it with
ds_read_b64_tr_b8, whose lane map was measured on gfx950: in each 16-lane
group, lane 8a + b receives byte b of the 8-byte units addressed by lanes
a, a + 2, ..., a + 14 of the group, in that order.

This file restates the kernel's address arithmetic (Pipe::init in
csrc/g9_gemm.hpp) for the two ways a chunk gets into LDS -- row-major scales
DMA'd as they are and transposed in place into the KM layout, K-major scales
DMA'd straight into the KL layout in whole 128-byte runs -- and checks the end
result against what the MFMAs need, derived independently: lane (g, rr) of
fragment F must hold, in byte 2 st + h, the scale of its row for MFMA step h
of stage st, i.e. group 8 st + 4 h + g of the chunk (the K values
32 (8 st + 4 h + g) .. of a 16x16x128 fragment's lane group g).  A wrong XOR,
a swapped octet, a transposed index or an out-of-place write fails at least
one check.
"""

import numpy as np
import pytest

SLOT = 16384
HALF = 4096  # one half tile's 128 rows x 32 groups


def tr_read(lds: np.ndarray, addrs: list[int]) -> list[bytes]:
    """ds_read_b64_tr_b8 of 64 lanes at the given byte addresses."""
    out = []
    for lane in range(64):
        grp, x = divmod(lane, 16)
        a, b = divmod(x, 8)
        out.append(bytes(int(lds[addrs[16 * grp + a + 2 * k] + b]) for k in range(8)))
    return out


def dma_row_major(lds, scales, hrow0, xw, ld):
    """The row-major chunk DMA of wave xw: part j, lane l fetches the 16-byte
    half of row 32 j + l // 2 that belongs in its LDS half (rows with bit 3
    set swapped) and writes it at 1024 j + 16 l of the wave's 4 KiB."""
    for j in range(4):
        for lane in range(64):
            row = 32 * j + (lane >> 1)
            half = (lane & 1) ^ ((row >> 3) & 1)
            src = scales[hrow0 + row, 16 * half:16 * half + 16]
            dst = xw * HALF + 1024 * j + 16 * lane
            lds[dst:dst + 16] = src


def k_major_dma_sources(j):
    """(group, first row) fetched by each lane of K-major part DMA j: lane l
    fills unit position l & 7 of group row G = 8 j + l // 8 with the 16 rows
    16 u .. of u = (l & 7) ^ (G >> 2)."""
    out = []
    for lane in range(64):
        G = 8 * j + (lane >> 3)
        out.append((G, 16 * ((lane & 7) ^ (G >> 2))))
    return out


def dma_k_major(lds, scales_km, hrow0, xw):
    """The K-major chunk DMA of wave xw (scales_km is groups x rows): part j
    writes its lanes' 16-byte units at 1024 j + 16 lane of the wave's 4 KiB."""
    for j in range(4):
        for lane, (G, r) in enumerate(k_major_dma_sources(j)):
            dst = xw * HALF + 1024 * j + 16 * lane
            lds[dst:dst + 16] = scales_km[G, hrow0 + r:hrow0 + r + 16]


def xform_read_addr(i, lane):
    g, k, a = lane >> 4, (lane >> 1) & 7, lane & 1
    return 512 * a + 256 * i + 32 * k + 16 * (((g >> 1) ^ a) ^ i) + 8 * (g & 1)


def xform_write_addr(lane):
    """tw: lane 16g + 8a + b writes its two units (group G = 8 (g ^ 2a) + b)
    at 32 p + 16 (a ^ (b & 1)), p = ((2 (g ^ 2a) + (b >> 2)) ^ (b & 2)) +
    8 (b & 3)."""
    g, a2, b = lane >> 4, (lane >> 3) & 1, lane & 7
    pg = ((2 * (g ^ (2 * a2)) + (b >> 2)) ^ (b & 2)) + 8 * (b & 3)
    return 32 * pg + 16 * (a2 ^ (b & 1))


def xform(lds, xw):
    """The in-place transpose of wave xw's four parts: two transpose reads
    per part (tb[i]: lane 16g + 2k + a at 512a + 256i + 32k + 16((g >> 1) ^
    a ^ i) + 8(g & 1)), then one 16-byte write per lane (xform_write_addr)
    of its two units, read 0's first."""
    msc = xw * HALF
    for j in range(4):
        got = [tr_read(lds, [msc + 1024 * j + xform_read_addr(i, lane) for lane in range(64)]) for i in range(2)]
        writes = []
        for lane in range(64):
            writes.append((msc + 1024 * j + xform_write_addr(lane), got[0][lane] + got[1][lane]))
        # The writes of a part cover exactly its KiB, once each.
        covered = sorted(w for w, _ in writes)
        assert covered == list(range(msc + 1024 * j, msc + 1024 * (j + 1), 16))
        for addr, data in writes:
            lds[addr:addr + 16] = np.frombuffer(data, dtype=np.uint8)


def mfma_read(lds, side, wave_col, F):
    """The chunk-scale read of fragment F of sub-buffer X = side (0..3) by a
    wave in row/column wave_col: bS[X >= 2][F & 1] + (X & 1) 4096 + (F / 2)
    1024, with lane 16g + 2k + a at 32 ((k ^ (g & 2)) + 8g) + 8 ((2 (F & 1) + a)
    ^ 2 (g & 1))."""
    addrs = []
    for lane in range(64):
        g, k, a = lane >> 4, (lane >> 1) & 7, lane & 1
        off = 32 * ((k ^ (g & 2)) + 8 * g) + 8 * ((2 * (F & 1) + a) ^ (2 * (g & 1)))
        base = (8192 if side >= 2 else 0) + 2048 * wave_col + off
        addrs.append(base + (side & 1) * 4096 + (F // 2) * 1024)
    return tr_read(lds, addrs), addrs


KSCALE_BASE = 131072  # the chunk slots' LDS offset (kScaleBase)


def mfma_read_kl(lds, side, wave_col, F):
    """The K-major kernel's chunk-scale read: bS[X >= 2][0] = kScaleBase +
    (8192 for B) + 128 (4k + g) + 8a + 16 ((4 wm) ^ k), XORed with 16 F,
    plus the immediate (X & 1) 4096 -- the kernel's arithmetic on the full
    address, so a XOR that reached past bits 4-5 would show."""
    addrs = []
    for lane in range(64):
        g, k, a = lane >> 4, (lane >> 1) & 7, lane & 1
        base = KSCALE_BASE + (8192 if side >= 2 else 0) + 128 * (4 * k + g) + 8 * a + 16 * ((4 * wave_col) ^ k)
        addrs.append(((base ^ (16 * F)) + (side & 1) * 4096) - KSCALE_BASE)
    return tr_read(lds, addrs), addrs


def check_mfma_reads(lds, tile_scales, read=mfma_read):
    """tile_scales: 512 rows (A then B) x 32 groups of the chunk."""
    for side in range(4):
        for wave_col in range(2):
            for F in range(4):
                got, _ = read(lds, side, wave_col, F)
                for lane in range(64):
                    g, rr = lane // 16, lane % 16
                    row = 128 * side + 64 * wave_col + 16 * F + rr
                    want = bytes(int(tile_scales[row, 8 * st + 4 * h + g]) for st in range(4) for h in range(2))
                    assert got[lane] == want, (side, wave_col, F, lane)


def _tile(seed):
    rng = np.random.default_rng(seed)
    return rng.integers(0, 256, (512, 32), dtype=np.uint8)


@pytest.mark.parametrize("seed", [0, 1])
def test_row_major_chunk_transposed_in_place_feeds_the_mfmas(seed):
    tile = _tile(seed)
    lds = np.zeros(SLOT, dtype=np.uint8)
    for xw in range(4):
        dma_row_major(lds, tile, 128 * xw, xw, 32)
    for xw in range(4):
        xform(lds, xw)
    check_mfma_reads(lds, tile)


@pytest.mark.parametrize("seed", [2, 3])
def test_k_major_chunk_feeds_the_mfmas(seed):
    tile = _tile(seed)
    lds = np.zeros(SLOT, dtype=np.uint8)
    for xw in range(4):
        dma_k_major(lds, tile.T.copy(), 128 * xw, xw)
    check_mfma_reads(lds, tile, read=mfma_read_kl)


def test_k_major_parts_fetch_whole_128_byte_runs():
    # Each part DMA reads eight group rows of 128 contiguous bytes (one
    # aligned run each for a 128-aligned tile row), and the wave's four
    # parts write every unit of its 4 KiB once.
    for j in range(4):
        src = k_major_dma_sources(j)
        for G in range(8 * j, 8 * j + 8):
            rows = sorted(r for g, r in src if g == G)
            assert rows == list(range(0, 128, 16))
    units = {(G, r) for j in range(4) for G, r in k_major_dma_sources(j)}
    assert len(units) == 32 * 8


def test_the_row_major_transpose_matches_the_k_major_dma_in_content():
    # The two layouts differ, but the bytes each MFMA lane receives agree.
    tile = _tile(4)
    a = np.zeros(SLOT, dtype=np.uint8)
    b = np.zeros(SLOT, dtype=np.uint8)
    for xw in range(4):
        dma_row_major(a, tile, 128 * xw, xw, 32)
        xform(a, xw)
        dma_k_major(b, tile.T.copy(), 128 * xw, xw)
    for side in range(4):
        for wave_col in range(2):
            for F in range(4):
                assert mfma_read(a, side, wave_col, F)[0] == mfma_read_kl(b, side, wave_col, F)[0]


def test_a_wrong_unit_swizzle_is_caught():
    # Plant a mistake in the model of the K-major read (no XOR of the unit
    # with k): the end-to-end check must fail.
    tile = _tile(5)
    lds = np.zeros(SLOT, dtype=np.uint8)
    for xw in range(4):
        dma_k_major(lds, tile.T.copy(), 128 * xw, xw)
    addrs = []
    for lane in range(64):
        g, k, a = lane >> 4, (lane >> 1) & 7, lane & 1
        addrs.append(128 * (4 * k + g) + 8 * a)
    got = tr_read(lds, addrs)
    want = [bytes(int(tile[lane % 16, 8 * st + 4 * h + lane // 16]) for st in range(4) for h in range(2))
            for lane in range(64)]
    assert got != want


def test_a_wrong_octet_swizzle_is_caught():
    # Plant a mistake in the model of the row-major path's read (no XOR on
    # the octet): the end-to-end check must fail.
    tile = _tile(5)
    lds = np.zeros(SLOT, dtype=np.uint8)
    for xw in range(4):
        dma_row_major(lds, tile, 128 * xw, xw, 32)
        xform(lds, xw)
    addrs = []
    for lane in range(64):
        g, k, a = lane >> 4, (lane >> 1) & 7, lane & 1
        addrs.append(32 * (k + 8 * g) + 8 * a)
    got = tr_read(lds, addrs)
    want = [bytes(int(tile[lane % 16, 8 * st + 4 * h + lane // 16]) for st in range(4) for h in range(2))
            for lane in range(64)]
    assert got != want


def _banks(addrs, width=8):
    return [((ad // 4) + d) % 64 for ad in addrs for d in range(width // 4)]


@pytest.mark.parametrize("read", [mfma_read, mfma_read_kl])
def test_mfma_reads_are_bank_conflict_free_per_32_lanes(read):
    # 64 banks x 4 bytes serve 32 lanes of an 8-byte read per cycle: each
    # half wave's units must fall on 64 distinct banks.
    lds = np.zeros(SLOT, dtype=np.uint8)
    for side in range(4):
        for wave_col in range(2):
            for F in range(4):
                _, addrs = read(lds, side, wave_col, F)
                for h in range(2):
                    banks = _banks(addrs[32 * h:32 * h + 32])
                    assert len(set(banks)) == 64, (side, wave_col, F, h)


def test_transpose_reads_are_bank_conflict_free_per_32_lanes():
    for i in range(2):
        addrs = [xform_read_addr(i, lane) for lane in range(64)]
        for h in range(2):
            assert len(set(_banks(addrs[32 * h:32 * h + 32]))) == 64


def test_transpose_writes_are_bank_conflict_free_per_8_lanes():
    # A 16-byte write is served 8 lanes at a time (the previous group-row
    # order, p = (G >> 2) + 8 (G & 3), measured 1152 conflict cycles per
    # workgroup, which this pass model gives as 8 per write): the 32 banks of
    # each pass of 8 lanes must be distinct.
    addrs = [xform_write_addr(lane) for lane in range(64)]
    for p0 in range(0, 64, 8):
        assert len(set(_banks(addrs[p0:p0 + 8], width=16))) == 32, p0
    old = []
    for lane in range(64):
        g, a2, b = lane >> 4, (lane >> 3) & 1, lane & 7
        old.append(32 * (2 * (g ^ (2 * a2)) + (b >> 2) + 8 * (b & 3)) + 16 * (a2 ^ (b & 1)))
    assert any(len(set(_banks(old[p0:p0 + 8], width=16))) < 32 for p0 in range(0, 64, 8))
