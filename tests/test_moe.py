"""CPU checks of the grouped (MoE) GEMM: argument validation of the C ABI
(status codes returned before any launch), kernel names, and a restatement
of the kernel's expert lookup (g9_gemm.hpp moe_find) showing that any offset
table keeps every access inside A, C and the experts' B, and that valid tables
give each expert's rows to exactly one tile."""

import numpy as np
import pytest

from gfx950_gluon_tutorials_amd import _lib

FAKE = 0x10000


def _moe16(T=512, N=256, K=256, E=4, sam=None, sbn=None, sbe=None, scm=None, dtype=_lib.G9_F16, off=FAKE):
    lib = _lib.load()
    return lib.g9_moe_a16w16(FAKE, FAKE, FAKE, off, T, N, K, E, K if sam is None else sam,
                             K if sbn is None else sbn, N * K * 2 if sbe is None else sbe,
                             N if scm is None else scm, dtype, None)


@pytest.mark.parametrize("kw,code", [
    (dict(E=0), _lib.G9_ERR_SHAPE),
    (dict(T=-1), _lib.G9_ERR_SHAPE),
    (dict(K=100), _lib.G9_ERR_SHAPE),
    (dict(N=0), _lib.G9_ERR_SHAPE),
    (dict(off=0), _lib.G9_ERR_LAYOUT),
    (dict(off=FAKE + 2), _lib.G9_ERR_LAYOUT),
    (dict(sbe=8), _lib.G9_ERR_LAYOUT),
    (dict(sam=100), _lib.G9_ERR_LAYOUT),
    (dict(scm=100), _lib.G9_ERR_LAYOUT),
    (dict(dtype=_lib.G9_FP4), _lib.G9_ERR_DTYPE),
    (dict(T=0), _lib.G9_OK),  # no tokens: nothing to launch
    (dict(T=0, K=100), _lib.G9_ERR_SHAPE),
])
def test_moe_a16w16_argument_validation(kw, code):
    assert _moe16(**kw) == code


def test_moe_a4w4_argument_validation():
    lib = _lib.load()
    T, N, K, E = 512, 256, 512, 4

    def call(out=_lib.G9_BF16, sasm=K // 32, sbse=N * K // 32, asc=FAKE):
        return lib.g9_moe_a4w4(FAKE, FAKE, FAKE, asc, FAKE, FAKE, T, N, K, E, K // 2, K // 2, N * K // 2,
                               sasm, K // 32, sbse, N, out, None)

    assert call(out=_lib.G9_BF8) == _lib.G9_ERR_DTYPE
    assert call(sasm=K // 32 - 4) == _lib.G9_ERR_LAYOUT
    assert call(sbse=6) == _lib.G9_ERR_LAYOUT
    assert call(asc=0) == _lib.G9_ERR_LAYOUT


def test_moe_a8w8_argument_validation():
    lib = _lib.load()
    T, N, K, E = 512, 256, 512, 4

    def call(out=_lib.G9_BF16, K_=K, sb=FAKE):
        return lib.g9_moe_a8w8(FAKE, FAKE, FAKE, FAKE, None, sb, T, N, K_, E, K_, K_, N * K_, N, out, None)

    assert call(out=_lib.G9_FP4) == _lib.G9_ERR_DTYPE
    assert call(K_=192) == _lib.G9_ERR_SHAPE  # K must be a multiple of 128
    assert call(sb=FAKE + 2) == _lib.G9_ERR_LAYOUT


def test_moe_kernel_names():
    pairs = [(_lib.G9_F16, _lib.G9_F16), (_lib.G9_BF16, _lib.G9_BF16), (_lib.G9_BF8, _lib.G9_BF16),
             (_lib.G9_BF8, _lib.G9_F16), (_lib.G9_FP4, _lib.G9_BF16), (_lib.G9_FP4, _lib.G9_F16)]
    names = {_lib.moe_kernel_name(dt, out) for dt, out in pairs}
    assert len(names) == 6 and all(n and n.endswith("_moe_4w") for n in names)
    assert _lib.moe_kernel_name(_lib.G9_F16, _lib.G9_BF16) is None


def moe_find(off, E, T, mt):
    """Restatement of the kernel's lookup: clamp each expert's [lo, hi) into [0, T], count its 256-row
    tiles, and return (expert, local m-tile, lo, rows) of m-tile mt, or None."""
    base = 0
    for e in range(E):
        lo = min(max(int(off[e]), 0), T)
        hi = min(max(int(off[e + 1]), lo), T)
        n = (hi - lo + 255) // 256
        if n and base <= mt < base + n:
            return e, mt - base, lo, hi - lo
        base += n
    return None


def test_moe_lookup_covers_valid_tables_exactly_once():
    rng = np.random.default_rng(0)
    for _ in range(200):
        E = int(rng.integers(1, 20))
        counts = rng.integers(0, 700, E)
        counts[rng.random(E) < 0.3] = 0
        off = np.concatenate([[0], np.cumsum(counts)])
        T = int(off[-1]) + int(rng.integers(0, 300))
        bound = -(-T // 256) + E
        owner = np.full(T, -1)
        for mt in range(bound):
            r = moe_find(off, E, T, mt)
            if r is None:
                continue
            e, lt, lo, rows = r
            assert 0 <= lt < -(-rows // 256)
            sl = slice(lo + 256 * lt, lo + min(256 * (lt + 1), rows))
            assert np.all(owner[sl] == -1)  # no row is computed twice
            owner[sl] = e
        for e in range(E):
            assert np.all(owner[off[e]:off[e + 1]] == e)
        assert np.all(owner[off[-1]:] == -1)


def test_moe_lookup_keeps_garbage_tables_in_bounds():
    rng = np.random.default_rng(1)
    for _ in range(300):
        E = int(rng.integers(1, 70))
        T = int(rng.integers(1, 3000))
        off = rng.integers(-5000, 8000, E + 1)
        bound = -(-T // 256) + E
        for mt in range(bound):
            r = moe_find(off, E, T, mt)
            if r is None:
                continue
            e, lt, lo, rows = r
            assert 0 <= e < E and 0 <= lo and lo + rows <= T
            # rows the tile reads from A and writes to C
            first, last = lo + 256 * lt, lo + min(256 * (lt + 1), rows)
            assert 0 <= first < last <= T
