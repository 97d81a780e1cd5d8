"""Writes the golden GEMM fixtures in tests/golden/ with exact arithmetic.

The reference ships no golden vectors (its correctness checks are print-only
``allclose``), so these fixtures are built from first principles: operands are
chosen so that every product and every partial sum is exactly representable,
and the expected output is the exact integer/rational result computed with
Python integers (no floating point, no BLAS, no oracle code), rounded once to
the output type.  Any K order, any accumulation tree and any correct kernel
must then reproduce them bit for bit; a transposed operand, a dropped K block,
a wrong nibble or scale index changes them.

Run from the repo root: ``python tests/golden/make_golden.py``.
"""

from __future__ import annotations

import os
import struct
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

# e2m1 magnitudes as exact fractions (OCP MX v1.0 table).
E2M1 = [Fraction(0), Fraction(1, 2), Fraction(1), Fraction(3, 2), Fraction(2), Fraction(3), Fraction(4), Fraction(6)]


def e2m1_exact(code: int) -> Fraction:
    v = E2M1[code & 7]
    return -v if code & 8 else v


def f16_bits_exact(q: Fraction) -> int:
    """Exact rational -> IEEE binary16 bits, round to nearest even (no overflow
    expected in these fixtures)."""
    return int(np.float16(float(q)).view(np.uint16)) if _f16_exact(q) else _round_f16(q)


def _f16_exact(q: Fraction) -> bool:
    return Fraction(float(np.float16(float(q)))) == q


def _round_f16(q: Fraction) -> int:
    raise ValueError(f"fixture value {q} not exactly representable in fp16")


def bf16_bits_rne(q: Fraction) -> int:
    """Exact rational -> bfloat16 bits with one round-to-nearest-even."""
    if q == 0:
        return 0
    sign = 0x8000 if q < 0 else 0
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    # a in [2^e, 2^(e+1)); bf16 keeps 8 significant bits.
    step = Fraction(2) ** (e - 7)
    n = a / step
    r = n.numerator // n.denominator
    rem = n - r
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and r % 2 == 1):
        r += 1
    val = r * step
    bits = struct.unpack("<I", struct.pack("<f", float(val)))[0]
    assert Fraction(struct.unpack("<f", struct.pack("<I", bits))[0]) == val
    return sign | (bits >> 16)


def exact_gemm_int(a: np.ndarray, b_nk: np.ndarray) -> np.ndarray:
    """Integer A . B^T with Python ints (object dtype)."""
    ao = a.astype(object)
    bo = b_nk.astype(object)
    return ao.dot(bo.T)


def make_a16w16(rng):
    M, N, K = 64, 96, 256
    a = rng.integers(-2, 3, size=(M, K))
    b = rng.integers(-2, 3, size=(N, K))
    c = exact_gemm_int(a, b)
    assert np.abs(c.astype(np.int64)).max() <= 2048  # integers exact in fp16 and bf16
    c16 = np.array([[f16_bits_exact(Fraction(int(v))) for v in row] for row in c], dtype=np.uint16)
    cbf = np.array([[bf16_bits_rne(Fraction(int(v))) for v in row] for row in c], dtype=np.uint16)
    np.savez(os.path.join(HERE, "a16w16_exact.npz"), a=a.astype(np.float16), b_nk=b.astype(np.float16),
             c_f16_bits=c16, c_bf16_bits=cbf)


def make_a8w8(rng):
    # e5m2 operands restricted to {0, +-1, +-2}: every K=256 sum is an integer
    # of magnitude <= 1024, exact in fp32 and in the fp16 output; with the
    # scales 0.75 * 0.125 = 3 * 2^-5 the scaled result is still exact in fp32.
    M, N, K = 80, 64, 256
    vals = np.array([0, 1, 2, -1, -2], dtype=np.float32)
    a = vals[rng.integers(0, len(vals), size=(M, K))]
    b = vals[rng.integers(0, len(vals), size=(N, K))]
    a4 = (a * 2).astype(np.int64)
    b4 = (b * 2).astype(np.int64)
    c = exact_gemm_int(a4, b4)  # = 4 * (A . B^T)
    codes_a = (a.astype(np.float16).view(np.uint16) >> 8).astype(np.uint8)
    codes_b = (b.astype(np.float16).view(np.uint16) >> 8).astype(np.uint8)
    # e5m2 is the high byte of fp16; these values need no low byte.
    assert np.array_equal((codes_a.astype(np.uint16) << 8).view(np.float16).astype(np.float32), a)
    c16 = np.array([[f16_bits_exact(Fraction(int(v), 4)) for v in row] for row in c], dtype=np.uint16)
    # Scaled, bf16 output: scales 0.75 and 2^-3.
    sa, sb = Fraction(3, 4), Fraction(1, 8)
    cbf = np.array([[bf16_bits_rne(Fraction(int(v), 4) * sa * sb) for v in row] for row in c], dtype=np.uint16)
    np.savez(os.path.join(HERE, "a8w8_exact.npz"), a_codes=codes_a, b_codes=codes_b, c_f16_bits=c16,
             c_bf16_scaled_bits=cbf, a_scale=np.float32(0.75), b_scale=np.float32(0.125))


def make_a4w4(rng):
    # Random e2m1 codes (all 16) and E8M0 scales in [124, 128) as the
    # reference's generator draws them (kernels/gemm/intra_wave/a4w4/bench.py:115-146).
    # Products are multiples of 2^-8 with magnitude <= 36, K=512 sums < 2^15:
    # exact in fp32 for any summation order.
    M, N, K = 64, 80, 512
    ca = rng.integers(0, 16, size=(M, K))
    cb = rng.integers(0, 16, size=(N, K))
    sa = rng.integers(124, 128, size=(M, K // 32))
    sb = rng.integers(124, 128, size=(N, K // 32))
    pa = ((ca[:, 0::2] & 0xF) | ((ca[:, 1::2] & 0xF) << 4)).astype(np.uint8)
    pb = ((cb[:, 0::2] & 0xF) | ((cb[:, 1::2] & 0xF) << 4)).astype(np.uint8)
    # Exact value * 2^8 as integers: e2m1 * 2 is an integer, scale 2^(s-127) * 2^3 is an integer.
    va = np.vectorize(lambda c: int(e2m1_exact(int(c)) * 2))(ca).astype(np.int64)
    vb = np.vectorize(lambda c: int(e2m1_exact(int(c)) * 2))(cb).astype(np.int64)
    fa = np.repeat((2 ** (sa - 124)).astype(np.int64), 32, axis=1)
    fb = np.repeat((2 ** (sb - 124)).astype(np.int64), 32, axis=1)
    c = exact_gemm_int(va * fa, vb * fb)  # = 2^2 * 2^6 * value = 2^8 * value
    cbf = np.array([[bf16_bits_rne(Fraction(int(v), 256)) for v in row] for row in c], dtype=np.uint16)
    np.savez(os.path.join(HERE, "a4w4_exact.npz"), a=pa, b=pb, a_scales=sa.astype(np.uint8),
             b_scales=sb.astype(np.uint8), c_bf16_bits=cbf)


def main():
    rng = np.random.default_rng(20261201)
    make_a16w16(rng)
    make_a8w8(rng)
    make_a4w4(rng)
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
