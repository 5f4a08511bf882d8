"""Pins the oracle's scalar numerics (a1, a2) against the reference's own
known answers and against independent closed forms / brute force."""
from fractions import Fraction
import math
import struct

import numpy as np
import pytest

import oracle


def f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def frac_e4m3(bits: int) -> Fraction:
    # Independent decode from the OCP e4m3 definition: bias 7, subnormal
    # 2^-6 * m/8.
    s = -1 if bits & 0x80 else 1
    e = (bits >> 3) & 15
    m = bits & 7
    mag = Fraction(m, 8) * Fraction(1, 64) if e == 0 else Fraction(8 + m, 8) * Fraction(2) ** (e - 7)
    return s * mag


FINITE_E4M3 = [b for b in range(256) if (b & 0x7F) != 0x7F]


def test_e2m1_sint8_known_answer():
    # tests/test_quantized_transforms.py:22-27
    packed = bytes((0x10, 0x87, 0xFE))
    out = []
    for v in packed:
        out += [oracle.e2m1_to_sint8(v & 15) & 0xFF, oracle.e2m1_to_sint8(v >> 4) & 0xFF]
    assert bytes(out) == bytes((0, 1, 12, 0, 248, 244))


def test_e2m1_e4m3_known_answer():
    # tests/test_quantized_transforms.py:38-42
    packed = bytes((0x10, 0xF8))
    out = []
    for v in packed:
        out += [oracle.e2m1_to_e4m3_bits(v & 15), oracle.e2m1_to_e4m3_bits(v >> 4)]
    assert bytes(out) == bytes((0x00, 0x30, 0x80, 0xCC))


def test_mxfp4_value_exhaustive_against_closed_form():
    # tests/test_quantized_transforms.py:30-50: value = code/2 * 2^(b-127),
    # byte 0 -> 2^-127; every (nibble, scale byte < 255) pair, bit-exact.
    mags = [Fraction(0), Fraction(1, 2), Fraction(1), Fraction(3, 2), Fraction(2), Fraction(3), Fraction(4), Fraction(6)]
    for b in range(255):
        scale = Fraction(2) ** (-127 if b == 0 else b - 127)
        assert Fraction(oracle.e8m0_scale(b)) == scale
        for n in range(16):
            expect = (-1 if n & 8 else 1) * mags[n & 7] * scale
            got = oracle.mxfp4_value(n, b)
            if abs(expect) >= Fraction(2) ** 128:  # beyond f32: overflows to +-inf
                assert math.isinf(got) and (got < 0) == (expect < 0), (n, b)
            else:
                assert Fraction(got) == expect, (n, b)
            # the sint8 route: code * (scale / 2)
            assert Fraction(oracle.e2m1_to_sint8(n)) * scale / 2 == expect


def test_e4m3_decode_matches_definition():
    for b in FINITE_E4M3:
        assert Fraction(float(oracle.e4m3_to_f32([b])[0])) == frac_e4m3(b), hex(b)


def _brute_e4m3(x: float) -> int:
    """Nearest finite e4m3 by exact distance; ties -> even code; |x| beyond
    the finite range -> 448 (saturation)."""
    if x != x:
        return 0x7F
    sign = 0x80 if math.copysign(1.0, x) < 0 else 0
    ax = Fraction(abs(x))
    best, best_d = None, None
    for b in range(0x7F):  # non-negative finite codes 0x00..0x7e
        d = abs(frac_e4m3(b) - ax)
        if best is None or d < best_d or (d == best_d and (b & 1) == 0 and (best & 1) == 1):
            best, best_d = b, d
    return sign | best


def test_e4m3_encode_against_brute_force():
    vals = set()
    pos = sorted({frac_e4m3(b) for b in range(0x7F)})
    for v in pos:
        vals.add(float(v))
    for a, b in zip(pos, pos[1:]):
        mid = (a + b) / 2
        fm = float(mid)
        vals.add(fm)
        vals.add(float(np.nextafter(np.float32(fm), np.float32(0))))
        vals.add(float(np.nextafter(np.float32(fm), np.float32(1e9))))
    vals.update([448.0, 449.0, 463.9, 464.0, 464.1, 480.0, 1e4, 2.0 ** -10, 2.0 ** -11, 1e-30, 0.0,
                 f32(0.0155), f32(2.0 ** -6 * 0.99)])
    rng = np.random.default_rng(0)
    vals.update(float(v) for v in rng.standard_normal(2000).astype(np.float32) * 10)
    vals.update(float(v) for v in rng.uniform(-1e-2, 1e-2, 500).astype(np.float32))
    vals = sorted(vals)
    vals = [f32(v) for v in vals] + [-f32(v) for v in vals]
    got = oracle.f32_to_e4m3(np.array(vals, np.float32))
    for v, g in zip(vals, got):
        assert int(g) == _brute_e4m3(v), (v, hex(int(g)), hex(_brute_e4m3(v)))


def test_pow2_scale_closed_form():
    # rounded_fp8_scale: the smallest power of two >= f32(max(amax,1e-4)/448).
    rng = np.random.default_rng(1)
    amaxes = list(rng.uniform(0, 20, 300).astype(np.float32)) + [0.0, 1e-5, 1e-4, 448.0, 896.0, 1.0, 0.5, 7.0]
    for a in amaxes:
        ratio = np.float32(max(np.float32(a), np.float32(1e-4))) / np.float32(448.0)
        m, e = math.frexp(float(ratio))  # ratio = m * 2^e, m in [0.5, 1)
        expect = 2.0 ** (e - 1) if m == 0.5 else 2.0 ** e
        assert oracle.pow2_fp8_scale(float(a)) == expect, a
        if a >= 1e-4:
            assert float(a) / expect <= 448.0 * (1 + 2 ** -20)


def test_quantize_blocks_known_answers_and_tail():
    # hidden = 1.0 (mxfp4_tests.rs:67-216 input): amax 1 -> scale 2^-8 -> code 256 = 0x78.
    one = np.full((1, 128), 0x3F80, np.uint16)
    q, s = oracle.quantize_blocks(one, pow2=True)
    assert s[0, 0] == 2.0 ** -8 and np.all(q == 0x78)
    q, s = oracle.quantize_blocks(one, pow2=False)  # amax/448 -> x/s = 448 -> 0x7e
    assert s[0, 0] == np.float32(1.0) / np.float32(448.0) and np.all(q == 0x7E)
    # zero block: pow2 scale from the 1e-4 floor; amax scale 1.0
    z = np.zeros((1, 160), np.uint16)
    q, s = oracle.quantize_blocks(z, pow2=True)
    assert s.shape == (1, 2) and np.all(q == 0) and s[0, 0] == oracle.pow2_fp8_scale(0.0)
    # tail block (K = 2880 = 22*128 + 64): its amax covers only the real columns
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((3, 2880)).astype(np.float32))
    xb = oracle.f32_to_bf16(x)
    q, s = oracle.quantize_blocks(xb, pow2=True)
    assert s.shape == (3, 23)
    xf = oracle.bf16_to_f32(xb)
    for r in range(3):
        for b in range(23):
            blk = xf[r, b * 128:(b + 1) * 128]
            assert s[r, b] == oracle.pow2_fp8_scale(float(np.max(np.abs(blk))))
        # decoded values equal x/s rounded; |q| never saturates
        deq = oracle.e4m3_to_f32(q[r]) * np.repeat(s[r], 128)[:2880]
        rel = np.abs(deq - xf[r]) / np.maximum(np.abs(xf[r]), 1e-3)
        assert np.all(np.abs(oracle.e4m3_to_f32(q[r])) <= 448)
        assert np.max(rel[np.abs(xf[r]) > 0.05]) <= 2.0 ** -4


def test_bf16_rounding_rne():
    vals = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 3.14159], np.float32)
    got = oracle.f32_to_bf16(vals)
    assert list(got) == [0x3F80, 0x3F80, 0x3F82, 0xC020, 0x4049]
    for v in (0.5, 1.5, -7.25, 1e-3):
        assert oracle.lib().o_f32_to_bf16(v) == int(oracle.f32_to_bf16(np.float32(v)))
