"""Pins of the oracle's block codec, decoder and products (CPU only).

* Block codec (``encoder.py:105-117``): pack/unpack round trips, over random arrays and, with
  hypothesis, over arbitrary 8-byte blocks.
* Decoder (``encoder.py:19-20`` gather, ``texelator_cuda.cu:141-152`` rounding): a known-answer
  block per palette mode whose weights are derived here in exact rational arithmetic
  (``fractions.Fraction``) with a non-power-of-two row scale, and the two independent
  restatements (numpy LUT gather, C palette recompute) equal bit for bit on random blocks, in
  the defined palette and in LUT mode with a perturbed table.
* Products (``texelator_cuda.cu:154-199``, ``cutlass_texture_mainloop.cu:203-249``): the numpy
  and C float64 matvec/GEMM agree with each other and with a pure-Python brute force.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle import bc4, clib
from tests.helpers import lognormal_scales, random_blocks


# ---------------------------------------------------------------------------------------------
# exact-arithmetic helpers (independent of numpy's float rounding)


def _round_to(fr: Fraction, significant_bits: int) -> Fraction:
    """Round an exact rational to ``significant_bits`` bits, ties to even (normal range)."""
    if fr == 0:
        return Fraction(0)
    sign = -1 if fr < 0 else 1
    mag = abs(fr)
    exponent = mag.numerator.bit_length() - mag.denominator.bit_length()
    if Fraction(2) ** exponent > mag:
        exponent -= 1
    quantum = Fraction(2) ** (exponent - significant_bits + 1)
    scaled = mag / quantum
    low = scaled.numerator // scaled.denominator
    rest = scaled - low
    if rest > Fraction(1, 2) or (rest == Fraction(1, 2) and low % 2 == 1):
        low += 1
    return sign * low * quantum


def _f32(fr: Fraction) -> Fraction:
    return _round_to(fr, 24)


def _bf16_bits(fr: Fraction) -> int:
    value = np.float32(float(_round_to(fr, 8)))
    return int(value.view(np.uint32)) >> 16


def _exact_weights(e0: int, e1: int, selectors: list[int], scale: np.float32) -> list[int]:
    """bf16 bits of ``RN_bf16(RN_f32(P[s] * scale))`` with P from the palette definition."""
    e0, e1 = max(e0, -127), max(e1, -127)
    base, end = _f32(Fraction(e0, 127)), _f32(Fraction(e1, 127))
    eight = e0 > e1
    step = _f32(Fraction(e1 - e0, 889 if eight else 635))
    palette = [base, end] + [_f32((s - 1) * step + base) for s in range(2, 8)]
    if not eight:
        palette[6], palette[7] = Fraction(-1), Fraction(1)
    s = Fraction(float(scale))
    return [_bf16_bits(_f32(palette[sel] * s)) for sel in selectors]


def _block(e0: int, e1: int, selectors: list[int]) -> np.ndarray:
    return bc4.pack_blocks(np.array([e0]), np.array([e1]), np.array([selectors]))


# ---------------------------------------------------------------------------------------------
# codec


def test_pack_unpack_round_trip_random():
    rng = np.random.default_rng(1)
    n = 4096
    e0 = rng.integers(-128, 128, n)
    e1 = rng.integers(-128, 128, n)
    sel = rng.integers(0, 8, (n, 16))
    blocks = bc4.pack_blocks(e0, e1, sel)
    assert blocks.shape == (n, 8) and blocks.dtype == np.uint8
    u0, u1, usel = bc4.unpack_blocks(blocks)
    assert np.array_equal(u0, e0) and np.array_equal(u1, e1) and np.array_equal(usel, sel)


def test_selector_bit_positions():
    """Selector of position p sits at bits 3p..3p+2 of the little-endian 48-bit field."""
    for p in range(16):
        sel = [0] * 16
        sel[p] = 5
        raw = _block(0, 0, sel)[0]
        field = int.from_bytes(bytes(raw[2:8]), "little")
        assert field == 5 << (3 * p)


@settings(max_examples=300, deadline=None)
@given(st.binary(min_size=8, max_size=8))
def test_unpack_pack_round_trip_any_block(raw):
    blocks = np.frombuffer(raw, dtype=np.uint8).reshape(1, 8)
    e0, e1, sel = bc4.unpack_blocks(blocks)
    assert bytes(bc4.pack_blocks(e0, e1, sel)[0]) == raw


# ---------------------------------------------------------------------------------------------
# decoder known answers


@pytest.mark.parametrize("e0,e1,scale", [
    (100, -50, 0.0173),      # 8-value mode
    (-128, 90, 0.0291),      # 6-value mode; -128 decodes as -127
    (-3, -3, 1.7),           # equal endpoints: 6-value mode, flat palette plus -1/+1
    (127, -127, 3.0e-3),     # widest 8-value span
])
def test_known_answer_block(e0, e1, scale):
    selectors = [p % 8 for p in range(16)]
    scale32 = np.float32(scale)
    want = np.array(_exact_weights(e0, e1, selectors, scale32), dtype=np.uint16)
    block = _block(e0, e1, selectors)
    scales = np.array([scale32], dtype=np.float32)
    assert np.array_equal(bc4.decode_bf16_bits(block, scales)[0], want)
    assert np.array_equal(clib.decode_bf16_bits(block, scales)[0], want)


def test_known_answer_six_value_constants():
    """In 6-value mode selectors 6 and 7 give exactly -scale and +scale (rounded to bf16)."""
    scale = np.float32(0.0123)
    block = _block(-20, 40, [6, 7] * 8)
    got = bc4.decode_bf16_bits(block, np.array([scale]))[0]
    neg, pos = _bf16_bits(-Fraction(float(scale))), _bf16_bits(Fraction(float(scale)))
    assert list(got) == [neg, pos] * 8


# ---------------------------------------------------------------------------------------------
# numpy and C restatements


def test_numpy_and_c_decoders_agree():
    m, k = 160, 512
    blocks = random_blocks(m, k, 31)
    scales = lognormal_scales(m, 32)
    scales[3] = 0.0
    scales[7] = 1e-30
    assert np.array_equal(bc4.decode_bf16_bits(blocks, scales), clib.decode_bf16_bits(blocks, scales))


def test_numpy_and_c_decoders_agree_in_lut_mode():
    """With a perturbed table both read the table (a decoder ignoring it would differ)."""
    m, k = 64, 256
    blocks = random_blocks(m, k, 33)
    scales = lognormal_scales(m, 34)
    table = bc4.palette().copy()
    rng = np.random.default_rng(35)
    table *= (1 + 1e-3 * rng.standard_normal(table.shape)).astype(np.float32)
    numpy_bits = bc4.decode_bf16_bits(blocks, scales, table)
    assert np.array_equal(numpy_bits, clib.decode_bf16_bits(blocks, scales, table))
    assert not np.array_equal(numpy_bits, bc4.decode_bf16_bits(blocks, scales))


def _brute_matvec(w_bits: np.ndarray, x_bits: np.ndarray) -> list[float]:
    w = bc4.bf16_bits_to_f32(w_bits)
    x = bc4.bf16_bits_to_f32(x_bits)
    # Every product of two bf16 values and every partial sum here is exact in Fraction.
    return [float(sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(row, x))) for row in w]


def test_matvec_numpy_c_and_brute_force_agree():
    m, k = 12, 96
    w_bits = bc4.decode_bf16_bits(random_blocks(m, k, 41), lognormal_scales(m, 42))
    x_bits = bc4.f32_to_bf16_bits(np.random.default_rng(43).standard_normal(k).astype(np.float32))
    exact = np.array(_brute_matvec(w_bits, x_bits))
    np.testing.assert_allclose(bc4.matvec_f64(w_bits, x_bits), exact, rtol=1e-12, atol=1e-15)
    np.testing.assert_allclose(clib.matvec_f64(w_bits, x_bits), exact, rtol=1e-12, atol=1e-15)


def test_gemm_numpy_and_c_agree_and_match_matvec():
    m, k, t = 72, 384, 9
    w_bits = bc4.decode_bf16_bits(random_blocks(m, k, 51), lognormal_scales(m, 52))
    x_bits = bc4.f32_to_bf16_bits(np.random.default_rng(53).standard_normal((t, k)).astype(np.float32))
    c = clib.gemm_f64(x_bits, w_bits)
    np.testing.assert_allclose(bc4.gemm_f64(x_bits, w_bits), c, rtol=1e-12, atol=1e-14)
    for row in (0, t - 1):   # a GEMM row is the matvec of that token (transposition check)
        np.testing.assert_allclose(c[row], clib.matvec_f64(w_bits, x_bits[row]), rtol=1e-12, atol=1e-14)


def test_fused_decode_matvec_f32_close_to_f64():
    """The C baseline's fused decode + fp32 matvec stays within fp32 accumulation error."""
    m, k = 48, 2048
    blocks = random_blocks(m, k, 61)
    scales = lognormal_scales(m, 62)
    x_bits = bc4.f32_to_bf16_bits(np.random.default_rng(63).standard_normal(k).astype(np.float32))
    ref = clib.matvec_f64(clib.decode_bf16_bits(blocks, scales), x_bits)
    got = clib.decode_matvec_f32(blocks, scales, x_bits)
    assert bc4.relative_error(ref, got) < 1e-5
