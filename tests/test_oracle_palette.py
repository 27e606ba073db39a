"""Pins of the CPU palette (the LUT of this build) against exact arithmetic.

The palette is defined in oracle/bc4.py. Checks here come from the mathematics, not from the
formula: exact rationals (fractions.Fraction), the BC4 mode rule, monotonicity, and agreement
of the two independent restatements (numpy and C).
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

from oracle import bc4, clib

PAL = bc4.palette()


def _cr(fr: Fraction) -> np.float32:
    """Correctly rounded float32 of an exact rational, by exhaustive neighbour search."""
    f = np.float32(float(fr))
    cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
    best = min(cands, key=lambda c: abs(Fraction(float(c)) - fr))
    ties = [c for c in cands if abs(Fraction(float(c)) - fr) == abs(Fraction(float(best)) - fr)]
    if len(ties) > 1:
        best = min(ties, key=lambda c: int(np.float32(c).view(np.uint32)) & 1)
    return np.float32(best)


def test_shape_and_layout():
    assert PAL.shape == (255, 255, 8) and PAL.dtype == np.float32
    # lut[e1+127][e0+127]: slot 0 is e0/127, slot 1 is e1/127
    assert PAL[127 + 5, 127 - 3, 0] == _cr(Fraction(-3, 127))
    assert PAL[127 + 5, 127 - 3, 1] == _cr(Fraction(5, 127))


def test_endpoints_correctly_rounded():
    for e in range(-127, 128):
        want = _cr(Fraction(e, 127))
        assert np.all(PAL[:, e + 127, 0] == want)
        assert np.all(PAL[e + 127, :, 1] == want)


def _header_constant(name: str) -> float:
    """A float literal of the device header (``constexpr float name = 0x...f;``)."""
    import re
    from pathlib import Path

    text = (Path(__file__).resolve().parents[1] / "texelator_amd/csrc/bc4_device.h").read_text()
    match = re.search(r"constexpr float " + name + r" = (-?0x[0-9a-fA-F.p+-]+)f;", text)
    assert match, name
    return float.fromhex(match.group(1))


def _split_reciprocal_quotient(n: np.ndarray, hi: float, lo: float) -> np.ndarray:
    """float32 fma(n, hi, RN32(n * lo)), the device's quotient: n*hi (n < 2^10, hi 24 bits) and
    the float32 n*lo are exact in float64 and so is their sum (< 50 significant bits), so the
    single float64 -> float32 conversion is the fma's one rounding."""
    n = n.astype(np.float64)
    inner = (n * np.float64(np.float32(lo))).astype(np.float32).astype(np.float64)
    return (n * np.float64(np.float32(hi)) + inner).astype(np.float32)


def test_seed_quotients_exactly_rounded_exhaustive():
    """Every seed quotient the decoders use, against exact rational rounding (fractions): the
    endpoint values RN(e/127), e = -127..127, and the step values RN(d/889) and RN(d/635) for every
    difference d = e1 - e0 in -254..254 under both denominators (1,273 quotients). Three methods
    must each give the correctly rounded float32: the oracle's float64 division, the double
    division rounded to float that builds the device's compile-time seed-table image, and the
    device's fma with a split reciprocal (constants read from the device header)."""
    cases = [(127, np.arange(-127, 128), "kInv127Hi", "kInv127Lo"),
             (889, np.arange(-254, 255), "kInv889Hi", "kInv889Lo"),
             (635, np.arange(-254, 255), "kInv635Hi", "kInv635Lo")]
    checked = 0
    for den, nums, hi_name, lo_name in cases:
        hi, lo = _header_constant(hi_name), _header_constant(lo_name)
        assert np.float32(hi) == _cr(Fraction(1, den))          # hi = RN(1/d)
        assert np.float32(lo) == _cr(Fraction(1, den) - Fraction(float(np.float32(hi))))
        exact = np.array([_cr(Fraction(int(n), den)) for n in nums], dtype=np.float32)
        image = np.array([np.float32(float(int(n)) / float(den)) for n in nums], dtype=np.float32)
        device = _split_reciprocal_quotient(nums, hi, lo)
        for got in (bc4.crdiv_f32(nums, den), image, device):
            assert np.array_equal(got.view(np.uint32), exact.view(np.uint32)), den
        # the 8x-prescaled pairs of the register decoder give the same quotients of 8n
        hi8, lo8 = _header_constant(hi_name) / 8.0, _header_constant(lo_name) / 8.0
        device8 = _split_reciprocal_quotient(8 * nums, hi8, lo8)
        assert np.array_equal(device8.view(np.uint32), exact.view(np.uint32)), den
        checked += nums.size
    assert checked == 255 + 2 * 509


def test_interpolants_close_to_exact_bc4_values():
    """Exhaustive over all 65,025 pairs. 8-value mode: ((8-s)e0 + (s-1)e1)/(7*127);
    6-value mode: ((6-s)e0 + (s-1)e1)/(5*127).

    |base| <= 1 and |t*step| < 2, so the three fp32 roundings stay below 2^-22 in absolute
    terms, while any wrong term, sign or index is off by at least 1/889 > 2^-10. The check
    ``|P*D - num| <= D * 2^-22`` is exact in float64 (P has 24 significant bits, D < 2^10).
    """
    e = np.arange(-127, 128, dtype=np.int64)
    e0 = np.broadcast_to(e[None, :], (255, 255))
    e1 = np.broadcast_to(e[:, None], (255, 255))
    eight = e0 > e1
    for s in range(2, 8):
        num = np.where(eight, (8 - s) * e0 + (s - 1) * e1, (6 - s) * e0 + (s - 1) * e1)
        den = np.where(eight, 889, 635)
        valid = eight | (s < 6)
        diff = np.abs(PAL[..., s].astype(np.float64) * den - num)
        assert np.all(diff[valid] <= den[valid] * 2.0 ** -22), s


def test_six_value_mode_constants_and_mode_rule():
    e = np.arange(-127, 128)
    six = e[None, :] <= e[:, None]      # [e1][e0]: e0 <= e1
    assert np.all(PAL[..., 6][six] == -1.0) and np.all(PAL[..., 7][six] == 1.0)
    # in 8-value mode slots 6 and 7 are interpolants strictly between the endpoints
    eight = ~six
    lo = np.minimum(PAL[..., 0], PAL[..., 1])
    hi = np.maximum(PAL[..., 0], PAL[..., 1])
    for s in (6, 7):
        assert np.all((PAL[..., s][eight] >= lo[eight]) & (PAL[..., s][eight] <= hi[eight]))


def test_monotone_interpolation():
    # 8-value order e0, s2..s7, e1 ; 6-value order e0, s2..s5, e1
    order8 = [0, 2, 3, 4, 5, 6, 7, 1]
    order6 = [0, 2, 3, 4, 5, 1]
    e = np.arange(-127, 128)
    e0 = np.broadcast_to(e[None, :], (255, 255))
    e1 = np.broadcast_to(e[:, None], (255, 255))
    seq8 = PAL[..., order8][e0 > e1]
    seq6 = PAL[..., order6][e0 < e1]
    assert np.all(np.diff(seq8, axis=1) <= 0)      # e0 > e1: non-increasing
    assert np.all(np.diff(seq6, axis=1) >= 0)      # e0 < e1: non-decreasing


def test_equal_endpoints_give_flat_palette():
    for e in (-127, -1, 0, 5, 127):
        row = PAL[e + 127, e + 127]
        assert np.all(row[:6] == _cr(Fraction(e, 127)))


def test_c_and_numpy_restatements_agree_bitwise():
    c = clib.palette()
    assert np.array_equal(c.view(np.uint32), PAL.view(np.uint32))


def test_palette_sha_is_stable():
    # Golden value of this build's palette; a change here changes every artifact's hash gate.
    assert bc4.palette_sha256() == "bd14120748c07e65ab6da1e4c36ac4de90ab1005e2a3970e9bdc4ddf2be86fdf"


@pytest.mark.parametrize("bits,expected", [
    (0x3F800000, 0x3F80), (0x3F808000, 0x3F80), (0x3F818000, 0x3F82), (0x3F80FFFF, 0x3F81),
    (0xBF808001, 0xBF81), (0x00000000, 0x0000), (0x80000000, 0x8000),
])
def test_bf16_round_to_nearest_even(bits, expected):
    v = np.array([bits], dtype=np.uint32).view(np.float32)
    assert int(bc4.f32_to_bf16_bits(v)[0]) == expected


def _blocks(m, k, seed):
    from tests.helpers import random_blocks
    return random_blocks(m, k, seed)


def test_fp16_path_weights_are_the_fp32_products():
    """decode_f32_weights is the fp32 product P * scale: with a power-of-two scale it is the
    palette value scaled exactly, and its bf16 rounding is the BF16 path's decoded weight."""
    m, k = 24, 256
    blocks = _blocks(m, k, 301)
    pal = bc4.decode_f32_palette(blocks, m)
    exact = bc4.decode_f32_weights(blocks, np.full(m, 0.125, np.float32))
    assert np.array_equal(exact, pal / np.float32(8))
    scales = (0.02 * np.exp(0.3 * np.random.default_rng(302).standard_normal(m))).astype(np.float32)
    w = bc4.decode_f32_weights(blocks, scales)
    assert np.array_equal(bc4.f32_to_bf16_bits(w), bc4.decode_bf16_bits(blocks, scales))


def test_fp16_weights_round_to_nearest_even():
    """Each fp16 weight is a nearest fp16 value of the fp32 product, and an exact tie picks the
    even significand -- checked from the fp16 neighbours, not by converting again."""
    m, k = 32, 512
    blocks = _blocks(m, k, 303)
    scales = (0.5 * np.exp(np.random.default_rng(304).standard_normal(m))).astype(np.float32)
    w = bc4.decode_f32_weights(blocks, scales).astype(np.float64).ravel()
    bits = bc4.decode_f16_bits(blocks, scales).ravel()
    h = bits.view(np.float16)
    up = np.nextafter(h, np.float16(np.inf)).astype(np.float64)
    down = np.nextafter(h, np.float16(-np.inf)).astype(np.float64)
    hv = h.astype(np.float64)
    err = np.abs(w - hv)
    assert np.all(err <= np.abs(w - up)) and np.all(err <= np.abs(w - down))
    ties = (err == np.abs(w - up)) | (err == np.abs(w - down))
    ties &= err > 0
    assert np.all((bits[ties] & 1) == 0)
    # a hand-made tie: 1 + 2^-11 lies halfway between 1 and 1 + 2^-10 and rounds to 1
    assert np.float32(1 + 2 ** -11).astype(np.float16) == np.float16(1.0)
