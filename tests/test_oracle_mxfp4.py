"""CPU pins of the MXFP4 restatement (oracle/mxfp4.py) against the OCP MX specification's
definitions, worked by hand: E2M1 grid round trips and ties-to-even midpoints, group scales from
the largest magnitude, saturation, the dequantization error bound, and the float64 GEMM."""
from __future__ import annotations

import numpy as np

from oracle import mxfp4


def test_e2m1_codes_round_trip_and_midpoints_round_to_even():
    for code in range(16):
        value = mxfp4.e2m1_value(np.array([code]))
        if code == 8:  # -0 keeps its sign bit
            assert mxfp4.e2m1_codes(np.array([-0.0]))[0] == 8
            continue
        assert mxfp4.e2m1_codes(value)[0] == code
    # midpoints between neighbouring magnitudes: the even code (even mantissa bit) wins
    midpoints = [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]
    expected = [0, 2, 2, 4, 4, 6, 6]
    assert mxfp4.e2m1_codes(np.array(midpoints)).tolist() == expected
    assert mxfp4.e2m1_codes(-np.array(midpoints)).tolist() == [c | 8 for c in expected]
    # just off the midpoints: the nearest value
    assert mxfp4.e2m1_codes(np.array([0.2500001, 0.7499999, 4.9999, 5.0001])).tolist() == [1, 1, 6, 7]
    # saturation at 6
    assert mxfp4.e2m1_codes(np.array([6.0, 7.9, 1e30, -100.0])).tolist() == [7, 7, 7, 15]


def _group(values):
    out = np.zeros(32, dtype=np.float32)
    out[: len(values)] = values
    return out[None, :]


def test_group_scale_from_the_largest_magnitude():
    # amax 6 -> floor(log2 6) = 2 -> X = 2^0, e = 127: values quantize on the plain grid
    codes, e = mxfp4.quantize(_group([6.0, 3.0, -0.25, 0.75, -1.75, 5.0]))
    assert e.tolist() == [[127]]
    assert codes[0, :6].tolist() == [7, 5, 8, 2, 12, 6]
    # amax 7 -> X = 1 too; 7 saturates to 6
    codes, e = mxfp4.quantize(_group([7.0, -7.0]))
    assert e.tolist() == [[127]] and codes[0, :2].tolist() == [7, 15]
    # amax 8 -> floor(log2 8) = 3 -> X = 2, e = 128: 8/2 = 4 (code 6), 1/2 = 0.5 (code 1),
    # -3/2 = -1.5 (code 3 with the sign bit)
    codes, e = mxfp4.quantize(_group([8.0, 1.0, -3.0]))
    assert e.tolist() == [[128]] and codes[0, :3].tolist() == [6, 1, 11]


def test_group_scale_edge_cases():
    # amax 0.75 -> floor(log2 0.75) = -1 -> X = 2^-3, e = 124: 0.75 / 0.125 = 6 (code 7)
    codes, e = mxfp4.quantize(_group([0.75, 0.1]))
    assert e.tolist() == [[124]] and codes[0, 0] == 7
    assert mxfp4.dequantize(codes, e)[0, 1] == 0.125  # 0.1/0.125 = 0.8 -> nearest 1.0
    # all-zero group: e = 0, codes zero
    codes, e = mxfp4.quantize(np.zeros((2, 64), dtype=np.float32))
    assert e.tolist() == [[0, 0], [0, 0]] and not codes.any()


def test_dequantization_error_bound_and_packing():
    rng = np.random.default_rng(5)
    values = (rng.standard_normal((8, 256)) * np.exp(rng.standard_normal((8, 1)))).astype(np.float32)
    codes, e = mxfp4.quantize(values)
    deq = mxfp4.dequantize(codes, e)
    x = np.ldexp(1.0, np.repeat(e.astype(np.int64), 32, axis=-1) - 127)
    # below the saturation point (6X) the error is at most half the grid step at that magnitude
    # (at most 2X for values in [4X, 6X)); every group's largest value is below 8X
    assert np.all(np.abs(values) < 8 * x)
    step = np.where(np.abs(values) < 2 * x, 0.5 * x, np.where(np.abs(values) < 4 * x, x, 2 * x))
    inside = np.abs(values) <= 6 * x
    assert np.all(np.abs(values - deq)[inside] <= step[inside] / 2 + 1e-30)
    assert np.all(np.abs(deq[~inside]) == 6 * x[~inside])
    assert np.array_equal(mxfp4.unpack(mxfp4.pack(codes)), codes)
    assert mxfp4.pack(np.array([[1, 2, 15, 8]], dtype=np.uint8)).tolist() == [[0x21, 0x8F]]


def test_gemm_f64_is_the_dequantized_product():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((3, 64)).astype(np.float32)
    w = rng.standard_normal((5, 64)).astype(np.float32)
    xc, xe = mxfp4.quantize(x)
    wc, we = mxfp4.quantize(w)
    y = mxfp4.gemm_f64(xc, xe, wc, we)
    dx, dw = mxfp4.dequantize(xc, xe), mxfp4.dequantize(wc, we)
    direct = np.array([[sum(dx[t, k] * dw[m, k] for k in range(64)) for m in range(5)] for t in range(3)])
    assert np.allclose(y, direct, rtol=1e-12, atol=0)
