"""numpy restatement of the FP4 hybrid prefill's formats -- TEST INFRASTRUCTURE ONLY (see the
package header): only tests may import it, as the checker.

Reference anchors (paths relative to the reference checkout):

* ``texelator/runtime.py:66-131`` -- the opt-in hybrid: at 512 tokens, for the MLP shapes, the
  activation and the decoded BC4 weight are quantized to FP4 and multiplied by a block-scaled
  FP4 GEMM (``torch._scaled_mm``, bf16 output, no bias).
* ``texelator/cuda/texelator_cuda.cu:1046-1152`` -- the quantizers: E2M1 values
  ``{0, 0.5, 1, 1.5, 2, 3, 4, 6}`` with the sign in bit 3, two values per byte (low nibble
  first), and a scale per group of 16 (NVFP4: E4M3 ``max/6``). The weight quantizer starts from
  the fp32 products ``palette * row scale`` (before any 16-bit rounding).

gfx950's block-scaled MFMA (``v_mfma_scale_f32_32x32x64_f8f6f4``) takes the OCP MX format
instead (Microscaling Formats Specification v1.0, section 6.3): E2M1 values as above and one
E8M0 scale (a power of two, ``2^(e - 127)``) per group of 32. This module defines MXFP4 as that
specification does:

* ``X = 2^(floor(log2(amax)) - 2)`` per group (2 = the largest E2M1 exponent), stored as
  ``e = floor(log2(amax)) - 2 + 127`` clamped to [0, 254]; an all-zero group stores e = 0;
* each value ``v / X`` rounded to E2M1 to nearest, ties to even (the code with an even mantissa
  bit), saturating at 6; the sign bit is the sign of v (a negative value that rounds to zero is
  code 8, -0).

Parity pins (tests/test_oracle_mxfp4.py): every E2M1 code round-trips, every midpoint between
neighbouring magnitudes rounds to the even code, hand-computed groups (scales from amax 6, 7, 8,
0.75 and 0; saturation), the dequantized error bound |v - deq(v)| <= X/2 below saturation, and
``gemm_f64`` against a direct sum.
"""
from __future__ import annotations

import numpy as np

GROUP = 32
E2M1_VALUES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def e2m1_codes(values: np.ndarray) -> np.ndarray:
    """Nearest E2M1 code (ties to even, saturating at 6) of each value, sign in bit 3."""
    v = np.asarray(values, dtype=np.float64)
    magnitude = np.abs(v)
    # distance to every grid point; ties broken towards the even code (lowest set of equal
    # distances among codes 0, 2, 4, 6 wins over 1, 3, 5, 7)
    distance = np.abs(magnitude[..., None] - E2M1_VALUES)
    best = distance.min(axis=-1, keepdims=True)
    candidates = distance == best
    even = candidates & (np.arange(8) % 2 == 0)
    pick = np.where(even.any(axis=-1), np.argmax(even, axis=-1), np.argmax(candidates, axis=-1))
    code = np.where(magnitude >= 6.0, 7, pick).astype(np.uint8)
    return code | np.where(np.signbit(v), 8, 0).astype(np.uint8)


def e2m1_value(codes: np.ndarray) -> np.ndarray:
    codes = np.asarray(codes, dtype=np.uint8)
    return np.where(codes & 8, -1.0, 1.0) * E2M1_VALUES[codes & 7]


def group_exponents(values: np.ndarray) -> np.ndarray:
    """E8M0 exponent of each group of 32 along the last axis (float32 inputs)."""
    v = np.asarray(values, dtype=np.float32)
    groups = v.reshape(*v.shape[:-1], v.shape[-1] // GROUP, GROUP)
    amax = np.abs(groups).max(axis=-1).astype(np.float64)
    _, exponent = np.frexp(amax)          # amax = f * 2^exponent, f in [0.5, 1): floor(log2) = exponent - 1
    e = np.where(amax > 0, exponent - 1 - 2 + 127, 0)
    return np.clip(e, 0, 254).astype(np.uint8)


def quantize(values: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """MXFP4 of ``values`` [..., K] (K a multiple of 32): (codes [..., K] uint8, E8M0 [..., K/32])."""
    v = np.asarray(values, dtype=np.float32)
    if v.shape[-1] % GROUP:
        raise ValueError("the last dimension must be a multiple of 32")
    e = group_exponents(v)
    scale = np.ldexp(1.0, 127 - np.repeat(e.astype(np.int64), GROUP, axis=-1))  # 1 / X, exact
    return e2m1_codes(v.astype(np.float64) * scale), e


def dequantize(codes: np.ndarray, exponents: np.ndarray) -> np.ndarray:
    x = np.ldexp(1.0, np.repeat(exponents.astype(np.int64), GROUP, axis=-1) - 127)
    return e2m1_value(codes) * x


def pack(codes: np.ndarray) -> np.ndarray:
    """Two codes per byte, even column in the low nibble (texelator_cuda.cu:1101-1105)."""
    c = np.asarray(codes, dtype=np.uint8)
    return (c[..., 0::2] | (c[..., 1::2] << 4)).astype(np.uint8)


def unpack(packed: np.ndarray) -> np.ndarray:
    p = np.asarray(packed, dtype=np.uint8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = p & 15
    out[..., 1::2] = p >> 4
    return out


def gemm_f64(x_codes, x_exponents, w_codes, w_exponents) -> np.ndarray:
    """y[t][m] = sum_k deq(x)[t][k] * deq(w)[m][k] in float64."""
    return dequantize(x_codes, x_exponents) @ dequantize(w_codes, w_exponents).T
