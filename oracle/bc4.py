"""numpy restatement of the BC4 weight path (test infrastructure only; see package header).

Reference anchors (paths relative to the reference checkout):

* block format -- ``texelator/encoder.py:105-117`` (``pack_blocks``): byte 0 = e0 (int8),
  byte 1 = e1 (int8), bytes 2..7 = 48-bit little-endian selector field, selector of
  position ``p`` at bits ``3p..3p+2``; position ``p`` of block ``b`` is input column
  ``16*b + p`` (``texelator/cuda/texelator_cuda.cu:127-131``, ``p = 4*qy + qx``).
* palette layout -- ``texelator/encoder.py:11-20``: ``lut[e1 + 127][e0 + 127][s]``,
  255 x 255 x 8 little-endian float32, as written by the probe
  (``texelator/cuda/texelator_cuda.cu:1542-1595``: ``out[(y*255 + x)*8 + s]``, x = e0+127).
* decoded weight -- ``texelator/cuda/texelator_cuda.cu:141-152``:
  ``bf16_rne(palette_value * scale[row])`` with an fp32 product.
* FP16 path -- the FP16 GEMV multiplies the unrounded fp32 product ``palette_value * scale``
  by the fp16 activation (``texelator_cuda.cu:75-83``, ``:94-139``); the FP16 prefill decodes
  ``fp16_rne(palette_value * scale)`` into its scratch matrix (``texelator_cuda.cu:604-628``).
* error metrics -- ``texelator/autotune.py:63-76`` and ``texelator/prefill.py:94-105``.

Palette definition (this build's; the reference's palette is measured from NVIDIA texture
hardware and is not reproducible, so the LUT itself is defined here):

* ``e0, e1`` are the signed endpoint bytes clamped to [-127, 127] (BC4 SNORM maps -128 to -1).
* ``base = RN(e0/127)``, ``end = RN(e1/127)`` (correctly rounded fp32).
* 8-value mode (``e0 > e1``): ``step = RN((e1-e0)/889)``; ``P[0]=base``, ``P[1]=end``,
  ``P[s] = fma_f32(s-1, step, base)`` for s = 2..7.
* 6-value mode (``e0 <= e1``): ``step = RN((e1-e0)/635)``; ``P[0]=base``, ``P[1]=end``,
  ``P[s] = fma_f32(s-1, step, base)`` for s = 2..5, ``P[6] = -1``, ``P[7] = +1``.

889 = 7*127 and 635 = 5*127, so ``P[s]`` approximates the BC4 interpolant
``((8-s)e0 + (s-1)e1)/7/127`` (resp. ``/5/127``) to within a few fp32 ulps.
"""
from __future__ import annotations

import hashlib
import math

import numpy as np

PAIRS = 255 * 255
PALETTE_SHAPE = (255, 255, 8)


# --------------------------------------------------------------------------------------
# fp32 helpers
# --------------------------------------------------------------------------------------

def crdiv_f32(numerator: np.ndarray, denominator) -> np.ndarray:
    """Correctly rounded float32 of ``numerator / denominator`` for small integers.

    The float64 quotient is correctly rounded; converting it to float32 can only
    double-round if the exact quotient lies within 2**-53 (relative) of a float32
    midpoint. For |n| <= 889 and odd D in {127, 635, 889} the exact quotient is either
    dyadic (D | n, no rounding at all) or at least ~2**-35 (relative) away from every
    midpoint, so the two-step conversion is exact. Pinned by
    ``tests/test_oracle_palette.py`` against ``fractions.Fraction``.
    """
    return (np.asarray(numerator, dtype=np.float64) / np.asarray(denominator, dtype=np.float64)).astype(np.float32)


def fma_f32(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """float32 fused multiply-add for the palette's operand ranges.

    ``a`` is a small integer (<= 6, 3 significant bits), ``b`` and ``c`` are float32 with
    |b| <= 0.4, |c| <= 1. The float64 expression ``a*b + c`` is then exact (at most ~37
    significant bits), so one rounding to float32 equals the fused operation.
    """
    return (np.asarray(a, np.float64) * np.asarray(b, np.float32).astype(np.float64)
            + np.asarray(c, np.float32).astype(np.float64)).astype(np.float32)


def f32_to_bf16_bits(values: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 (round-to-nearest-even), returning the uint16 bit patterns.

    Restates ``__float2bfloat16`` (RNE, ``cutlass/bfloat16.h:116-120``) for finite inputs.
    """
    bits = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# --------------------------------------------------------------------------------------
# palette
# --------------------------------------------------------------------------------------

def palette_values(e0: np.ndarray, e1: np.ndarray) -> np.ndarray:
    """Palette rows for (already clamped) endpoint arrays; returns ``shape + (8,)`` float32."""
    e0 = np.asarray(e0, dtype=np.int64)
    e1 = np.asarray(e1, dtype=np.int64)
    e0, e1 = np.broadcast_arrays(e0, e1)
    eight = e0 > e1
    base = crdiv_f32(e0, 127)
    end = crdiv_f32(e1, 127)
    step = crdiv_f32(e1 - e0, np.where(eight, 889, 635))
    out = np.empty(e0.shape + (8,), dtype=np.float32)
    out[..., 0] = base
    out[..., 1] = end
    for s in range(2, 8):
        out[..., s] = fma_f32(s - 1, step, base)
    out[..., 6] = np.where(eight, out[..., 6], np.float32(-1.0))
    out[..., 7] = np.where(eight, out[..., 7], np.float32(1.0))
    return out


def palette() -> np.ndarray:
    """The full 255 x 255 x 8 LUT, indexed ``[e1 + 127][e0 + 127][s]`` (``encoder.py:19-20``)."""
    e = np.arange(-127, 128, dtype=np.int64)
    return palette_values(e[None, :], e[:, None])


def palette_bytes() -> bytes:
    return palette().astype("<f4", copy=False).tobytes()


def palette_sha256() -> str:
    return hashlib.sha256(palette_bytes()).hexdigest()


# --------------------------------------------------------------------------------------
# block codec
# --------------------------------------------------------------------------------------

def pack_blocks(e0: np.ndarray, e1: np.ndarray, sel: np.ndarray) -> np.ndarray:
    """Pack endpoints ``[N]`` and selectors ``[N,16]`` into ``[N,8]`` uint8 blocks (``encoder.py:105-117``)."""
    sel = np.asarray(sel, dtype=np.uint64)
    bits = np.zeros(sel.shape[0], dtype=np.uint64)
    for p in range(16):
        bits |= (sel[:, p] & 7) << np.uint64(3 * p)
    out = np.empty((sel.shape[0], 8), dtype=np.uint8)
    out[:, 0] = np.asarray(e0, dtype=np.int64).astype(np.int8).view(np.uint8)
    out[:, 1] = np.asarray(e1, dtype=np.int64).astype(np.int8).view(np.uint8)
    for byte in range(6):
        out[:, 2 + byte] = ((bits >> np.uint64(8 * byte)) & np.uint64(255)).astype(np.uint8)
    return out


def unpack_blocks(blocks: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Inverse of :func:`pack_blocks`: raw int8 endpoints and ``[N,16]`` selectors."""
    blocks = np.asarray(blocks, dtype=np.uint8).reshape(-1, 8)
    e0 = blocks[:, 0].view(np.int8).astype(np.int16)
    e1 = blocks[:, 1].view(np.int8).astype(np.int16)
    bits = np.zeros(blocks.shape[0], dtype=np.uint64)
    for byte in range(6):
        bits |= blocks[:, 2 + byte].astype(np.uint64) << np.uint64(8 * byte)
    sel = np.empty((blocks.shape[0], 16), dtype=np.uint8)
    for p in range(16):
        sel[:, p] = ((bits >> np.uint64(3 * p)) & np.uint64(7)).astype(np.uint8)
    return e0, e1, sel


def clamp_endpoint(e: np.ndarray) -> np.ndarray:
    return np.maximum(np.asarray(e, dtype=np.int16), -127)


# --------------------------------------------------------------------------------------
# decoder and products
# --------------------------------------------------------------------------------------

def decode_f32_palette(blocks: np.ndarray, m: int, lut: np.ndarray | None = None) -> np.ndarray:
    """Palette value of every weight, ``[M, K]`` float32 (``encoder.actual_palette`` gather)."""
    lut = palette() if lut is None else lut
    e0, e1, sel = unpack_blocks(blocks)
    e0 = clamp_endpoint(e0).astype(np.int64)
    e1 = clamp_endpoint(e1).astype(np.int64)
    rows = lut[e1 + 127, e0 + 127]                 # [N, 8]
    vals = np.take_along_axis(rows, sel.astype(np.int64), axis=1)  # [N, 16]
    return vals.reshape(m, -1)


def decode_bf16_bits(blocks: np.ndarray, scales: np.ndarray, lut: np.ndarray | None = None) -> np.ndarray:
    """Decoded weights as bf16 bit patterns ``[M, K]``: ``bf16_rne(fp32(P * scale[m]))``."""
    scales = np.asarray(scales, dtype=np.float32)
    m = scales.shape[0]
    pal = decode_f32_palette(blocks, m, lut)
    prod = (pal * scales[:, None]).astype(np.float32)  # float32 * float32 -> correctly rounded
    return f32_to_bf16_bits(prod)


def decode_f32_weights(blocks: np.ndarray, scales: np.ndarray, lut: np.ndarray | None = None) -> np.ndarray:
    """Unrounded FP16-path weights ``fp32(P * scale[m])`` ``[M, K]`` (``texelator_cuda.cu:75-83``)."""
    scales = np.asarray(scales, dtype=np.float32)
    pal = decode_f32_palette(blocks, scales.shape[0], lut)
    return (pal * scales[:, None]).astype(np.float32)


def decode_f16_bits(blocks: np.ndarray, scales: np.ndarray, lut: np.ndarray | None = None) -> np.ndarray:
    """FP16 prefill weights as fp16 bit patterns ``[M, K]``: ``fp16_rne(fp32(P * scale[m]))``
    (``texelator_cuda.cu:624``, ``__float2half``)."""
    return decode_f32_weights(blocks, scales, lut).astype(np.float16).view(np.uint16)


def matvec_f64(w_bits: np.ndarray, x: np.ndarray) -> np.ndarray:
    """``y = W x`` in float64 on the decoded bf16 weights; ``x`` given as float values or bf16 bits."""
    w = bf16_bits_to_f32(w_bits).astype(np.float64)
    xv = _as_f64(x)
    return w @ xv


def gemm_f64(x: np.ndarray, w_bits: np.ndarray) -> np.ndarray:
    """``Y[T, M] = X[T, K] W[M, K]^T`` in float64."""
    w = bf16_bits_to_f32(w_bits).astype(np.float64)
    return _as_f64(x) @ w.T


def _as_f64(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x)
    if x.dtype == np.uint16:
        return bf16_bits_to_f32(x).astype(np.float64)
    return x.astype(np.float64)


# --------------------------------------------------------------------------------------
# metrics (texelator/autotune.py:63-76, texelator/prefill.py:94-105)
# --------------------------------------------------------------------------------------

def error_metrics(reference: np.ndarray, candidate: np.ndarray) -> dict:
    ref = np.asarray(reference, dtype=np.float64)
    val = np.asarray(candidate, dtype=np.float64)
    delta = val - ref
    ref_rms = math.sqrt(float(np.mean(ref * ref)))
    denom = math.sqrt(float(np.sum(ref * ref)) * float(np.sum(val * val)))
    return {
        "max_abs": float(np.max(np.abs(delta))),
        "mean_abs": float(np.mean(np.abs(delta))),
        "relative_rms": math.sqrt(float(np.mean(delta * delta))) / max(ref_rms, 1e-30),
        "cosine": float(np.sum(ref * val)) / max(denom, 1e-30),
        "bitwise_equal": bool(np.array_equal(np.asarray(reference), np.asarray(candidate))),
    }


def relative_rms(reference: np.ndarray, candidate: np.ndarray) -> float:
    return error_metrics(reference, candidate)["relative_rms"]


def relative_error(reference: np.ndarray, candidate: np.ndarray) -> float:
    """Norm-wise relative error ``||c - r|| / ||r||``."""
    ref = np.asarray(reference, dtype=np.float64)
    val = np.asarray(candidate, dtype=np.float64)
    return float(np.linalg.norm(val - ref) / max(np.linalg.norm(ref), 1e-300))
