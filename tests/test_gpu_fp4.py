"""GPU parity of the FP4 hybrid prefill staging and GEMM (MXFP4 on gfx950) against the oracle's
restatement of the OCP MX format (oracle/mxfp4.py).

Reference: ``texelator/runtime.py:66-131`` (the opt-in hybrid), ``texelator_cuda.cu:1046-1260``
(the quantizers, NVFP4 there). Bars: the activation and weight quantizers bitwise equal to the
oracle (codes and E8M0 scales); the block-scaled GEMM within bf16 rounding of the float64 product
of the dequantized operands (a wrong operand layout or scale placement is off by O(1)); the bias
added with a second rounding; the hybrid dispatch bitwise equal to the explicit pipeline.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import bc4, mxfp4
from texelator_amd import runtime
from tests.helpers import bf16_vector, lognormal_scales, random_blocks

pytestmark = pytest.mark.gpu


def _pack(ext, blocks, scales, bias=None):
    return ext.pack_encoded(torch.from_numpy(np.ascontiguousarray(blocks).reshape(-1)),
                            torch.from_numpy(np.ascontiguousarray(scales)), bias)


def _activations(tokens, k, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((tokens, k)) * np.exp(1.5 * rng.standard_normal((tokens, 1)))
    x[0, :64] = 0.0                      # an all-zero group
    if tokens > 1:
        x[1, :32] = [6.0, 3.0, -0.25, 0.75, -1.75, 5.0, 7.0, -8.0] * 4   # midpoints and saturation
        x[1, 32:64] = 1e-40              # subnormal group maximum
    return torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16)


@pytest.mark.parametrize("tokens,k", [(1, 64), (37, 1024), (130, 5120)])
def test_activation_quantizer_bitwise(ext, tokens, k):
    x = _activations(tokens, k, 801)
    packed, scales = ext.quantize_activation_fp4(x.cuda())
    torch.cuda.synchronize()
    codes, exponents = mxfp4.quantize(x.float().numpy())
    assert np.array_equal(scales.cpu().numpy(), exponents)
    assert np.array_equal(packed.cpu().numpy(), mxfp4.pack(codes))


@pytest.mark.parametrize("m,k", [(16, 128), (37, 1024), (300, 2048)])
def test_weight_quantizer_bitwise(ext, m, k):
    blocks = random_blocks(m, k, 811)
    scales = lognormal_scales(m, 812)
    handle = _pack(ext, blocks, scales)
    try:
        packed, group_scales = ext.decode_weight_fp4(handle)
        torch.cuda.synchronize()
    finally:
        ext.free(handle)
    codes, exponents = mxfp4.quantize(bc4.decode_f32_weights(blocks, scales))
    assert np.array_equal(group_scales.cpu().numpy(), exponents)
    assert np.array_equal(packed.cpu().numpy(), mxfp4.pack(codes))


def test_weight_quantizer_reads_the_palette_table_in_lut_mode(ext):
    """A LUT-mode handle (another GPU's palette) quantizes the products of ITS table's values, as
    every other kernel of that handle decodes them: bitwise the oracle on the table's palette, and
    different from the arithmetic palette's codes (so a quantizer that ignored the table fails)."""
    from tests.test_gpu_lut import foreign_palette

    m, k = 300, 2048
    blocks = random_blocks(m, k, 815)
    scales = lognormal_scales(m, 816)
    lut = foreign_palette(17)
    handle = _pack(ext, blocks, scales)
    try:
        ext.set_palette_table(handle, torch.from_numpy(lut.reshape(-1)).cuda())
        packed, group_scales = ext.decode_weight_fp4(handle)
        torch.cuda.synchronize()
    finally:
        ext.free(handle)
    codes, exponents = mxfp4.quantize(bc4.decode_f32_weights(blocks, scales, lut))
    assert np.array_equal(group_scales.cpu().numpy(), exponents)
    assert np.array_equal(packed.cpu().numpy(), mxfp4.pack(codes))
    plain, _ = mxfp4.quantize(bc4.decode_f32_weights(blocks, scales))
    assert not np.array_equal(mxfp4.pack(plain), mxfp4.pack(codes))


@pytest.mark.parametrize("tokens,m,k", [(1, 64, 64), (37, 200, 1024), (130, 300, 5120), (256, 128, 128)])
def test_fp4_gemm_matches_dequantized_product(ext, tokens, m, k):
    x = _activations(tokens, k, 821)
    w = _activations(m, k, 822)
    xc, xe = mxfp4.quantize(x.float().numpy())
    wc, we = mxfp4.quantize(w.float().numpy())
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    bias = bf16_vector((m,), 823, scale=0.5)
    y = ext.fp4_gemm(dev(mxfp4.pack(xc)), dev(xe), dev(mxfp4.pack(wc)), dev(we))
    yb = ext.fp4_gemm(dev(mxfp4.pack(xc)), dev(xe), dev(mxfp4.pack(wc)), dev(we), bias=bias.cuda())
    torch.cuda.synchronize()
    ref = mxfp4.gemm_f64(xc, xe, wc, we)
    got = y.double().cpu().numpy()
    # one bf16 rounding of an fp32 sum: within 2^-8 of each value plus the fp32 accumulation error
    scale = np.abs(mxfp4.dequantize(xc, xe)) @ np.abs(mxfp4.dequantize(wc, we)).T
    assert np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-4 * scale + 1e-38)
    assert torch.equal(yb, (y.float() + bias.cuda().float()[None, :]).to(torch.bfloat16))


@pytest.mark.parametrize("tokens,m,k", [(37, 200, 1024), (130, 300, 5120), (256, 128, 128)])
def test_fp4_gemm_staged_and_direct_kernels_agree_bitwise(ext, tokens, m, k):
    """K a multiple of 128 with word-aligned scales takes the LDS-staged kernel; the same scales one
    byte off a word boundary take the direct kernel. Same MFMAs in the same K order: same bits."""
    x = _activations(tokens, k, 841)
    w = _activations(m, k, 842)
    xc, xe = mxfp4.quantize(x.float().numpy())
    wc, we = mxfp4.quantize(w.float().numpy())
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()

    def shifted(scales):  # the same bytes at an address one past a word boundary
        flat = torch.empty(scales.size + 4, dtype=torch.uint8, device="cuda")
        view = flat[1:1 + scales.size].view(scales.shape)
        view.copy_(dev(scales))
        return view

    xp, wp = dev(mxfp4.pack(xc)), dev(mxfp4.pack(wc))
    staged = ext.fp4_gemm(xp, dev(xe), wp, dev(we))
    direct = ext.fp4_gemm(xp, shifted(xe), wp, shifted(we))
    assert torch.equal(staged, direct)


@pytest.mark.parametrize("m,k", sorted(runtime.FP4_HYBRID_SHAPES))
def test_fp4_hybrid_dispatch_on_a_reference_shape(ext, m, k):
    """At 512 tokens on the reference's MLP shapes the hybrid runs the explicit pipeline (bitwise)
    and stays within FP4 quantization error of the bf16 prefill of the same weights; at 511 tokens
    the same handle keeps the bf16 prefill, bit for bit."""
    tokens = runtime.FP4_HYBRID_TOKENS
    blocks = random_blocks(m, k, 831 + m)
    scales = lognormal_scales(m, 832 + m)
    x = bf16_vector((tokens, k), 833 + m, scale=0.5).cuda()
    x511 = x[:tokens - 1].contiguous()
    handle = _pack(ext, blocks, scales)
    try:
        exact = runtime._linear_dispatch(handle, x)
        exact511 = ext.linear(handle, x511)
        runtime.set_fp4_hybrid(True)
        hybrid = runtime._linear_dispatch(handle, x)
        hybrid511 = runtime._linear_dispatch(handle, x511)
        xp, xs = ext.quantize_activation_fp4(x)
        wp, ws = ext.decode_weight_fp4(handle)
        explicit = ext.fp4_gemm(xp, xs, wp, ws)
        torch.cuda.synchronize()
    finally:
        runtime.free([handle])
    assert not runtime._Fp4State.enabled
    assert torch.equal(hybrid, explicit)
    assert torch.equal(hybrid511, exact511)
    assert bc4.relative_rms(exact.double().cpu().numpy(), hybrid.double().cpu().numpy()) <= 0.3


def test_fp4_errors(ext):
    with pytest.raises(RuntimeError, match="divisible by 32"):
        ext.quantize_activation_fp4(torch.zeros((2, 48), dtype=torch.bfloat16, device="cuda"))
    z = torch.zeros((4, 16), dtype=torch.uint8, device="cuda")
    s = torch.zeros((4, 1), dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError, match="multiple of 64"):
        ext.fp4_gemm(z, s, z, s)
