"""GPU parity of the dense-scratch prefill backend (the reference's backend 1,
``texelator/cuda/texelator_cuda.cu:937-990``): rows decoded ``tile_rows`` at a time into the
caller's workspace, one hipBLASLt GEMM per row tile, the bias added afterwards with a second
rounding (``:982-989``). The workspace holds the decoded rows and 8 MiB for the library GEMM.

Bars: within 1e-2 relative RMS of the float64 CPU GEMM on the oracle's decoded weights (the
library GEMM accumulates in its own order, so it is not bitwise equal to the tile candidates);
the biased output is exactly round(unbiased + bias); LUT-mode decode with the device palette gives
bitwise the same output; the workspace is min(tile_rows, M) decoded rows plus the GEMM's 8 MiB.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import bc4, clib
from tests.helpers import bf16_bits, bf16_vector, f16_vector, lognormal_scales, random_blocks

pytestmark = pytest.mark.gpu

PREFILL_RRMS_TOL = 1e-2
DENSE = 1


def _pack(ext, blocks, scales, bias=None):
    return ext.pack_encoded(torch.from_numpy(np.ascontiguousarray(blocks).reshape(-1)),
                            torch.from_numpy(np.ascontiguousarray(scales)), bias)


def _dense(ext, handle, tile_rows):
    ext.set_prefill(handle, 16, tile_rows)
    ext.set_prefill_backend(handle, DENSE)


@pytest.mark.parametrize("m,k,tokens,tile_rows", [(200, 1280, 40, 64), (300, 2064, 129, 1024), (96, 27648, 32, 48)])
def test_dense_backend_matches_oracle_with_row_tiles(ext, oracle_threads, m, k, tokens, tile_rows):
    blocks = random_blocks(m, k, 701)
    scales = lognormal_scales(m, 702)
    x = (bf16_vector((tokens, k), 703).float() * 0.125).to(torch.bfloat16)
    bias = bf16_vector((m,), 704, scale=0.1)
    plain = _pack(ext, blocks, scales)
    biased = _pack(ext, blocks, scales, bias.cuda())
    try:
        for handle in (plain, biased):
            _dense(ext, handle, tile_rows)
        assert ext.handle_info(plain)[3:5] == [tile_rows, DENSE]
        rows = min(tile_rows, m)
        assert ext.workspace_bytes(plain, tokens) == (rows * k * 2 + 255) // 256 * 256 + 256 + (8 << 20)
        y0 = ext.linear(plain, x.cuda())
        y1 = ext.linear(biased, x.cuda())
        tile = ext.prefill(plain, 6, x.cuda())
        torch.cuda.synchronize()
    finally:
        ext.free(plain)
        ext.free(biased)
    assert torch.equal(y1, (y0.float() + bias.cuda().float()[None, :]).to(torch.bfloat16))
    w = clib.decode_bf16_bits(blocks, scales)
    ref = clib.gemm_f64(bf16_bits(x), w)
    assert bc4.relative_rms(ref, y0.float().cpu().numpy()) <= PREFILL_RRMS_TOL
    assert bc4.relative_rms(ref + bias.float().numpy()[None, :], y1.float().cpu().numpy()) <= PREFILL_RRMS_TOL
    # the tile kernels and the library GEMM agree to a few bf16 ulps
    assert bc4.relative_rms(tile.float().cpu().numpy(), y0.float().cpu().numpy()) <= 4e-3


def test_dense_backend_f16(ext, oracle_threads):
    m, k, tokens = 160, 1280, 33
    blocks = random_blocks(m, k, 711)
    scales = lognormal_scales(m, 712)
    x = f16_vector((tokens, k), 713, scale=0.125)
    bias = f16_vector((m,), 714, scale=0.1)
    plain = _pack(ext, blocks, scales)
    biased = _pack(ext, blocks, scales, bias.cuda())
    try:
        for handle in (plain, biased):
            _dense(ext, handle, 64)
        y0 = ext.linear(plain, x.cuda())
        y1 = ext.linear(biased, x.cuda())
        torch.cuda.synchronize()
    finally:
        ext.free(plain)
        ext.free(biased)
    assert y0.dtype == torch.float16
    assert torch.equal(y1, (y0.float() + bias.cuda().float()[None, :]).to(torch.float16))
    w = bc4.decode_f16_bits(blocks, scales).view(np.float16).astype(np.float64)
    ref = x.double().numpy() @ w.T
    assert bc4.relative_rms(ref, y0.double().cpu().numpy()) <= PREFILL_RRMS_TOL


def test_dense_backend_lut_mode_agrees(ext):
    """LUT-mode decode with the device's own palette feeds the GEMM the same weights."""
    m, k, tokens = 256, 2048, 64
    blocks = random_blocks(m, k, 721)
    scales = lognormal_scales(m, 722)
    x = bf16_vector((tokens, k), 723, scale=0.125).cuda()
    handle = _pack(ext, blocks, scales)
    table = ext.palette_probe().reshape(-1).cuda()
    try:
        _dense(ext, handle, 128)
        plain = ext.linear(handle, x)
        torch.cuda.synchronize()
        ext.set_palette_table(handle, table)
        lut = ext.linear(handle, x)
        torch.cuda.synchronize()
    finally:
        ext.free(handle)
    assert torch.equal(plain, lut)


def test_dense_backend_below_threshold_uses_gemv(ext):
    """Calls below the prefill threshold keep the GEMV whatever the backend."""
    m, k = 64, 512
    blocks = random_blocks(m, k, 731)
    scales = lognormal_scales(m, 732)
    x = bf16_vector((1, k), 733).cuda()
    handle = _pack(ext, blocks, scales)
    try:
        before = ext.linear(handle, x)
        _dense(ext, handle, 64)
        after = ext.linear(handle, x)
        torch.cuda.synchronize()
    finally:
        ext.free(handle)
    assert torch.equal(before, after)
