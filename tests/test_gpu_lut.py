"""LUT-mode decode on the GPU: every kernel reading its block palettes from a table
(``tx_set_palette_table``) instead of computing this build's palette.

The tables used are a perturbed copy of the defined palette (no closed form can reproduce it,
so a kernel that ignored the table would fail) and the defined palette itself (the table path
must then agree bit for bit with the arithmetic path). The checker is the oracle's LUT gather
``decode_f32_palette(blocks, m, lut)``, the reference's ``actual_palette`` (``encoder.py:19-20``).
"""
from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from oracle import bc4
from tests.helpers import (bf16_bits, bf16_vector, f16_vector, lognormal_scales, max_rel_err_floor, random_blocks,
                           rel_err)
from texelator_amd import artifacts, hardware, runtime

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-3
PREFILL_RRMS_TOL = 1e-2


def foreign_palette(seed: int = 7) -> np.ndarray:
    """A palette no arithmetic decoder reproduces: the defined one with 1% noise on every value."""
    rng = np.random.default_rng(seed)
    lut = bc4.palette()
    return (lut * (1 + 0.01 * rng.standard_normal(lut.shape))).astype(np.float32)


def _pack(ext, blocks, scales, table=None, bias=None):
    handle = ext.pack_encoded(torch.from_numpy(np.ascontiguousarray(blocks).reshape(-1)),
                              torch.from_numpy(np.ascontiguousarray(scales)), bias)
    if table is not None:
        ext.set_palette_table(handle, torch.from_numpy(table).cuda())
    return handle


def lut_weights_f32(blocks, scales, lut):
    pal = bc4.decode_f32_palette(blocks, scales.shape[0], lut)
    return (pal * scales[:, None]).astype(np.float32)


@pytest.mark.parametrize("m,k,seed", [(16, 128, 501), (37, 272, 502), (64, 4096, 503)])
def test_lut_decode_dense_bit_exact(ext, m, k, seed):
    lut = foreign_palette(seed)
    blocks = random_blocks(m, k, seed)
    scales = lognormal_scales(m, seed + 1)
    handle = _pack(ext, blocks, scales, lut)
    try:
        got16 = bf16_bits(ext.decode_dense(handle).cpu())
        gotf16 = ext.decode_dense(handle, torch.float16).cpu().view(torch.int16).numpy().view(np.uint16)
    finally:
        ext.free(handle)
    assert np.array_equal(got16, bc4.decode_bf16_bits(blocks, scales, lut))
    assert np.array_equal(gotf16, lut_weights_f32(blocks, scales, lut).astype(np.float16).view(np.uint16))
    # and the table really was used: the defined palette decodes these blocks differently
    assert not np.array_equal(got16, bc4.decode_bf16_bits(blocks, scales))


def test_defined_palette_as_table_is_bitwise_the_arithmetic_path(ext):
    m, k = 300, 2064
    blocks = random_blocks(m, k, 511)
    scales = lognormal_scales(m, 512)
    x1 = bf16_vector((1, k), 513).cuda()
    x40 = (bf16_vector((40, k), 514).float() * 0.125).to(torch.bfloat16).cuda()
    plain = _pack(ext, blocks, scales)
    table = _pack(ext, blocks, scales, bc4.palette())
    try:
        for h in (plain, table):
            ext.set_prefill(h, 16, 1024)
        assert torch.equal(ext.decode_dense(plain), ext.decode_dense(table))
        assert torch.equal(ext.linear_f32(plain, x1), ext.linear_f32(table, x1))
        assert torch.equal(ext.linear(plain, x40), ext.linear(table, x40))
        ext.set_palette_table(table, None)      # back to the arithmetic decode
        assert torch.equal(ext.linear_f32(plain, x1), ext.linear_f32(table, x1))
    finally:
        ext.free(plain)
        ext.free(table)


@pytest.mark.parametrize("m,k,tokens,lookahead", [(1024, 5120, 1, 1), (37, 272, 1, 4), (64, 27648, 1, 2),
                                                  (272, 3072, 5, 1), (5120, 5120, 1, 8)])
def test_lut_gemv_within_tolerance(ext, m, k, tokens, lookahead):
    lut = foreign_palette(m)
    blocks = random_blocks(m, k, 521 + m)
    scales = lognormal_scales(m, 522 + m)
    x = bf16_vector((tokens, k), 523 + m)
    handle = _pack(ext, blocks, scales, lut)
    try:
        ext.set_lookahead(handle, lookahead)
        ext.set_prefill(handle, 1 << 20, 1024)
        y = ext.linear_f32(handle, x.cuda()).cpu().numpy()
    finally:
        ext.free(handle)
    w = bc4.decode_bf16_bits(blocks, scales, lut)
    ref = bc4.gemm_f64(bf16_bits(x), w)
    for t in range(tokens):
        assert rel_err(ref[t], y[t]) <= GEMV_TOL
        assert max_rel_err_floor(ref[t], y[t]) <= GEMV_TOL


def test_lut_gemv_f16(ext):
    m, k = 333, 2048
    lut = foreign_palette(9)
    blocks = random_blocks(m, k, 531)
    scales = lognormal_scales(m, 532)
    x = f16_vector((1, k), 533)
    handle = _pack(ext, blocks, scales, lut)
    try:
        y = ext.linear(handle, x.cuda()).double().cpu().numpy()
    finally:
        ext.free(handle)
    ref = x.double().numpy() @ lut_weights_f32(blocks, scales, lut).astype(np.float64).T
    assert rel_err(ref[0], y[0]) <= GEMV_TOL
    assert max_rel_err_floor(ref[0], y[0]) <= 2 ** -11 + GEMV_TOL


@pytest.mark.parametrize("m,k,tokens", [(200, 1280, 17), (200, 1280, 128), (300, 27648, 32)])
def test_lut_prefill_candidates_bitwise_equal_and_within_rrms(ext, m, k, tokens):
    lut = foreign_palette(11)
    blocks = random_blocks(m, k, 541)
    scales = lognormal_scales(m, 542)
    x = (bf16_vector((tokens, k), 543).float() * 0.125).to(torch.bfloat16)
    handle = _pack(ext, blocks, scales, lut)
    try:
        outputs = [ext.prefill(handle, c, x.cuda()) for c in range(5, 10)]
        torch.cuda.synchronize()
    finally:
        ext.free(handle)
    for c, value in zip(range(6, 10), outputs[1:]):
        assert torch.equal(outputs[0], value), f"candidate {c} differs"
    ref = bc4.gemm_f64(bf16_bits(x), bc4.decode_bf16_bits(blocks, scales, lut))
    assert bc4.relative_rms(ref, outputs[0].float().cpu().numpy()) <= PREFILL_RRMS_TOL


def test_artifact_with_a_foreign_palette_runs_in_lut_mode(ext, tmp_path):
    """An artifact naming another GPU's palette and bundling it (hardware/common/palette.bin) is
    packed in LUT mode; the reference would refuse it (``standalone.py:68-76``)."""
    lut = foreign_palette(13)
    m, k = 96, 512
    blocks = random_blocks(m, k, 551)
    scales = lognormal_scales(m, 552)
    bundled = tmp_path / "palette.bin"
    lut.astype("<f4").tofile(bundled)
    digest = artifacts.sha256_file(bundled)
    art = artifacts.write_artifact(tmp_path / "art", [("model.layers.0.mlp.down_proj", blocks, scales)], digest)
    (art / "hardware" / "common").mkdir(parents=True, exist_ok=True)
    (art / "hardware" / "common" / "palette.bin").write_bytes(bundled.read_bytes())
    table = runtime.artifact_palette(art)
    assert table is not None and table.numel() == 255 * 255 * 8
    entry = json.loads((artifacts.weights_dir(art) / "metadata.json").read_text())["entries"][0]
    handles = runtime.pack_entry_handles(artifacts.weights_dir(art), entry, palette=table)
    x = bf16_vector((1, k), 553)
    try:
        y = ext.linear_f32(handles[0], x.cuda()).cpu().numpy()
    finally:
        runtime.free(handles)
    ref = bc4.matvec_f64(bc4.decode_bf16_bits(blocks, scales, lut), bf16_bits(x[0]))
    assert rel_err(ref, y[0]) <= GEMV_TOL
    # a corrupt bundle is refused, and an artifact of the defined palette needs no table
    (art / "hardware" / "common" / "palette.bin").write_bytes(bundled.read_bytes()[:-4] + b"\0\0\0\0")
    with pytest.raises(RuntimeError, match="palette"):
        runtime.artifact_palette(art)
    plain = artifacts.write_artifact(tmp_path / "plain", [("model.layers.0.mlp.down_proj", blocks, scales)],
                                     hardware.PALETTE_SHA256)
    assert runtime.artifact_palette(plain) is None
