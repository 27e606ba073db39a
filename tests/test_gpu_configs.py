"""The BASELINE configurations at their full sizes on the GPU, against the CPU oracle.

* Config 1: the 4096 x 4096 matrix encoded by this build's PTQ encoder (its bytes pinned by the
  reference encoder's golden hashes), all 16.8 M decoded weights bit-exact, the fp32 GEMV within
  1e-3 of the float64 matvec norm-wise and per element.
* Config 2: every 27B-class decode shape (q/o 5120->5120, k/v 5120->1024, gate/up
  5120->27648, down 27648->5120) encoded on the GPU from ``N(0, 0.02^2) * LogNormal(0, 0.3)``
  per input channel: decoded weights bit-exact, bf16-input GEMV within 1e-3.
* Config 3: the prefill GEMM at T = 32, 128 and 512 on the q/o, k/v, gate/up and down shapes: all
  five tile candidates bitwise equal (the reference autotuner's gate, ``autotune.py:150-168``),
  the whole output within relative RMS 1e-2 of the float64 GEMM, and every output row within it
  as well (a wrong row tile cannot hide in the whole-matrix figure).
* Configs 4 and 5: the Qwen2.5-3B-style and 27B-class decoders built at full size, the
  reference's 32-token prefill gate (``prefill.py:88-108``, relative RMS <= 0.02 between the
  GEMV-only and the prefill-GEMM paths), and graph-replayed decode equal to eager decode.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import bc4, clib
from tests.golden.cases import config1_inputs
from tests.helpers import bf16_bits, bf16_vector, max_rel_err_floor, rel_err
from texelator_amd import encoder, hardware, modeling, prefill

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-3
PREFILL_RRMS_TOL = 1e-2
GOLDEN = Path(__file__).resolve().parent / "golden"

# BASELINE config 2 / 3 shapes: name -> (M, K)
SHAPES = {"q_o": (5120, 5120), "k_v": (1024, 5120), "gate_up": (27648, 5120), "down": (5120, 27648)}


def _pack(ext, blocks, scales):
    return ext.pack_encoded(torch.from_numpy(np.ascontiguousarray(blocks).reshape(-1)),
                            torch.from_numpy(np.ascontiguousarray(scales)))


def _check_gemv(y: np.ndarray, ref: np.ndarray) -> None:
    assert rel_err(ref, y) <= GEMV_TOL
    assert max_rel_err_floor(ref, y) <= GEMV_TOL


# ---------------------------------------------------------------------------------------------
# config 1


def test_config1_encoded_matrix(ext, oracle_threads):
    record = json.loads((GOLDEN / "encoder_vectors.json").read_text())
    weight, hdiag = config1_inputs()
    blocks, scales = encoder.encode_matrix(weight, hdiag, torch.from_numpy(bc4.palette()), rows_per_chunk=128)
    assert hashlib.sha256(blocks.tobytes()).hexdigest() == record["blocks_sha256"]
    assert hashlib.sha256(scales.tobytes()).hexdigest() == record["scales_sha256"]
    x = bf16_vector((1, 4096), 20260827)
    handle = _pack(ext, blocks, scales)
    try:
        dense = bf16_bits(ext.decode_dense(handle).cpu())
        y32 = ext.linear_f32(handle, x.cuda()).cpu().numpy()[0]
        y16 = ext.linear(handle, x.cuda()).float().cpu().numpy()[0]
    finally:
        ext.free(handle)
    w = clib.decode_bf16_bits(blocks, scales)
    mismatches = int(np.count_nonzero(dense != w))
    assert mismatches == 0, f"{mismatches} of {w.size} decoded weights differ"
    ref = clib.matvec_f64(w, bf16_bits(x[0]))
    _check_gemv(y32, ref)
    assert max_rel_err_floor(ref, y16) <= 2 ** -8 + GEMV_TOL


# ---------------------------------------------------------------------------------------------
# configs 2 and 3: matrices encoded once per shape on the GPU


@pytest.fixture(scope="module")
def encoded():
    """name -> (blocks uint8 [M, K/16*8], scales f32 [M], decoded bf16 bits [M, K])."""
    lut = hardware.device_palette("cuda")
    cache = {}

    def get(name: str):
        if name not in cache:
            m, k = SHAPES[name]
            g = torch.Generator(device="cuda").manual_seed(20260827 + m + 7 * k)
            w = torch.randn((m, k), device="cuda", generator=g) * 0.02
            w *= torch.exp(0.3 * torch.randn(k, device="cuda", generator=g))[None, :]
            blocks, scales = encoder.encode_matrix(w, torch.ones(k), lut, rows_per_chunk=2048)
            del w
            cache[name] = (blocks, scales, clib.decode_bf16_bits(blocks, scales))
        return cache[name]

    yield get
    cache.clear()


@pytest.mark.parametrize("name", list(SHAPES))
def test_config2_gemv_full_shape(ext, oracle_threads, encoded, name):
    blocks, scales, w = encoded(name)
    m, k = SHAPES[name]
    x = bf16_vector((1, k), 31 + m)
    handle = _pack(ext, blocks, scales)
    try:
        dense = bf16_bits(ext.decode_dense(handle).cpu())
        y = ext.linear_f32(handle, x.cuda()).cpu().numpy()[0]
        again = ext.linear_f32(handle, x.cuda()).cpu().numpy()[0]
    finally:
        ext.free(handle)
    mismatches = int(np.count_nonzero(dense != w))
    assert mismatches == 0, f"{mismatches} of {w.size} decoded weights differ"
    _check_gemv(y, clib.matvec_f64(w, bf16_bits(x[0])))
    assert np.array_equal(y, again)   # deterministic split-K order


@pytest.mark.parametrize("tokens", [32, 128, 512])
@pytest.mark.parametrize("name", list(SHAPES))
def test_config3_prefill_full_shape(ext, oracle_threads, encoded, name, tokens):
    blocks, scales, w = encoded(name)
    m, k = SHAPES[name]
    x = bf16_vector((tokens, k), 41 + tokens)
    handle = _pack(ext, blocks, scales)
    try:
        xd = x.cuda()
        outputs = {c: ext.prefill(handle, c, xd) for c in range(5, 10)}
        ext.set_prefill(handle, 1, 1024)
        via_linear = ext.linear(handle, xd)
        torch.cuda.synchronize()
    finally:
        ext.free(handle)
    base = outputs[5]
    for candidate, value in outputs.items():
        assert torch.equal(base, value), f"candidate {candidate} differs from candidate 5"
    assert torch.equal(base, via_linear)
    ref = clib.gemm_f64(bf16_bits(x), w)          # every output row and token
    got = base.float().cpu().numpy()
    assert bc4.relative_rms(ref, got) <= PREFILL_RRMS_TOL
    per_row = np.sqrt(np.sum((got - ref) ** 2, axis=0) / np.maximum(np.sum(ref ** 2, axis=0), 1e-300))
    worst = int(np.argmax(per_row))
    assert per_row[worst] <= PREFILL_RRMS_TOL, f"row {worst}: relative RMS {per_row[worst]:.3g}"


@pytest.mark.parametrize("tokens", [300, 512])
def test_prefill_pair_tile_full_and_partial_token_tiles(ext, oracle_threads, tokens):
    """M = 1024, K = 5120 with a bias: the 256-token pair tile runs a full first token tile and a
    partial (300) or full (512) second one, with K splits; all tiles bitwise equal and within the
    rrms bar of the float64 GEMM on every row."""
    from tests.helpers import lognormal_scales, random_blocks

    m, k = 1024, 5120
    blocks = random_blocks(m, k, 71)
    scales = lognormal_scales(m, 72)
    x = bf16_vector((tokens, k), 73)
    bias = bf16_vector((m,), 74, scale=0.1)
    handle = ext.pack_encoded(torch.from_numpy(blocks.reshape(-1)), torch.from_numpy(scales), bias.cuda())
    try:
        assert ext.workspace_bytes(handle, tokens) > 0, "shape expected to split"
        outputs = [ext.prefill(handle, c, x.cuda()) for c in range(5, 10)]
        torch.cuda.synchronize()
    finally:
        ext.free(handle)
    for c, value in zip(range(6, 10), outputs[1:]):
        assert torch.equal(outputs[0], value), f"candidate {c} differs"
    w = clib.decode_bf16_bits(blocks, scales)
    ref = clib.gemm_f64(bf16_bits(x), w) + bias.float().numpy()[None, :]
    assert bc4.relative_rms(ref, outputs[0].float().cpu().numpy()) <= PREFILL_RRMS_TOL


# ---------------------------------------------------------------------------------------------
# configs 4 and 5: whole decoders


@pytest.mark.parametrize("config_name", ["qwen25_3b_style", "class_27b"])
def test_decoder_prefill_gate_and_graph_decode(ext, config_name):
    """The decoder as ``bench.py`` builds it (same seed): ``benchmark_prefill`` on a 512-token
    prompt applies the reference's gate to its first 32 tokens and raises above 0.02; then six
    greedy tokens, graph-replayed and eager, must be the same."""
    config = getattr(modeling.DecoderConfig, config_name)()
    model = modeling.BC4Decoder(config, max_context=1024, seed=20260827)
    try:
        result = prefill.benchmark_prefill(model, tokens=512, warmup=0, runs=1)
        assert result["correctness"]["tokens"] == prefill.CORRECTNESS_TOKENS
        assert result["correctness"]["relative_rms"] <= prefill.RRMS_LIMIT
        assert result["correctness"]["cosine"] > 0.999
        ids = prefill.prompt_ids(model, 64)
        eager = model.generate(ids, 6, eager=True)
        graphed = model.generate(ids, 6, eager=False)
        assert torch.equal(eager, graphed)
        assert int(graphed.max()) < config.vocab
    finally:
        model.close()
