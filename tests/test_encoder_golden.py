"""The PTQ encoder (texelator_amd.encoder) against golden vectors written by the reference's own
encoder (texelator/encoder.py:35-157) with this build's palette; see tests/golden/make_encoder_vectors.py.
Bar: identical block bytes and scale bits."""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import bc4
from tests.golden.cases import config1_inputs, small_cases
from texelator_amd import encoder

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def vectors():
    with np.load(GOLDEN / "encoder_vectors.npz", allow_pickle=False) as data:
        return {key: data[key] for key in data.files}


@pytest.fixture(scope="module")
def lut():
    return torch.from_numpy(bc4.palette())


@pytest.mark.parametrize("name", list(small_cases()))
def test_small_cases_match_reference_encoder(vectors, lut, name):
    weight, hdiag, rows_per_chunk = small_cases()[name]
    assert np.array_equal(vectors[f"{name}/weight"], weight.numpy())   # inputs regenerate exactly
    assert np.array_equal(vectors[f"{name}/hdiag"], hdiag.numpy())
    blocks, scales = encoder.encode_matrix(weight, hdiag, lut, rows_per_chunk=int(vectors[f"{name}/rows_per_chunk"]))
    assert np.array_equal(scales.view(np.uint32), vectors[f"{name}/scales"].view(np.uint32))
    mismatched = int(np.count_nonzero(blocks != vectors[f"{name}/blocks"]))
    assert mismatched == 0, f"{mismatched} block bytes differ"


def test_config1_matches_reference_encoder(lut):
    record = json.loads((GOLDEN / "encoder_vectors.json").read_text())
    assert record["palette_sha256"] == bc4.palette_sha256()
    weight, hdiag = config1_inputs()
    blocks, scales = encoder.encode_matrix(weight, hdiag, lut, rows_per_chunk=128)
    assert blocks[0, :64].tobytes().hex() == record["first_row_blocks_hex"]
    assert hashlib.sha256(scales.tobytes()).hexdigest() == record["scales_sha256"]
    assert hashlib.sha256(blocks.tobytes()).hexdigest() == record["blocks_sha256"]


def test_encoded_weights_decode_close_to_source(vectors):
    """Independent sanity check of the golden data itself: the LUT decode of the reference's
    blocks reconstructs W to within BC4's 3-bit resolution."""
    weight = vectors["lognormal_128x256_hvaried_chunk32/weight"]
    blocks = vectors["lognormal_128x256_hvaried_chunk32/blocks"]
    scales = vectors["lognormal_128x256_hvaried_chunk32/scales"]
    decoded = bc4.bf16_bits_to_f32(bc4.decode_bf16_bits(blocks, scales))
    rel = np.linalg.norm(decoded - weight) / np.linalg.norm(weight)
    assert rel < 0.2
    assert np.array_equal(scales, np.maximum(np.abs(weight).max(axis=1), 1e-12).astype(np.float32))
