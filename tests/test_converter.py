"""CPU tests of the calibration and conversion pipeline (reference: texelator/converter.py:62-233).

A tiny random Qwen2 model runs on the CPU; the encoder searches this build's palette (the
oracle's table). Checks:
- the collected moments against E[x^2] recomputed independently for layer 0's q_proj input
  (embedding, then the layer's RMSNorm, done here by hand), and the invariants that q/k/v and
  gate/up see the same input;
- every entry is the encoder's output for that weight with those moments as hdiag (and differs
  from an uncalibrated encode), in the reference's artifact layout;
- an interrupted conversion resumes without re-encoding finished entries and ends with the same
  bytes as an uninterrupted one; a corrupted finished entry is re-encoded; a finished artifact
  is reused, and one with another calibration size is refused.
"""
from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from oracle import bc4
from texelator_amd import artifacts, converter, encoder

transformers = pytest.importorskip("transformers")

TOKENS = 96


@pytest.fixture(scope="module")
def model():
    torch.manual_seed(0)
    config = transformers.Qwen2Config(vocab_size=300, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=256,
                                      tie_word_embeddings=False, attn_implementation="eager")
    return transformers.Qwen2ForCausalLM(config).eval()


@pytest.fixture(scope="module")
def lut():
    return torch.from_numpy(bc4.palette())


@pytest.fixture(scope="module")
def ids(tmp_path_factory):
    rng = np.random.default_rng(7)
    path = tmp_path_factory.mktemp("calib") / "ids.npy"
    np.save(path, rng.integers(0, 300, size=TOKENS + 10).astype(np.int32))
    return converter.read_token_ids(path, TOKENS)


def _convert(model, path, ids, lut, **kwargs):
    return converter.convert_model(model, path, ids, source="tiny-qwen2", chunk=40, lut=lut, **kwargs)


def test_token_sources(tmp_path):
    text = tmp_path / "ids.txt"
    text.write_text("5 6 7\n8 9")
    assert converter.read_token_ids(text, 4).tolist() == [5, 6, 7, 8]
    with pytest.raises(RuntimeError, match="need 9"):
        converter.read_token_ids(text, 9)

    class Tokenizer:
        def __call__(self, value, return_tensors, add_special_tokens):
            assert not add_special_tokens
            return type("Encoded", (), {"input_ids": torch.tensor([[len(word) for word in value.split()]])})

    prose = tmp_path / "prose.txt"
    prose.write_text("a bb ccc dddd")
    assert converter.read_token_ids(prose, 3, tokenizer=Tokenizer()).tolist() == [1, 2, 3]


def test_moments_match_direct_computation(model, ids):
    specs = [s for s in converter.discover_linears(model) if s.supported]
    moments = converter.collect_moments(model, {s.module_name: s.artifact_key for s in specs}, ids, chunk=40)
    key = {s.module_name: s.artifact_key for s in specs}
    # layer 0's q_proj input, by hand: RMSNorm(embed(ids)) with the layer's norm weight
    layer = model.model.layers[0]
    with torch.no_grad():
        h = model.model.embed_tokens(ids).double()
        eps = model.config.rms_norm_eps
        x = h * torch.rsqrt(h.square().mean(-1, keepdim=True) + eps) * layer.input_layernorm.weight.double()
    want = x.square().mean(0)
    got = moments[key["model.layers.0.self_attn.q_proj"]].double()
    assert torch.allclose(got, want, rtol=2e-5, atol=0)
    for i in range(2):
        base = f"model.layers.{i}"
        q = moments[key[f"{base}.self_attn.q_proj"]]
        assert torch.equal(q, moments[key[f"{base}.self_attn.k_proj"]])
        assert torch.equal(q, moments[key[f"{base}.self_attn.v_proj"]])
        assert torch.equal(moments[key[f"{base}.mlp.gate_proj"]], moments[key[f"{base}.mlp.up_proj"]])
        assert all(bool((m > 0).all()) for m in moments.values())


def test_conversion_encodes_with_moments_in_reference_layout(model, ids, lut, tmp_path):
    path = _convert(model, tmp_path / "art", ids, lut)
    manifest = artifacts.read_manifest(path)
    assert manifest["format"] == "texelator-bc4-v1" and manifest["calibration"]["tokens"] == TOKENS
    metadata = json.loads((path / "weights" / "metadata.json").read_text())
    assert len(metadata["entries"]) == 14 and not (path / "weights" / "progress.json").exists()
    assert artifacts.validate_encoded(path / "weights")["ok"]
    moments = converter._load_moments(path / converter.MOMENTS_FILE)
    differs = 0
    for entry in metadata["entries"][:4] + metadata["entries"][-3:]:
        weight = model.get_submodule(entry["module_name"]).weight.detach()
        blocks = np.fromfile(path / "weights" / entry["blocks_file"], dtype=np.uint8).reshape(entry["M"], -1)
        scales = np.fromfile(path / "weights" / entry["scales_file"], dtype="<f4")
        want_blocks, want_scales = encoder.encode_matrix(weight, moments[entry["artifact_key"]], lut)
        assert np.array_equal(blocks, want_blocks) and np.array_equal(scales, want_scales)
        plain, _ = encoder.encode_matrix(weight, torch.ones(entry["K"]), lut)
        differs += int(not np.array_equal(blocks, plain))
    assert differs > 0


def test_interrupted_conversion_resumes(model, ids, lut, tmp_path, monkeypatch):
    reference = _convert(model, tmp_path / "whole", ids, lut)
    calls = []
    real = converter.encode_linear_e3

    def counting(*args, **kwargs):
        calls.append(args[3].name)
        return real(*args, **kwargs)

    monkeypatch.setattr(converter, "encode_linear_e3", counting)
    path = _convert(model, tmp_path / "parts", ids, lut, stop_after=5)
    assert len(calls) == 5 and not (path / artifacts.MANIFEST).exists()
    progress = json.loads((path / "weights" / "progress.json").read_text())["entries"]
    # a corrupted finished entry is encoded again
    (path / "weights" / progress[1]["blocks_file"]).write_bytes(b"\0" * progress[1]["blocks_bytes"])
    calls.clear()
    _convert(model, path, ids, lut)
    assert len(calls) == 14 - 5 + 1
    whole = json.loads((reference / "weights" / "metadata.json").read_text())["entries"]
    parts = json.loads((path / "weights" / "metadata.json").read_text())["entries"]
    assert [(e["module_name"], e["blocks_sha256"], e["scales_sha256"]) for e in whole] == \
           [(e["module_name"], e["blocks_sha256"], e["scales_sha256"]) for e in parts]
    calls.clear()
    _convert(model, path, ids, lut)          # finished: verified and reused
    assert calls == []
    with pytest.raises(RuntimeError, match="different source"):
        _convert(model, path, ids[:TOKENS - 8], lut)
