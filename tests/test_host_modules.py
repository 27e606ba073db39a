"""CPU tests of the host-side modules: artifact layout, naming, profile keys and gates, metrics.

Modelled on the reference's CPU contract tests (tests/test_adapters.py, tests/test_runtime_layout.py,
tests/test_store.py) and on the numeric gates its commands apply (autotune.py:63-85,
tuning.py:66-81). Device queries are replaced by monkeypatched fakes; no GPU is used.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch
from torch import nn

from oracle import bc4
from tests.helpers import lognormal_scales, random_blocks
from texelator_amd import adapters, artifacts, autotune, hardware, runtime, tuning


def _write_small_artifact(path: Path, shapes=((32, 64), (48, 128)), palette=None) -> Path:
    matrices = []
    for index, (m, k) in enumerate(shapes):
        matrices.append((f"model.layers.{index}.mlp.up_proj", random_blocks(m, k, 100 + index),
                         lognormal_scales(m, 200 + index)))
    return artifacts.write_artifact(path, matrices, palette or hardware.PALETTE_SHA256)


def test_palette_constant_matches_oracle():
    assert hardware.PALETTE_SHA256 == bc4.palette_sha256()


def test_artifact_layout_and_validation(tmp_path):
    art = _write_small_artifact(tmp_path / "art")
    manifest = artifacts.read_manifest(art)
    assert manifest["format"] == "texelator-bc4-v1" and manifest["runtime_dtype"] == "bfloat16"
    metadata = json.loads((art / "weights" / "metadata.json").read_text())
    assert [e["M"] for e in metadata["entries"]] == [32, 48]
    assert [e["K"] for e in metadata["entries"]] == [64, 128]
    first = metadata["entries"][0]
    assert (art / "weights" / first["blocks_file"]).stat().st_size == 32 * 64 // 2
    assert (art / "weights" / first["scales_file"]).stat().st_size == 32 * 4
    assert artifacts.validate_encoded(art / "weights")["ok"]
    # a flipped byte is caught by the checksum gate (artifacts.py:76-87)
    blob = bytearray((art / "weights" / first["blocks_file"]).read_bytes())
    blob[3] ^= 1
    (art / "weights" / first["blocks_file"]).write_bytes(bytes(blob))
    report = artifacts.validate_encoded(art / "weights")
    assert not report["ok"] and report["failures"][0]["module_name"] == first["module_name"]


def test_missing_manifest_is_rejected(tmp_path):
    with pytest.raises(RuntimeError, match="not a Texelator artifact"):
        artifacts.read_manifest(tmp_path)


def test_artifact_key_is_stable_safe_and_unique():
    names = ["model.layers.0.self_attn.q_proj", "model.layers.0.self_attn.k_proj",
             "model.layers.10.mlp.down_proj", "model.layers.1.mlp.down_proj", "weird name/with:chars"]
    keys = [adapters.artifact_key(n) for n in names]
    assert len(set(keys)) == len(keys)
    assert keys == [adapters.artifact_key(n) for n in names]
    for key in keys:
        assert all(c.isalnum() or c in "_.-" for c in key)
    assert keys[0].startswith("model__layers__0__self_attn__q_proj--") and len(keys[0].split("--")[-1]) == 10


@pytest.mark.parametrize("name,layer", [("model.layers.7.mlp.up_proj", 7), ("transformer.h.3.attn", 3),
                                        ("decoder.layers.12.fc1", 12), ("lm_head", None)])
def test_layer_index(name, layer):
    assert adapters.layer_index(name) == layer


def test_resolve_top_level_module():
    model = nn.Module()
    model.lm_head = nn.Linear(4, 8, bias=False)
    parent, child = adapters.resolve_parent(model, "lm_head")
    assert parent is model and child == "lm_head"
    with pytest.raises(RuntimeError, match="does not exist"):
        adapters.resolve_parent(model, "missing")


def test_texelator_linear_requires_handles():
    with pytest.raises(ValueError, match="at least one"):
        runtime.TexelatorLinear([])


def test_decode_only_linear_routes_single_tokens():
    calls = []

    class Tag(nn.Module):
        def __init__(self, tag):
            super().__init__()
            self.tag = tag

        def forward(self, x):
            calls.append(self.tag)
            return x

    module = runtime.DecodeOnlyLinear(Tag("dense"), Tag("bc4"))
    module(torch.zeros(1, 1, 8))
    module(torch.zeros(1, 3, 8))
    assert calls == ["bc4", "dense"]


def test_fp4_hybrid_dispatch(monkeypatch):
    """The hybrid takes only bf16 calls of 512 tokens on its MLP shapes while it is on
    (reference runtime.py:119-131); ``free`` turns it off."""
    calls = []

    class Ext:
        @staticmethod
        def shape(handle):
            return {1: (5120, 17408), 2: (17408, 5120), 3: (5120, 5120)}[handle]

        @staticmethod
        def linear(handle, x):
            calls.append(("linear", handle, x.shape[0]))
            return torch.zeros(x.shape[0], Ext.shape(handle)[0])

        @staticmethod
        def quantize_activation_fp4_out(x, packed, scales):
            assert packed.shape == (x.shape[0], x.shape[1] // 2) and scales.shape == (x.shape[0], x.shape[1] // 32)
            calls.append(("quantize", x.shape[0]))

        @staticmethod
        def decode_weight_fp4_out(handle, packed, scales):
            calls.append(("decode", handle))

        @staticmethod
        def fp4_gemm(xp, xs, wp, ws):
            calls.append(("gemm", xp.shape[0], wp.shape[0]))
            return torch.zeros(xp.shape[0], wp.shape[0], dtype=torch.bfloat16)

        @staticmethod
        def free(handle):
            calls.append(("free", handle))

    monkeypatch.setattr(runtime, "extension", lambda verbose=False: Ext)
    x512 = torch.zeros(512, 17408, dtype=torch.bfloat16)
    runtime._linear_dispatch(1, x512)
    assert calls == [("linear", 1, 512)]          # off by default
    calls.clear()
    runtime.set_fp4_hybrid(True)
    assert runtime._linear_dispatch(1, x512).shape == (512, 5120)
    assert calls == [("quantize", 512), ("decode", 1), ("gemm", 512, 5120)]
    calls.clear()
    runtime._linear_dispatch(1, torch.zeros(511, 17408, dtype=torch.bfloat16))
    runtime._linear_dispatch(1, torch.zeros(512, 17408, dtype=torch.float16))
    runtime._linear_dispatch(3, torch.zeros(512, 5120, dtype=torch.bfloat16))
    assert [c[0] for c in calls] == ["linear", "linear", "linear"]
    calls.clear()
    runtime.free([1])
    runtime._linear_dispatch(2, torch.zeros(512, 5120, dtype=torch.bfloat16))
    assert calls == [("free", 1), ("linear", 2, 512)]


@pytest.mark.parametrize("tokens,bucket", [(1, 32), (32, 32), (33, 128), (512, 512), (513, 2048), (65535, 65535)])
def test_token_buckets(tokens, bucket):
    assert autotune.token_bucket(tokens) == bucket
    assert autotune.dispatch_key(tokens, 5120, 27648) == f"tokens<={bucket}:M=5120:K=27648"


@pytest.mark.parametrize("tokens", [0, 65536])
def test_token_bucket_limits(tokens):
    with pytest.raises(ValueError):
        autotune.token_bucket(tokens)


def test_candidates_match_library_names():
    from texelator_amd import _lib

    lib = _lib.load()
    assert list(autotune.CANDIDATES) == [lib.tx_candidate_name(i).decode() for i in range(5, 10)]
    assert autotune.BASELINE in autotune.CANDIDATES


def test_kernel_source_hash_tracks_sources(tmp_path, monkeypatch):
    first = autotune.kernel_source_sha256()
    assert first == autotune.kernel_source_sha256()
    fake = tmp_path / "pkg"
    (fake / "csrc").mkdir(parents=True)
    for path in (runtime.PACKAGE_ROOT / "csrc").iterdir():
        (fake / "csrc" / path.name).write_bytes(path.read_bytes())
    monkeypatch.setattr(autotune, "PACKAGE_ROOT", fake)
    assert autotune.kernel_source_sha256() == first
    (fake / "csrc" / "gemv.hip").write_bytes((fake / "csrc" / "gemv.hip").read_bytes() + b"\n")
    assert autotune.kernel_source_sha256() != first


def test_error_metrics_match_oracle():
    rng = np.random.default_rng(5)
    ref = rng.standard_normal((7, 33)).astype(np.float32)
    val = ref + 0.01 * rng.standard_normal(ref.shape).astype(np.float32)
    got = autotune._error(torch.from_numpy(ref), torch.from_numpy(val))
    want = bc4.error_metrics(ref, val)
    for key in ("max_abs", "mean_abs", "relative_rms", "cosine"):
        assert got[key] == pytest.approx(want[key], rel=1e-5)
    assert got["bitwise_equal"] is False
    assert autotune._error(torch.from_numpy(ref), torch.from_numpy(ref.copy()))["bitwise_equal"] is True
    # closed form: a uniform relative scaling by (1+e) has rrms = e and cosine = 1
    scaled = autotune._error(torch.ones(10), torch.full((10,), 1.25))
    assert scaled["relative_rms"] == pytest.approx(0.25) and scaled["cosine"] == pytest.approx(1.0)


def test_eligibility():
    assert autotune._eligible("small_32x128x128", 17, 48) == (True, None)
    assert autotune._eligible("small_32x128x128", 16, 40)[0] is False


@pytest.fixture()
def fake_device(monkeypatch):
    class Props:
        multi_processor_count = 256
        total_memory = 288 << 30
        name = "AMD Instinct MI355X"

    monkeypatch.setattr(torch.cuda, "get_device_name", lambda *a, **k: "AMD Instinct MI355X")
    monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)
    monkeypatch.setattr(torch.cuda, "get_device_properties", lambda *a, **k: Props())
    monkeypatch.setattr(autotune, "device_key", lambda: "gfx950")
    monkeypatch.setattr(tuning, "device_key", lambda: "gfx950")
    return Props


def test_profile_gate_rejects_foreign_profiles(fake_device):
    good = {"kernel_source_sha256": autotune.kernel_source_sha256(),
            "device": {"arch": "gfx950", "multiprocessor_count": 256}}
    autotune.check_profile_device(good)
    with pytest.raises(RuntimeError, match="kernel hash"):
        autotune.check_profile_device({**good, "kernel_source_sha256": "0" * 64})
    with pytest.raises(RuntimeError, match="architecture"):
        autotune.check_profile_device({**good, "device": {"arch": "gfx942", "multiprocessor_count": 256}})
    with pytest.raises(RuntimeError, match="CU count"):
        autotune.check_profile_device({**good, "device": {"arch": "gfx950", "multiprocessor_count": 304}})


def test_profile_paths_and_selected_profile_gates(tmp_path, fake_device, monkeypatch):
    monkeypatch.setattr(autotune, "STATE_HOME", tmp_path / "state")
    monkeypatch.setattr(tuning, "STATE_HOME", tmp_path / "state")
    art = _write_small_artifact(tmp_path / "art")
    assert autotune.selected_profile(art)[0] is None
    assert tuning.selected_lookahead(art) == (1, None)
    target = autotune.profile_path(art)
    assert target.name == "gfx950-amd-instinct-mi355x-prefill.json"
    metadata_sha = artifacts.sha256_file(art / "weights" / "metadata.json")
    assert target.parent.name == metadata_sha[:20]
    profile = {"metadata_sha256": metadata_sha, "kernel_source_sha256": autotune.kernel_source_sha256()}
    target.parent.mkdir(parents=True)
    target.write_text(json.dumps(profile))
    assert autotune.selected_profile(art)[0] == profile
    target.write_text(json.dumps({**profile, "metadata_sha256": "x"}))
    with pytest.raises(RuntimeError, match="encoded weights"):
        autotune.selected_profile(art)
    # decode profile: the palette hash of the artifact must match
    decode = tuning._profile_path(art)
    decode.write_text(json.dumps({"weights_metadata_sha256": metadata_sha, "palette_sha256": "other",
                                  "selected_lookahead": 4}))
    with pytest.raises(RuntimeError, match="palette"):
        tuning.selected_lookahead(art)
    decode.write_text(json.dumps({"weights_metadata_sha256": metadata_sha,
                                  "palette_sha256": hardware.PALETTE_SHA256, "selected_lookahead": 4}))
    assert tuning.selected_lookahead(art) == (4, decode)


def test_runtime_dtype_gate():
    """bfloat16 and float16 artifacts are accepted; float16 is the default (``tuning.py``)."""
    assert tuning._runtime_dtype({"runtime_dtype": "bfloat16"}) is torch.bfloat16
    assert tuning._runtime_dtype({"runtime_dtype": "float16"}) is torch.float16
    assert tuning._runtime_dtype({}) is torch.float16
    with pytest.raises(RuntimeError, match="unsupported"):
        tuning._runtime_dtype({"runtime_dtype": "float32"})


def test_device_block_packing_matches_host_packing():
    """``pack_blocks_tensor`` (on the endpoints' device) writes the bytes of ``pack_blocks``,
    extreme endpoints and every selector value included."""
    from texelator_amd import encoder

    g = torch.Generator().manual_seed(11)
    n = 257
    e0 = torch.randint(-127, 128, (n,), generator=g, dtype=torch.int16)
    e1 = torch.randint(-127, 128, (n,), generator=g, dtype=torch.int16)
    e0[:3] = torch.tensor([-127, 127, 0], dtype=torch.int16)
    e1[:3] = torch.tensor([127, -127, -1], dtype=torch.int16)
    idx = torch.randint(0, 8, (n, 16), generator=g, dtype=torch.uint8)
    idx[0] = 7
    want = encoder.pack_blocks(e0, e1, idx)
    got = encoder.pack_blocks_tensor(e0, e1, idx).numpy()
    assert got.dtype == np.uint8 and got.shape == (n, 8)
    assert np.array_equal(got, want)


def test_tensor_encoder_matches_array_encoder():
    """``encode_matrix_tensor`` keeps the result on the device and returns the bytes and scales of
    ``encode_matrix`` for the same rows (here on the CPU, rows in several chunks)."""
    from texelator_amd import encoder

    g = torch.Generator().manual_seed(12)
    w = torch.randn(37, 64, generator=g) * 0.02
    hdiag = torch.ones(64)
    lut = torch.from_numpy(bc4.palette())
    want_blocks, want_scales = encoder.encode_matrix(w, hdiag, lut, rows_per_chunk=16)
    blocks, scales = encoder.encode_matrix_tensor(w, hdiag, lut, rows_per_chunk=16)
    assert np.array_equal(blocks.numpy(), want_blocks)
    assert np.array_equal(scales.numpy(), want_scales)


def test_qwen2_config_of_decoder_config():
    """The Hugging Face model that stands in for BASELINE config 4 has its shapes."""
    pytest.importorskip("transformers")
    from texelator_amd import hf, modeling

    c = modeling.DecoderConfig.qwen25_3b_style()
    q = hf.qwen2_config(c)
    assert (q.num_hidden_layers, q.hidden_size, q.intermediate_size) == (36, 2048, 11008)
    assert (q.num_attention_heads, q.num_key_value_heads, q.head_dim) == (16, 2, 128)
    assert (q.vocab_size, q.rms_norm_eps, q.tie_word_embeddings) == (151936, 1e-6, False)
    assert q.rope_parameters["rope_theta"] == 1e6


def test_texelator_attention_registration_and_refusals():
    """``use_texelator_attention`` registers the ``"texelator"`` implementation and switches a
    Hugging Face model to it; the attention function refuses, before any launch, the calls its
    kernels do not take (head_dim other than 128, batch > 1, a mask, a prompt not at position 0)."""
    transformers = pytest.importorskip("transformers")
    from texelator_amd import hf
    from texelator_amd._lib import TexelatorError

    config = transformers.Qwen2Config(vocab_size=64, hidden_size=64, intermediate_size=128, num_hidden_layers=1,
                                      num_attention_heads=4, num_key_value_heads=2, head_dim=16,
                                      tie_word_embeddings=False)
    model = transformers.Qwen2ForCausalLM(config).eval()
    hf.use_texelator_attention(model)
    assert model.config._attn_implementation == hf.ATTENTION
    module = model.model.layers[0].self_attn
    positions = torch.arange(3)[None]

    def call(q_shape, k_shape, mask=None, position_ids=positions):
        q, k = torch.zeros(q_shape, dtype=torch.bfloat16), torch.zeros(k_shape, dtype=torch.bfloat16)
        return hf.texelator_attention(module, q, k, k, mask, scaling=0.1, position_ids=position_ids)

    with pytest.raises(TexelatorError, match="head_dim 128"):
        call((1, 4, 3, 16), (1, 2, 8, 16))
    with pytest.raises(TexelatorError, match="batch 1"):
        call((2, 4, 3, 128), (2, 2, 8, 128))
    with pytest.raises(TexelatorError, match="no mask"):
        call((1, 4, 3, 128), (1, 2, 8, 128), mask=torch.ones(1, 1, 3, 8, dtype=torch.bool))
    with pytest.raises(TexelatorError, match="position 0"):
        call((1, 4, 3, 128), (1, 2, 8, 128), position_ids=torch.arange(2, 5)[None])
    with pytest.raises(TexelatorError, match="at most 8"):
        call((1, 36, 1, 128), (1, 2, 8, 128), position_ids=torch.tensor([[4]]))


def test_texelator_norm_replacement_and_restore():
    """``use_texelator_norms`` swaps every bf16 RMSNorm of a Hugging Face model (two per layer and the
    final one) for ``TexelatorRMSNorm`` sharing the weight, and ``restore_modules`` puts them back;
    fp32 norms are left alone."""
    transformers = pytest.importorskip("transformers")
    from texelator_amd import hf

    config = transformers.Qwen2Config(vocab_size=64, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                                      num_attention_heads=4, num_key_value_heads=2, head_dim=16,
                                      tie_word_embeddings=False)
    model = transformers.Qwen2ForCausalLM(config).eval()
    assert hf.use_texelator_norms(model) == []  # fp32 weights
    model.to(torch.bfloat16)
    original = model.model.layers[1].post_attention_layernorm
    replaced = hf.use_texelator_norms(model)
    assert len(replaced) == 2 * 2 + 1
    swapped = model.model.layers[1].post_attention_layernorm
    assert isinstance(swapped, hf.TexelatorRMSNorm) and swapped.weight is original.weight
    assert swapped.variance_epsilon == original.variance_epsilon
    assert hf.use_texelator_norms(model) == []  # already swapped
    hf.restore_modules(replaced)
    assert model.model.layers[1].post_attention_layernorm is original


def test_texelator_mlp_replacement_and_restore():
    """``use_texelator_mlp`` swaps a Hugging Face gated SiLU MLP whose gate and up projections are
    single-handle TexelatorLinear modules without a separate bias (no GPU call: only the module
    tree changes), leaves dense MLPs, biased, sharded or non-SiLU ones alone, and
    ``restore_modules`` puts the originals back."""
    transformers = pytest.importorskip("transformers")
    from texelator_amd import hf
    from texelator_amd.runtime import TexelatorLinear

    config = transformers.Qwen2Config(vocab_size=64, hidden_size=64, intermediate_size=128, num_hidden_layers=4,
                                      num_attention_heads=4, num_key_value_heads=2, head_dim=16,
                                      tie_word_embeddings=False)
    model = transformers.Qwen2ForCausalLM(config).eval()
    assert hf.use_texelator_mlp(model) == []  # dense linears
    layers = model.model.layers
    for i, layer in enumerate(layers):
        layer.mlp.gate_proj = TexelatorLinear([10 * i + 1])
        layer.mlp.up_proj = TexelatorLinear([10 * i + 2])
        layer.mlp.down_proj = TexelatorLinear([10 * i + 3])
    layers[1].mlp.gate_proj = TexelatorLinear([11], bias=nn.Parameter(torch.zeros(128)))  # a separate bias
    layers[2].mlp.up_proj = TexelatorLinear([22, 23])  # two row shards
    layers[3].mlp.act_fn = nn.GELU()
    originals = [layer.mlp for layer in layers]
    replaced = hf.use_texelator_mlp(model)
    assert [r[2] for r in replaced] == [originals[0]]
    fused = layers[0].mlp
    assert isinstance(fused, hf.TexelatorMLP) and fused.original is originals[0]
    assert (fused.gate, fused.up) == (1, 2)
    assert all(layers[i].mlp is originals[i] for i in (1, 2, 3))
    assert hf.use_texelator_mlp(model) == []  # already swapped
    hf.restore_modules(replaced)
    assert [layer.mlp for layer in layers] == originals


def test_texelator_rope_forward_replacement_and_restore():
    """``use_texelator_rope`` gives every Qwen2 attention module a forward that runs the module's own
    steps around the rotary embedding; off the GPU (here: fp32 on the CPU) it takes Hugging Face's
    ``apply_rotary_pos_emb``, so the model's logits are bitwise the unchanged model's; a second call
    changes nothing and ``restore_rope`` gives back the class's forward."""
    transformers = pytest.importorskip("transformers")
    from texelator_amd import hf

    config = transformers.Qwen2Config(vocab_size=64, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                                      num_attention_heads=4, num_key_value_heads=2, head_dim=16,
                                      tie_word_embeddings=False)
    torch.manual_seed(5)
    model = transformers.Qwen2ForCausalLM(config).eval()
    ids = torch.randint(0, 64, (1, 9), generator=torch.Generator().manual_seed(6))
    with torch.no_grad():
        want = model(ids).logits
        changed = hf.use_texelator_rope(model)
        assert len(changed) == 2 and all("forward" in m.__dict__ for m in changed)
        assert hf.use_texelator_rope(model) == []
        got = model(ids).logits
    assert torch.equal(want, got)
    hf.restore_rope(changed)
    assert all("forward" not in m.__dict__ for m in changed)


def test_texelator_residuals_forward_replacement_and_restore():
    """``use_texelator_residuals`` gives every Qwen2 decoder layer a forward with the layer's own steps;
    with Hugging Face's norm modules (here: fp32 on the CPU) it adds and normalizes as the layer does,
    so the logits are bitwise the unchanged model's (also with ``use_texelator_rope`` on); ``use_texelator_qkv``
    joins nothing without installed linears; ``restore_rope`` undoes both overrides."""
    transformers = pytest.importorskip("transformers")
    from texelator_amd import hf

    config = transformers.Qwen2Config(vocab_size=64, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                                      num_attention_heads=4, num_key_value_heads=2, head_dim=16,
                                      tie_word_embeddings=False)
    torch.manual_seed(7)
    model = transformers.Qwen2ForCausalLM(config).eval()
    ids = torch.randint(0, 64, (1, 9), generator=torch.Generator().manual_seed(8))
    with torch.no_grad():
        want = model(ids).logits
        changed = hf.use_texelator_residuals(model)
        assert len(changed) == 2 and hf.use_texelator_residuals(model) == []
        assert torch.equal(want, model(ids).logits)
        rope = hf.use_texelator_rope(model)
        assert hf.use_texelator_qkv(model) == []
        assert torch.equal(want, model(ids).logits)
    hf.restore_rope(changed + rope)
    assert all("forward" not in m.__dict__ for m in changed + rope)


def test_prefill_benchmark_rejects_plain_models():
    from texelator_amd import prefill

    with pytest.raises(TypeError, match="installed Texelator linears"):
        prefill._Target(nn.Linear(4, 4))
