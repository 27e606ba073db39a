"""GPU tests of the tuners and of runtime installation (reference: texelator/tuning.py,
texelator/autotune.py, texelator/runtime.py:179-274), on small synthetic artifacts."""
from __future__ import annotations

import json

import numpy as np
import pytest
import torch
from torch import nn

from oracle import clib
from tests.helpers import bf16_bits, bf16_vector, lognormal_scales, random_blocks, rel_err
from texelator_amd import artifacts, autotune, hardware, runtime, tuning

pytestmark = pytest.mark.gpu

SHAPES = ((64, 256), (200, 1280), (40, 512))


@pytest.fixture()
def state(tmp_path, monkeypatch):
    for module in (autotune, tuning, hardware):
        monkeypatch.setattr(module, "STATE_HOME", tmp_path / "state")
    return tmp_path / "state"


def _artifact(path, palette=None, runtime_dtype="bfloat16"):
    matrices = [(f"model.layers.{i}.mlp.down_proj", random_blocks(m, k, 300 + i), lognormal_scales(m, 400 + i))
                for i, (m, k) in enumerate(SHAPES)]
    return artifacts.write_artifact(path, matrices, palette or hardware.PALETTE_SHA256,
                                    runtime_dtype=runtime_dtype), matrices


def test_ensure_hardware_caches_the_defined_palette(ext, state):
    path = hardware.ensure_hardware(force=True)
    assert artifacts.sha256_file(path) == hardware.PALETTE_SHA256
    payload = hardware.doctor_payload()
    assert payload["palette_sha256"] == hardware.PALETTE_SHA256 and payload["endpoint_pairs"] == 65025


@pytest.mark.parametrize("runtime_dtype", ["bfloat16", "float16"])
def test_lookahead_tuner_selects_and_persists(ext, state, tmp_path, runtime_dtype):
    art, _ = _artifact(tmp_path / "art", runtime_dtype=runtime_dtype)
    profile = tuning.tune_artifact(art, warmup=1, measured=3, runs=2)
    assert profile["selected_lookahead"] in tuning.CANDIDATES
    assert all(row["max_abs_vs_k1"] == 0.0 for row in profile["candidates"])
    assert tuning.selected_lookahead(art)[0] == profile["selected_lookahead"]


def test_lookahead_tuner_rejects_foreign_palette(ext, state, tmp_path):
    art, _ = _artifact(tmp_path / "art", palette="0" * 64)
    with pytest.raises(RuntimeError, match="palette does not match"):
        tuning.tune_artifact(art, warmup=0, measured=1, runs=1)


def test_prefill_autotuner_profile_and_apply(ext, state, tmp_path):
    art, matrices = _artifact(tmp_path / "art")
    profile = autotune.tune_artifact(art, None, tokens=[32, 100], warmup=3, measured=10)
    assert profile["status"] == "complete"
    assert len(profile["selections"]) == 2 * len(SHAPES)
    for record in profile["selections"].values():
        assert not record["rejected"], record["rejected"]          # every tile is bitwise equal
        assert record["winner"] in autotune.CANDIDATES
    loaded, _ = autotune.selected_profile(art)
    assert loaded["selections"] == json.loads(json.dumps(profile["selections"]))

    handles = []
    try:
        for _, blocks, scales in matrices:
            handles.extend(runtime.pack_arrays(blocks, scales))
        assert autotune.apply_profile(handles, 100, loaded)
        for handle, (m, k) in zip(handles, SHAPES):
            key = autotune.dispatch_key(100, m, k)
            assert ext.handle_info(handle)[2] == 1
            assert ext.handle_info(handle)[4] == profile["selections"][key]["backend"]
        # an unprofiled bucket falls back to the large tile and reports it
        assert not autotune.apply_profile(handles, 600, loaded)
        assert all(ext.handle_info(h)[4] == autotune.CANDIDATES[autotune.BASELINE] for h in handles)
        # threshold 1 still sends a single token to the GEMV: same result as the f32 GEMV, rounded once
        x = bf16_vector((1, SHAPES[0][1]), 9).cuda()
        y16 = ext.linear(handles[0], x).float()
        y32 = ext.linear_f32(handles[0], x)
        assert torch.equal(y16, y32.to(torch.bfloat16).float())
    finally:
        runtime.free(handles)


def test_texelator_linear_row_split_and_install(ext, oracle_threads):
    m, k = 100, 512
    blocks = random_blocks(m, k, 11)
    scales = lognormal_scales(m, 12)
    handles = runtime.pack_arrays(blocks, scales, max_rows=48)       # 48 + 48 + 4 rows
    assert len(handles) == 3
    module = runtime.TexelatorLinear(handles)
    x = bf16_vector((2, 3, k), 13)
    try:
        y = module(x.cuda()).float().cpu().numpy().reshape(-1, m)
    finally:
        runtime.free(handles)
    w = clib.decode_bf16_bits(blocks, scales)
    ref = clib.gemm_f64(bf16_bits(x.reshape(-1, k)), w)
    for t in range(ref.shape[0]):
        assert rel_err(ref[t], y[t]) <= 2 ** -8


def test_install_replaces_linears_from_artifact(ext, tmp_path):
    art, matrices = _artifact(tmp_path / "art")

    class Layer(nn.Module):
        def __init__(self, m, k):
            super().__init__()
            self.mlp = nn.Module()
            self.mlp.down_proj = nn.Linear(k, m, bias=False)

    model = nn.Module()
    model.model = nn.Module()
    model.model.layers = nn.ModuleList([Layer(m, k) for m, k in SHAPES]).cuda()
    for i, (name, _, _) in enumerate(matrices):
        assert name == f"model.layers.{i}.mlp.down_proj"
    handles = runtime.install(model, art / "weights")
    try:
        assert len(handles) == len(SHAPES)
        for i, (m, k) in enumerate(SHAPES):
            layer = model.model.layers[i].mlp.down_proj
            assert isinstance(layer, runtime.TexelatorLinear)
            out = layer(torch.randn(1, k, device="cuda").to(torch.bfloat16))
            assert out.shape == (1, m) and bool(torch.isfinite(out.float()).all())
    finally:
        runtime.free(handles)
