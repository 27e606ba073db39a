"""Hugging Face integration on the GPU (reference: ``runtime.install`` :210-239 driving a stock
``transformers`` Qwen2 model, and ``cli._generate`` / ``standalone.py`` generation).

A tiny random Qwen2 model is encoded with this build's PTQ encoder running on the GPU (the
reference's ``endpoint_opt`` with the LUT on a CUDA device), written as an artifact, installed
with ``runtime.install`` and compared with the same architecture whose linears hold the decoded
BC4 weights as dense bf16 matrices. Attention runs through torch's flash kernel only, so no
bf16 batched product of the math path is issued.
"""
from __future__ import annotations

import copy
import json

import numpy as np
import pytest
import torch
from torch.nn.attention import SDPBackend, sdpa_kernel

from texelator_amd import artifacts, encoder, hardware, layers, runtime

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")

LINEARS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
           "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


def rrms(ref: torch.Tensor, got: torch.Tensor) -> float:
    ref, got = ref.float(), got.float()
    return float(torch.sqrt(torch.mean((got - ref) ** 2)) / torch.sqrt(torch.mean(ref ** 2)))


@pytest.fixture(scope="module")
def qwen_pair(ext, tmp_path_factory):
    """(BC4-installed model, dense model on the decoded weights, handles)."""
    torch.manual_seed(0)
    config = transformers.Qwen2Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=1024,
                                      rope_theta=1e6, tie_word_embeddings=False, attn_implementation="sdpa")
    dense = transformers.Qwen2ForCausalLM(config).to(device="cuda", dtype=torch.bfloat16).eval()
    lut = hardware.device_palette("cuda")
    matrices = []
    for layer in range(config.num_hidden_layers):
        for name in LINEARS:
            module = dense.get_submodule(f"model.layers.{layer}.{name}")
            blocks, scales = encoder.encode_matrix(module.weight.float(), torch.ones(module.in_features), lut)
            matrices.append((f"model.layers.{layer}.{name}", blocks, scales))
    path = artifacts.write_artifact(tmp_path_factory.mktemp("qwen") / "art", matrices, hardware.PALETTE_SHA256)
    quantized = copy.deepcopy(dense)
    handles = runtime.install(quantized, artifacts.weights_dir(path))
    # the reference model: the same BC4 weights, decoded, as plain dense linears
    for module_name, handle_module in [(n, quantized.get_submodule(n)) for n, _, _ in matrices]:
        target = dense.get_submodule(module_name)
        decoded = torch.cat([ext.decode_dense(h) for h in handle_module.handles], dim=0)
        with torch.no_grad():
            target.weight.copy_(decoded)
    yield quantized, dense, handles
    runtime.free(handles)


def test_gpu_encoder_matches_cpu_encoder(ext):
    """The PTQ encoder on the GPU chooses the CPU's endpoints and selectors for almost every block
    (fp32 reductions may round differently on rare near-ties), with the same reconstruction error."""
    g = torch.Generator().manual_seed(5)
    w = torch.randn(192, 512, generator=g) * 0.02 * torch.exp(0.3 * torch.randn(512, generator=g))[None, :]
    hdiag = torch.exp(torch.randn(512, generator=g))
    lut_gpu = hardware.device_palette("cuda")
    gpu_blocks, gpu_scales = encoder.encode_matrix(w.cuda(), hdiag, lut_gpu)
    cpu_blocks, cpu_scales = encoder.encode_matrix(w, hdiag, lut_gpu.cpu())
    assert np.array_equal(gpu_scales, cpu_scales)
    same = np.all(gpu_blocks.reshape(-1, 8) == cpu_blocks.reshape(-1, 8), axis=1)
    assert same.mean() >= 0.999


def test_installed_linears_are_texelator(qwen_pair):
    quantized, _, handles = qwen_pair
    assert len(handles) == 14
    assert type(quantized.get_submodule("model.layers.1.mlp.down_proj")).__name__ == "TexelatorLinear"


@pytest.mark.parametrize("tokens", [1, 7, 40])
def test_logits_match_dense_decoded_model(qwen_pair, tokens):
    """Decode GEMV (1 and 7 tokens) and prefill GEMM (40 tokens) inside the HF forward."""
    quantized, dense, _ = qwen_pair
    ids = torch.randint(0, 512, (1, tokens), generator=torch.Generator().manual_seed(tokens)).cuda()
    with torch.inference_mode(), sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
        got = quantized(ids).logits
        want = dense(ids).logits
    assert torch.isfinite(got).all()
    assert rrms(want, got) < 2e-2


def test_hf_generate_greedy(qwen_pair):
    """HF ``generate`` (prefill, then cached one-token steps) through the BC4 linears."""
    quantized, dense, _ = qwen_pair
    ids = torch.randint(0, 512, (1, 24), generator=torch.Generator().manual_seed(3)).cuda()
    with torch.inference_mode(), sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
        got = quantized.generate(ids, max_new_tokens=12, do_sample=False, pad_token_id=0)
        want = dense.generate(ids, max_new_tokens=12, do_sample=False, pad_token_id=0)
    assert got.shape == want.shape == (1, 36)
    assert torch.equal(got[:, :24], ids)
    assert (got[:, 24:] == want[:, 24:]).float().mean() >= 0.75


def test_calibrated_artifact_installed_standalone_matches_dense(ext, tmp_path):
    """BASELINE-style offline pipeline (reference: converter.py:62-233, runtime.py:242-263,
    standalone.py:102-158): E[x^2] moments from a local token file drive the GPU encoder into a
    resumable artifact; ``install_standalone`` puts its handles into a meta-initialised Qwen2
    whose remaining tensors are then assigned (as the standalone loader does); its logits match
    the dense model holding the decoded weights, in the decode GEMV and the prefill GEMM."""
    from accelerate import init_empty_weights

    from texelator_amd import converter

    torch.manual_seed(1)
    config = transformers.Qwen2Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=1024,
                                      rope_theta=1e6, tie_word_embeddings=False, attn_implementation="sdpa")
    source = transformers.Qwen2ForCausalLM(config).to("cuda").eval()
    ids_file = tmp_path / "calibration.npy"
    np.save(ids_file, np.random.default_rng(2).integers(0, 512, size=600).astype(np.int64))
    ids = converter.read_token_ids(ids_file, 512)
    with torch.no_grad(), sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.MATH]):
        path = converter.convert_model(source, tmp_path / "art", ids, source="tiny-qwen2", chunk=256,
                                       lut=hardware.device_palette("cuda"))
    assert artifacts.read_manifest(path)["calibration"]["tokens"] == 512
    entries = json.loads((artifacts.weights_dir(path) / "metadata.json").read_text())["entries"]
    assert len(entries) == 14

    with init_empty_weights():
        model = transformers.Qwen2ForCausalLM(config)
    handles = runtime.install_standalone(model, artifacts.weights_dir(path), entries, name_mapper=lambda name: name)
    try:
        linears = {entry["module_name"] for entry in entries}
        residual = {name: value.to(torch.bfloat16) for name, value in source.state_dict().items()
                    if name.rsplit(".", 1)[0] not in linears or not name.endswith(".weight")}
        model.load_state_dict(residual, strict=False, assign=True)
        model.to("cuda").eval()
        assert not [name for name, value in model.named_parameters() if value.device.type == "meta"]
        assert isinstance(model.get_submodule("model.layers.0.self_attn.q_proj"), runtime.TexelatorLinear)

        dense = source.to(torch.bfloat16)
        with torch.no_grad():
            for entry in entries:
                module = model.get_submodule(entry["module_name"])
                decoded = torch.cat([ext.decode_dense(h) for h in module.handles], dim=0)
                dense.get_submodule(entry["module_name"]).weight.copy_(decoded)
        for tokens in (1, 40):
            x = torch.randint(0, 512, (1, tokens), generator=torch.Generator().manual_seed(tokens)).cuda()
            with torch.inference_mode(), sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
                got = model(x).logits
                want = dense(x).logits
            assert torch.isfinite(got).all()
            assert rrms(want, got) < 2e-2
    finally:
        runtime.free(handles)


def test_build_qwen2_reference_prefill_protocol_and_generate(ext):
    """The reference's calling path at BASELINE config-4 shapes (4 of its 36 layers, so the test
    stays short): ``hf.build_qwen2`` puts TexelatorLinear modules holding GPU-encoded random-init
    weights into a meta-initialised Qwen2, ``prefill.benchmark_prefill`` runs the reference's
    protocol on it (``model.model(input_ids=...)``, scalar-vs-hybrid gate on 32 tokens), and
    greedy ``generate`` decodes through the same linears."""
    from dataclasses import replace

    from texelator_amd import hf, modeling, prefill

    config = replace(modeling.DecoderConfig.qwen25_3b_style(), layers=4)
    model, handles = hf.build_qwen2(config, seed=7)
    try:
        assert len(handles) == 4 * 7
        assert isinstance(model.get_submodule("model.layers.3.mlp.down_proj"), runtime.TexelatorLinear)
        result = prefill.benchmark_prefill(model, tokens=128, warmup=0, runs=1)
        assert result["correctness"]["tokens"] == prefill.CORRECTNESS_TOKENS
        assert result["correctness"]["relative_rms"] <= prefill.RRMS_LIMIT
        assert result["model"]["num_hidden_layers"] == 4
        assert result["fused_bc4_mfma"]["gpu_tokens_per_second"] > 0
        timing = hf.benchmark_generate(model, prompt_tokens=64, new_tokens=4, runs=1)
        assert timing["new_tokens"] == 4 and timing["decode_tok_s"] > 0
    finally:
        runtime.free(handles)


@pytest.fixture(scope="module")
def tiny_bc4(ext):
    """A two-layer Qwen2 (head_dim 128) whose linears are GPU-encoded BC4 handles."""
    from texelator_amd import hf, modeling

    model, handles = hf.build_qwen2(modeling.DecoderConfig.tiny(), seed=11)
    yield model
    runtime.free(handles)


def test_texelator_attention_prompt_matches_flash(tiny_bc4):
    """The ``"texelator"`` attention (the library's prompt attention kernel) inside the Hugging Face
    forward gives the logits of torch's flash attention on a 40-token prompt."""
    from texelator_amd import hf

    ids = torch.randint(0, 512, (1, 40), generator=torch.Generator().manual_seed(21)).cuda()
    try:
        with torch.inference_mode(), sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
            tiny_bc4.set_attn_implementation("sdpa")
            want = tiny_bc4(ids).logits
            hf.use_texelator_attention(tiny_bc4)
            got = tiny_bc4(ids).logits
    finally:
        tiny_bc4.set_attn_implementation("sdpa")
    assert torch.isfinite(got).all()
    assert rrms(want, got) < 2e-2


def test_graphed_greedy_replays_equal_eager_steps(tiny_bc4):
    """``GraphedGreedy``: every graph replay (embedding, BC4 linears, decode attention over the
    static cache, norms, argmax) yields the token of the same step run eagerly, twice over from a
    reset cache; and the tokens mostly agree with Hugging Face ``generate`` on flash attention and a
    dynamic cache (bf16 attention sums differ in rounding)."""
    from texelator_amd import hf

    ids = torch.randint(0, 512, (1, 30), generator=torch.Generator().manual_seed(22)).cuda()
    try:
        runner = hf.GraphedGreedy(tiny_bc4, max_cache_len=256)
        eager = runner.generate(ids, 24, eager=True)
        graphed = runner.generate(ids, 24)
        again = runner.generate(ids, 24)
        assert torch.equal(eager, graphed) and torch.equal(graphed, again)
        with torch.inference_mode(), sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
            tiny_bc4.set_attn_implementation("sdpa")
            want = tiny_bc4.generate(ids, max_new_tokens=24, do_sample=False, pad_token_id=0)[0, 30:]
        assert (graphed == want).float().mean() >= 0.75
        timing = runner.benchmark(prompt_tokens=30, new_tokens=16)
        assert timing["decode_tok_s"] > 0
        # with the norms on the library kernel too: replays still equal eager steps
        replaced = hf.use_texelator_norms(tiny_bc4)
        try:
            assert len(replaced) == 2 * 2 + 1
            runner = hf.GraphedGreedy(tiny_bc4, max_cache_len=256)
            assert torch.equal(runner.generate(ids, 24, eager=True), runner.generate(ids, 24))
        finally:
            hf.restore_modules(replaced)
    finally:
        tiny_bc4.set_attn_implementation("sdpa")


def test_texelator_mlp_matches_the_module_and_replays(tiny_bc4):
    """``use_texelator_mlp``: one token through the fused gate/up SwiGLU GEMV gives the Hugging
    Face MLP's output up to the product's single rounding (``bf16(silu(G) * U)`` against
    ``bf16(bf16(silu(G)) * U)`` before the down projection); longer inputs take the module itself,
    bitwise; ``GraphedGreedy`` replays still equal eager steps, with tokens mostly those of the
    unfused model; and the modules come back on restore."""
    from texelator_amd import hf

    hidden = tiny_bc4.config.hidden_size
    g = torch.Generator(device="cuda").manual_seed(23)
    ids = torch.randint(0, 512, (1, 30), generator=torch.Generator().manual_seed(24)).cuda()
    try:
        runner = hf.GraphedGreedy(tiny_bc4, max_cache_len=256)
        unfused = runner.generate(ids, 24)
        originals = [layer.mlp for layer in tiny_bc4.model.layers]
        replaced = hf.use_texelator_mlp(tiny_bc4)
        try:
            assert [r[2] for r in replaced] == originals
            assert all(isinstance(layer.mlp, hf.TexelatorMLP) for layer in tiny_bc4.model.layers)
            assert hf.use_texelator_mlp(tiny_bc4) == []  # nothing left to replace
            mlp = tiny_bc4.model.layers[0].mlp
            with torch.inference_mode():
                x = torch.randn(1, 1, hidden, device="cuda", generator=g).to(torch.bfloat16)
                got, want = mlp(x), mlp.original(x)
                assert mlp.fused and got.shape == want.shape and got.dtype == torch.bfloat16
                assert rrms(want, got) < 1e-2
                xs = torch.randn(1, 5, hidden, device="cuda", generator=g).to(torch.bfloat16)
                assert torch.equal(mlp(xs), mlp.original(xs))
            runner = hf.GraphedGreedy(tiny_bc4, max_cache_len=256)
            eager = runner.generate(ids, 24, eager=True)
            graphed = runner.generate(ids, 24)
            assert torch.equal(eager, graphed)
            assert (graphed == unfused).float().mean() >= 0.75
        finally:
            hf.restore_modules(replaced)
        assert [layer.mlp for layer in tiny_bc4.model.layers] == originals
    finally:
        tiny_bc4.set_attn_implementation("sdpa")


@pytest.mark.parametrize("batch,tokens,heads,kv_heads,dim", [(1, 1, 16, 2, 128), (1, 7, 16, 2, 128),
                                                            (2, 5, 8, 8, 64), (1, 3, 40, 8, 128)])
def test_rope_rotate_half_matches_hf(ext, batch, tokens, heads, kv_heads, dim):
    """``layers.rope_rotate_half`` == Hugging Face's ``apply_rotary_pos_emb`` on bf16 q, k and the
    model's own cos/sin, bit for bit (the same bf16 roundings of both products and of the sum)."""
    from transformers import Qwen2Config
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RotaryEmbedding, apply_rotary_pos_emb

    from texelator_amd import layers

    g = torch.Generator(device="cuda").manual_seed(tokens * heads + dim)
    q = (3 * torch.randn(batch, tokens, heads, dim, device="cuda", generator=g)).to(torch.bfloat16)
    k = (3 * torch.randn(batch, tokens, kv_heads, dim, device="cuda", generator=g)).to(torch.bfloat16)
    config = Qwen2Config(hidden_size=heads * dim, num_attention_heads=heads, num_key_value_heads=kv_heads,
                         head_dim=dim, rope_theta=1e6)
    rotary = Qwen2RotaryEmbedding(config).to("cuda")
    positions = torch.randint(0, 4096, (batch, tokens), device="cuda", generator=g)
    cos, sin = rotary(q, positions)
    want_q, want_k = apply_rotary_pos_emb(q.transpose(1, 2), k.transpose(1, 2), cos, sin)
    got_q, got_k = layers.rope_rotate_half(q, k, cos.contiguous(), sin.contiguous())
    assert torch.equal(want_q.transpose(1, 2), got_q) and torch.equal(want_k.transpose(1, 2), got_k)


def test_texelator_rope_model_is_bitwise_the_module(tiny_bc4):
    """``use_texelator_rope`` on the BC4 Qwen2: prompt logits bitwise those of the unchanged model
    (the kernel reproduces the module's rotary embedding exactly), ``GraphedGreedy`` tokens the
    unchanged runner's, replays equal to eager steps; ``restore_rope`` undoes it."""
    from texelator_amd import hf

    ids = torch.randint(0, 512, (1, 30), generator=torch.Generator().manual_seed(25)).cuda()
    try:
        tiny_bc4.set_attn_implementation("sdpa")
        with torch.inference_mode():
            want = tiny_bc4(ids).logits
        runner = hf.GraphedGreedy(tiny_bc4, max_cache_len=256)
        unchanged = runner.generate(ids, 24)
        changed = hf.use_texelator_rope(tiny_bc4)
        try:
            assert len(changed) == len(tiny_bc4.model.layers)
            tiny_bc4.set_attn_implementation("sdpa")
            with torch.inference_mode():
                assert torch.equal(want, tiny_bc4(ids).logits)
            runner = hf.GraphedGreedy(tiny_bc4, max_cache_len=256)
            eager = runner.generate(ids, 24, eager=True)
            graphed = runner.generate(ids, 24)
            assert torch.equal(eager, graphed) and torch.equal(graphed, unchanged)
        finally:
            hf.restore_rope(changed)
        assert all("forward" not in layer.self_attn.__dict__ for layer in tiny_bc4.model.layers)
    finally:
        tiny_bc4.set_attn_implementation("sdpa")


def test_kv_cache_append_matches_the_static_layer_update(ext):
    """``_cache_update`` on a Hugging Face static cache: one token's k and v (views, as the attention
    forward passes them) land where ``StaticLayer.update`` puts them, the length advances the same and
    the same tensors come back, step after step; a full cache is left as it is; a prompt of several
    tokens takes the cache's own update."""
    import transformers

    from texelator_amd import hf

    config = transformers.Qwen2Config(vocab_size=64, hidden_size=256, intermediate_size=512, num_hidden_layers=1,
                                      num_attention_heads=4, num_key_value_heads=2, head_dim=64)
    ours = transformers.StaticCache(config=config, max_cache_len=8)
    theirs = transformers.StaticCache(config=config, max_cache_len=8)
    g = torch.Generator(device="cuda").manual_seed(30)

    def token_kv(tokens):
        k = torch.randn(1, tokens, 2, 64, device="cuda", generator=g).to(torch.bfloat16).transpose(1, 2)
        v = torch.randn(1, tokens, 2, 64, device="cuda", generator=g).to(torch.bfloat16).transpose(1, 2)
        return k, v

    k, v = token_kv(3)
    hf._cache_update(ours, 0, k, v)
    theirs.update(k, v, 0)
    for step in range(7):
        k, v = token_kv(1)
        got = hf._cache_update(ours, 0, k, v)
        want = theirs.update(k, v, 0) if step < 5 else (theirs.layers[0].keys, theirs.layers[0].values)
        assert got[0] is ours.layers[0].keys and got[1] is ours.layers[0].values
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1]), step
        assert int(ours.layers[0].cumulative_length) == min(4 + step, 8)


def test_texelator_qkv_joins_the_projections(ext, tiny_bc4):
    """``use_texelator_qkv`` (with ``use_texelator_rope``'s forward) on the BC4 Qwen2 with non-zero
    biases: one token's q, k and v from the joined handle match the three projections within bf16
    rounding (the joined GEMV may split K differently); prompts still take the three projections
    (logits bitwise the unchanged model's); graphed tokens equal eager ones and mostly the
    unchanged runner's; ``restore_qkv`` undoes it."""
    from texelator_amd import hf

    ids = torch.randint(0, 512, (1, 30), generator=torch.Generator().manual_seed(26)).cuda()
    attention = [layer.self_attn for layer in tiny_bc4.model.layers]
    saved = [[p.bias.detach().clone() for p in (a.q_proj, a.k_proj, a.v_proj)] for a in attention]
    g = torch.Generator(device="cuda").manual_seed(27)
    try:
        for a in attention:
            for p in (a.q_proj, a.k_proj, a.v_proj):
                p.bias.data.copy_((0.3 * torch.randn(p.bias.shape, device="cuda", generator=g)).to(torch.bfloat16))
        tiny_bc4.set_attn_implementation("sdpa")
        with torch.inference_mode():
            want = tiny_bc4(ids).logits
        unchanged = hf.GraphedGreedy(tiny_bc4, max_cache_len=256).generate(ids, 24)
        changed = hf.use_texelator_rope(tiny_bc4)
        created = hf.use_texelator_qkv(tiny_bc4)
        try:
            assert len(created) == len(attention) and hf.use_texelator_qkv(tiny_bc4) == []
            x = torch.randn(1, 1, tiny_bc4.config.hidden_size, device="cuda", generator=g).to(torch.bfloat16)
            for a in attention:
                got = hf._projections(a, x)
                for part, p in zip(got, (a.q_proj, a.k_proj, a.v_proj)):
                    ref = p(x).float()
                    assert part.shape == ref.shape
                    assert float((part.float() - ref).norm() / ref.norm()) < 1e-2
            tiny_bc4.set_attn_implementation("sdpa")
            with torch.inference_mode():
                assert torch.equal(want, tiny_bc4(ids).logits)
            runner = hf.GraphedGreedy(tiny_bc4, max_cache_len=256)
            eager = runner.generate(ids, 24, eager=True)
            graphed = runner.generate(ids, 24)
            assert torch.equal(eager, graphed)
            assert (graphed == unchanged).float().mean() >= 0.75
        finally:
            hf.restore_rope(changed)
            hf.restore_qkv(tiny_bc4, created)
        assert all("_texelator_qkv" not in a.__dict__ for a in attention)
    finally:
        for a, biases in zip(attention, saved):
            for p, b in zip((a.q_proj, a.k_proj, a.v_proj), biases):
                p.bias.data.copy_(b)
        tiny_bc4.set_attn_implementation("sdpa")


@pytest.mark.parametrize("shape", [(1, 1, 2048), (3, 5120), (2, 12288), (5, 36)])
def test_add_rmsnorm_bf16_matches_torch_and_the_fp32_kernel(ext, shape):
    """The bf16-residual kernel: its sum is torch's bf16 add bit for bit, and its norm of that sum
    (or of the residual alone) is bitwise the fp32-residual kernel's on the same values (same
    reduction order; 12288 columns take the two-pass path); against Hugging Face's RMSNorm at most
    one bf16 step apart."""
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm

    g = torch.Generator(device="cuda").manual_seed(shape[-1] + len(shape))
    residual = (torch.randn(shape, device="cuda", generator=g) * 3).to(torch.bfloat16)
    delta = (torch.randn(shape, device="cuda", generator=g) * 2).to(torch.bfloat16)
    weight = (1 + 0.1 * torch.randn(shape[-1], device="cuda", generator=g)).to(torch.bfloat16)
    total, got = layers.add_rmsnorm_bf16(residual, delta, weight, 1e-6)
    assert torch.equal(total, residual + delta) and got.shape == residual.shape
    flat = total.reshape(-1, shape[-1]).float()
    assert torch.equal(got.reshape(flat.shape), layers.add_rmsnorm(flat.clone(), None, weight, 1e-6))
    none, alone = layers.add_rmsnorm_bf16(residual, None, weight, 1e-6)
    assert none is None
    assert torch.equal(alone.reshape(flat.shape), layers.add_rmsnorm(residual.reshape(flat.shape).float(), None, weight, 1e-6))
    module = Qwen2RMSNorm(shape[-1], eps=1e-6).to(device="cuda", dtype=torch.bfloat16)
    module.weight.data.copy_(weight)
    want = module(total)
    step = torch.maximum(want.float().abs(), got.float().abs()) * 2.0 ** -7
    assert bool(((got.float() - want.float()).abs() <= step + 1e-30).all())


def test_texelator_residuals_are_bitwise_the_norm_modules(tiny_bc4):
    """``use_texelator_residuals`` after ``use_texelator_norms`` and ``use_texelator_mlp``: the attention's
    residual add fused into the post-attention norm and the MLP's residual add fused into the down
    GEMV give the same bits as the separate adds (one token's MLP output with the residual, prompt
    logits and graphed tokens equal); ``restore_rope`` gives the layers their class's forward back."""
    from texelator_amd import hf

    ids = torch.randint(0, 512, (1, 30), generator=torch.Generator().manual_seed(28)).cuda()
    replaced = hf.use_texelator_norms(tiny_bc4)
    replaced += hf.use_texelator_mlp(tiny_bc4)
    try:
        mlp = tiny_bc4.model.layers[0].mlp
        assert isinstance(mlp, hf.TexelatorMLP)
        g = torch.Generator(device="cuda").manual_seed(29)
        hidden = tiny_bc4.config.hidden_size
        for scale in (1.0, 30.0):
            x = (torch.randn(1, 1, hidden, device="cuda", generator=g)).to(torch.bfloat16)
            r = (scale * torch.randn(1, 1, hidden, device="cuda", generator=g)).to(torch.bfloat16)
            assert torch.equal(mlp.forward_residual(x, r), r + mlp(x))
        tiny_bc4.set_attn_implementation("sdpa")
        with torch.inference_mode():
            want = tiny_bc4(ids).logits
        unchanged = hf.GraphedGreedy(tiny_bc4, max_cache_len=256).generate(ids, 24)
        changed = hf.use_texelator_residuals(tiny_bc4)
        try:
            assert len(changed) == len(tiny_bc4.model.layers)
            tiny_bc4.set_attn_implementation("sdpa")
            with torch.inference_mode():
                assert torch.equal(want, tiny_bc4(ids).logits)
            runner = hf.GraphedGreedy(tiny_bc4, max_cache_len=256)
            eager = runner.generate(ids, 24, eager=True)
            graphed = runner.generate(ids, 24)
            assert torch.equal(eager, graphed) and torch.equal(graphed, unchanged)
        finally:
            hf.restore_rope(changed)
        assert all("forward" not in layer.__dict__ for layer in tiny_bc4.model.layers)
    finally:
        hf.restore_modules(replaced)
        tiny_bc4.set_attn_implementation("sdpa")


@pytest.mark.parametrize("shape", [(7, 256), (1, 3, 2048), (2, 5120)])
def test_texelator_rmsnorm_matches_hf_rmsnorm(ext, shape):
    """``TexelatorRMSNorm`` against the Hugging Face module on the same weight: the same formula and
    roundings, so almost every value is bitwise equal and none is more than one bf16 step apart
    (the fp32 sums of squares add in different orders)."""
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm

    from texelator_amd import hf

    g = torch.Generator(device="cuda").manual_seed(shape[-1])
    x = (torch.randn(shape, device="cuda", generator=g) * 3).to(torch.bfloat16)
    norm = Qwen2RMSNorm(shape[-1], eps=1e-6).to(device="cuda", dtype=torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.2 * torch.randn(shape[-1], device="cuda", generator=g))
        want = norm(x)
        got = hf.TexelatorRMSNorm(norm.weight, norm.variance_epsilon)(x)
    assert got.shape == want.shape and got.dtype == torch.bfloat16
    assert (got == want).float().mean() >= 0.99
    assert torch.allclose(got.float(), want.float(), rtol=2 ** -7, atol=0)
