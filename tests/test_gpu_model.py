"""Model-level GPU tests of the BC4 decoder (texelator_amd.modeling): its hidden states against a
float32 PyTorch restatement on the decoded weights, graph replay against eager decode, the
KV-cached decode against a full recomputation, and the reference's prefill correctness gate
(texelator/prefill.py:88-108)."""
from __future__ import annotations

import math

import pytest
import torch
from torch.nn import functional

from texelator_amd import modeling, prefill

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tiny(ext):
    model = modeling.BC4Decoder(modeling.DecoderConfig.tiny(), max_context=1024, seed=3)
    yield model
    model.close()


def reference_hidden(model: modeling.BC4Decoder, ids: torch.Tensor, ext) -> torch.Tensor:
    """Float32 forward of the same architecture on the dense decoded weights."""
    c = model.config
    t = ids.numel()
    pos = torch.arange(t, device=ids.device)
    inv = 1.0 / (c.rope_theta ** (torch.arange(0, c.head_dim, 2, device=ids.device).float() / c.head_dim))
    ang = pos.float()[:, None] * inv[None, :]
    ang = torch.cat([ang, ang], -1)
    cos, sin = ang.cos()[:, None, :], ang.sin()[:, None, :]

    def norm(x, w):
        return w.float() * (x * torch.rsqrt(x.square().mean(-1, keepdim=True) + c.rms_eps))

    def rope(x):
        h = x.shape[-1] // 2
        return x * cos + torch.cat([-x[..., h:], x[..., :h]], -1) * sin

    def lin(layer, name, x):
        w = ext.decode_dense(layer.linears[name].handles[0]).float()
        y = x @ w.t().contiguous()
        return y + layer.biases[name].float() if name in layer.biases else y

    h = model.embed.float()[ids]  # fp32 residual stream, as the decoder keeps it
    group = c.heads // c.kv_heads
    mask = torch.triu(torch.ones(t, t, dtype=torch.bool, device=ids.device), 1)
    for layer in model.layers:
        x = norm(h, layer.input_norm)
        q = rope(lin(layer, "self_attn.q_proj", x).view(t, c.heads, c.head_dim))
        k = rope(lin(layer, "self_attn.k_proj", x).view(t, c.kv_heads, c.head_dim))
        v = lin(layer, "self_attn.v_proj", x).view(t, c.kv_heads, c.head_dim)
        k = k.repeat_interleave(group, 1)
        v = v.repeat_interleave(group, 1)
        scores = torch.einsum("thd,shd->hts", q, k) / math.sqrt(c.head_dim)
        probs = torch.softmax(scores.masked_fill(mask, float("-inf")), -1)
        attn = torch.einsum("hts,shd->thd", probs, v).reshape(t, -1)
        h = h + lin(layer, "self_attn.o_proj", attn)
        x = norm(h, layer.post_norm)
        h = h + lin(layer, "mlp.down_proj", functional.silu(lin(layer, "mlp.gate_proj", x)) * lin(layer, "mlp.up_proj", x))
    return norm(h, model.final_norm)


def rrms(ref: torch.Tensor, got: torch.Tensor) -> float:
    ref, got = ref.float(), got.float()
    return float(torch.sqrt(torch.mean((got - ref) ** 2)) / torch.sqrt(torch.mean(ref ** 2)))


@pytest.mark.parametrize("tokens,threshold", [(20, 16), (20, 1 << 30), (77, 1), (5, 16)])
def test_hidden_states_match_fp32_reference(ext, tiny, tokens, threshold):
    ids = prefill.prompt_ids(tiny, tokens, seed=tokens)
    tiny.set_prefill(threshold)
    try:
        with torch.inference_mode():
            got = tiny.hidden_states(ids, tiny.key_positions[:tokens], tokens)
            want = reference_hidden(tiny, ids, ext)
    finally:
        tiny.set_prefill(16)
    assert torch.isfinite(got.float()).all()
    assert rrms(want, got) < 2e-2


def test_graph_decode_equals_eager_decode_and_recompute(ext, tiny):
    ids = prefill.prompt_ids(tiny, 30, seed=1)
    eager = tiny.generate(ids, 12, eager=True)
    graphed = tiny.generate(ids, 12, eager=False)
    assert torch.equal(eager, graphed)
    # the cached decode's last hidden state equals a full recomputation of the whole sequence
    sequence = torch.cat([ids, graphed[:-1]])
    with torch.inference_mode():
        tiny.prefill(ids)
        tiny.decode(11, 30, eager=True)
        full = tiny.hidden_states(sequence, tiny.key_positions[:sequence.numel()], sequence.numel())
        # one more eager step from the same state gives the hidden state of the last token
        step_hidden = tiny.hidden_states(graphed[-2:-1], tiny.key_positions[40:41], 41)
    assert rrms(full[-1:], step_hidden) < 2e-2


def test_decode_crosses_context_buckets(ext, tiny):
    ids = prefill.prompt_ids(tiny, 500, seed=2)
    out = tiny.generate(ids, 30)          # positions 500..529 cross the 512 bucket boundary
    assert out.shape == (30,) and int(out.max()) < tiny.config.vocab


def test_benchmark_prefill_gate_and_report(ext, tiny):
    result = prefill.benchmark_prefill(tiny, tokens=64, warmup=1, runs=2)
    assert result["correctness"]["relative_rms"] <= prefill.RRMS_LIMIT
    assert result["fused_bc4_mfma"]["tokens"] == 64 and result["scalar_gemv"]["gpu_seconds_median"] > 0


def test_benchmark_decode_reports_buckets(ext, tiny):
    result = prefill.benchmark_decode(tiny, prompt_tokens=100, context=600)
    assert result["steps"] == 500 and set(result["per_bucket"]) == {"512", "1024"}
    assert result["gpu_tokens_per_second"] > 0
