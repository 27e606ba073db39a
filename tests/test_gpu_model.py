"""Model-level GPU tests of the BC4 decoder (texelator_amd.modeling): its hidden states against a
float32 PyTorch restatement on the decoded weights, graph replay against eager decode, the
KV-cached decode against a full recomputation, and the reference's prefill correctness gate
(texelator/prefill.py:88-108)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
from torch.nn import functional

from texelator_amd import _lib, layers, modeling, prefill, runtime

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tiny(ext):
    model = modeling.BC4Decoder(modeling.DecoderConfig.tiny(), max_context=1024, seed=3)
    yield model
    model.close()


@pytest.fixture(scope="module")
def tiny_torch(ext):
    model = modeling.BC4Decoder(modeling.DecoderConfig.tiny(), max_context=1024, seed=3, fused=False)
    yield model
    model.close()


def reference_hidden(model: modeling.BC4Decoder, ids: torch.Tensor, ext) -> torch.Tensor:
    """Float32 forward of the same architecture on the dense decoded weights (attention in fp32)."""
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

    def lin(index, name, x):
        return x @ model.dense_weight(index, name).float().t().contiguous()

    h = model.embed.float()[ids]  # fp32 residual stream, as the decoder keeps it
    group = c.heads // c.kv_heads
    mask = torch.triu(torch.ones(t, t, dtype=torch.bool, device=ids.device), 1)
    for index, layer in enumerate(model.layers):
        x = norm(h, layer.input_norm)
        q = rope(lin(index, "self_attn.q_proj", x).view(t, c.heads, c.head_dim))
        k = rope(lin(index, "self_attn.k_proj", x).view(t, c.kv_heads, c.head_dim))
        v = lin(index, "self_attn.v_proj", x).view(t, c.kv_heads, c.head_dim)
        k = k.repeat_interleave(group, 1)
        v = v.repeat_interleave(group, 1)
        scores = torch.einsum("thd,shd->hts", q, k) / math.sqrt(c.head_dim)
        probs = torch.softmax(scores.masked_fill(mask, float("-inf")), -1)
        attn = torch.einsum("hts,shd->thd", probs, v).reshape(t, -1)
        h = h + lin(index, "self_attn.o_proj", attn)
        x = norm(h, layer.post_norm)
        h = h + lin(index, "mlp.down_proj",
                    functional.silu(lin(index, "mlp.gate_proj", x)) * lin(index, "mlp.up_proj", x))
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


def test_fused_path_matches_torch_path(ext, tiny, tiny_torch):
    """Same seed, same BC4 weights: the fused kernels agree with the plain PyTorch layer glue."""
    ids = prefill.prompt_ids(tiny, 40, seed=5)
    with torch.inference_mode():
        a = tiny.hidden_states(ids, tiny.key_positions[:40], 40)
        b = tiny_torch.hidden_states(ids, tiny_torch.key_positions[:40], 40)
    assert rrms(b, a) < 1e-2
    # decode: the split-length attention against the torch attention over the cache
    ga = tiny.generate(ids, 8, eager=True)
    gb = tiny_torch.generate(ids, 8, eager=True)
    with torch.inference_mode():
        ha = tiny.hidden_states(ga[-1:], tiny.key_positions[47:48], 48)
        hb = tiny_torch.hidden_states(ga[-1:], tiny_torch.key_positions[47:48], 48)
    assert rrms(hb, ha) < 2e-2
    assert (ga == gb).float().mean() >= 0.75


def test_add_rmsnorm_kernel(ext):
    g = torch.Generator(device="cuda").manual_seed(7)
    h = torch.randn(5, 5120, device="cuda", generator=g)
    d = torch.randn(5, 5120, device="cuda", generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(5120, device="cuda", generator=g)).to(torch.bfloat16)
    want_h = h + d.float()
    want = w.float() * (want_h * torch.rsqrt(want_h.square().mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16).float()
    got = layers.add_rmsnorm(h, d, w, 1e-6)
    assert torch.equal(h, want_h)
    assert rrms(want, got) < 4e-3


def test_rope_kv_cache_kernel(ext, tiny):
    c = tiny.config
    g = torch.Generator(device="cuda").manual_seed(8)
    t = 6
    width = (c.heads + 2 * c.kv_heads) * c.head_dim
    qkv = torch.randn(t, width, device="cuda", generator=g).to(torch.bfloat16)
    positions = torch.tensor([0, 3, 7, 100, 511, 1023], device="cuda")
    kc = torch.zeros(c.kv_heads, 1024, c.head_dim, device="cuda", dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    q = layers.rope_kv_cache(qkv, positions, tiny.rope_cos, tiny.rope_sin, c.heads, c.kv_heads, c.head_dim, kc, vc)
    qs = c.heads * c.head_dim
    ks = c.kv_heads * c.head_dim
    want_q = tiny._rope(qkv[:, :qs].reshape(t, c.heads, c.head_dim), positions).reshape(t, -1)
    want_k = tiny._rope(qkv[:, qs:qs + ks].reshape(t, c.kv_heads, c.head_dim), positions)
    assert torch.equal(q, want_q)
    assert torch.equal(kc[:, positions].transpose(0, 1), want_k)
    assert torch.equal(vc[:, positions].transpose(0, 1), qkv[:, qs + ks:].reshape(t, c.kv_heads, c.head_dim))


@pytest.mark.parametrize("position,length,ctx", [(0, 512, 1024), (100, 512, 1024), (511, 512, 1024), (700, 1024, 1024),
                                                 (1023, 1024, 1024), (33000, 33024, 33024)])
@pytest.mark.parametrize("heads,kv", [(40, 8), (64, 8), (8, 8)])
def test_decode_attention_kernel(ext, position, length, ctx, heads, kv):
    """Against an fp32 reference, up to 516 chunks, at 5, 8 (the most the kernel takes) and 1 query
    heads per KV head; a second call on the same workspace repeats the output."""
    d = 128
    g = torch.Generator(device="cuda").manual_seed(position)
    kc = torch.randn(kv, ctx, d, device="cuda", generator=g).to(torch.bfloat16)
    vc = torch.randn(kv, ctx, d, device="cuda", generator=g).to(torch.bfloat16)
    q = (torch.randn(heads * d, device="cuda", generator=g) * 0.3).to(torch.bfloat16)
    pos = torch.tensor([position], device="cuda")
    ws = torch.empty(layers.decode_attention_workspace_bytes(heads, length), dtype=torch.uint8, device="cuda")
    first = layers.decode_attention(q, kc, vc, pos, length, heads, kv, 1 / math.sqrt(d), ws).clone()
    got = layers.decode_attention(q, kc, vc, pos, length, heads, kv, 1 / math.sqrt(d), ws)
    assert torch.equal(first, got)
    got = got.float()
    qf = q.float().view(kv, heads // kv, d)
    keys, values = kc[:, :position + 1].float(), vc[:, :position + 1].float()
    scores = torch.einsum("kgd,ksd->kgs", qf, keys) / math.sqrt(d)
    want = torch.einsum("kgs,ksd->kgd", torch.softmax(scores, -1), values).reshape(1, -1)
    assert rrms(want, got) < 5e-3


def test_swiglu_kernel(ext):
    g = torch.Generator(device="cuda").manual_seed(9)
    gu = (torch.randn(3, 2 * 1024, device="cuda", generator=g) * 3).to(torch.bfloat16)
    got = layers.swiglu(gu).float()
    f = gu.float()
    want = (functional.silu(f[:, :1024]) * f[:, 1024:]).to(torch.bfloat16).float()
    assert rrms(want, got) < 4e-3


def _random_handle(ext, m, k, seed, bias=False):
    g = torch.Generator(device="cuda").manual_seed(seed)
    blocks = torch.randint(0, 256, (m * k // 2,), device="cuda", dtype=torch.uint8, generator=g)
    scales = 0.02 * torch.exp(0.3 * torch.randn(m, device="cuda", generator=g))
    b = (0.1 * torch.randn(m, device="cuda", generator=g)).to(torch.bfloat16) if bias else None
    return ext.pack_encoded_device(blocks, scales.float(), b)


@pytest.mark.parametrize("m,k,bias,ks", [(5120, 5120, False, 4), (5120, 5120, True, 4), (16384, 256, True, 1),
                                         (256, 512, False, 1), (8192, 1024, True, 2), (3072, 4096, False, 6),
                                         (2048, 4096, True, 8)])
def test_add_rmsnorm_split_is_bit_identical(ext, m, k, bias, ks):
    """linear_split + add_rmsnorm_split == linear + add_rmsnorm, bit for bit, for K split counts
    that take the kernel's loop-free variants (1, 2, 4) and its generic loop (6, 8)."""
    handle = _random_handle(ext, m, k, seed=m + k, bias=bias)
    try:
        assert ext.gemv_plan(handle)[0] == ks
        g = torch.Generator(device="cuda").manual_seed(11)
        x = torch.randn(1, k, device="cuda", generator=g).to(torch.bfloat16)
        w = (1 + 0.1 * torch.randn(m, device="cuda", generator=g)).to(torch.bfloat16)
        h0 = torch.randn(1, m, device="cuda", generator=g)
        h1, h2 = h0.clone(), h0.clone()
        want = layers.add_rmsnorm(h1, ext.linear(handle, x), w, 1e-6)
        layers.linear_split(handle, x)
        got = layers.add_rmsnorm_split(h2, handle, w, 1e-6, out=torch.empty_like(want))
        assert torch.equal(h1, h2)
        assert torch.equal(want, got)
    finally:
        ext.free(handle)


@pytest.mark.parametrize("heads,kv,k,bias", [(40, 8, 5120, True), (4, 2, 256, False)])
def test_rope_kv_cache_split_is_bit_identical(ext, heads, kv, k, bias):
    d, ctx = 128, 1024
    handle = _random_handle(ext, (heads + 2 * kv) * d, k, seed=heads, bias=bias)
    try:
        g = torch.Generator(device="cuda").manual_seed(13)
        x = torch.randn(1, k, device="cuda", generator=g).to(torch.bfloat16)
        angles = torch.rand(ctx, d, device="cuda", generator=g) * 6
        cos, sin = angles.cos().contiguous(), angles.sin().contiguous()
        pos = torch.tensor([517], device="cuda")
        caches = [torch.zeros(kv, ctx, d, device="cuda", dtype=torch.bfloat16) for _ in range(4)]
        want = layers.rope_kv_cache(ext.linear(handle, x), pos, cos, sin, heads, kv, d, caches[0], caches[1])
        layers.linear_split(handle, x)
        got = layers.rope_kv_cache_split(handle, pos, cos, sin, heads, kv, d, caches[2], caches[3],
                                         torch.empty(heads * d, device="cuda", dtype=torch.bfloat16))
        assert torch.equal(want.view(-1), got)
        assert torch.equal(caches[0], caches[2]) and torch.equal(caches[1], caches[3])
    finally:
        ext.free(handle)


@pytest.mark.parametrize("vocab,hidden", [(151936, 2048), (32003, 5120), (1000, 128), (17, 256)])
def test_lm_head_argmax_matches_float64_logits(ext, vocab, hidden):
    """The lm_head GEMV + argmax: its bf16 logits are the float64 products rounded once (to fp32
    summation error), and the token is the first row among the largest of those logits, as
    torch.argmax picks it."""
    g = torch.Generator(device="cuda").manual_seed(vocab + hidden)
    w = (torch.randn(vocab, hidden, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(1, hidden, device="cuda", generator=g).to(torch.bfloat16)
    ws = torch.empty(layers.lm_head_argmax_workspace_bytes(), dtype=torch.uint8, device="cuda")
    logits = torch.empty(vocab, dtype=torch.bfloat16, device="cuda")
    token = layers.lm_head_argmax(w, x, ws, logits=logits)
    ref = (w.double() @ x.double().t()).view(-1)
    err = (logits.double() - ref).abs()
    assert bool((err <= ref.abs() * 2.0 ** -8 + 1e-4).all())
    assert int(token) == int(torch.argmax(logits.float()))


def test_lm_head_argmax_takes_the_first_of_equal_logits(ext):
    """Rows that are copies of one another tie exactly; the first of them wins, across workgroups."""
    vocab, hidden = 40000, 1024
    g = torch.Generator(device="cuda").manual_seed(3)
    w = (torch.randn(vocab, hidden, device="cuda", generator=g) * 0.01).to(torch.bfloat16)
    x = torch.randn(1, hidden, device="cuda", generator=g).to(torch.bfloat16)
    best = torch.randn(hidden, device="cuda", generator=g).sign().to(torch.bfloat16) * x.view(-1).sign()
    for row in (39000, 777, 20001):  # the same winning row at three places, the smallest not first written
        w[row] = best
    ws = torch.empty(layers.lm_head_argmax_workspace_bytes(), dtype=torch.uint8, device="cuda")
    assert int(layers.lm_head_argmax(w, x, ws)) == 777


def test_decoder_greedy_token_agrees_with_torch_head(ext, tiny):
    """The decoder's fused head picks torch's argmax token, or one whose logit is within rounding
    of it (the two sum the dot products in different orders)."""
    ids = prefill.prompt_ids(tiny, 40, seed=12)
    with torch.inference_mode():
        hidden = tiny.hidden_states(ids, tiny.key_positions[:40], 40)
        for t in range(40):
            h = hidden[t:t + 1].contiguous()
            got = int(tiny.greedy_token(h))
            logits = tiny.logits(h).float().view(-1)
            assert logits[got] >= logits.max() - 2.0 ** -7 * logits.abs().max()


def _prefill_workspace(ext, handle, tokens):
    return torch.empty(max(ext.workspace_bytes(handle, tokens), 16), dtype=torch.uint8, device="cuda")


@pytest.mark.parametrize("m,k,tokens,bias", [(5120, 5120, 512, True), (2048, 11008, 512, False),
                                             (5120, 27648, 300, True), (2048, 4096, 64, True), (5120, 5120, 20, False),
                                             (27648, 5120, 32, True)])
def test_add_rmsnorm_prefill_split_is_bit_identical(ext, m, k, tokens, bias):
    """prefill_split + add_rmsnorm_prefill_split == linear + add_rmsnorm over several tokens, bit
    for bit (the prefill reduce's rounding: the bias added after the sum's bf16 rounding), for split
    counts that take the consumer's loop-free variants and its generic loop. 27648 rows at 32
    tokens split four ways, where linear runs the split-group tile (no partials) and prefill_split
    the partial-writing 32-token tile."""
    handle = _random_handle(ext, m, k, seed=m + k + tokens, bias=bias)
    try:
        g = torch.Generator(device="cuda").manual_seed(tokens)
        x = torch.randn(tokens, k, device="cuda", generator=g).to(torch.bfloat16)
        w = (1 + 0.1 * torch.randn(m, device="cuda", generator=g)).to(torch.bfloat16)
        h0 = torch.randn(tokens, m, device="cuda", generator=g)
        h1, h2 = h0.clone(), h0.clone()
        want = layers.add_rmsnorm(h1, ext.linear(handle, x), w, 1e-6)
        ws = _prefill_workspace(ext, handle, tokens)
        splits = layers.prefill_split(handle, x, ws)
        assert splits > 1
        got = layers.add_rmsnorm_prefill_split(h2, handle, ws, w, 1e-6, out=torch.empty_like(want))
        assert torch.equal(h1, h2)
        assert torch.equal(want, got)
    finally:
        ext.free(handle)


@pytest.mark.parametrize("heads,kv,k,tokens", [(40, 8, 5120, 512), (16, 2, 2048, 300), (28, 4, 3584, 64)])
def test_rope_kv_cache_prefill_split_is_bit_identical(ext, heads, kv, k, tokens):
    """prefill_split + rope_kv_cache_prefill_split == linear + rope_kv_cache over a prompt, bit for
    bit, with a nonzero q/k/v bias (added after the sum's bf16 rounding, as the prefill reduce does)."""
    d, ctx = 128, 1024
    handle = _random_handle(ext, (heads + 2 * kv) * d, k, seed=heads + tokens, bias=True)
    try:
        g = torch.Generator(device="cuda").manual_seed(17)
        x = torch.randn(tokens, k, device="cuda", generator=g).to(torch.bfloat16)
        angles = torch.rand(ctx, d, device="cuda", generator=g) * 6
        cos, sin = angles.cos().contiguous(), angles.sin().contiguous()
        pos = torch.arange(100, 100 + tokens, device="cuda")
        caches = [torch.zeros(kv, ctx, d, device="cuda", dtype=torch.bfloat16) for _ in range(4)]
        want = layers.rope_kv_cache(ext.linear(handle, x), pos, cos, sin, heads, kv, d, caches[0], caches[1])
        ws = _prefill_workspace(ext, handle, tokens)
        assert layers.prefill_split(handle, x, ws) > 1
        got = layers.rope_kv_cache_prefill_split(handle, ws, pos, cos, sin, heads, kv, d, caches[2], caches[3])
        assert torch.equal(want, got)
        assert torch.equal(caches[0], caches[2]) and torch.equal(caches[1], caches[3])
    finally:
        ext.free(handle)


def test_prefill_split_refusals(ext):
    """prefill_split runs nothing where its call would not split K (a 512-token gate GEMM on the
    wide tile), below the prefill threshold, or on the dense backend: UnsupportedError."""
    handle = _random_handle(ext, 27648, 5120, seed=3)
    try:
        x = torch.zeros(512, 5120, device="cuda", dtype=torch.bfloat16)
        ws = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
        with pytest.raises(_lib.UnsupportedError):
            layers.prefill_split(handle, x, ws)
        ext.set_prefill(handle, 64, 1024)
        with pytest.raises(_lib.UnsupportedError):
            layers.prefill_split(handle, x[:32], ws)
        ext.set_prefill(handle, 16, 1024)
        ext.set_prefill_backend(handle, 1)
        with pytest.raises(_lib.UnsupportedError):
            layers.prefill_split(handle, x[:64], ws)
    finally:
        ext.free(handle)


@pytest.mark.parametrize("config", ["class_27b", "qwen25_3b_style"])
def test_decoder_prefill_with_split_consumers_is_bit_identical(ext, config):
    """Two layers of the 27B- and 3B-class decoders: the 512-token prefill whose q|k|v, o and down
    GEMMs leave their K-split partials to RoPE and add+RMSNorm gives the hidden states, keys and
    values of the GEMM + reduce path, bit for bit."""
    from dataclasses import replace

    model = modeling.BC4Decoder(replace(getattr(modeling.DecoderConfig, config)(), layers=2), max_context=512, seed=7)
    try:
        ids = prefill.prompt_ids(model, 512)
        positions = model.key_positions[:512]
        with torch.inference_mode():
            split = model.hidden_states(ids, positions, 512).clone()
            kc, vc = model.k_cache.clone(), model.v_cache.clone()
            model.split_prefill = False
            plain = model.hidden_states(ids, positions, 512)
        assert torch.equal(split, plain)
        assert torch.equal(kc, model.k_cache) and torch.equal(vc, model.v_cache)
    finally:
        model.close()


@pytest.mark.parametrize("heads,kv,k,bias,position,length,ks", [
    (40, 8, 5120, True, 517, 1024, 3), (40, 8, 5120, False, 0, 512, 3), (4, 2, 256, False, 63, 512, 1),
    (4, 2, 256, True, 64, 1024, 1), (48, 8, 1024, True, 300, 512, 2), (16, 4, 4096, False, 1000, 1024, 6),
    (8, 4, 4096, True, 127, 1024, 8)])
def test_decode_attention_split_is_bit_identical(ext, heads, kv, k, bias, position, length, ks):
    """RoPE + KV write inside the attention kernel == rope_kv_cache_split + decode_attention, bit
    for bit: output and both caches; repeated on the same workspace. The qkv split counts cover the
    kernel's loop-free partial reads (1-3) and its generic loop (6, 8)."""
    d, ctx = 128, 1024
    handle = _random_handle(ext, (heads + 2 * kv) * d, k, seed=heads + position, bias=bias)
    try:
        assert ext.gemv_plan(handle)[0] == ks
        g = torch.Generator(device="cuda").manual_seed(position + 5)
        x = torch.randn(1, k, device="cuda", generator=g).to(torch.bfloat16)
        angles = torch.rand(ctx, d, device="cuda", generator=g) * 6
        cos, sin = angles.cos().contiguous(), angles.sin().contiguous()
        pos = torch.tensor([position], device="cuda")
        kc = torch.randn(kv, ctx, d, device="cuda", generator=g).to(torch.bfloat16)
        vc = torch.randn(kv, ctx, d, device="cuda", generator=g).to(torch.bfloat16)
        caches = [kc.clone(), vc.clone(), kc.clone(), vc.clone()]
        ws = torch.empty(layers.decode_attention_workspace_bytes(heads, length), dtype=torch.uint8, device="cuda")
        scale = 1 / math.sqrt(d)
        layers.linear_split(handle, x)
        q = layers.rope_kv_cache_split(handle, pos, cos, sin, heads, kv, d, caches[0], caches[1],
                                       torch.empty(heads * d, device="cuda", dtype=torch.bfloat16))
        want = layers.decode_attention(q, caches[0], caches[1], pos, length, heads, kv, scale, ws).clone()
        for _ in range(2):
            rope_row = torch.cat([cos[position], sin[position]])
            got = layers.decode_attention_split(handle, pos, rope_row, heads, kv, d, caches[2], caches[3], length,
                                                scale, ws)
            assert torch.equal(want, got)
            assert torch.equal(caches[0], caches[2]) and torch.equal(caches[1], caches[3])
    finally:
        ext.free(handle)


@pytest.mark.parametrize("inter,k,bias,lookahead", [(8192, 1024, False, 1), (11008, 2048, True, 2),
                                                    (27648, 5120, False, 4), (16384, 4096, True, 8)])
def test_linear_swiglu_is_bit_identical(ext, inter, k, bias, lookahead):
    """The gate|up GEMV with the SwiGLU epilogue == linear + swiglu, bit for bit."""
    handle = _random_handle(ext, 2 * inter, k, seed=inter + k, bias=bias)
    try:
        ext.set_lookahead(handle, lookahead)
        assert ext.gemv_plan(handle) == (1, False)
        g = torch.Generator(device="cuda").manual_seed(17)
        for scale in (1.0, 30.0):  # large inputs drive silu into both saturated ends
            x = (scale * torch.randn(1, k, device="cuda", generator=g)).to(torch.bfloat16)
            want = layers.swiglu(ext.linear(handle, x))
            got = layers.linear_swiglu(handle, x)
            assert got.shape == (1, inter)
            assert torch.equal(want, got)
    finally:
        ext.free(handle)


def test_linear_swiglu_refuses_unsupported_handles(ext):
    split = _random_handle(ext, 512, 4096, seed=1)       # 32 row groups x 32 tile columns: K splits 8 ways
    odd = _random_handle(ext, 48, 256, seed=2)           # halves of 24 rows
    x = torch.zeros(1, 4096, device="cuda", dtype=torch.bfloat16)
    try:
        assert ext.gemv_plan(split)[0] > 1
        with pytest.raises(_lib.UnsupportedError):
            layers.linear_swiglu(split, x)
        with pytest.raises(_lib.TexelatorError, match="16-row aligned"):
            layers.linear_swiglu(odd, x[:, :256])
    finally:
        ext.free(split)
        ext.free(odd)


@pytest.mark.parametrize("inter,k,lookahead", [(11008, 2048, 1), (27648, 5120, 2), (1000, 1024, 4)])
def test_linear_swiglu_pair_is_bit_identical(ext, inter, k, lookahead):
    """The SwiGLU GEMV over separate gate and up handles == the SwiGLU GEMV of the merged [gate | up]
    handle of the same blocks and == linear + swiglu of that (unsplit) handle, bit for bit (inter %
    16 == 0); against linear + linear + swiglu of the two handles, whose GEMVs may split K and sum
    in another order, within bf16 rounding. 1000 rows leave the last row group partly empty."""
    g = torch.Generator(device="cuda").manual_seed(inter + k)
    blocks = [torch.randint(0, 256, (inter * k // 2,), device="cuda", dtype=torch.uint8, generator=g) for _ in range(2)]
    scales = [(0.02 * torch.exp(0.3 * torch.randn(inter, device="cuda", generator=g))).float() for _ in range(2)]
    gate = ext.pack_encoded_device(blocks[0], scales[0], None)
    up = ext.pack_encoded_device(blocks[1], scales[1], None)
    merged = ext.pack_encoded_device(torch.cat(blocks), torch.cat(scales), None) if inter % 16 == 0 else None
    try:
        for h in (gate, up, merged):
            if h is not None:
                ext.set_lookahead(h, lookahead)
        for scale in (1.0, 30.0):  # large inputs drive silu into both saturated ends
            x = (scale * torch.randn(1, k, device="cuda", generator=g)).to(torch.bfloat16)
            got = layers.linear_swiglu_pair(gate, up, x)
            assert got.shape == (1, inter)
            near = layers.swiglu(torch.cat([ext.linear(gate, x), ext.linear(up, x)], dim=-1)).float()
            err = (got.float() - near).norm() / near.norm()
            assert err < 1e-2, f"relative RMS {err:.3g}"
            if merged is not None:
                assert ext.gemv_plan(merged)[0] == 1
                assert torch.equal(layers.linear_swiglu(merged, x), got)
                assert torch.equal(layers.swiglu(ext.linear(merged, x)), got)
            again = torch.empty_like(got)
            layers.linear_swiglu_pair(gate, up, x, again)
            assert torch.equal(got, again)
    finally:
        for h in (gate, up, merged):
            if h is not None:
                ext.free(h)


def test_linear_swiglu_pair_refusals(ext):
    gate = _random_handle(ext, 256, 1024, seed=5)
    up_bias = _random_handle(ext, 256, 1024, seed=6, bias=True)
    other = _random_handle(ext, 512, 1024, seed=7)
    x = torch.zeros(1, 1024, device="cuda", dtype=torch.bfloat16)
    try:
        with pytest.raises(_lib.UnsupportedError):
            layers.linear_swiglu_pair(gate, up_bias, x)
        with pytest.raises(_lib.TexelatorError, match="same shape"):
            layers.linear_swiglu_pair(gate, other, x)
        with pytest.raises(_lib.TexelatorError, match="wrong length"):
            layers.linear_swiglu_pair(gate, gate, x[:, :512])
    finally:
        for h in (gate, up_bias, other):
            ext.free(h)


@pytest.mark.parametrize("m,k", [(2560, 2048), (5120, 5120), (1024, 5120), (16384, 256), (1000, 1024)])
def test_linear_add_bias_is_bit_identical(ext, m, k):
    """linear_add_bias == linear(x) + bias in bf16 (two roundings), bit for bit, whatever the
    handle's one-token plan: every K split in one workgroup, split partials plus the reduce kernel,
    or unsplit; at two lookaheads and at inputs large enough that the second rounding matters."""
    handle = _random_handle(ext, m, k, seed=m + k)
    try:
        g = torch.Generator(device="cuda").manual_seed(m - k)
        bias = (0.5 * torch.randn(m, device="cuda", generator=g)).to(torch.bfloat16)
        for la in (1, 2):
            ext.set_lookahead(handle, la)
            for scale in (1.0, 40.0):
                x = (scale * torch.randn(1, k, device="cuda", generator=g)).to(torch.bfloat16)
                want = ext.linear(handle, x) + bias
                got = layers.linear_add_bias(handle, x, bias)
                assert got.shape == (1, m)
                assert torch.equal(got, want), (la, scale)
        module = runtime.TexelatorLinear([handle], bias=torch.nn.Parameter(bias, requires_grad=False))
        x3 = x.reshape(1, 1, k)
        assert torch.equal(module(x3), (ext.linear(handle, x) + bias).reshape(1, 1, m))
    finally:
        ext.free(handle)


@pytest.mark.parametrize("rows,k,bias", [((2048, 256, 256), 2048, False), ((5120, 1024, 1024), 5120, True),
                                         ((64, 48, 100), 1024, True)])
def test_concat_rows_joins_the_matrices(ext, rows, k, bias):
    """A joined handle decodes to the sources' dense weights stacked in order, bit for bit (the tile
    copy keeps every row group and scale in place, the last source's ragged rows included), and
    its GEMV and prefill results match the sources' within bf16 rounding (the joined shape may split
    K differently); settings follow the first handle; the sources keep working."""
    handles = [_random_handle(ext, m, k, seed=m + i, bias=bias) for i, m in enumerate(rows)]
    ext.set_lookahead(handles[0], 2)
    joined = ext.concat_rows(handles)
    try:
        assert ext.shape(joined) == (sum(rows), k) and ext.lookahead(joined) == 2
        assert torch.equal(ext.decode_dense(joined), torch.cat([ext.decode_dense(h) for h in handles]))
        g = torch.Generator(device="cuda").manual_seed(k)
        for tokens in (1, 40):
            x = torch.randn(tokens, k, device="cuda", generator=g).to(torch.bfloat16)
            want = torch.cat([ext.linear(h, x) for h in handles], dim=-1).float()
            got = ext.linear(joined, x).float()
            assert got.shape == want.shape
            assert float((got - want).norm() / want.norm()) < 1e-2, tokens
    finally:
        ext.free(joined)
        for h in handles:
            ext.free(h)


def test_concat_rows_refusals(ext):
    a = _random_handle(ext, 100, 1024, seed=1)
    b = _random_handle(ext, 128, 1024, seed=2)
    c = _random_handle(ext, 128, 2048, seed=3)
    d = _random_handle(ext, 128, 1024, seed=4, bias=True)
    try:
        with pytest.raises(_lib.TexelatorError, match="multiple of 16"):
            ext.concat_rows([a, b])
        with pytest.raises(_lib.TexelatorError, match="share K"):
            ext.concat_rows([b, c])
        with pytest.raises(_lib.TexelatorError, match="bias"):
            ext.concat_rows([b, d])
        joined = ext.concat_rows([b, a])  # ragged rows last is fine
        ext.free(joined)
    finally:
        for h in (a, b, c, d):
            ext.free(h)


def test_linear_add_bias_refuses_a_handle_with_its_own_bias(ext):
    handle = _random_handle(ext, 256, 1024, seed=9, bias=True)
    try:
        x = torch.zeros(1, 1024, device="cuda", dtype=torch.bfloat16)
        bias = torch.zeros(256, device="cuda", dtype=torch.bfloat16)
        with pytest.raises(_lib.TexelatorError, match="own bias"):
            layers.linear_add_bias(handle, x, bias)
        with pytest.raises(_lib.TexelatorError, match="one token"):
            layers.linear_add_bias(handle, torch.zeros(2, 1024, device="cuda", dtype=torch.bfloat16), bias)
    finally:
        ext.free(handle)


def test_split_decode_with_fused_swiglu_is_bit_identical(ext):
    """A model whose gate|up GEMV runs unsplit takes the fused SwiGLU epilogue in its split decode
    step; the step still equals the unsplit fused step bit for bit."""
    config = modeling.DecoderConfig(layers=2, hidden=512, heads=4, kv_heads=2, head_dim=128, intermediate=8192,
                                    vocab=512)
    model = modeling.BC4Decoder(config, max_context=256, seed=5)
    try:
        assert ext.gemv_plan(model.layers[0].handles["gate_up"]) == (1, False)
        ids = prefill.prompt_ids(model, 20, seed=8)
        with torch.inference_mode():
            model.prefill(ids)
            token = ids[-1:]
            model.split_decode = False
            a = model.hidden_states(token, model.key_positions[20:21], 128).clone()
            model.split_decode = True
            b = model.hidden_states(token, model.key_positions[20:21], 128)
        assert torch.equal(a, b)
    finally:
        model.close()


def test_capture_after_the_cache_is_full(ext):
    """A decode that fills the cache leaves the model at position max_context. Capturing a step
    from there (benchmark_decode captures before its prefill) runs the warm-up step at the last row,
    inside the RoPE table, and leaves the cache, the token and the position as they were; the
    benchmark then runs twice in a row on a model whose context is its whole cache."""
    model = modeling.BC4Decoder(modeling.DecoderConfig.tiny(), max_context=96, seed=5)
    try:
        ids = prefill.prompt_ids(model, 40, seed=4)
        with torch.inference_mode():
            model.prefill(ids)
            model.decode(56, 40)  # positions 40..95: the cache is full
            assert int(model.position) == 96
            k, v, token = model.k_cache.clone(), model.v_cache.clone(), model.token.clone()
            model.graphs.clear()
            model.capture(96)
            torch.cuda.synchronize()
        assert int(model.position) == 96 and torch.equal(model.token, token)
        assert torch.equal(model.k_cache, k) and torch.equal(model.v_cache, v)
        for _ in range(2):
            assert prefill.benchmark_decode(model, prompt_tokens=40, context=96)["steps"] == 56
    finally:
        model.close()


@pytest.mark.parametrize("attention_in_o,norm_in_gemv", [(True, True), (True, False), (False, True), (False, False)])
def test_split_decode_step_is_bit_identical(ext, tiny, attention_in_o, norm_in_gemv):
    """A decode step through the split-K consumers equals the unsplit fused step, bit for bit, with
    the attention's chunk merge inside the o GEMV or as its own kernel, and the add+RMSNorms inside
    the following GEMVs or as their own kernels."""
    ids = prefill.prompt_ids(tiny, 30, seed=6)
    try:
        tiny.attention_in_o = attention_in_o
        tiny.norm_in_gemv = norm_in_gemv
        with torch.inference_mode():
            tiny.prefill(ids)
            token = ids[-1:]
            tiny.split_decode = False
            a = tiny.hidden_states(token, tiny.key_positions[30:31], 512).clone()
            ka = tiny.k_cache[:, :, 30].clone()
            tiny.split_decode = True
            b = tiny.hidden_states(token, tiny.key_positions[30:31], 512)
            kb = tiny.k_cache[:, :, 30].clone()
    finally:
        tiny.attention_in_o = True
        tiny.norm_in_gemv = True
    assert torch.equal(a, b)
    assert torch.equal(ka, kb)


def _norm_reference(ext, delta, hidden, g, bias_scale=1.0):
    """Residual, weight and eps for a norm-consumer test, with delta's partials written."""
    k = _hip_shape_k(ext, delta)
    layers.linear_split(delta, (torch.randn(1, k, device="cuda", generator=g) * bias_scale).to(torch.bfloat16))
    h0 = torch.randn(1, hidden, device="cuda", generator=g)
    w = (1 + 0.1 * torch.randn(hidden, device="cuda", generator=g)).to(torch.bfloat16)
    return h0, w, 1e-6


def _hip_shape_k(ext, handle):
    from texelator_amd import _hip
    return _hip.shape(handle)[1]


@pytest.mark.parametrize("hidden,dk,cm,bias", [(2048, 2048, 2560, True), (2048, 11008, 2048, False),
                                               (256, 512, 1024, True), (1024, 4096, 1024, False)])
def test_linear_split_norm_is_bit_identical(ext, hidden, dk, cm, bias):
    """add_rmsnorm_split + linear_split == linear_split_norm, bit for bit: the updated residual and
    the consumer's split partials (read back through add_rmsnorm_split), for producers split 1-8 ways
    and consumers split 1-4 ways, twice in a row."""
    delta = _random_handle(ext, hidden, dk, seed=hidden + dk, bias=bias)
    consumer = _random_handle(ext, cm, hidden, seed=cm + 1, bias=bias)
    try:
        g = torch.Generator(device="cuda").manual_seed(hidden + cm)
        h0, w, eps = _norm_reference(ext, delta, hidden, g)
        w2 = (1 + 0.1 * torch.randn(cm, device="cuda", generator=g)).to(torch.bfloat16)
        r0 = torch.randn(1, cm, device="cuda", generator=g)
        h_want = h0.clone()
        x = layers.add_rmsnorm_split(h_want, delta, w, eps, torch.empty(1, hidden, device="cuda", dtype=torch.bfloat16))
        layers.linear_split(consumer, x)
        r_want = r0.clone()
        read_want = layers.add_rmsnorm_split(r_want, consumer, w2, eps, torch.empty(1, cm, device="cuda", dtype=torch.bfloat16))
        for _ in range(2):
            h_in, h_out = h0.clone(), torch.full_like(h0, float("nan"))
            assert layers.linear_split_norm(consumer, h_in, h_out, delta, w, eps)
            r_got = r0.clone()
            read_got = layers.add_rmsnorm_split(r_got, consumer, w2, eps, torch.empty(1, cm, device="cuda", dtype=torch.bfloat16))
            assert torch.equal(h_out, h_want) and torch.equal(h_in, h0)
            assert torch.equal(r_got, r_want) and torch.equal(read_got, read_want)
    finally:
        ext.free(delta)
        ext.free(consumer)


@pytest.mark.parametrize("hidden,dk,inter,bias", [(2048, 2048, 11008, True), (256, 512, 512, False),
                                                  (1024, 4096, 8192, True)])
def test_linear_swiglu_norm_is_bit_identical(ext, hidden, dk, inter, bias):
    """add_rmsnorm_split + linear_swiglu == linear_swiglu_norm, bit for bit (the activations and the
    updated residual), twice in a row."""
    delta = _random_handle(ext, hidden, dk, seed=hidden + dk + 3, bias=bias)
    gate_up = _random_handle(ext, 2 * inter, hidden, seed=inter, bias=bias)
    try:
        assert ext.gemv_plan(gate_up) == (1, False)
        g = torch.Generator(device="cuda").manual_seed(inter)
        h0, w, eps = _norm_reference(ext, delta, hidden, g)
        h_want = h0.clone()
        x = layers.add_rmsnorm_split(h_want, delta, w, eps, torch.empty(1, hidden, device="cuda", dtype=torch.bfloat16))
        want = layers.linear_swiglu(gate_up, x).clone()
        for _ in range(2):
            h_in, h_out = h0.clone(), torch.full_like(h0, float("nan"))
            got = torch.full_like(want, float("nan"))
            assert layers.linear_swiglu_norm(gate_up, h_in, h_out, delta, w, eps, got)
            assert torch.equal(got, want) and torch.equal(h_out, h_want) and torch.equal(h_in, h0)
    finally:
        ext.free(delta)
        ext.free(gate_up)


@pytest.mark.parametrize("hidden,cm,vocab,token", [(2048, 2560, 4096, 17), (256, 1024, 512, 511), (1024, 1024, 300, 1000)])
def test_linear_split_embed_norm_is_bit_identical(ext, hidden, cm, vocab, token):
    """Embedding row + add_rmsnorm (no delta) + linear_split == linear_split_embed_norm, bit for bit
    (the residual and the consumer's partials read back through add_rmsnorm_split); a token past the
    table takes its last row."""
    consumer = _random_handle(ext, cm, hidden, seed=cm + vocab, bias=True)
    try:
        g = torch.Generator(device="cuda").manual_seed(hidden + token)
        embed = torch.randn(vocab, hidden, device="cuda", generator=g).to(torch.bfloat16)
        w = (1 + 0.1 * torch.randn(hidden, device="cuda", generator=g)).to(torch.bfloat16)
        w2 = (1 + 0.1 * torch.randn(cm, device="cuda", generator=g)).to(torch.bfloat16)
        r0 = torch.randn(1, cm, device="cuda", generator=g)
        tok = torch.tensor([token], device="cuda")
        h_want = embed[min(token, vocab - 1)].float().view(1, hidden).clone()
        x = layers.add_rmsnorm(h_want, None, w, 1e-6)
        layers.linear_split(consumer, x)
        r_want = r0.clone()
        read_want = layers.add_rmsnorm_split(r_want, consumer, w2, 1e-6, torch.empty(1, cm, device="cuda", dtype=torch.bfloat16))
        h_got = torch.full((1, hidden), float("nan"), device="cuda")
        assert layers.linear_split_embed_norm(consumer, embed, tok, h_got, w, 1e-6)
        r_got = r0.clone()
        read_got = layers.add_rmsnorm_split(r_got, consumer, w2, 1e-6, torch.empty(1, cm, device="cuda", dtype=torch.bfloat16))
        assert torch.equal(h_got, h_want)
        assert torch.equal(r_got, r_want) and torch.equal(read_got, read_want)
    finally:
        ext.free(consumer)


def test_linear_norm_refusals(ext):
    """The same buffer for both residuals is refused; a 27B-class gate|up GEMV (hidden 5120, above
    the 2048 the prologue holds) returns False and launches nothing."""
    from texelator_amd._lib import TexelatorError

    delta = _random_handle(ext, 5120, 5120, seed=1)
    gate_up = _random_handle(ext, 2 * 27648, 5120, seed=2)
    try:
        layers.linear_split(delta, torch.ones(1, 5120, device="cuda", dtype=torch.bfloat16))
        h = torch.zeros(1, 5120, device="cuda")
        w = torch.ones(5120, device="cuda", dtype=torch.bfloat16)
        with pytest.raises(TexelatorError, match="another buffer"):
            layers.linear_split_norm(delta, h, h, delta, w, 1e-6)
        out = torch.zeros(1, 27648, device="cuda", dtype=torch.bfloat16)
        h_out = torch.zeros_like(h)
        assert not layers.linear_swiglu_norm(gate_up, h, h_out, delta, w, 1e-6, out)
        torch.cuda.synchronize()
        assert not out.any() and not h_out.any()
    finally:
        ext.free(delta)
        ext.free(gate_up)


@pytest.mark.parametrize("heads,kv,k,position,length,bias", [
    (16, 2, 2048, 600, 768, True), (16, 2, 2048, 0, 64, False), (16, 2, 2048, 1023, 1024, True),
    (16, 2, 2048, 100, 512, False), (12, 2, 1536, 300, 640, True), (40, 8, 5120, 200, 256, True),
    (8, 8, 1024, 63, 128, False)])
def test_decode_attention_o_split_is_bit_identical(ext, heads, kv, k, position, length, bias):
    """RoPE + attention with the chunk merge inside the o GEMV == decode_attention_split +
    linear_split(o), bit for bit: the add+RMSNorm read of o's split partials, the residual and both
    caches; group sizes 8, 6, 5 and 1, o split 1-4 ways, 1-16 chunks, twice on the same workspace."""
    d, ctx = 128, 1024
    qkv = _random_handle(ext, (heads + 2 * kv) * d, k, seed=heads + position, bias=bias)
    o = _random_handle(ext, k, heads * d, seed=heads + position + 1, bias=bias)
    try:
        g = torch.Generator(device="cuda").manual_seed(position + 9)
        x = torch.randn(1, k, device="cuda", generator=g).to(torch.bfloat16)
        angles = torch.rand(ctx, d, device="cuda", generator=g) * 6
        rope_row = torch.cat([angles[position].cos(), angles[position].sin()]).contiguous()
        pos = torch.tensor([position], device="cuda")
        kc = torch.randn(kv, ctx, d, device="cuda", generator=g).to(torch.bfloat16)
        vc = torch.randn(kv, ctx, d, device="cuda", generator=g).to(torch.bfloat16)
        h0 = torch.randn(1, k, device="cuda", generator=g)
        w = (1 + 0.1 * torch.randn(k, device="cuda", generator=g)).to(torch.bfloat16)
        ws = torch.empty(layers.decode_attention_workspace_bytes(heads, length), dtype=torch.uint8, device="cuda")
        scale = 1 / math.sqrt(d)
        layers.linear_split(qkv, x)
        caches = [kc.clone(), vc.clone()]
        attn = layers.decode_attention_split(qkv, pos, rope_row, heads, kv, d, caches[0], caches[1], length, scale, ws)
        layers.linear_split(o, attn)
        h_want = h0.clone()
        want = layers.add_rmsnorm_split(h_want, o, w, 1e-6, torch.empty(1, k, device="cuda", dtype=torch.bfloat16))
        for _ in range(2):
            got_caches = [kc.clone(), vc.clone()]
            assert layers.decode_attention_o_split(qkv, o, pos, rope_row, heads, kv, d, got_caches[0], got_caches[1],
                                                   length, scale, ws)
            h_got = h0.clone()
            got = layers.add_rmsnorm_split(h_got, o, w, 1e-6, torch.empty(1, k, device="cuda", dtype=torch.bfloat16))
            assert torch.equal(want, got) and torch.equal(h_want, h_got)
            assert torch.equal(caches[0], got_caches[0]) and torch.equal(caches[1], got_caches[1])
    finally:
        ext.free(qkv)
        ext.free(o)


def test_decode_attention_o_split_refusals(ext):
    """Where the merge does not fit the o GEMV (more than 16 chunks, or 40 heads x 16 chunks per o
    workgroup) the call returns False and launches nothing: the caches stay as they were."""
    heads, kv, k, d, ctx = 40, 8, 5120, 128, 2048
    qkv = _random_handle(ext, (heads + 2 * kv) * d, k, seed=3)
    o = _random_handle(ext, k, heads * d, seed=4)
    try:
        kc = torch.zeros(kv, ctx, d, device="cuda", dtype=torch.bfloat16)
        vc = torch.zeros_like(kc)
        pos = torch.tensor([5], device="cuda")
        rope_row = torch.ones(2 * d, device="cuda")
        layers.linear_split(qkv, torch.ones(1, k, device="cuda", dtype=torch.bfloat16))
        for length in (1088, 1024):
            ws = torch.empty(layers.decode_attention_workspace_bytes(heads, length), dtype=torch.uint8, device="cuda")
            assert not layers.decode_attention_o_split(qkv, o, pos, rope_row, heads, kv, d, kc, vc, length, 0.1, ws)
        torch.cuda.synchronize()
        assert not kc.any() and not vc.any()
    finally:
        ext.free(qkv)
        ext.free(o)


def test_prompt_flash_attention_matches_cached_attention(ext, tiny):
    """The prompt path (causal flash attention over the prompt's own cache rows) agrees with the
    cached fp32 attention that any other multi-token call uses."""
    ids = prefill.prompt_ids(tiny, 48, seed=9)
    with torch.inference_mode():
        a = tiny.hidden_states(ids, tiny.key_positions[:48], 48).clone()
        tiny.flash_prompt_attention = False
        try:
            b = tiny.hidden_states(ids, tiny.key_positions[:48], 48)
        finally:
            tiny.flash_prompt_attention = True
    assert rrms(b, a) < 1e-2


@pytest.mark.parametrize("inter,k,tokens,bias,tile", [
    (27648, 5120, 512, False, None),    # the 27B gate|up: its default prefill is the wide tile, unsplit
    (11008, 2048, 512, True, None),     # the 3B gate|up: the 128-token tile, unsplit
    (1024, 512, 512, True, 7),
    (208, 272, 300, False, 7),          # a partial row tile, K not a multiple of 128, a partial token tile
    (2048, 384, 700, True, 7),          # two token tiles
    (1024, 512, 128, True, 6),
    (208, 272, 100, False, 6),
    (1024, 512, 64, False, 8),
    (208, 272, 40, True, 8),
    (1024, 512, 32, True, 9),
    (208, 272, 17, False, 9),
])
def test_linear_swiglu_prefill_is_bit_identical(ext, inter, k, tokens, bias, tile):
    """The gate|up prefill GEMM with the SwiGLU epilogue == linear + swiglu, bit for bit, on the
    wide tile and the 128-, 64- and 32-token tiles."""
    handle = _random_handle(ext, 2 * inter, k, seed=inter + tokens, bias=bias)
    try:
        if tile is not None:
            ext.set_prefill_backend(handle, tile)
        g = torch.Generator(device="cuda").manual_seed(19)
        for scale in (1.0, 30.0):  # large inputs drive silu into both saturated ends
            x = (scale * torch.randn(tokens, k, device="cuda", generator=g)).to(torch.bfloat16)
            want = layers.swiglu(ext.linear(handle, x))
            got = layers.linear_swiglu_prefill(handle, x)
            assert got.shape == (tokens, inter)
            assert torch.equal(want, got)
    finally:
        ext.free(handle)


def test_linear_swiglu_prefill_lut_mode_is_bit_identical(ext):
    """The same with the palette read from a table (a perturbed palette)."""
    from oracle import bc4

    rng = np.random.default_rng(23)
    table = (bc4.palette() * (1 + 0.01 * rng.standard_normal((255, 255, 8)))).astype(np.float32)
    handle = _random_handle(ext, 2 * 512, 640, seed=29, bias=True)
    try:
        ext.set_palette_table(handle, torch.from_numpy(table).cuda())
        ext.set_prefill_backend(handle, 7)
        x = torch.randn(512, 640, device="cuda", generator=torch.Generator(device="cuda").manual_seed(31)).to(torch.bfloat16)
        want = layers.swiglu(ext.linear(handle, x))
        assert torch.equal(want, layers.linear_swiglu_prefill(handle, x))
    finally:
        ext.free(handle)


def test_linear_swiglu_prefill_refuses_other_calls(ext):
    handle = _random_handle(ext, 2 * 1024, 5120, seed=3)
    odd = _random_handle(ext, 48, 256, seed=4)
    x = torch.zeros(128, 5120, device="cuda", dtype=torch.bfloat16)
    try:
        with pytest.raises(_lib.UnsupportedError):   # 128 tokens over 40 tile columns: K is split
            layers.linear_swiglu_prefill(handle, x)
        with pytest.raises(_lib.UnsupportedError):   # below the prefill threshold
            layers.linear_swiglu_prefill(handle, x[:8])
        ext.set_prefill_backend(odd, 5)
        ext.set_prefill_backend(handle, 5)
        with pytest.raises(_lib.UnsupportedError):   # the pair tile has no SwiGLU epilogue
            layers.linear_swiglu_prefill(handle, torch.zeros(512, 5120, device="cuda", dtype=torch.bfloat16))
        with pytest.raises(_lib.TexelatorError, match="16-row aligned"):
            layers.linear_swiglu_prefill(odd, x[:, :256].contiguous())
    finally:
        ext.free(handle)
        ext.free(odd)


def test_decoder_prefill_with_fused_swiglu_is_bit_identical(ext):
    """Two layers of the 27B-class decoder: the 512-token prefill whose gate|up GEMM applies SwiGLU
    in its epilogue gives the hidden states of the GEMM + SwiGLU kernels, bit for bit."""
    from dataclasses import replace

    model = modeling.BC4Decoder(replace(modeling.DecoderConfig.class_27b(), layers=2), max_context=512, seed=5)
    try:
        ids = prefill.prompt_ids(model, 512)
        positions = model.key_positions[:512]
        x = torch.zeros(512, model.config.hidden, device="cuda", dtype=torch.bfloat16)
        layers.linear_swiglu_prefill(model.layers[0].handles["gate_up"], x)   # the fused path applies
        with torch.inference_mode():
            fused = model.hidden_states(ids, positions, 512).clone()
            model.gate_up_swiglu_prefill = False
            plain = model.hidden_states(ids, positions, 512)
        assert torch.equal(fused, plain)
    finally:
        model.close()


@pytest.mark.parametrize("tokens,heads,kv_heads", [(512, 40, 8), (300, 16, 2), (64, 4, 4), (1, 8, 1), (1000, 12, 4)])
def test_prefill_attention_matches_fp32_reference(ext, tokens, heads, kv_heads):
    """The prompt-attention kernel against a float32 causal softmax attention on the same bf16
    inputs; cache rows past the prompt hold NaN, which must not reach any output."""
    d, ctx = 128, 1088
    g = torch.Generator(device="cuda").manual_seed(tokens + heads)
    q = (torch.randn(tokens, heads * d, device="cuda", generator=g) * 2).to(torch.bfloat16)
    kc = torch.full((kv_heads, ctx, d), float("nan"), device="cuda").to(torch.bfloat16)
    vc = kc.clone()
    kc[:, :tokens] = torch.randn(kv_heads, tokens, d, device="cuda", generator=g).to(torch.bfloat16)
    vc[:, :tokens] = torch.randn(kv_heads, tokens, d, device="cuda", generator=g).to(torch.bfloat16)
    scale = 1 / math.sqrt(d)
    got = layers.prefill_attention(q, kc, vc, heads, kv_heads, scale)
    torch.cuda.synchronize()
    group = heads // kv_heads
    qf = q.float().view(tokens, heads, d).transpose(0, 1)                        # [H, T, d]
    kf = kc[:, :tokens].float().repeat_interleave(group, 0)                     # [H, T, d]
    vf = vc[:, :tokens].float().repeat_interleave(group, 0)
    scores = torch.matmul(qf, kf.transpose(1, 2).contiguous()) * scale          # fp32
    mask = torch.triu(torch.ones(tokens, tokens, dtype=torch.bool, device="cuda"), 1)
    probs = torch.softmax(scores.masked_fill(mask, float("-inf")), dim=-1)
    want = torch.matmul(probs, vf).transpose(0, 1).reshape(tokens, heads * d)
    assert torch.isfinite(got.float()).all()
    assert rrms(want, got.float()) < 5e-3


def test_decoder_prompt_attention_kernel_matches_flash(ext, tiny):
    """The decoder's prompt with this library's attention kernel and with torch's flash kernel give
    hidden states equal to within bf16 noise."""
    ids = torch.randint(0, tiny.config.vocab, (200,), device="cuda", generator=torch.Generator(device="cuda").manual_seed(37))
    positions = tiny.key_positions[:200]
    with torch.inference_mode():
        assert tiny.prompt_attention_kernel
        own = tiny.hidden_states(ids, positions, 200).clone()
        tiny.prompt_attention_kernel = False
        try:
            flash = tiny.hidden_states(ids, positions, 200)
        finally:
            tiny.prompt_attention_kernel = True
    assert rrms(flash.float(), own.float()) < 1e-2
