"""A Qwen2-style decoder whose q/k/v/o/gate/up/down linears are BC4 handles.

This is the model-level harness for decode and prefill tok/s. The reference installs its
``TexelatorLinear`` into Hugging Face modules (``runtime.py:210-263``,
``standalone.py:102-158``) and decodes through ``model.generate``. Here the same linears drive a
compact decoder with a static KV cache, so that a whole decode step (all layers, sampling and
the cache update) can be captured once as a HIP graph and replayed per token. The host then
does no per-token work, and decode speed is set by the GPU.

Layer math follows Qwen2, the architecture of BASELINE configs 4 and 5:
- RMSNorm in fp32 with ``weight * x``;
- rotate-half RoPE with ``theta``;
- grouped-query attention with q/k/v biases;
- SwiGLU MLP.

The residual stream and the SwiGLU product are kept in fp32; every linear reads and writes bf16.

Attention uses plain batched products whose right operands are contiguous (no transposed
views), with the softmax in fp32.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
from torch.nn import functional

from .runtime import TexelatorLinear, extension, free


@dataclass(frozen=True)
class DecoderConfig:
    layers: int
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    rms_eps: float = 1e-6
    rope_theta: float = 1e6
    qkv_bias: bool = True

    @staticmethod
    def qwen25_3b_style() -> "DecoderConfig":
        """BASELINE config 4."""
        return DecoderConfig(layers=36, hidden=2048, heads=16, kv_heads=2, head_dim=128, intermediate=11008,
                             vocab=151936)

    @staticmethod
    def class_27b() -> "DecoderConfig":
        """BASELINE config 5."""
        return DecoderConfig(layers=64, hidden=5120, heads=40, kv_heads=8, head_dim=128, intermediate=27648,
                             vocab=151936)

    @staticmethod
    def tiny() -> "DecoderConfig":
        return DecoderConfig(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=64, intermediate=512, vocab=512)

    def linear_shapes(self) -> list[tuple[str, int, int]]:
        """(name, M = out features, K = in features) of one layer's seven linears."""
        q, kv = self.heads * self.head_dim, self.kv_heads * self.head_dim
        return [("self_attn.q_proj", q, self.hidden), ("self_attn.k_proj", kv, self.hidden),
                ("self_attn.v_proj", kv, self.hidden), ("self_attn.o_proj", self.hidden, q),
                ("mlp.gate_proj", self.intermediate, self.hidden), ("mlp.up_proj", self.intermediate, self.hidden),
                ("mlp.down_proj", self.hidden, self.intermediate)]

    def bc4_bytes(self) -> int:
        return self.layers * sum(m * k // 2 + 4 * m for _, m, k in self.linear_shapes())


def random_bc4(m: int, k: int, generator: torch.Generator, device: torch.device,
               std: float = 0.02) -> tuple[torch.Tensor, torch.Tensor]:
    """Random BC4 matrix on the device: uniform block bytes (every endpoint and selector value
    occurs) and row scales 1.75 * std * LogNormal(0, 0.1). Uniform blocks decode to palette
    values with standard deviation ~0.57, so the weights have standard deviation ~std."""
    blocks = torch.randint(0, 256, (m * (k // 16) * 8,), dtype=torch.uint8, device=device, generator=generator)
    scales = 1.75 * std * torch.exp(0.1 * torch.randn(m, device=device, generator=generator))
    return blocks, scales


def init_std(config: "DecoderConfig", name: str, depth_scaled: bool) -> float:
    """Random-init standard deviation of a linear: Hugging Face's ``initializer_range`` 0.02.
    With ``depth_scaled``, the two projections that write into the residual stream (o_proj,
    down_proj) also get GPT-2's 1/sqrt(2 * layers)."""
    if depth_scaled and name in ("self_attn.o_proj", "mlp.down_proj"):
        return 0.02 / math.sqrt(2 * config.layers)
    return 0.02


class _Layer:
    def __init__(self):
        self.linears: dict[str, TexelatorLinear] = {}
        self.biases: dict[str, torch.Tensor] = {}
        self.input_norm: torch.Tensor | None = None
        self.post_norm: torch.Tensor | None = None


class BC4Decoder:
    """Decoder with BC4 linears, a static KV cache and graph-captured decode steps."""

    def __init__(self, config: DecoderConfig, max_context: int, device: torch.device | str = "cuda", seed: int = 0,
                 lookahead: int = 1, linear_source=None, depth_scaled: bool = True, embed_std: float = 1.0):
        """``linear_source(layer, name, m, k)`` may return ``(blocks, scales)`` device tensors for a
        linear (reference block layout). By default every linear is a seeded random BC4 matrix.

        The random init follows Hugging Face's for Qwen2: weights N(0, 0.02) (here as BC4), norms
        1, and q/k/v biases 0. The biases are still passed to the handles, so the kernels' bias
        epilogues run.

        Two defaults condition the deep random network, so that rounding differences between
        the decode and prefill kernels are not amplified chaotically through 64 layers:
        - ``depth_scaled``: GPT-2's 1/sqrt(2 * layers) on o_proj and down_proj;
        - a unit-scale embedding (``embed_std``).
        ``depth_scaled=False, embed_std=0.02`` gives Hugging Face's plain init."""
        self.config = config
        self.device = torch.device(device)
        self.max_context = int(max_context)
        ext = extension()
        c = config
        g = torch.Generator(device=self.device).manual_seed(seed)
        bf16 = torch.bfloat16

        def normal(*shape, std=0.02):
            return (torch.randn(shape, device=self.device, generator=g) * std).to(bf16)

        self.embed = normal(c.vocab, c.hidden, std=embed_std)
        self.lm_head = normal(c.vocab, c.hidden)
        self.final_norm = torch.ones(c.hidden, device=self.device, dtype=bf16)
        self.handles: list[int] = []
        self.layers: list[_Layer] = []
        try:
            for index in range(c.layers):
                layer = _Layer()
                layer.input_norm = torch.ones(c.hidden, device=self.device, dtype=bf16)
                layer.post_norm = torch.ones(c.hidden, device=self.device, dtype=bf16)
                for name, m, k in c.linear_shapes():
                    source = linear_source(index, name, m, k) if linear_source else None
                    blocks, scales = source if source is not None else random_bc4(
                        m, k, g, self.device, init_std(c, name, depth_scaled))
                    bias = (torch.zeros(m, device=self.device, dtype=bf16)
                            if c.qkv_bias and name in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj")
                            else None)
                    handle = ext.pack_encoded_device(blocks, scales, bias)
                    if bias is not None:
                        layer.biases[name] = bias
                    self.handles.append(handle)
                    ext.set_lookahead(handle, lookahead)
                    layer.linears[name] = TexelatorLinear([handle])
                    del blocks, scales
                self.layers.append(layer)
        except Exception:
            free(self.handles)
            raise
        # K cache [layer, kv_head, position, head_dim]; V cache transposed [layer, kv_head, head_dim, position]
        self.k_cache = torch.zeros((c.layers, c.kv_heads, self.max_context, c.head_dim), device=self.device, dtype=bf16)
        self.v_cache = torch.zeros((c.layers, c.kv_heads, c.head_dim, self.max_context), device=self.device, dtype=bf16)
        inv_freq = 1.0 / (c.rope_theta ** (torch.arange(0, c.head_dim, 2, device=self.device, dtype=torch.float32)
                                           / c.head_dim))
        angles = torch.arange(self.max_context, device=self.device, dtype=torch.float32)[:, None] * inv_freq[None, :]
        angles = torch.cat([angles, angles], dim=-1)
        self.rope_cos, self.rope_sin = angles.cos(), angles.sin()
        self.key_positions = torch.arange(self.max_context, device=self.device)
        # decode-step state (static buffers read and advanced by the captured graphs)
        self.token = torch.zeros(1, dtype=torch.long, device=self.device)
        self.position = torch.zeros(1, dtype=torch.long, device=self.device)
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self._pool = None

    # ---------------------------------------------------------------- building blocks
    def set_prefill(self, threshold: int, tile_rows: int = 1024) -> None:
        ext = extension()
        for handle in self.handles:
            ext.set_prefill(handle, threshold, tile_rows)

    def set_prefill_backend(self, backend: int) -> None:
        ext = extension()
        for handle in self.handles:
            ext.set_prefill_backend(handle, backend)

    def _rms_norm(self, x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
        """RMSNorm of the fp32 residual stream, returned as the bf16 input of the next linears."""
        xf = x.float()
        xf = xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + self.config.rms_eps)
        return weight * xf.to(torch.bfloat16)

    def _rope(self, x: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        # x: [T, heads, head_dim]
        cos = self.rope_cos.index_select(0, positions)[:, None, :]
        sin = self.rope_sin.index_select(0, positions)[:, None, :]
        xf = x.float()
        half = xf.shape[-1] // 2
        rotated = torch.cat([-xf[..., half:], xf[..., :half]], dim=-1)
        return (xf * cos + rotated * sin).to(torch.bfloat16)

    def _attention(self, index: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, positions: torch.Tensor,
                   length: int) -> torch.Tensor:
        """q [T, heads, d], k/v [T, kv, d] at ``positions``; attends keys 0..length-1 causally.

        Keys are cached as rows ([kv, position, d]) and values transposed ([kv, d, position]), so
        scores^T = K q^T and out^T = V^T P^T are batched products whose right operands are
        contiguous and whose left operands are row-strided cache slices."""
        c = self.config
        tokens = q.shape[0]
        group = c.heads // c.kv_heads
        self.k_cache[index].index_copy_(1, positions, k.transpose(0, 1))
        self.v_cache[index].index_copy_(2, positions, v.permute(1, 2, 0))
        keys = self.k_cache[index, :, :length]                      # [kv, L, d]
        values_t = self.v_cache[index, :, :, :length]               # [kv, d, L]
        # queries as [kv, d, group * T] (column = g * T + t), contiguous
        qt = q.view(tokens, c.kv_heads, group, c.head_dim).permute(1, 3, 2, 0).reshape(
            c.kv_heads, c.head_dim, group * tokens).contiguous()
        # scores accumulate and stay in fp32 (as flash attention keeps them), never rounded to bf16
        scores = torch.bmm(keys, qt, out_dtype=torch.float32) * (1.0 / math.sqrt(c.head_dim))   # [kv, L, G*T]
        future = self.key_positions[:length, None] > positions.repeat(group)[None, :]
        scores = scores.masked_fill(future, float("-inf"))
        probs = torch.softmax(scores, dim=1).to(torch.bfloat16)     # [kv, L, G*T], contiguous
        out_t = torch.bmm(values_t, probs)                          # [kv, d, G*T]
        return out_t.view(c.kv_heads, c.head_dim, group, tokens).permute(3, 0, 2, 1).reshape(
            tokens, c.heads * c.head_dim)

    def hidden_states(self, ids: torch.Tensor, positions: torch.Tensor, length: int) -> torch.Tensor:
        """Final-norm hidden states [T, hidden] (bf16) for tokens ``ids`` at ``positions``.

        The residual stream is kept in fp32 and the SwiGLU product is formed in fp32; every
        linear reads bf16 activations and writes bf16 outputs."""
        c = self.config
        h = self.embed.index_select(0, ids).float()
        for index, layer in enumerate(self.layers):
            x = self._rms_norm(h, layer.input_norm)
            lin = layer.linears
            q = lin["self_attn.q_proj"](x).view(-1, c.heads, c.head_dim)
            k = lin["self_attn.k_proj"](x).view(-1, c.kv_heads, c.head_dim)
            v = lin["self_attn.v_proj"](x).view(-1, c.kv_heads, c.head_dim)
            q, k = self._rope(q, positions), self._rope(k, positions)
            h = h + lin["self_attn.o_proj"](self._attention(index, q, k, v, positions, length)).float()
            x = self._rms_norm(h, layer.post_norm)
            act = functional.silu(lin["mlp.gate_proj"](x).float()) * lin["mlp.up_proj"](x).float()
            h = h + lin["mlp.down_proj"](act.to(torch.bfloat16)).float()
        return self._rms_norm(h, self.final_norm)

    def logits(self, hidden: torch.Tensor) -> torch.Tensor:
        return functional.linear(hidden, self.lm_head)

    # ---------------------------------------------------------------- prefill and decode
    @torch.inference_mode()
    def prefill(self, ids: torch.Tensor) -> torch.Tensor:
        """Run the prompt (positions 0..T-1), fill the cache, return the next greedy token [1]."""
        tokens = ids.numel()
        if tokens > self.max_context:
            raise ValueError("prompt longer than the cache")
        positions = self.key_positions[:tokens]
        hidden = self.hidden_states(ids.view(-1), positions, tokens)
        next_token = self.logits(hidden[-1:]).argmax(-1)
        self.token.copy_(next_token)
        self.position.fill_(tokens)
        return next_token

    def _bucket(self, position: int) -> int:
        return min(self.max_context, (position // 512 + 1) * 512)

    def _step(self, length: int) -> None:
        hidden = self.hidden_states(self.token, self.position, length)
        self.token.copy_(self.logits(hidden).argmax(-1))
        self.position.add_(1)

    @torch.inference_mode()
    def capture(self, length: int) -> torch.cuda.CUDAGraph:
        """Capture one decode step attending to ``length`` cache positions (a multiple of 512)."""
        if length in self.graphs:
            return self.graphs[length]
        saved_token, saved_position = self.token.clone(), self.position.clone()
        stream = torch.cuda.Stream(self.device)
        stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(stream):
            self._step(length)                       # warm-up outside the graph
        torch.cuda.current_stream(self.device).wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self._pool, stream=stream):
            self._step(length)
        if self._pool is None:
            self._pool = graph.pool()
        self.graphs[length] = graph
        self.token.copy_(saved_token)
        self.position.copy_(saved_position)
        return graph

    @torch.inference_mode()
    def decode(self, steps: int, position: int, eager: bool = False) -> None:
        """Advance ``steps`` greedy tokens from host-known ``position`` (the cache holds 0..position-1)."""
        if position + steps > self.max_context:
            raise ValueError("decode would run past the cache")
        for p in range(position, position + steps):
            length = self._bucket(p)
            if eager:
                self._step(length)
            else:
                self.capture(length).replay()

    def generate(self, ids: torch.Tensor, new_tokens: int, eager: bool = False) -> torch.Tensor:
        """Greedy generation; returns the ``new_tokens`` generated ids (one host sync per token)."""
        out = [self.prefill(ids).clone()]
        position = ids.numel()
        for _ in range(new_tokens - 1):
            self.decode(1, position, eager=eager)
            position += 1
            out.append(self.token.clone())
        return torch.cat(out)

    def close(self) -> None:
        self.graphs.clear()
        free(self.handles)
        self.handles = []
