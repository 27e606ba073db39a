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

from torch.nn.attention import SDPBackend, sdpa_kernel

from . import layers
from ._lib import UnsupportedError
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
        return DecoderConfig(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=128, intermediate=512, vocab=512)

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


def encoded_bc4(m: int, k: int, generator: torch.Generator, lut: torch.Tensor, std: float = 0.02
                ) -> tuple[torch.Tensor, torch.Tensor]:
    """A random-init dense weight ``N(0, std^2)`` [M, K], BC4-encoded on the device by this build's
    PTQ encoder (no activation moments): ``(blocks, scales)`` device tensors in the reference's
    block layout. This is what a converted random-init model holds."""
    from .encoder import encode_matrix_tensor

    weight = torch.randn((m, k), device=lut.device, generator=generator) * std
    blocks, scales = encode_matrix_tensor(weight, torch.ones(k, device=lut.device), lut)
    del weight
    return blocks.reshape(-1), scales


def init_std(config: "DecoderConfig", name: str, depth_scaled: bool) -> float:
    """Random-init standard deviation of a linear: Hugging Face's ``initializer_range`` 0.02.
    With ``depth_scaled``, the two projections that write into the residual stream (o_proj,
    down_proj) also get GPT-2's 1/sqrt(2 * layers)."""
    if depth_scaled and name in ("self_attn.o_proj", "mlp.down_proj"):
        return 0.02 / math.sqrt(2 * config.layers)
    return 0.02


# Longest prompt the decoder sends to this library's prompt-attention kernel: it is faster than
# torch's flash kernel at 512 tokens (25 vs 36 us for 40/8 heads) and slower at 2048 (210 vs 164 us).
PROMPT_ATTENTION_MAX_TOKENS = 1024


def prompt_attention_supported(config: "DecoderConfig") -> bool:
    """Whether the prompt-attention kernel handles this configuration (head_dim 128, grouped heads)."""
    return config.head_dim == 128 and config.heads % config.kv_heads == 0


# Distinct encoded weight sets of a random-init model (layer i uses set i % DISTINCT_LAYERS; each
# layer still holds its own copy in memory, so every decode step streams the whole model from HBM).
DISTINCT_LAYERS = 4


# Merged handles of a layer: rows of q, k, v (one launch) and of gate, up (one launch).
MERGED = {
    "qkv": ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"),
    "o": ("self_attn.o_proj",),
    "gate_up": ("mlp.gate_proj", "mlp.up_proj"),
    "down": ("mlp.down_proj",),
}


class _Layer:
    def __init__(self):
        self.linears: dict[str, TexelatorLinear] = {}     # keys of MERGED
        self.handles: dict[str, int] = {}                  # keys of MERGED -> library handle
        self.rows: dict[str, tuple[int, int]] = {}         # reference linear name -> (first row, rows)
        self.biases: dict[str, torch.Tensor] = {}          # merged key -> bias
        self.input_norm: torch.Tensor | None = None
        self.post_norm: torch.Tensor | None = None


class BC4Decoder:
    """Decoder with BC4 linears, a static KV cache and graph-captured decode steps.

    The seven linears of a layer are packed as four handles: q|k|v and gate|up are merged along
    the output rows (one launch each), o and down stay single. With ``fused`` (the default) the
    layer glue runs as this library's kernels (``texelator_amd.layers``): add+RMSNorm, RoPE+KV
    write, split-length decode attention and SwiGLU. Without it, the same math runs as plain
    PyTorch ops (the cross-check path).

    With ``split_decode`` (the default; needs ``fused``) a one-token step hands the split-K
    partials of qkv, o and down straight to their consumer kernels (the decode attention, which
    applies RoPE and writes the KV caches itself, and add+RMSNorm), and the gate|up GEMV applies
    SwiGLU in its epilogue, so a layer is eight kernels instead of thirteen; the results are
    bit-identical to the unsplit fused path."""

    def __init__(self, config: DecoderConfig, max_context: int, device: torch.device | str = "cuda", seed: int = 0,
                 lookahead: int = 1, linear_source=None, depth_scaled: bool = True, embed_std: float = 1.0,
                 fused: bool = True, split_decode: bool = True, gate_up_lookahead: int = 1,
                 weights: str = "encoded", distinct_layers: int = DISTINCT_LAYERS):
        """``linear_source(layer, name, m, k)`` may return ``(blocks, scales)`` device tensors for a
        linear (reference block layout). By default every linear is a seeded random BC4 matrix.

        ``lookahead`` is the decode GEMV lookahead of every handle but gate|up, which takes
        ``gate_up_lookahead``. Since the GEMV prologue copies x and the seed tables into LDS
        without VALU work, one tile in flight is fastest for the fused SwiGLU GEMV too (37.8 vs
        39.7 us per call at two, interleaved on one GPU); before that, two measured 2% faster on
        the decode step. Lookahead 2-4 makes the split q|k|v, o and down GEMVs slower.

        The random init follows Hugging Face's for Qwen2: weights N(0, 0.02) (here as BC4), norms
        1, and q/k/v biases 0. The biases are still passed to the handles, so the kernels' bias
        epilogues run.

        Two defaults condition the deep random network, so that rounding differences between
        the decode and prefill kernels are not amplified chaotically through 64 layers:
        - ``depth_scaled``: GPT-2's 1/sqrt(2 * layers) on o_proj and down_proj;
        - a unit-scale embedding (``embed_std``).
        ``depth_scaled=False, embed_std=0.02`` gives Hugging Face's plain init.

        ``weights`` chooses the BC4 data of the linears that ``linear_source`` does not supply:
        ``"encoded"`` (the default) encodes dense ``N(0, std^2)`` weights with this build's PTQ
        encoder on the GPU, as a converted random-init model holds; ``distinct_layers`` such
        weight sets are encoded and layer i takes set ``i % distinct_layers`` (each layer still
        has its own copy in memory). ``"uniform"`` draws every block byte uniformly (every
        endpoint and selector value occurs), with row scales setting the weights' spread."""
        if weights not in ("encoded", "uniform"):
            raise ValueError("weights must be 'encoded' or 'uniform'")
        if distinct_layers < 1:
            raise ValueError("distinct_layers must be positive")
        self.weights = weights
        self.config = config
        self.device = torch.device(device)
        self.max_context = int(max_context)
        self.fused = fused
        self.split_decode = fused and split_decode
        self.flash_prompt_attention = fused
        # prefill of the merged gate|up handle with the SwiGLU epilogue where the call allows it
        self.gate_up_swiglu_prefill = fused
        # prefill GEMMs that split K leave their partials to RoPE and add+RMSNorm (no reduce kernel)
        self.split_prefill = fused
        # greedy next token by this library's lm_head GEMV + argmax (else torch's linear + argmax)
        self.fused_head = fused and config.hidden % 128 == 0
        # short caches: the attention's chunk merge inside the o GEMV (tx_decode_attention_o_split)
        self.attention_in_o = fused
        # the add+RMSNorms inside the following GEMV where it fits (tx_linear_swiglu_norm, _split_norm)
        self.norm_in_gemv = fused
        # a prompt's causal attention with this library's kernel (else torch's flash attention)
        self.prompt_attention_kernel = fused and prompt_attention_supported(config)
        ext = extension()
        c = config
        if fused and not layers.decode_attention_supported(c):
            raise ValueError("the fused decode attention needs head_dim 128 and at most 8 query heads per KV head")
        g = torch.Generator(device=self.device).manual_seed(seed)
        bf16 = torch.bfloat16

        def normal(*shape, std=0.02):
            return (torch.randn(shape, device=self.device, generator=g) * std).to(bf16)

        self.embed = normal(c.vocab, c.hidden, std=embed_std)
        self.lm_head = normal(c.vocab, c.hidden)
        self.final_norm = torch.ones(c.hidden, device=self.device, dtype=bf16)
        self.handles: list[int] = []
        self.layers: list[_Layer] = []
        shapes = {name: (m, k) for name, m, k in c.linear_shapes()}
        encoded_sets: dict[tuple[int, str], tuple[torch.Tensor, torch.Tensor]] = {}
        lut = None
        if weights == "encoded" and linear_source is None:
            from .hardware import device_palette

            lut = device_palette(self.device).reshape(255, 255, 8)

        def weight_source(index: int, name: str, m: int, k: int):
            if linear_source is not None:
                source = linear_source(index, name, m, k)
                if source is not None:
                    return source
            std = init_std(c, name, depth_scaled)
            if weights == "uniform":
                return random_bc4(m, k, g, self.device, std)
            key = (index % distinct_layers, name)
            if key not in encoded_sets:
                encoded_sets[key] = encoded_bc4(m, k, g, lut, std)
            return encoded_sets[key]

        try:
            for index in range(c.layers):
                layer = _Layer()
                layer.input_norm = torch.ones(c.hidden, device=self.device, dtype=bf16)
                layer.post_norm = torch.ones(c.hidden, device=self.device, dtype=bf16)
                for key, names in MERGED.items():
                    parts_blocks, parts_scales, row = [], [], 0
                    for name in names:
                        m, k = shapes[name]
                        blocks, scales = weight_source(index, name, m, k)
                        parts_blocks.append(blocks.reshape(-1))
                        parts_scales.append(scales.reshape(-1).float())
                        layer.rows[name] = (row, m)
                        row += m
                    blocks = torch.cat(parts_blocks) if len(parts_blocks) > 1 else parts_blocks[0]
                    scales = torch.cat(parts_scales) if len(parts_scales) > 1 else parts_scales[0]
                    bias = torch.zeros(row, device=self.device, dtype=bf16) if (c.qkv_bias and key == "qkv") else None
                    handle = ext.pack_encoded_device(blocks.contiguous(), scales.contiguous(), bias)
                    self.handles.append(handle)
                    ext.set_lookahead(handle, gate_up_lookahead if key == "gate_up" else lookahead)
                    layer.linears[key] = TexelatorLinear([handle])
                    layer.handles[key] = handle
                    if bias is not None:
                        layer.biases[key] = bias
                    del blocks, scales, parts_blocks, parts_scales
                self.layers.append(layer)
        except Exception:
            free(self.handles)
            raise
        finally:
            encoded_sets.clear()
        # K and V caches [layer, kv_head, position, head_dim]
        shape = (c.layers, c.kv_heads, self.max_context, c.head_dim)
        self.k_cache = torch.zeros(shape, device=self.device, dtype=bf16)
        self.v_cache = torch.zeros(shape, device=self.device, dtype=bf16)
        inv_freq = 1.0 / (c.rope_theta ** (torch.arange(0, c.head_dim, 2, device=self.device, dtype=torch.float32)
                                           / c.head_dim))
        angles = torch.arange(self.max_context, device=self.device, dtype=torch.float32)[:, None] * inv_freq[None, :]
        angles = torch.cat([angles, angles], dim=-1)
        self.rope_cos, self.rope_sin = angles.cos().contiguous(), angles.sin().contiguous()
        # [cos | sin] per position, and the row of the current decode step (gathered once per token)
        self.rope_cs = torch.cat([self.rope_cos, self.rope_sin], dim=1).contiguous()
        self.rope_row = torch.empty(1, 2 * c.head_dim, dtype=torch.float32, device=self.device)
        self.key_positions = torch.arange(self.max_context, device=self.device)
        self.attention_workspace = torch.empty(
            layers.decode_attention_workspace_bytes(c.heads, self.max_context) if fused else 16,
            dtype=torch.uint8, device=self.device)
        # decode-step state (static buffers read and advanced by the captured graphs)
        self.attn_buffer = torch.empty(1, c.heads * c.head_dim, dtype=bf16, device=self.device)
        self.act_buffer = torch.empty((1, c.intermediate), dtype=bf16, device=self.device)
        self.token = torch.zeros(1, dtype=torch.long, device=self.device)
        self.head_workspace = torch.empty(layers.lm_head_argmax_workspace_bytes() if self.fused_head else 16,
                                          dtype=torch.uint8, device=self.device)
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

    def dense_weight(self, index: int, name: str) -> torch.Tensor:
        """Decoded bf16 weight ``[M, K]`` of one reference linear (for checks)."""
        layer = self.layers[index]
        key = next(k for k, names in MERGED.items() if name in names)
        first, rows = layer.rows[name]
        return extension().decode_dense(layer.linears[key].handles[0])[first:first + rows]

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

    def _prompt_attention(self, index: int, q: torch.Tensor) -> torch.Tensor:
        """Causal attention of a prompt (positions 0..T-1) over its own keys, q [T, heads, d]; the
        prompt's keys and values are the cache rows 0..T-1 that ``rope_kv_cache`` just wrote. This
        library's prompt-attention kernel (bf16 in, online fp32 softmax) up to
        ``PROMPT_ATTENTION_MAX_TOKENS`` tokens, else (or with ``prompt_attention_kernel`` off) torch's
        flash-attention kernel (only the flash backend is allowed, so an unsupported shape raises
        instead of running the unfused math path)."""
        c = self.config
        tokens = q.shape[0]
        if self.prompt_attention_kernel and tokens <= PROMPT_ATTENTION_MAX_TOKENS:
            return layers.prefill_attention(q.reshape(tokens, c.heads * c.head_dim), self.k_cache[index],
                                            self.v_cache[index], c.heads, c.kv_heads, 1.0 / math.sqrt(c.head_dim))
        keys = self.k_cache[index, :, :tokens].unsqueeze(0)        # [1, kv, T, d]
        values = self.v_cache[index, :, :tokens].unsqueeze(0)
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
            out = functional.scaled_dot_product_attention(q.permute(1, 0, 2).unsqueeze(0), keys, values,
                                                          is_causal=True, enable_gqa=c.heads != c.kv_heads)
        return out[0].permute(1, 0, 2).reshape(tokens, c.heads * c.head_dim)

    def _cached_attention(self, index: int, q: torch.Tensor, positions: torch.Tensor, length: int) -> torch.Tensor:
        """q [T, heads, d] at ``positions`` over cache positions 0..length-1, causally.

        scores^T = K q^T and out = P V are batched products whose right operands are
        contiguous or row-strided cache slices (never transposed views); scores and softmax in fp32."""
        c = self.config
        tokens = q.shape[0]
        group = c.heads // c.kv_heads
        keys = self.k_cache[index, :, :length]                      # [kv, L, d]
        values = self.v_cache[index, :, :length]                    # [kv, L, d]
        qt = q.reshape(tokens, c.kv_heads, group, c.head_dim).permute(1, 3, 2, 0).reshape(
            c.kv_heads, c.head_dim, group * tokens).contiguous()   # column = g * T + t
        scores = torch.bmm(keys, qt, out_dtype=torch.float32) * (1.0 / math.sqrt(c.head_dim))   # [kv, L, G*T]
        future = self.key_positions[:length, None] > positions.repeat(group)[None, :]
        probs = torch.softmax(scores.masked_fill(future, float("-inf")), dim=1)
        probs = probs.to(torch.bfloat16).transpose(1, 2).contiguous()              # [kv, G*T, L]
        out = torch.bmm(probs, values)                                             # [kv, G*T, d]
        return out.view(c.kv_heads, group, tokens, c.head_dim).permute(2, 0, 1, 3).reshape(tokens, c.heads * c.head_dim)

    def _layer_torch(self, index: int, layer: _Layer, h: torch.Tensor, positions: torch.Tensor, length: int) -> torch.Tensor:
        c = self.config
        q_rows, kv_rows = c.heads * c.head_dim, c.kv_heads * c.head_dim
        x = self._rms_norm(h, layer.input_norm)
        qkv = layer.linears["qkv"](x)
        q = self._rope(qkv[:, :q_rows].reshape(-1, c.heads, c.head_dim), positions)
        k = self._rope(qkv[:, q_rows:q_rows + kv_rows].reshape(-1, c.kv_heads, c.head_dim), positions)
        v = qkv[:, q_rows + kv_rows:].reshape(-1, c.kv_heads, c.head_dim)
        self.k_cache[index].index_copy_(1, positions, k.transpose(0, 1))
        self.v_cache[index].index_copy_(1, positions, v.transpose(0, 1))
        h = h + layer.linears["o"](self._cached_attention(index, q, positions, length)).float()
        x = self._rms_norm(h, layer.post_norm)
        gu = layer.linears["gate_up"](x).float()
        act = functional.silu(gu[:, :c.intermediate]) * gu[:, c.intermediate:]
        return h + layer.linears["down"](act.to(torch.bfloat16)).float()

    def hidden_states(self, ids: torch.Tensor, positions: torch.Tensor, length: int) -> torch.Tensor:
        """Final-norm hidden states [T, hidden] (bf16) for tokens ``ids`` at ``positions``.

        The residual stream is kept in fp32; every linear reads bf16 activations and writes bf16
        outputs. On the fused path a single token uses the split-length decode attention, a prompt
        (positions ``key_positions[:T]``, ``length == T``) torch's causal flash attention, and any
        other multi-token call the cached fp32 attention."""
        c = self.config
        if self.fused and ids.numel() == 1 and self.split_decode:
            return self._decode_split(ids, positions, length, 1.0 / math.sqrt(c.head_dim))
        h = self.embed.index_select(0, ids).float()
        if not self.fused:
            for index, layer in enumerate(self.layers):
                h = self._layer_torch(index, layer, h, positions, length)
            return self._rms_norm(h, self.final_norm)
        tokens = ids.numel()
        scale = 1.0 / math.sqrt(c.head_dim)
        x = layers.add_rmsnorm(h, None, self.layers[0].input_norm, c.rms_eps)
        # a prompt at positions 0..T-1 attending to itself only: causal flash attention
        prompt = (tokens > 1 and length == tokens and positions.data_ptr() == self.key_positions.data_ptr()
                  and self.flash_prompt_attention)
        workspace = self._split_workspace(tokens)
        for index, layer in enumerate(self.layers):
            if self._prefill_partials(layer.handles["qkv"], x, workspace):
                q = layers.rope_kv_cache_prefill_split(layer.handles["qkv"], workspace, positions, self.rope_cos,
                                                       self.rope_sin, c.heads, c.kv_heads, c.head_dim,
                                                       self.k_cache[index], self.v_cache[index])
            else:
                qkv = layer.linears["qkv"](x)
                q = layers.rope_kv_cache(qkv, positions, self.rope_cos, self.rope_sin, c.heads, c.kv_heads, c.head_dim,
                                         self.k_cache[index], self.v_cache[index])
            if tokens == 1:
                attn = layers.decode_attention(q, self.k_cache[index], self.v_cache[index], positions, length, c.heads,
                                               c.kv_heads, scale, self.attention_workspace)
            elif prompt:
                attn = self._prompt_attention(index, q.view(tokens, c.heads, c.head_dim))
            else:
                attn = self._cached_attention(index, q.view(tokens, c.heads, c.head_dim), positions, length)
            self._add_rmsnorm_tokens(h, layer.handles["o"], layer.linears["o"], attn, layer.post_norm, x, workspace)
            act = self._gate_up_swiglu_tokens(layer, x)
            following = self.layers[index + 1].input_norm if index + 1 < len(self.layers) else self.final_norm
            self._add_rmsnorm_tokens(h, layer.handles["down"], layer.linears["down"], act, following, x, workspace)
        return x

    def _split_workspace(self, tokens: int) -> torch.Tensor | None:
        """Workspace for the partials of this call's K-split prefill GEMMs (None if none is used)."""
        if not self.split_prefill or tokens < 2:
            return None
        ext = extension()
        layer = self.layers[0]
        need = max(ext.workspace_bytes(layer.handles[key], tokens) for key in ("qkv", "o", "down"))
        return torch.empty(max(need, 16), dtype=torch.uint8, device=self.device) if need else None

    def _prefill_partials(self, handle: int, x: torch.Tensor, workspace: torch.Tensor | None) -> bool:
        """The prefill GEMM of ``x`` leaving its K-split partials in ``workspace``; False (nothing
        run) where the call does not split K, so the caller runs the plain linear."""
        if workspace is None or x.shape[0] < 2:
            return False
        try:
            layers.prefill_split(handle, x, workspace)
        except UnsupportedError:
            return False
        return True

    def _add_rmsnorm_tokens(self, h: torch.Tensor, handle: int, linear: TexelatorLinear, x_in: torch.Tensor,
                            weight: torch.Tensor, out: torch.Tensor, workspace: torch.Tensor | None) -> None:
        """``h += linear(x_in)``, ``out = rmsnorm(h) * weight``: from the GEMM's K-split partials where
        it splits (bit-identical, one reduce launch fewer), else through the linear's output."""
        if self._prefill_partials(handle, x_in, workspace):
            layers.add_rmsnorm_prefill_split(h, handle, workspace, weight, self.config.rms_eps, out=out)
        else:
            layers.add_rmsnorm(h, linear(x_in), weight, self.config.rms_eps, out=out)

    def _decode_split(self, ids: torch.Tensor, positions: torch.Tensor, length: int, scale: float) -> torch.Tensor:
        """One token through every layer with the split-K consumers (eight kernels a layer; seven where
        the attention's merge runs inside the o GEMV, five where the two add+RMSNorms also run inside
        the gate|up and the next q|k|v GEMVs, whose updated residual then alternates between h and a
        second buffer)."""
        c = self.config
        torch.index_select(self.rope_cs, 0, positions, out=self.rope_row)
        h = torch.empty((1, c.hidden), dtype=torch.float32, device=self.device)
        x = torch.empty((1, c.hidden), dtype=torch.bfloat16, device=self.device)
        other = torch.empty_like(h) if self.norm_in_gemv else None
        # the embedding row, the first input norm and the first q|k|v GEMV: one launch where it fits
        qkv_done = self.norm_in_gemv and layers.linear_split_embed_norm(
            self.layers[0].handles["qkv"], self.embed, ids.view(1), h, self.layers[0].input_norm, c.rms_eps)
        if not qkv_done:
            h.copy_(self.embed.index_select(0, ids.view(1)))
            layers.add_rmsnorm(h, None, self.layers[0].input_norm, c.rms_eps, out=x)
        for index, layer in enumerate(self.layers):
            if not qkv_done:
                layers.linear_split(layer.handles["qkv"], x)
            if not (self.attention_in_o and layers.decode_attention_o_split(
                    layer.handles["qkv"], layer.handles["o"], positions, self.rope_row, c.heads, c.kv_heads, c.head_dim,
                    self.k_cache[index], self.v_cache[index], length, scale, self.attention_workspace)):
                attn = layers.decode_attention_split(layer.handles["qkv"], positions, self.rope_row, c.heads, c.kv_heads,
                                                     c.head_dim, self.k_cache[index], self.v_cache[index], length, scale,
                                                     self.attention_workspace, out=self.attn_buffer)
                layers.linear_split(layer.handles["o"], attn)
            gate_up = layer.handles["gate_up"]
            if (self.norm_in_gemv and self._gate_up_unsplit(layer)
                    and layers.linear_swiglu_norm(gate_up, h, other, layer.handles["o"], layer.post_norm, c.rms_eps,
                                                  self.act_buffer)):
                h, other = other, h
                act = self.act_buffer
            else:
                layers.add_rmsnorm_split(h, layer.handles["o"], layer.post_norm, c.rms_eps, out=x)
                act = self._gate_up_swiglu(layer, x)
            layers.linear_split(layer.handles["down"], act)
            qkv_done = False
            if index + 1 < len(self.layers):
                following = self.layers[index + 1]
                if self.norm_in_gemv and layers.linear_split_norm(following.handles["qkv"], h, other,
                                                                  layer.handles["down"], following.input_norm,
                                                                  c.rms_eps):
                    h, other = other, h
                    qkv_done = True
                    continue
                layers.add_rmsnorm_split(h, layer.handles["down"], following.input_norm, c.rms_eps, out=x)
            else:
                layers.add_rmsnorm_split(h, layer.handles["down"], self.final_norm, c.rms_eps, out=x)
        return x

    def _gate_up_unsplit(self, layer: _Layer) -> bool:
        """Whether the merged gate|up GEMV of one token runs unsplit (its SwiGLU epilogue applies)."""
        splits, lut = extension().gemv_plan(layer.handles["gate_up"])
        return splits == 1 and not lut and self.config.intermediate % 16 == 0

    def _gate_up_swiglu(self, layer: _Layer, x: torch.Tensor) -> torch.Tensor:
        """SwiGLU of the merged gate|up projection of one token: one GEMV with the SwiGLU epilogue
        when the handle's GEMV runs unsplit (bit-identical to the GEMV + SwiGLU kernels it
        replaces), else those two kernels."""
        handle = layer.handles["gate_up"]
        if self._gate_up_unsplit(layer):
            return layers.linear_swiglu(handle, x, out=self.act_buffer)
        return layers.swiglu(layer.linears["gate_up"](x))

    def _gate_up_swiglu_tokens(self, layer: _Layer, x: torch.Tensor) -> torch.Tensor:
        """SwiGLU of the merged gate|up projection of several tokens: one prefill GEMM with the
        SwiGLU epilogue where the call's tile supports it unsplit (bit-identical to the GEMM +
        SwiGLU kernels it replaces), else those two kernels."""
        if x.shape[0] > 1 and self.gate_up_swiglu_prefill:
            try:
                return layers.linear_swiglu_prefill(layer.handles["gate_up"], x)
            except UnsupportedError:
                pass
        return layers.swiglu(layer.linears["gate_up"](x))

    def logits(self, hidden: torch.Tensor) -> torch.Tensor:
        return functional.linear(hidden, self.lm_head)

    def greedy_token(self, hidden: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """``argmax(logits(hidden))`` of one hidden state [1, hidden] (int64 [1]): the lm_head GEMV
        with the argmax in its epilogue (the first of equal bf16 logits, as argmax picks it), or
        torch's linear + argmax without ``fused_head``."""
        if self.fused_head:
            return layers.lm_head_argmax(self.lm_head, hidden, self.head_workspace, out=out)
        token = self.logits(hidden).argmax(-1)
        if out is None:
            return token
        out.copy_(token)
        return out

    # ---------------------------------------------------------------- prefill and decode
    @torch.inference_mode()
    def prefill(self, ids: torch.Tensor) -> torch.Tensor:
        """Run the prompt (positions 0..T-1), fill the cache, return the next greedy token [1]."""
        tokens = ids.numel()
        if tokens > self.max_context:
            raise ValueError("prompt longer than the cache")
        positions = self.key_positions[:tokens]
        hidden = self.hidden_states(ids.view(-1), positions, tokens)
        next_token = self.greedy_token(hidden[-1:])
        self.token.copy_(next_token)
        self.position.fill_(tokens)
        return next_token

    def _bucket(self, position: int) -> int:
        return min(self.max_context, (position // 512 + 1) * 512)

    def _step(self, length: int) -> None:
        hidden = self.hidden_states(self.token, self.position, length)
        self.greedy_token(hidden, out=self.token)
        self.position.add_(1)

    @torch.inference_mode()
    def capture(self, length: int) -> torch.cuda.CUDAGraph:
        """Capture one decode step attending to ``length`` cache positions (a multiple of 512)."""
        if length in self.graphs:
            return self.graphs[length]
        saved_token, saved_position = self.token.clone(), self.position.clone()
        # The warm-up step runs for real: at the model's position, which after a decode that filled
        # the cache is max_context, a row past the RoPE table (whose gather traps on it). It runs at
        # the last row then, and the cache rows it writes are put back afterwards.
        row = min(int(saved_position), self.max_context - 1)
        self.position.fill_(row)
        saved_rows = (self.k_cache[:, :, row].clone(), self.v_cache[:, :, row].clone())
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
        self.k_cache[:, :, row] = saved_rows[0]
        self.v_cache[:, :, row] = saved_rows[1]
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
