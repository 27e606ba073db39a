"""The reference's own calling path at a BASELINE model size: a Hugging Face Qwen2 whose seven
linears per layer are :class:`~texelator_amd.runtime.TexelatorLinear` modules.

The reference loads its standalone artifact into a meta-initialised Hugging Face model, puts
``TexelatorLinear`` modules in place of the linears (``standalone.py:102-158`` through
``runtime.install_standalone`` :242-263), assigns the remaining tensors, then decodes with
``model.generate`` (``cli._generate`` :189-219) and measures prefill with ``model.model(...)``
(``prefill.py:24-26``). :func:`build_qwen2` does the same for a random-init BASELINE config 4 or 5
model, its linears BC4-encoded on the GPU (or uniform blocks) with the same initialisation rules as
:class:`~texelator_amd.modeling.BC4Decoder`; :func:`benchmark_generate` times greedy ``generate``.

Attention runs through torch's flash kernel (``sdpa``): the math path would issue bf16 batched
products with transposed operands. :func:`use_texelator_attention` switches a model to this
library's decode and prompt attention kernels instead (the ``"texelator"`` attention
implementation), and :class:`GraphedGreedy` decodes such a model from a static KV cache with the
one-token forward captured in a HIP graph, which removes the per-token host cost of the Hugging Face
modules.
"""
from __future__ import annotations

import statistics
import time

import torch
from torch import nn

from ._lib import TexelatorError
from .modeling import DISTINCT_LAYERS, DecoderConfig, encoded_bc4, init_std, random_bc4
from .runtime import PREFILL_THRESHOLD, PREFILL_TILE_ROWS, TexelatorLinear, extension, free

LINEARS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
           "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


def qwen2_config(config: DecoderConfig):
    """The ``transformers.Qwen2Config`` of a BASELINE decoder config (untied lm_head, sdpa)."""
    import transformers

    return transformers.Qwen2Config(
        vocab_size=config.vocab, hidden_size=config.hidden, intermediate_size=config.intermediate,
        num_hidden_layers=config.layers, num_attention_heads=config.heads, num_key_value_heads=config.kv_heads,
        head_dim=config.head_dim, rms_norm_eps=config.rms_eps, rope_theta=config.rope_theta,
        max_position_embeddings=32768, tie_word_embeddings=False, attn_implementation="sdpa",
        torch_dtype=torch.bfloat16)


def build_qwen2(config: DecoderConfig, seed: int = 0, weights: str = "encoded", distinct_layers: int = DISTINCT_LAYERS,
                depth_scaled: bool = True, embed_std: float = 1.0, lookahead: int = 1,
                device: str = "cuda") -> tuple[nn.Module, list[int]]:
    """A Qwen2ForCausalLM on ``device`` whose linears are BC4 handles; returns ``(model, handles)``
    (free the handles with :func:`texelator_amd.runtime.free`). No dense linear weight is ever
    materialised in the model: it is built on the meta device, the TexelatorLinear modules are
    swapped in, and only embeddings, norms, lm_head and the q/k/v biases (zeros) are assigned."""
    import transformers
    from accelerate import init_empty_weights

    if weights not in ("encoded", "uniform"):
        raise ValueError("weights must be 'encoded' or 'uniform'")
    ext = extension()
    hf_config = qwen2_config(config)
    with init_empty_weights():
        model = transformers.Qwen2ForCausalLM(hf_config)
    g = torch.Generator(device=device).manual_seed(seed)
    lut = None
    if weights == "encoded":
        from .hardware import device_palette

        lut = device_palette(device).reshape(255, 255, 8)
    shapes = {name: (m, k) for name, m, k in config.linear_shapes()}
    cache: dict[tuple[int, str], tuple[torch.Tensor, torch.Tensor]] = {}
    handles: list[int] = []
    try:
        for index in range(config.layers):
            for name in LINEARS:
                m, k = shapes[name]
                std = init_std(config, name, depth_scaled)
                if weights == "uniform":
                    blocks, scales = random_bc4(m, k, g, torch.device(device), std)
                else:
                    key = (index % distinct_layers, name)
                    if key not in cache:
                        cache[key] = encoded_bc4(m, k, g, lut, std)
                    blocks, scales = cache[key]
                handle = ext.pack_encoded_device(blocks.reshape(-1).contiguous(), scales.float().contiguous(), None)
                handles.append(handle)
                ext.set_lookahead(handle, lookahead)
                ext.set_prefill(handle, PREFILL_THRESHOLD, PREFILL_TILE_ROWS)
                bias = None
                if name in LINEARS[:3]:
                    bias = nn.Parameter(torch.zeros(m, device=device, dtype=torch.bfloat16), requires_grad=False)
                parent = model.get_submodule(f"model.layers.{index}.{name.rsplit('.', 1)[0]}")
                setattr(parent, name.rsplit(".", 1)[1], TexelatorLinear([handle], bias=bias))
        bf16 = torch.bfloat16

        def normal(*shape, std):
            return (torch.randn(shape, device=device, generator=g) * std).to(bf16)

        rest = {"model.embed_tokens.weight": normal(config.vocab, config.hidden, std=embed_std),
                "lm_head.weight": normal(config.vocab, config.hidden, std=0.02),
                "model.norm.weight": torch.ones(config.hidden, device=device, dtype=bf16)}
        for index in range(config.layers):
            for norm in ("input_layernorm", "post_attention_layernorm"):
                rest[f"model.layers.{index}.{norm}.weight"] = torch.ones(config.hidden, device=device, dtype=bf16)
        model.load_state_dict(rest, strict=False, assign=True)
        model.to(device)
        left = [n for n, p in model.named_parameters() if p.device.type == "meta"]
        if left:
            raise RuntimeError(f"parameters left uninitialised: {left[:4]}")
        model.eval()
    except BaseException:
        free(handles)
        raise
    finally:
        cache.clear()
    model._texelator_handles = handles
    return model, handles


ATTENTION = "texelator"


def texelator_attention(module: nn.Module, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                        attention_mask: torch.Tensor | None, scaling: float | None = None, dropout: float = 0.0,
                        **kwargs) -> tuple[torch.Tensor, None]:
    """The Hugging Face attention implementation ``"texelator"`` (see :func:`use_texelator_attention`):
    one query token through the library's decode attention kernel, a prompt starting at position 0
    through its prompt attention kernel. Arguments as Hugging Face passes them to an attention
    function: ``query`` ``[1, heads, T, 128]`` after RoPE, ``key``/``value`` the layer's whole cache
    ``[1, kv_heads, L, 128]`` just updated (a static cache's ``L`` is its capacity; the keys that
    count are those at positions 0..position), ``position_ids`` ``[1, T]`` in ``kwargs``. No mask is
    read: decode attends to positions 0..position, a prompt causally. Returns ``[1, T, heads, 128]``
    as the Hugging Face attention functions do. No reference counterpart: the reference runs the
    stock ``sdpa`` attention (``runtime.py:210-239`` replaces only the linears)."""
    from . import layers

    batch, heads, tokens, head_dim = query.shape
    kv_heads, length = key.shape[1], key.shape[2]
    positions = kwargs.get("position_ids")
    if batch != 1 or head_dim != 128 or heads % kv_heads or dropout or positions is None:
        raise TexelatorError("texelator attention: batch 1, head_dim 128, heads a multiple of kv_heads, "
                             "no dropout, position_ids given")
    if attention_mask is not None:
        raise TexelatorError("texelator attention reads no mask (padding is not supported)")
    k_cache, v_cache = key[0], value[0]
    scale = float(scaling if scaling is not None else head_dim ** -0.5)
    if tokens == 1:
        if heads // kv_heads > 8:
            raise TexelatorError("texelator attention: at most 8 query heads per KV head in decode")
        workspace = torch.empty(layers.decode_attention_workspace_bytes(heads, length), dtype=torch.uint8,
                                device=query.device)
        out = layers.decode_attention(query.reshape(heads * head_dim), k_cache, v_cache, positions.reshape(1), length,
                                      heads, kv_heads, scale, workspace)
        return out.view(1, 1, heads, head_dim), None
    if int(positions[0, 0]) != 0:
        raise TexelatorError("texelator attention: a prompt must start at position 0 (no chunked prefill)")
    q = query.transpose(1, 2).reshape(tokens, heads * head_dim)
    out = layers.prefill_attention(q, k_cache, v_cache, heads, kv_heads, scale)
    return out.view(1, tokens, heads, head_dim), None


def use_texelator_attention(model: nn.Module) -> None:
    """Register :func:`texelator_attention` with Hugging Face as ``"texelator"`` and switch
    ``model`` to it."""
    from transformers import AttentionInterface

    AttentionInterface.register(ATTENTION, texelator_attention)
    model.set_attn_implementation(ATTENTION)


class TexelatorRMSNorm(nn.Module):
    """A Hugging Face RMSNorm (Qwen2/Llama form: ``weight * bf16(x * rsqrt(mean(x^2) + eps))``, x in
    fp32) through the library's bf16 add+RMSNorm kernel: one launch instead of the module's six or
    seven elementwise ones. The same formula and roundings; the fp32 sum of squares runs in the
    kernel's order, so a row's result can differ from torch's in the last bit where the two sums
    round apart. bf16 activations and weight, hidden a multiple of 4."""

    def __init__(self, weight: nn.Parameter, eps: float):
        super().__init__()
        self.weight = weight
        self.variance_epsilon = float(eps)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        from . import layers

        if x.dtype == torch.bfloat16 and x.is_cuda and x.is_contiguous() and x.data_ptr() % 8 == 0:
            return layers.add_rmsnorm_bf16(x, None, self.weight, self.variance_epsilon)[1]
        shape = x.shape
        h = x.reshape(-1, shape[-1]).float()
        return layers.add_rmsnorm(h, None, self.weight, self.variance_epsilon).view(shape)


def use_texelator_norms(model: nn.Module) -> list[tuple[nn.Module, str, nn.Module]]:
    """Replace every bf16 ``*RMSNorm`` module of ``model`` (weight and ``variance_epsilon``, hidden a
    multiple of 4) with :class:`TexelatorRMSNorm`; returns ``(parent, name, original)`` per
    replacement, for :func:`restore_modules`."""
    replaced = []
    for name, module in list(model.named_modules()):
        weight = getattr(module, "weight", None)
        if (not type(module).__name__.endswith("RMSNorm") or isinstance(module, TexelatorRMSNorm)
                or not hasattr(module, "variance_epsilon") or weight is None or weight.dtype != torch.bfloat16
                or weight.dim() != 1 or weight.numel() % 4):
            continue
        parent_name, _, child = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        setattr(parent, child, TexelatorRMSNorm(weight, module.variance_epsilon))
        replaced.append((parent, child, module))
    return replaced


class TexelatorMLP(nn.Module):
    """A Hugging Face gated MLP (``down(act(gate(x)) * up(x))`` with SiLU, Qwen2/Llama form) whose
    gate and up projections are single-handle :class:`~texelator_amd.runtime.TexelatorLinear`
    modules: one token runs gate, up and the SwiGLU product as one kernel
    (:func:`~texelator_amd.layers.linear_swiglu_pair`) instead of two GEMVs, their reductions and
    two elementwise kernels; longer inputs, and handles the fused kernel refuses (a bias, LUT mode),
    run the original module. The product is ``bf16(silu(G) * U)`` from the bf16 projections G and
    U, one rounding, where the original rounds ``silu(G)`` first: a token's result can differ from
    the module's in the last bit."""

    def __init__(self, original: nn.Module):
        super().__init__()
        self.original = original
        self.gate = int(original.gate_proj.handles[0])
        self.up = int(original.up_proj.handles[0])
        self.fused = True

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        from . import layers
        from ._lib import UnsupportedError

        if self.fused and x.dtype == torch.bfloat16 and x.numel() == x.shape[-1]:
            xc = x.contiguous()
            if xc.data_ptr() % 16:
                xc = xc.clone()
            try:
                act = layers.linear_swiglu_pair(self.gate, self.up, xc.view(-1))
            except UnsupportedError:
                self.fused = False
            else:
                return self.original.down_proj(act.view(*x.shape[:-1], act.shape[-1]))
        return self.original(x)

    def forward_residual(self, x: torch.Tensor, residual: torch.Tensor) -> torch.Tensor | None:
        """``residual + self(x)`` for one bf16 token with the residual added in the down projection's
        GEMV epilogue (:func:`~texelator_amd.layers.linear_add_bias` with the residual as the vector:
        the bf16 projection plus the residual rounded again, bit for bit the separate add); ``None``
        (nothing computed) where that path does not apply."""
        from . import layers
        from ._lib import UnsupportedError

        down = self.original.down_proj
        if not (self.fused and isinstance(down, TexelatorLinear) and len(down.handles) == 1 and down.bias is None
                and x.dtype == residual.dtype == torch.bfloat16 and x.is_cuda and x.numel() == x.shape[-1]
                and residual.shape == x.shape and residual.is_contiguous() and residual.data_ptr() % 2 == 0):
            return None
        xc = x.contiguous()
        if xc.data_ptr() % 16:
            xc = xc.clone()
        try:
            act = layers.linear_swiglu_pair(self.gate, self.up, xc.view(-1))
        except UnsupportedError:
            self.fused = False
            return None
        try:
            return layers.linear_add_bias(down.handles[0], act, residual.view(-1)).view(residual.shape)
        except TexelatorError:  # a down handle with its own bias: the separate add
            return residual + down(act.view(*x.shape[:-1], act.shape[-1]))


def use_texelator_mlp(model: nn.Module) -> list[tuple[nn.Module, str, nn.Module]]:
    """Replace every gated SiLU MLP of ``model`` whose gate and up projections are single-handle
    TexelatorLinear modules without a separate bias with :class:`TexelatorMLP`; returns ``(parent,
    name, original)`` per replacement, for :func:`restore_modules`."""
    from .runtime import TexelatorLinear

    replaced = []
    wrapped = [name for name, module in model.named_modules() if isinstance(module, TexelatorMLP)]
    for name, module in list(model.named_modules()):
        if any(name == w or name.startswith(w + ".") for w in wrapped):
            continue  # a TexelatorMLP or the original it holds
        gate, up = getattr(module, "gate_proj", None), getattr(module, "up_proj", None)
        act = getattr(module, "act_fn", None)
        if (not isinstance(gate, TexelatorLinear)
                or not isinstance(up, TexelatorLinear) or getattr(module, "down_proj", None) is None
                or len(gate.handles) != 1 or len(up.handles) != 1 or gate.bias is not None or up.bias is not None
                or not (isinstance(act, nn.SiLU) or "SiLU" in type(act).__name__)):
            continue
        parent_name, _, child = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        setattr(parent, child, TexelatorMLP(module))
        replaced.append((parent, child, module))
    return replaced


def _rope_attention_forward(self, hidden_states: torch.Tensor, position_embeddings: tuple[torch.Tensor, torch.Tensor],
                            attention_mask: torch.Tensor | None, past_key_values=None, **kwargs):
    """A Qwen2 attention module's forward with its rotary embedding on the library's kernel
    (:func:`~texelator_amd.layers.rope_rotate_half`: one launch, bitwise the module's result) and
    every other step as the module does it: the projections, the cache update, the configured
    attention function and the output projection."""
    import sys

    from . import layers

    hf_module = sys.modules[type(self).__module__]
    input_shape = hidden_states.shape[:-1]
    hidden_shape = (*input_shape, -1, self.head_dim)
    q, k, v = _projections(self, hidden_states)
    q = q.view(hidden_shape)  # [batch, tokens, heads, head_dim]
    k = k.view(hidden_shape)
    v = v.view(hidden_shape).transpose(1, 2)
    cos, sin = position_embeddings  # [batch, tokens, head_dim]
    if q.is_cuda and q.dtype == cos.dtype == torch.bfloat16 and cos.shape[:-1] == q.shape[:-2]:
        q, k = layers.rope_rotate_half(q.contiguous(), k.contiguous(), cos.contiguous(), sin.contiguous())
        q, k = q.transpose(1, 2), k.transpose(1, 2)
    else:
        q, k = hf_module.apply_rotary_pos_emb(q.transpose(1, 2), k.transpose(1, 2), cos, sin)
    if past_key_values is not None:
        k, v = _cache_update(past_key_values, self.layer_idx, k, v)
    attention = hf_module.ALL_ATTENTION_FUNCTIONS.get_interface(self.config._attn_implementation,
                                                                 hf_module.eager_attention_forward)
    out, weights = attention(self, q, k, v, attention_mask, dropout=0.0 if not self.training else self.attention_dropout,
                             scaling=self.scaling, sliding_window=self.sliding_window, **kwargs)
    return self.o_proj(out.reshape(*input_shape, -1).contiguous()), weights


def _cache_update(cache, index: int, k: torch.Tensor, v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``cache.update(k, v, index)``; for one bf16 token into an initialized, not offloaded static
    layer, its two index copies and length update as one launch
    (:func:`~texelator_amd.layers.kv_cache_append`), the same cache contents and returned tensors."""
    from . import layers

    stack = getattr(cache, "layers", None)
    layer = stack[index] if stack is not None and index < len(stack) else None
    length = getattr(layer, "cumulative_length", None)
    if (layer is not None and type(layer).__name__ == "StaticLayer" and getattr(layer, "is_initialized", False)
            and not getattr(cache, "offloading", False) and k.is_cuda and k.dtype == v.dtype == torch.bfloat16
            and k.dim() == 4 and k.shape[0] == 1 and k.shape[-2] == 1 and v.shape == k.shape
            and layer.keys.dtype == torch.bfloat16 and layer.keys.shape[-1] == k.shape[-1]
            and layer.keys.shape[1] == k.shape[1] and isinstance(length, torch.Tensor) and length.is_cuda
            and length.dtype == torch.int64 and length.numel() == 1):
        layers.kv_cache_append(k, v, layer.keys, layer.values, length)
        return layer.keys, layer.values
    return cache.update(k, v, index)


def _projections(self, hidden_states: torch.Tensor) -> tuple[torch.Tensor, ...]:
    """q, k and v of an attention module: for one bf16 token of a module :func:`use_texelator_qkv`
    joined, one GEMV over its q|k|v handle with the three biases in the GEMV's epilogue (views of
    one output); otherwise the module's three projections."""
    from . import layers

    joined = self.__dict__.get("_texelator_qkv")
    x = hidden_states
    if (joined is not None and x.is_cuda and x.dtype == torch.bfloat16 and x.numel() == x.shape[-1]
            and x.is_contiguous() and x.data_ptr() % 16 == 0):
        handle, bias, sizes = joined
        out = layers.linear_add_bias(handle, x, bias) if bias is not None else extension().linear(handle, x)
        return out.split(sizes, dim=-1)
    return self.q_proj(x), self.k_proj(x), self.v_proj(x)


def use_texelator_qkv(model: nn.Module) -> list[int]:
    """Join the q, k and v projections of every Qwen2 attention module whose three projections are
    single-handle :class:`TexelatorLinear` modules of one K (q and k rows multiples of 16; all with
    bf16 separate biases or none) into one handle (``concat_rows``), so that a one-token forward runs
    one GEMV for the three. Takes effect in the forward :func:`use_texelator_rope` installs; the
    biases are copied now. Returns the new handles; :func:`restore_qkv` drops and frees them."""
    ext = extension()
    created = []
    for module in model.modules():
        if type(module).__name__ != "Qwen2Attention" or "_texelator_qkv" in module.__dict__:
            continue
        projections = [module.q_proj, module.k_proj, module.v_proj]
        if not all(isinstance(p, TexelatorLinear) and len(p.handles) == 1 for p in projections):
            continue
        biases = [p.bias for p in projections]
        if any(b is None for b in biases):
            if not all(b is None for b in biases):
                continue
            bias = None
        elif all(b.dtype == torch.bfloat16 and b.is_cuda for b in biases):
            bias = torch.cat([b.detach().reshape(-1) for b in biases]).contiguous()
        else:
            continue
        try:
            handle = ext.concat_rows([p.handles[0] for p in projections])
        except TexelatorError:
            continue
        module._texelator_qkv = (handle, bias, [ext.shape(p.handles[0])[0] for p in projections])
        created.append(handle)
    return created


def restore_qkv(model: nn.Module, created: list[int]) -> None:
    """Undo :func:`use_texelator_qkv`: the modules run their three projections again and the joined
    handles are freed."""
    for module in model.modules():
        module.__dict__.pop("_texelator_qkv", None)
    if torch.cuda.is_available():
        torch.cuda.synchronize()
    ext = extension()
    for handle in created:
        ext.free(handle)


def _decoder_layer_forward(self, hidden_states: torch.Tensor, attention_mask: torch.Tensor | None = None,
                           position_ids: torch.Tensor | None = None, past_key_values=None, use_cache: bool | None = False,
                           position_embeddings: tuple[torch.Tensor, torch.Tensor] | None = None, **kwargs) -> torch.Tensor:
    """A Qwen2 decoder layer's forward with the attention's residual add and the post-attention
    RMSNorm in one launch (:func:`~texelator_amd.layers.add_rmsnorm_bf16`: ``bf16(residual +
    attention)`` as torch adds, then the norm of that sum as :class:`TexelatorRMSNorm` computes it)
    and, under :class:`TexelatorMLP`, the MLP's residual add in the down projection's GEMV
    (:meth:`TexelatorMLP.forward_residual`); every other step as the layer does it."""
    from . import layers

    residual = hidden_states
    hidden_states = self.input_layernorm(hidden_states)
    hidden_states, _ = self.self_attn(hidden_states=hidden_states, attention_mask=attention_mask,
                                      position_ids=position_ids, past_key_values=past_key_values, use_cache=use_cache,
                                      position_embeddings=position_embeddings, **kwargs)
    norm = self.post_attention_layernorm
    if (isinstance(norm, TexelatorRMSNorm) and residual.is_cuda and residual.dtype == hidden_states.dtype == torch.bfloat16
            and residual.is_contiguous() and hidden_states.is_contiguous() and residual.shape == hidden_states.shape
            and residual.data_ptr() % 8 == 0 and hidden_states.data_ptr() % 8 == 0):
        residual, hidden_states = layers.add_rmsnorm_bf16(residual, hidden_states, norm.weight, norm.variance_epsilon)
    else:
        hidden_states = residual + hidden_states
        residual = hidden_states
        hidden_states = norm(hidden_states)
    if isinstance(self.mlp, TexelatorMLP):
        out = self.mlp.forward_residual(hidden_states, residual)
        if out is not None:
            return out
    hidden_states = self.mlp(hidden_states)
    return residual + hidden_states


def use_texelator_residuals(model: nn.Module) -> list[nn.Module]:
    """Give every Qwen2 decoder layer of ``model`` :func:`_decoder_layer_forward` (the attention's
    residual add fused into the post-attention RMSNorm when :func:`use_texelator_norms` made it a
    :class:`TexelatorRMSNorm`); returns the layers changed, for :func:`restore_rope`, which gives
    them their class's forward back the same way."""
    import types

    changed = []
    for module in model.modules():
        if type(module).__name__ != "Qwen2DecoderLayer" or "forward" in module.__dict__:
            continue
        module.forward = types.MethodType(_decoder_layer_forward, module)
        changed.append(module)
    return changed


def use_texelator_rope(model: nn.Module) -> list[nn.Module]:
    """Give every Qwen2 attention module of ``model`` :func:`_rope_attention_forward` (its rotary
    embedding as one library kernel instead of Hugging Face's elementwise ones, bit for bit the
    same); returns the modules changed, for :func:`restore_rope`."""
    import types

    changed = []
    for module in model.modules():
        if type(module).__name__ != "Qwen2Attention" or "forward" in module.__dict__:
            continue
        module.forward = types.MethodType(_rope_attention_forward, module)
        changed.append(module)
    return changed


def restore_rope(changed: list[nn.Module]) -> None:
    """Give the modules :func:`use_texelator_rope` changed their class's forward back."""
    for module in changed:
        module.__dict__.pop("forward", None)


def restore_modules(replaced: list[tuple[nn.Module, str, nn.Module]]) -> None:
    """Put back the modules :func:`use_texelator_norms` or :func:`use_texelator_mlp` replaced."""
    for parent, child, original in replaced:
        setattr(parent, child, original)


class GraphedGreedy:
    """Greedy decoding of a Hugging Face causal LM at batch 1 with a static KV cache, the
    one-token forward captured once in a HIP graph: each replay embeds the previous token, runs
    every layer (the BC4 linears, the ``"texelator"`` attention, Hugging Face's norms, RoPE and
    cache writes), appends to the cache and leaves the argmax as the next input. The host only
    replays; nothing syncs between tokens. The prompt runs eagerly (:meth:`prefill`). Switches
    ``model`` to the ``"texelator"`` attention. The same model and cache work without the graph
    (``eager=True``), token for token the same."""

    def __init__(self, model: nn.Module, max_cache_len: int):
        import transformers

        use_texelator_attention(model)
        self.model = model
        self.max_cache_len = int(max_cache_len)
        self.cache = transformers.StaticCache(config=model.config, max_cache_len=self.max_cache_len)
        self.token = torch.zeros((1, 1), dtype=torch.long, device=model.device)
        self.length = 0  # tokens in the cache, as the host counts them
        self.graph: torch.cuda.CUDAGraph | None = None

    def _step(self) -> None:
        logits = self.model(input_ids=self.token, past_key_values=self.cache, use_cache=True).logits
        torch.argmax(logits[:, -1], dim=-1, keepdim=True, out=self.token)

    @torch.inference_mode()
    def prefill(self, ids: torch.Tensor) -> torch.Tensor:
        """Reset the cache, run the prompt ``ids`` ``[1, T]`` and return the first new token."""
        if ids.dim() != 2 or ids.shape[0] != 1 or not 0 < ids.shape[1] < self.max_cache_len:
            raise ValueError("prefill takes one prompt [1, T] shorter than the cache")
        self.cache.reset()
        logits = self.model(input_ids=ids, past_key_values=self.cache, use_cache=True, logits_to_keep=1).logits
        torch.argmax(logits[:, -1], dim=-1, keepdim=True, out=self.token)
        self.length = ids.shape[1]
        return self.token.clone()

    @torch.inference_mode()
    def _capture(self) -> None:
        # a warm-up step outside the graph, then the capture; the cache lengths and the token are
        # put back, so the cache holds exactly the prompt afterwards
        lengths = [layer.cumulative_length.clone() for layer in self.cache.layers]
        token = self.token.clone()
        stream = torch.cuda.Stream(self.token.device)
        stream.wait_stream(torch.cuda.current_stream(self.token.device))
        with torch.cuda.stream(stream):
            self._step()
        torch.cuda.current_stream(self.token.device).wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            self._step()
        for layer, saved in zip(self.cache.layers, lengths):
            layer.cumulative_length.copy_(saved)
        self.token.copy_(token)
        self.graph = graph

    @torch.inference_mode()
    def decode(self, steps: int, out: torch.Tensor | None = None, eager: bool = False) -> None:
        """``steps`` greedy tokens after the current one; token i goes to ``out[i]`` when given."""
        if self.length == 0:
            raise RuntimeError("prefill first")
        if self.length + steps >= self.max_cache_len:
            raise ValueError("decode would run past the static cache")
        if not eager and self.graph is None:
            self._capture()
        for i in range(steps):
            if eager:
                self._step()
            else:
                self.graph.replay()
            if out is not None:
                out[i].copy_(self.token[0, 0])
        self.length += steps

    def generate(self, ids: torch.Tensor, new_tokens: int, eager: bool = False) -> torch.Tensor:
        """Greedy generation: the ``new_tokens`` new token ids (the first from the prompt's logits)."""
        out = torch.empty(new_tokens, dtype=torch.long, device=self.token.device)
        out[0] = self.prefill(ids)[0, 0]
        self.decode(new_tokens - 1, out=out[1:], eager=eager)
        return out

    def benchmark(self, prompt_tokens: int, new_tokens: int) -> dict:
        """Decode tok/s of graph replays after a seeded random prompt (device clock, prompt excluded)."""
        generator = torch.Generator(device="cpu").manual_seed(0)
        vocab = self.model.get_input_embeddings().weight.shape[0]
        ids = torch.randint(0, vocab, (1, prompt_tokens), generator=generator).to(self.token.device)
        self.prefill(ids)
        self.decode(4)  # capture and first replays
        self.prefill(ids)
        torch.cuda.synchronize()
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        begin.record()
        self.decode(new_tokens)
        end.record()
        end.synchronize()
        seconds = begin.elapsed_time(end) / 1000.0
        return {"prompt_tokens": prompt_tokens, "new_tokens": new_tokens, "seconds": seconds,
                "decode_tok_s": new_tokens / seconds}


def _generate(model: nn.Module, ids: torch.Tensor, new_tokens: int) -> torch.Tensor:
    from torch.nn.attention import SDPBackend, sdpa_kernel

    with torch.inference_mode(), sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
        return model.generate(ids, max_new_tokens=new_tokens, min_new_tokens=new_tokens, do_sample=False,
                              use_cache=True, pad_token_id=0)


def benchmark_generate(model: nn.Module, prompt_tokens: int, new_tokens: int, runs: int = 3) -> dict:
    """Greedy ``model.generate`` from a seeded random prompt, timed on the host clock around
    synchronised calls: ``new_tokens`` tokens and, separately, one token (the prompt's prefill and
    the first step), so that the decode rate excludes the prefill. Medians of ``runs``."""
    if new_tokens < 2:
        raise ValueError("new_tokens must be at least 2")
    generator = torch.Generator(device="cpu").manual_seed(0)
    vocab = model.get_input_embeddings().weight.shape[0]
    ids = torch.randint(0, vocab, (1, prompt_tokens), generator=generator).to(model.device)

    def seconds(count: int) -> float:
        torch.cuda.synchronize()
        start = time.perf_counter()
        out = _generate(model, ids, count)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - start
        if out.shape[1] != prompt_tokens + count:
            raise RuntimeError(f"generate returned {out.shape[1] - prompt_tokens} tokens, expected {count}")
        return elapsed

    seconds(2)  # warm-up: kernels, allocator, HF caches
    full = statistics.median(seconds(new_tokens) for _ in range(runs))
    first = statistics.median(seconds(1) for _ in range(runs))
    decode = max(full - first, 1e-9)
    return {"prompt_tokens": prompt_tokens, "new_tokens": new_tokens, "runs": runs,
            "generate_seconds": full, "prefill_and_first_token_seconds": first,
            "decode_tok_s": (new_tokens - 1) / decode, "generate_tok_s": new_tokens / full}
