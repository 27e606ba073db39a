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
products with transposed operands.
"""
from __future__ import annotations

import statistics
import time

import torch
from torch import nn

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
