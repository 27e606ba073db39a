"""Decoder-layer helpers of ``libtexelator_hip.so`` on torch tensors (no reference counterpart:
the reference leaves these layers to Hugging Face modules; see ``include/texelator_hip.h``).

Every function checks shapes, dtypes and devices on the host before the launch, and launches on
the current stream. Nothing here allocates unless an output is not supplied.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._hip import _stream as _device_stream
from ._hip import shape as _hip_shape
from ._lib import TexelatorError, check


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr() if t is not None else None)


def _stream(t: torch.Tensor) -> ctypes.c_void_p:
    return _device_stream(t.device)


def _expect(condition: bool, message: str) -> None:
    if not condition:
        raise TexelatorError(message)


def add_rmsnorm(residual: torch.Tensor, delta: torch.Tensor | None, weight: torch.Tensor, eps: float,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """``residual += delta`` (in place, fp32) then ``out = bf16(weight * bf16(rmsnorm(residual)))``."""
    _expect(residual.is_cuda and residual.dtype == torch.float32 and residual.is_contiguous() and residual.dim() == 2,
            "residual must be a contiguous CUDA float32 [rows, hidden]")
    rows, hidden = residual.shape
    _expect(weight.dtype == torch.bfloat16 and weight.is_contiguous() and weight.numel() == hidden, "weight must be bf16 [hidden]")
    if delta is not None:
        _expect(delta.dtype == torch.bfloat16 and delta.is_contiguous() and delta.shape == residual.shape,
                "delta must be a contiguous bf16 tensor shaped like the residual")
    if out is None:
        out = torch.empty((rows, hidden), dtype=torch.bfloat16, device=residual.device)
    _expect(out.dtype == torch.bfloat16 and out.is_contiguous() and out.shape == residual.shape, "bad output")
    check(_lib.load().tx_add_rmsnorm(_ptr(residual), _ptr(delta), _ptr(weight), float(eps), _ptr(out), rows, hidden,
                                     _stream(residual)))
    return out


def add_rmsnorm_bf16(residual: torch.Tensor, delta: torch.Tensor | None, weight: torch.Tensor,
                     eps: float) -> tuple[torch.Tensor | None, torch.Tensor]:
    """RMSNorm over a bf16 residual ``[..., hidden]`` kept in bf16: with ``delta``, ``(bf16(residual +
    delta), norm of that sum)`` (torch's bf16 add, then Hugging Face's RMSNorm roundings); without,
    ``(None, norm of residual)``. One launch; outputs shaped like ``residual``."""
    _expect(residual.is_cuda and residual.dtype == torch.bfloat16 and residual.is_contiguous()
            and residual.data_ptr() % 8 == 0, "residual must be a contiguous, 8-byte aligned CUDA bf16 tensor")
    hidden = residual.shape[-1]
    rows = residual.numel() // hidden if hidden else 0
    _expect(weight.is_cuda and weight.dtype == torch.bfloat16 and weight.is_contiguous() and weight.numel() == hidden,
            "weight must be bf16 [hidden]")
    total = None
    if delta is not None:
        _expect(delta.dtype == torch.bfloat16 and delta.is_contiguous() and delta.shape == residual.shape
                and delta.device == residual.device, "delta must be a contiguous bf16 tensor shaped like the residual")
        total = torch.empty_like(residual)
    out = torch.empty_like(residual)
    check(_lib.load().tx_add_rmsnorm_bf16(_ptr(residual), _ptr(delta), _ptr(weight), float(eps), _ptr(total), _ptr(out),
                                          rows, hidden, _stream(residual)))
    return total, out


def rope_kv_cache(qkv: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, heads: int,
                  kv_heads: int, head_dim: int, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  q_out: torch.Tensor | None = None) -> torch.Tensor:
    """RoPE on the q and k heads of packed ``[q | k | v]`` rows; k and v go into the caches at
    ``positions``; returns the rotated q ``[tokens, heads * head_dim]``."""
    _expect(qkv.dtype == torch.bfloat16 and qkv.dim() == 2 and qkv.stride(1) == 1, "qkv must be bf16 [tokens, width]")
    tokens = qkv.shape[0]
    _expect(qkv.shape[1] >= (heads + 2 * kv_heads) * head_dim, "qkv row too short for the heads")
    _expect(positions.dtype == torch.int64 and positions.is_contiguous() and positions.numel() == tokens,
            "positions must be int64 [tokens]")
    max_ctx = k_cache.shape[1]
    for cache in (k_cache, v_cache):
        _expect(cache.dtype == torch.bfloat16 and cache.is_contiguous() and tuple(cache.shape) == (kv_heads, max_ctx, head_dim),
                "caches must be contiguous bf16 [kv_heads, max_context, head_dim]")
    for table in (cos, sin):
        _expect(table.dtype == torch.float32 and table.is_contiguous() and tuple(table.shape) == (max_ctx, head_dim),
                "rope tables must be float32 [max_context, head_dim]")
    if q_out is None:
        q_out = torch.empty((tokens, heads * head_dim), dtype=torch.bfloat16, device=qkv.device)
    _expect(q_out.dtype == torch.bfloat16 and q_out.is_contiguous() and q_out.numel() == tokens * heads * head_dim, "bad q_out")
    check(_lib.load().tx_rope_kv_cache(_ptr(qkv), qkv.stride(0), tokens, _ptr(positions), _ptr(cos), _ptr(sin), heads,
                                       kv_heads, head_dim, _ptr(q_out), _ptr(k_cache), _ptr(v_cache), max_ctx,
                                       _stream(qkv)))
    return q_out


def decode_attention_supported(config) -> bool:
    """The fused decode attention handles head_dim 128 and at most 8 query heads per KV head."""
    return config.head_dim == 128 and config.heads % config.kv_heads == 0 and config.heads // config.kv_heads <= 8


def decode_attention_workspace_bytes(heads: int, length: int) -> int:
    out = ctypes.c_int64(0)
    check(_lib.load().tx_decode_attention_workspace(int(heads), int(length), ctypes.byref(out)))
    return int(out.value)


def decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, position: torch.Tensor, length: int,
                     heads: int, kv_heads: int, scale: float, workspace: torch.Tensor,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """One-token grouped-query attention over cache positions 0..position (device int64 [1])."""
    head_dim = k_cache.shape[2]
    _expect(q.dtype == torch.bfloat16 and q.is_contiguous() and q.numel() == heads * head_dim, "q must be bf16 [heads*head_dim]")
    _expect(position.dtype == torch.int64 and position.numel() == 1, "position must be int64 [1]")
    for cache in (k_cache, v_cache):
        _expect(cache.dtype == torch.bfloat16 and cache.is_contiguous() and cache.shape[0] == kv_heads, "bad cache")
    need = decode_attention_workspace_bytes(heads, length)
    _expect(workspace.is_cuda and workspace.numel() * workspace.element_size() >= need, "decode attention workspace too small")
    if out is None:
        out = torch.empty((1, heads * head_dim), dtype=torch.bfloat16, device=q.device)
    check(_lib.load().tx_decode_attention(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(position), int(length), heads,
                                          kv_heads, head_dim, k_cache.shape[1], float(scale), _ptr(workspace),
                                          workspace.numel() * workspace.element_size(), _ptr(out), _stream(q)))
    return out


def prefill_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, heads: int, kv_heads: int,
                      scale: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """Causal self-attention of a prompt: ``q`` bf16 ``[tokens, heads * head_dim]`` (rows 16-byte
    aligned) at positions 0..tokens-1 against cache rows 0..tokens-1 of ``k_cache``/``v_cache``
    (bf16 ``[kv_heads, max_context, head_dim]``). Returns bf16 ``[tokens, heads * head_dim]``."""
    _expect(q.is_cuda and q.dtype == torch.bfloat16 and q.dim() == 2 and q.stride(1) == 1, "q must be bf16 [tokens, width]")
    head_dim = k_cache.shape[2]
    tokens = q.shape[0]
    _expect(q.shape[1] == heads * head_dim, "q width must be heads * head_dim")
    for cache in (k_cache, v_cache):
        _expect(cache.dtype == torch.bfloat16 and cache.is_contiguous() and cache.shape[0] == kv_heads and
                cache.device == q.device, "bad cache")
    if out is None:
        out = torch.empty((tokens, heads * head_dim), dtype=torch.bfloat16, device=q.device)
    _expect(out.dtype == torch.bfloat16 and out.dim() == 2 and out.stride(1) == 1 and out.shape == (tokens, heads * head_dim),
            "bad output")
    check(_lib.load().tx_prefill_attention(_ptr(q), q.stride(0), _ptr(k_cache), _ptr(v_cache), tokens, heads, kv_heads,
                                           head_dim, k_cache.shape[1], float(scale), _ptr(out), out.stride(0),
                                           _stream(q)))
    return out


def decode_attention_split(qkv_handle: int, positions: torch.Tensor, rope_row: torch.Tensor, heads: int,
                           kv_heads: int, head_dim: int, k_cache: torch.Tensor, v_cache: torch.Tensor, length: int,
                           scale: float, workspace: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """:func:`rope_kv_cache_split` then :func:`decode_attention` with one kernel launch fewer
    (bit-identical to the two calls): one token whose ``[q | k | v]`` row is the last
    :func:`linear_split` of ``qkv_handle``; ``rope_row`` holds the RoPE tables' rows at
    ``positions[0]`` (fp32 ``[cos (head_dim) | sin (head_dim)]``). The key and value are written to
    the caches at ``positions[0]``."""
    _expect(positions.dtype == torch.int64 and positions.is_contiguous() and positions.numel() == 1,
            "positions must be int64 [1]")
    _expect(rope_row.dtype == torch.float32 and rope_row.is_contiguous() and rope_row.numel() == 2 * head_dim,
            "rope_row must be float32 [2 * head_dim]")
    max_ctx = k_cache.shape[1]
    for cache in (k_cache, v_cache):
        _expect(cache.dtype == torch.bfloat16 and cache.is_contiguous() and tuple(cache.shape) == (kv_heads, max_ctx, head_dim),
                "caches must be contiguous bf16 [kv_heads, max_context, head_dim]")
    need = decode_attention_workspace_bytes(heads, length)
    _expect(workspace.is_cuda and workspace.numel() * workspace.element_size() >= need, "decode attention workspace too small")
    if out is None:
        out = torch.empty((1, heads * head_dim), dtype=torch.bfloat16, device=k_cache.device)
    _expect(out.dtype == torch.bfloat16 and out.is_contiguous() and out.numel() == heads * head_dim, "bad out")
    check(_lib.load().tx_decode_attention_split(qkv_handle, _ptr(positions), _ptr(rope_row), int(length), heads,
                                                kv_heads, head_dim, _ptr(k_cache), _ptr(v_cache), max_ctx, float(scale),
                                                _ptr(workspace), workspace.numel() * workspace.element_size(),
                                                _ptr(out), _stream(positions)))
    return out


def decode_attention_o_split(qkv_handle: int, o_handle: int, positions: torch.Tensor, rope_row: torch.Tensor,
                             heads: int, kv_heads: int, head_dim: int, k_cache: torch.Tensor, v_cache: torch.Tensor,
                             length: int, scale: float, workspace: torch.Tensor) -> bool:
    """:func:`decode_attention_split` then :func:`linear_split` of ``o_handle`` on its output, with
    the attention's chunk merge done inside the o GEMV (one launch fewer, o's split-K partials
    bitwise the same; read them with :func:`add_rmsnorm_split`). Returns False, with nothing
    launched, where the merge does not fit the o GEMV (more than 16 chunks of 64 positions, too many
    heads per o split, a LUT handle): then make the two calls."""
    _expect(positions.dtype == torch.int64 and positions.is_contiguous() and positions.numel() == 1,
            "positions must be int64 [1]")
    _expect(rope_row.dtype == torch.float32 and rope_row.is_contiguous() and rope_row.numel() == 2 * head_dim,
            "rope_row must be float32 [2 * head_dim]")
    max_ctx = k_cache.shape[1]
    for cache in (k_cache, v_cache):
        _expect(cache.dtype == torch.bfloat16 and cache.is_contiguous() and tuple(cache.shape) == (kv_heads, max_ctx, head_dim),
                "caches must be contiguous bf16 [kv_heads, max_context, head_dim]")
    need = decode_attention_workspace_bytes(heads, length)
    _expect(workspace.is_cuda and workspace.numel() * workspace.element_size() >= need, "decode attention workspace too small")
    status = _lib.load().tx_decode_attention_o_split(qkv_handle, o_handle, _ptr(positions), _ptr(rope_row), int(length),
                                                    heads, kv_heads, head_dim, _ptr(k_cache), _ptr(v_cache), max_ctx,
                                                    float(scale), _ptr(workspace),
                                                    workspace.numel() * workspace.element_size(), _stream(positions))
    if status == _lib.TX_ERR_UNSUPPORTED:
        return False
    check(status)
    return True


def linear_split(handle: int, x: torch.Tensor) -> None:
    """One-token decode GEMV of ``handle`` (``x`` bf16 ``[K]``) whose output stays as split-K
    partials inside the handle, for :func:`add_rmsnorm_split` or :func:`rope_kv_cache_split`."""
    _expect(x.is_cuda and x.dtype == torch.bfloat16 and x.is_contiguous() and x.data_ptr() % 16 == 0,
            "x must be a contiguous, 16-byte aligned CUDA bf16 tensor")
    _expect(x.numel() == _hip_shape(handle)[1], "x has the wrong length for this handle")
    check(_lib.load().tx_linear_split(handle, _ptr(x), _stream(x)))


def linear_swiglu(handle: int, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``swiglu(linear(handle, x))`` for one token of a merged ``[gate | up]`` handle, in one kernel
    (bit-identical to the two calls). Raises ``UnsupportedError`` for a handle whose GEMV is split
    or in LUT mode."""
    _expect(x.is_cuda and x.dtype == torch.bfloat16 and x.is_contiguous() and x.data_ptr() % 16 == 0,
            "x must be a contiguous, 16-byte aligned CUDA bf16 tensor")
    m, k = _hip_shape(handle)
    _expect(x.numel() == k, "x has the wrong length for this handle")
    if out is None:
        out = torch.empty((1, m // 2), dtype=torch.bfloat16, device=x.device)
    _expect(out.dtype == torch.bfloat16 and out.is_contiguous() and out.numel() == m // 2, "bad output")
    check(_lib.load().tx_linear_swiglu(handle, _ptr(x), _ptr(out), _stream(x)))
    return out


def linear_add_bias(handle: int, x: torch.Tensor, bias: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``linear(handle, x) + bias`` for one bf16 token and a separate bf16 bias ``[M]`` (the handle
    has none of its own): the GEMV's bf16 output plus the bias rounded again, bit for bit the two
    operations, in the GEMV's own launches. Returns ``[..., M]`` shaped like ``x``."""
    _expect(x.is_cuda and x.dtype == torch.bfloat16 and x.is_contiguous() and x.data_ptr() % 16 == 0,
            "x must be a contiguous, 16-byte aligned CUDA bf16 tensor")
    m, k = _hip_shape(handle)
    _expect(x.numel() == k and x.shape[-1] == k, "x must be one token of this handle's K")
    _expect(bias.is_cuda and bias.dtype == torch.bfloat16 and bias.is_contiguous() and bias.numel() == m,
            "bias must be a contiguous CUDA bf16 [M]")
    if out is None:
        out = torch.empty((*x.shape[:-1], m), dtype=torch.bfloat16, device=x.device)
    _expect(out.dtype == torch.bfloat16 and out.is_contiguous() and out.numel() == m, "bad output")
    check(_lib.load().tx_linear_add_bias(handle, _ptr(x), _ptr(bias), _ptr(out), _stream(x)))
    return out


def linear_swiglu_pair(gate: int, up: int, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``swiglu(linear(gate, x), linear(up, x))`` for one token over two handles of one shape, in one
    kernel: bit for bit :func:`linear_swiglu` of the merged ``[gate | up]`` handle. Raises
    ``UnsupportedError`` for LUT-mode handles or handles with a bias."""
    _expect(x.is_cuda and x.dtype == torch.bfloat16 and x.is_contiguous() and x.data_ptr() % 16 == 0,
            "x must be a contiguous, 16-byte aligned CUDA bf16 tensor")
    m, k = _hip_shape(gate)
    _expect(_hip_shape(up) == (m, k), "gate and up must have the same shape")
    _expect(x.numel() == k, "x has the wrong length for these handles")
    if out is None:
        out = torch.empty((1, m), dtype=torch.bfloat16, device=x.device)
    _expect(out.dtype == torch.bfloat16 and out.is_contiguous() and out.numel() == m, "bad output")
    check(_lib.load().tx_linear_swiglu_pair(gate, up, _ptr(x), _ptr(out), _stream(x)))
    return out


def _norm_args(residual_in: torch.Tensor, residual_out: torch.Tensor, weight: torch.Tensor, k: int) -> None:
    for name, t in (("residual_in", residual_in), ("residual_out", residual_out)):
        _expect(t.is_cuda and t.dtype == torch.float32 and t.is_contiguous() and t.numel() == k and t.data_ptr() % 16 == 0,
                f"{name} must be a contiguous, 16-byte aligned CUDA float32 row of K values")
    _expect(residual_in.data_ptr() != residual_out.data_ptr(), "residual_out must be another buffer than residual_in")
    _expect(weight.dtype == torch.bfloat16 and weight.is_contiguous() and weight.numel() == k and weight.data_ptr() % 16 == 0,
            "weight must be a contiguous, 16-byte aligned bf16 [K]")


def linear_split_norm(handle: int, residual_in: torch.Tensor, residual_out: torch.Tensor, delta_handle: int,
                      weight: torch.Tensor, eps: float) -> bool:
    """:func:`add_rmsnorm_split` of ``residual_in`` and ``delta_handle``'s last :func:`linear_split`,
    then :func:`linear_split` of ``handle`` on the result, in one launch: the GEMV's workgroups
    normalize their x themselves (bitwise the same partials) and the updated residual goes to
    ``residual_out``. Returns False, with nothing launched, where that does not fit the GEMV (K
    above 2048, a delta split more than 8 ways, a LUT handle, or too many workgroups); then make the
    two calls."""
    _norm_args(residual_in, residual_out, weight, _hip_shape(handle)[1])
    status = _lib.load().tx_linear_split_norm(handle, _ptr(residual_in), _ptr(residual_out), delta_handle, _ptr(weight),
                                             float(eps), _stream(residual_in))
    if status == _lib.TX_ERR_UNSUPPORTED:
        return False
    check(status)
    return True


def linear_split_embed_norm(handle: int, embed: torch.Tensor, token: torch.Tensor, residual_out: torch.Tensor,
                            weight: torch.Tensor, eps: float) -> bool:
    """The first layer's :func:`linear_split_norm`: ``residual_out`` = row ``token`` (device int64
    [1], clamped into the table) of the bf16 embedding table ``embed`` [vocab, K] in fp32, then
    :func:`add_rmsnorm` of it (no delta) and :func:`linear_split` of ``handle``, in one launch.
    False, with nothing launched, where that does not fit the GEMV."""
    k = _hip_shape(handle)[1]
    _expect(embed.is_cuda and embed.dtype == torch.bfloat16 and embed.is_contiguous() and embed.dim() == 2 and
            embed.shape[1] == k and embed.data_ptr() % 16 == 0, "embed must be a contiguous CUDA bf16 [vocab, K] table")
    _expect(token.dtype == torch.int64 and token.numel() == 1 and token.is_contiguous(), "token must be int64 [1]")
    _expect(residual_out.is_cuda and residual_out.dtype == torch.float32 and residual_out.is_contiguous() and
            residual_out.numel() == k and residual_out.data_ptr() % 16 == 0, "residual_out must be float32 [K]")
    _expect(weight.dtype == torch.bfloat16 and weight.is_contiguous() and weight.numel() == k and weight.data_ptr() % 16 == 0,
            "weight must be a contiguous, 16-byte aligned bf16 [K]")
    status = _lib.load().tx_linear_split_embed_norm(handle, _ptr(embed), embed.shape[0], _ptr(token), _ptr(residual_out),
                                                   _ptr(weight), float(eps), _stream(residual_out))
    if status == _lib.TX_ERR_UNSUPPORTED:
        return False
    check(status)
    return True


def linear_swiglu_norm(handle: int, residual_in: torch.Tensor, residual_out: torch.Tensor, delta_handle: int,
                       weight: torch.Tensor, eps: float, out: torch.Tensor) -> bool:
    """:func:`linear_split_norm` for :func:`linear_swiglu`: the add+RMSNorm of the residual and
    ``delta_handle``'s partials, then the gate|up GEMV with its SwiGLU epilogue into ``out``, in one
    launch; False, with nothing launched, where that does not fit."""
    m, k = _hip_shape(handle)
    _norm_args(residual_in, residual_out, weight, k)
    _expect(out.dtype == torch.bfloat16 and out.is_contiguous() and out.numel() == m // 2, "bad output")
    status = _lib.load().tx_linear_swiglu_norm(handle, _ptr(residual_in), _ptr(residual_out), delta_handle, _ptr(weight),
                                              float(eps), _ptr(out), _stream(residual_in))
    if status == _lib.TX_ERR_UNSUPPORTED:
        return False
    check(status)
    return True


def linear_swiglu_prefill(handle: int, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``swiglu(linear(handle, x))`` for a prefill-sized ``x`` [tokens, K] of a merged ``[gate | up]``
    handle, in one GEMM whose epilogue applies SwiGLU (bit-identical to the two calls). Raises
    ``UnsupportedError`` where the call's prefill would run the pair tile or the dense backend, or
    split K."""
    _expect(x.is_cuda and x.dtype == torch.bfloat16 and x.is_contiguous() and x.dim() == 2 and x.data_ptr() % 16 == 0,
            "x must be a contiguous, 16-byte aligned CUDA bf16 [tokens, K] tensor")
    m, k = _hip_shape(handle)
    _expect(x.shape[1] == k, "x has the wrong width for this handle")
    tokens = x.shape[0]
    if out is None:
        out = torch.empty((tokens, m // 2), dtype=torch.bfloat16, device=x.device)
    _expect(out.dtype == torch.bfloat16 and out.is_contiguous() and out.shape == (tokens, m // 2), "bad output")
    check(_lib.load().tx_linear_swiglu_prefill(handle, _ptr(x), tokens, _ptr(out), _stream(x)))
    return out


def prefill_split(handle: int, x: torch.Tensor, workspace: torch.Tensor) -> int:
    """The prefill GEMM of ``x`` [tokens, K] (bf16, at or above the handle's prefill threshold)
    leaving its fp32 K-split partials in ``workspace`` (at least ``workspace_bytes(handle, tokens)``
    bytes) for :func:`add_rmsnorm_prefill_split` or :func:`rope_kv_cache_prefill_split`; returns
    the split count. Raises ``UnsupportedError`` when the call does not split K or runs the dense
    backend (then :func:`linear` is the path)."""
    _expect(x.is_cuda and x.dtype == torch.bfloat16 and x.is_contiguous() and x.dim() == 2 and x.data_ptr() % 16 == 0,
            "x must be a contiguous, 16-byte aligned CUDA bf16 [tokens, K] tensor")
    _expect(x.shape[1] == _hip_shape(handle)[1], "x has the wrong width for this handle")
    _expect(workspace.is_cuda and workspace.is_contiguous() and workspace.data_ptr() % 16 == 0,
            "workspace must be a contiguous, 16-byte aligned CUDA tensor")
    splits = ctypes.c_int(0)
    check(_lib.load().tx_prefill_split(handle, _ptr(x), x.shape[0], _ptr(workspace),
                                       workspace.numel() * workspace.element_size(), ctypes.byref(splits), _stream(x)))
    return splits.value


def add_rmsnorm_prefill_split(residual: torch.Tensor, delta_handle: int, partials: torch.Tensor, weight: torch.Tensor,
                              eps: float, out: torch.Tensor) -> torch.Tensor:
    """:func:`add_rmsnorm` of ``tokens`` rows whose delta is ``linear(delta_handle, x)``, read from
    the partials :func:`prefill_split` left (bit-identical)."""
    _expect(residual.is_cuda and residual.dtype == torch.float32 and residual.is_contiguous() and residual.dim() == 2,
            "residual must be a contiguous CUDA float32 [tokens, hidden]")
    tokens, hidden = residual.shape
    _expect(_hip_shape(delta_handle)[0] == hidden, "the delta handle's output size must equal hidden")
    _expect(weight.dtype == torch.bfloat16 and weight.is_contiguous() and weight.numel() == hidden, "weight must be bf16 [hidden]")
    _expect(out.dtype == torch.bfloat16 and out.is_contiguous() and out.shape == residual.shape, "bad output")
    _expect(partials.is_cuda and partials.is_contiguous(), "partials must be the workspace prefill_split filled")
    check(_lib.load().tx_add_rmsnorm_prefill_split(_ptr(residual), delta_handle, _ptr(partials), tokens, _ptr(weight),
                                                   float(eps), _ptr(out), hidden, _stream(residual)))
    return out


def rope_kv_cache_prefill_split(qkv_handle: int, partials: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor,
                                sin: torch.Tensor, heads: int, kv_heads: int, head_dim: int, k_cache: torch.Tensor,
                                v_cache: torch.Tensor, q_out: torch.Tensor | None = None) -> torch.Tensor:
    """:func:`rope_kv_cache` of ``tokens`` tokens whose ``[q | k | v]`` rows are
    ``linear(qkv_handle, x)``, read from the partials :func:`prefill_split` left (bit-identical);
    returns the rotated q ``[tokens, heads * head_dim]``."""
    _expect(_hip_shape(qkv_handle)[0] >= (heads + 2 * kv_heads) * head_dim, "qkv handle too narrow for the heads")
    _expect(positions.dtype == torch.int64 and positions.is_contiguous() and positions.dim() == 1,
            "positions must be int64 [tokens]")
    tokens = positions.numel()
    max_ctx = k_cache.shape[1]
    for cache in (k_cache, v_cache):
        _expect(cache.dtype == torch.bfloat16 and cache.is_contiguous() and tuple(cache.shape) == (kv_heads, max_ctx, head_dim),
                "caches must be contiguous bf16 [kv_heads, max_context, head_dim]")
    for table in (cos, sin):
        _expect(table.dtype == torch.float32 and table.is_contiguous() and tuple(table.shape) == (max_ctx, head_dim),
                "rope tables must be float32 [max_context, head_dim]")
    _expect(partials.is_cuda and partials.is_contiguous(), "partials must be the workspace prefill_split filled")
    if q_out is None:
        q_out = torch.empty((tokens, heads * head_dim), dtype=torch.bfloat16, device=positions.device)
    _expect(q_out.dtype == torch.bfloat16 and q_out.is_contiguous() and q_out.numel() == tokens * heads * head_dim, "bad q_out")
    check(_lib.load().tx_rope_kv_cache_prefill_split(qkv_handle, _ptr(partials), tokens, _ptr(positions), _ptr(cos),
                                                     _ptr(sin), heads, kv_heads, head_dim, _ptr(q_out), _ptr(k_cache),
                                                     _ptr(v_cache), max_ctx, _stream(positions)))
    return q_out


def add_rmsnorm_split(residual: torch.Tensor, delta_handle: int, weight: torch.Tensor, eps: float,
                      out: torch.Tensor) -> torch.Tensor:
    """:func:`add_rmsnorm` of one row whose delta is the last :func:`linear_split` of ``delta_handle``."""
    _expect(residual.is_cuda and residual.dtype == torch.float32 and residual.is_contiguous() and residual.numel() ==
            weight.numel(), "residual must be a contiguous CUDA float32 row of hidden values")
    hidden = residual.numel()
    _expect(_hip_shape(delta_handle)[0] == hidden, "the delta handle's output size must equal hidden")
    _expect(weight.dtype == torch.bfloat16 and weight.is_contiguous(), "weight must be bf16 [hidden]")
    _expect(out.dtype == torch.bfloat16 and out.is_contiguous() and out.numel() == hidden, "bad output")
    check(_lib.load().tx_add_rmsnorm_split(_ptr(residual), delta_handle, _ptr(weight), float(eps), _ptr(out), hidden,
                                           _stream(residual)))
    return out


def rope_kv_cache_split(qkv_handle: int, positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, heads: int,
                        kv_heads: int, head_dim: int, k_cache: torch.Tensor, v_cache: torch.Tensor,
                        q_out: torch.Tensor) -> torch.Tensor:
    """:func:`rope_kv_cache` of one token whose ``[q | k | v]`` row is the last :func:`linear_split`
    of ``qkv_handle``."""
    _expect(_hip_shape(qkv_handle)[0] >= (heads + 2 * kv_heads) * head_dim, "qkv handle too narrow for the heads")
    _expect(positions.dtype == torch.int64 and positions.is_contiguous() and positions.numel() == 1,
            "positions must be int64 [1]")
    max_ctx = k_cache.shape[1]
    for cache in (k_cache, v_cache):
        _expect(cache.dtype == torch.bfloat16 and cache.is_contiguous() and tuple(cache.shape) == (kv_heads, max_ctx, head_dim),
                "caches must be contiguous bf16 [kv_heads, max_context, head_dim]")
    for table in (cos, sin):
        _expect(table.dtype == torch.float32 and table.is_contiguous() and tuple(table.shape) == (max_ctx, head_dim),
                "rope tables must be float32 [max_context, head_dim]")
    _expect(q_out.dtype == torch.bfloat16 and q_out.is_contiguous() and q_out.numel() == heads * head_dim, "bad q_out")
    check(_lib.load().tx_rope_kv_cache_split(qkv_handle, _ptr(positions), _ptr(cos), _ptr(sin), heads, kv_heads,
                                             head_dim, _ptr(q_out), _ptr(k_cache), _ptr(v_cache), max_ctx,
                                             _stream(positions)))
    return q_out


def lm_head_argmax_workspace_bytes() -> int:
    """Device scratch of :func:`lm_head_argmax`."""
    out = ctypes.c_int64(0)
    check(_lib.load().tx_lm_head_argmax_workspace(ctypes.byref(out)))
    return int(out.value)


def lm_head_argmax(weight: torch.Tensor, x: torch.Tensor, workspace: torch.Tensor, out: torch.Tensor | None = None,
                   logits: torch.Tensor | None = None) -> torch.Tensor:
    """Greedy next token ``argmax(bf16(x @ weight^T))`` (the first row among equal maxima) for one
    bf16 hidden state ``x`` [hidden] or [1, hidden], written to ``out`` (int64 [1]); the bf16
    logits [vocab] too when ``logits`` is given."""
    _expect(weight.is_cuda and weight.dtype == torch.bfloat16 and weight.is_contiguous() and weight.dim() == 2,
            "weight must be a contiguous CUDA bf16 [vocab, hidden] tensor")
    vocab, hidden = weight.shape
    _expect(x.dtype == torch.bfloat16 and x.is_contiguous() and x.numel() == hidden and x.data_ptr() % 16 == 0,
            "x must be one contiguous, 16-byte aligned bf16 hidden state")
    _expect(workspace.is_cuda and workspace.is_contiguous(), "workspace must be a contiguous CUDA tensor")
    if out is None:
        out = torch.empty(1, dtype=torch.int64, device=x.device)
    _expect(out.dtype == torch.int64 and out.is_contiguous() and out.numel() == 1, "out must be int64 [1]")
    if logits is not None:
        _expect(logits.dtype == torch.bfloat16 and logits.is_contiguous() and logits.numel() == vocab, "logits must be bf16 [vocab]")
    check(_lib.load().tx_lm_head_argmax(_ptr(weight), vocab, hidden, _ptr(x), _ptr(logits), _ptr(workspace),
                                        workspace.numel() * workspace.element_size(), _ptr(out), _stream(x)))
    return out


def rope_rotate_half(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Hugging Face's ``apply_rotary_pos_emb`` (rotate-half form) on ``q`` ``[..., tokens, heads,
    dim]`` and ``k`` ``[..., tokens, kv_heads, dim]`` (contiguous bf16, the projections' own layout)
    with ``cos``/``sin`` ``[..., tokens, dim]`` bf16, bit for bit, in one kernel; returns new
    ``(q, k)`` of the same shapes."""
    _expect(all(t.is_cuda and t.dtype == torch.bfloat16 and t.is_contiguous() for t in (q, k, cos, sin)),
            "q, k, cos and sin must be contiguous CUDA bf16 tensors")
    dim = q.shape[-1]
    tokens = cos.numel() // dim
    _expect(cos.shape == sin.shape and cos.shape[-1] == dim and k.shape[-1] == dim and q.dim() >= 2 and k.dim() >= 2,
            "cos and sin must be [tokens, dim] rows of the heads' dim")
    _expect(q.numel() % (tokens * dim) == 0 and k.numel() % (tokens * dim) == 0, "q and k must hold whole tokens")
    heads, kv_heads = q.numel() // (tokens * dim), k.numel() // (tokens * dim)
    _expect(q.shape[-2] == heads and k.shape[-2] == kv_heads, "q and k must be [tokens, heads, dim]")
    q_out, k_out = torch.empty_like(q), torch.empty_like(k)
    check(_lib.load().tx_rope_rotate_half(_ptr(q), _ptr(k), tokens, heads, kv_heads, dim, _ptr(cos), _ptr(sin),
                                          _ptr(q_out), _ptr(k_out), _stream(q)))
    return q_out, k_out


def kv_cache_append(k: torch.Tensor, v: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                    length: torch.Tensor) -> None:
    """One token's ``k`` and ``v`` (``kv_heads x dim`` bf16 each, any view of one token) into a static
    cache ``keys``/``values`` ``[1, kv_heads, max_len, dim]`` at row ``length`` (a CUDA int64 scalar
    tensor), then ``length += 1``, in one launch; a full cache is left unchanged."""
    _expect(keys.is_cuda and keys.dtype == values.dtype == torch.bfloat16 and keys.is_contiguous()
            and values.is_contiguous() and keys.dim() == 4 and keys.shape[0] == 1 and keys.shape == values.shape,
            "keys and values must be contiguous CUDA bf16 [1, kv_heads, max_len, dim]")
    _, kv_heads, max_len, dim = keys.shape
    _expect(k.dtype == v.dtype == torch.bfloat16 and k.numel() == v.numel() == kv_heads * dim
            and k.device == v.device == keys.device, "k and v must be one token's bf16 [kv_heads, dim]")
    _expect(length.is_cuda and length.dtype == torch.int64 and length.numel() == 1 and length.device == keys.device,
            "length must be a CUDA int64 scalar")
    k, v = k.reshape(kv_heads, dim).contiguous(), v.reshape(kv_heads, dim).contiguous()
    check(_lib.load().tx_kv_cache_append(_ptr(k), _ptr(v), kv_heads, dim, _ptr(keys), _ptr(values), max_len,
                                         _ptr(length), _stream(keys)))


def swiglu(gate_up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``bf16(silu(g) * u)`` for rows ``[g | u]``."""
    _expect(gate_up.dtype == torch.bfloat16 and gate_up.is_contiguous() and gate_up.dim() == 2 and gate_up.shape[1] % 2 == 0,
            "gate_up must be contiguous bf16 [rows, 2 * intermediate]")
    rows, width = gate_up.shape
    if out is None:
        out = torch.empty((rows, width // 2), dtype=torch.bfloat16, device=gate_up.device)
    check(_lib.load().tx_swiglu(_ptr(gate_up), rows, width // 2, _ptr(out), _stream(gate_up)))
    return out
