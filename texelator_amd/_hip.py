"""The native operator module of the gfx950 build.

Same function names, argument meaning and error behaviour as the reference's pybind11
module (``texelator/cuda/extension.cpp:27-48``); every call goes through the C ABI of
``libtexelator_hip.so``. PyTorch provides device memory and the current stream only.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import TexelatorError, UnsupportedError, check

_SHAPES: dict[int, tuple[int, int]] = {}
# LUT-mode palette tables, kept alive for as long as a handle uses them.
_PALETTES: dict[int, torch.Tensor] = {}
_DTYPE_CODE = {torch.float16: _lib.TX_DTYPE_F16, torch.bfloat16: _lib.TX_DTYPE_BF16}

# Reference kernel-info names -> prefill candidate ids (autotune.CANDIDATES values).
_KERNEL_INFO_IDS = {
    "cutlass_texture_kernel_info": 5,
    "cutlass_t1_kernel_info": 6,
    "cutlass_t2_kernel_info": 7,
    "cutlass_t3_kernel_info": 8,
    "cutlass_smalln_kernel_info": 9,
}


def _require(condition: bool, message: str) -> None:
    if not condition:
        raise TexelatorError(message)


# torch's raw current-stream query (~0.1 us) where this torch build has it; building a Stream
# object per call (~2 us) was a fifth of a one-token linear's host cost.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device) -> ctypes.c_void_p:
    if _raw_stream is not None:
        return ctypes.c_void_p(_raw_stream(device.index if device.index is not None else torch.cuda.current_device()))
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _aligned(x: torch.Tensor) -> torch.Tensor:
    return x if x.data_ptr() % 16 == 0 else x.clone()


def workspace_bytes(handle: int, tokens: int) -> int:
    """Device scratch the prefill path needs for ``tokens`` tokens (``tx_workspace_bytes``)."""
    out = ctypes.c_int64(0)
    check(_lib.load().tx_workspace_bytes(handle, int(tokens), ctypes.byref(out)))
    return int(out.value)


def _workspace(handle: int, tokens: int, device: torch.device):
    """Stream-ordered scratch from the caching allocator (None when the shape needs none): the
    prefill split-K partials, or a one-token GEMV's, so that calls on one handle from several
    streams never share the handle's own buffer."""
    nbytes = workspace_bytes(handle, tokens) if tokens >= 1 else 0
    if nbytes == 0:
        return None, ctypes.c_void_p(None), 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    return ws, ctypes.c_void_p(ws.data_ptr()), nbytes


def shape(handle: int) -> tuple[int, int]:
    """(M, K) of a handle, cached."""
    cached = _SHAPES.get(handle)
    if cached is None:
        info = handle_info(handle)
        cached = (int(info[0]), int(info[1]))
        _SHAPES[handle] = cached
    return cached


def pack_encoded(blocks: torch.Tensor, scales: torch.Tensor, bias: torch.Tensor | None = None) -> int:
    """Upload one encoded matrix (``texelator_cuda.cu:1260-1327``); returns a handle."""
    _require(not blocks.is_cuda and blocks.dtype == torch.uint8 and blocks.is_contiguous(),
             "blocks must be contiguous CPU uint8")
    _require(not scales.is_cuda and scales.dtype == torch.float32 and scales.is_contiguous(),
             "scales must be contiguous CPU float32")
    rows = scales.numel()
    _require(rows > 0 and blocks.numel() % (rows * 8) == 0, "invalid encoded size")
    bias_ptr = None
    bias_code = -1
    device = torch.cuda.current_device()
    if bias is not None and bias.numel():
        bias = bias.detach().contiguous()
        _require(bias.is_cuda and bias.dtype in _DTYPE_CODE and bias.numel() == rows,
                 "bias must be CUDA FP16 or BF16 [M]")
        bias_ptr = ctypes.c_void_p(bias.data_ptr())
        bias_code = _DTYPE_CODE[bias.dtype]
        device = bias.device.index if bias.device.index is not None else device
    out = ctypes.c_uint64(0)
    lib = _lib.load()
    check(lib.tx_pack_encoded(ctypes.c_void_p(blocks.data_ptr()), blocks.numel(),
                              ctypes.c_void_p(scales.data_ptr()), rows, bias_ptr, bias_code, device,
                              ctypes.byref(out)))
    handle = int(out.value)
    _SHAPES[handle] = (rows, blocks.numel() // rows // 8 * 16)
    return handle


def pack_encoded_device(blocks: torch.Tensor, scales: torch.Tensor, bias: torch.Tensor | None = None) -> int:
    """``pack_encoded`` from device tensors (``tx_pack_encoded_device``): blocks CUDA uint8
    ``[M * K/16 * 8]``, scales CUDA float32 ``[M]``, on the same device."""
    _require(blocks.is_cuda and blocks.dtype == torch.uint8 and blocks.is_contiguous(),
             "blocks must be contiguous CUDA uint8")
    _require(scales.is_cuda and scales.dtype == torch.float32 and scales.is_contiguous(),
             "scales must be contiguous CUDA float32")
    _require(blocks.device == scales.device, "blocks and scales must be on one device")
    rows = scales.numel()
    _require(rows > 0 and blocks.numel() % (rows * 8) == 0, "invalid encoded size")
    bias_ptr, bias_code = None, -1
    if bias is not None and bias.numel():
        bias = bias.detach().contiguous()
        _require(bias.is_cuda and bias.dtype in _DTYPE_CODE and bias.numel() == rows and bias.device == blocks.device,
                 "bias must be CUDA FP16 or BF16 [M]")
        bias_ptr, bias_code = ctypes.c_void_p(bias.data_ptr()), _DTYPE_CODE[bias.dtype]
    out = ctypes.c_uint64(0)
    check(_lib.load().tx_pack_encoded_device(ctypes.c_void_p(blocks.data_ptr()), blocks.numel(),
                                             ctypes.c_void_p(scales.data_ptr()), rows, bias_ptr, bias_code,
                                             blocks.device.index, ctypes.byref(out)))
    handle = int(out.value)
    _SHAPES[handle] = (rows, blocks.numel() // rows // 8 * 16)
    return handle


def concat_rows(handles: list[int]) -> int:
    """A new handle with the rows of ``handles`` (one K) in order (``tx_concat_rows``); every handle
    but the last needs a multiple of 16 rows. The sources stay valid; free the result on its own."""
    handles = [int(handle) for handle in handles]
    array = (ctypes.c_uint64 * len(handles))(*handles)
    out = ctypes.c_uint64(0)
    check(_lib.load().tx_concat_rows(array, len(handles), ctypes.byref(out)))
    handle = int(out.value)
    _SHAPES[handle] = (sum(shape(h)[0] for h in handles), shape(handles[0])[1])
    return handle


def linear(handle: int, x: torch.Tensor) -> torch.Tensor:
    """``y = x W^T (+ bias)`` (``texelator_cuda.cu:1329-1469``); output dtype = input dtype."""
    _require(bool(handle), "null Texelator handle")
    _require(x.is_cuda and x.dtype in _DTYPE_CODE and x.is_contiguous(),
             "input must be contiguous CUDA FP16 or BF16")
    m, k = shape(handle)
    _require(x.dim() >= 1 and x.size(-1) == k, "input shape/device mismatch")
    out_shape = list(x.shape)
    out_shape[-1] = m
    y = torch.empty(out_shape, dtype=x.dtype, device=x.device)
    x = _aligned(x)
    tokens = x.numel() // k
    ws, ws_ptr, ws_bytes = _workspace(handle, tokens, x.device)
    check(_lib.load().tx_linear(handle, ctypes.c_void_p(x.data_ptr()), _DTYPE_CODE[x.dtype], x.numel(),
                                x.size(-1), x.device.index, ctypes.c_void_p(y.data_ptr()), ws_ptr, ws_bytes,
                                _stream(x.device)))
    del ws
    return y


def linear_noalloc_into(handle: int, x: torch.Tensor, y: torch.Tensor) -> None:
    """``linear`` into a caller-provided ``y`` (x's dtype, ``[..., M]``) through
    ``tx_linear_noalloc``: the library allocates nothing and keeps split-K partials in its static
    per-GPU scratch, so calls that overlap on one GPU must be serialised by the caller."""
    m, k = shape(handle)
    if (x.dtype not in _DTYPE_CODE or y.dtype != x.dtype or not x.is_contiguous() or not y.is_contiguous()
            or x.size(-1) != k or y.size(-1) != m or x.numel() // k != y.numel() // m or x.data_ptr() % 16):
        raise TexelatorError("linear_noalloc_into: expected aligned contiguous fp16/bf16 x [..., K] and y [..., M]")
    check(_lib.load().tx_linear_noalloc(handle, ctypes.c_void_p(x.data_ptr()), _DTYPE_CODE[x.dtype], x.numel(), k,
                                        x.device.index, ctypes.c_void_p(y.data_ptr()), _stream(x.device)))


def noalloc_scratch_bytes() -> int:
    out = ctypes.c_int64(0)
    check(_lib.load().tx_noalloc_scratch_bytes(ctypes.byref(out)))
    return int(out.value)


def linear_f32(handle: int, x: torch.Tensor) -> torch.Tensor:
    """Decode GEMV with a float32 output and no bias (parity entry point, ``tx_linear_f32``)."""
    _require(x.is_cuda and x.dtype == torch.bfloat16 and x.is_contiguous(), "input must be contiguous CUDA BF16")
    m, k = shape(handle)
    _require(x.size(-1) == k, "input shape/device mismatch")
    out_shape = list(x.shape)
    out_shape[-1] = m
    y = torch.empty(out_shape, dtype=torch.float32, device=x.device)
    x = _aligned(x)
    check(_lib.load().tx_linear_f32(handle, ctypes.c_void_p(x.data_ptr()), x.numel() // k,
                                    ctypes.c_void_p(y.data_ptr()), _stream(x.device)))
    return y


def linear_f32_into(handle: int, x: torch.Tensor, y: torch.Tensor) -> None:
    """``linear_f32`` writing into a caller-provided float32 ``y`` (no allocation; graph-capturable).

    ``x`` must be a contiguous, 16-byte aligned CUDA bf16 tensor of ``[..., K]`` and ``y`` a
    contiguous CUDA float32 tensor of ``[..., M]`` with the same leading shape."""
    m, k = shape(handle)
    if (x.dtype != torch.bfloat16 or y.dtype != torch.float32 or not x.is_contiguous() or not y.is_contiguous()
            or x.size(-1) != k or y.size(-1) != m or x.numel() // k != y.numel() // m or x.data_ptr() % 16):
        raise TexelatorError("linear_f32_into: expected aligned contiguous bf16 x [..., K] and f32 y [..., M]")
    check(_lib.load().tx_linear_f32(handle, ctypes.c_void_p(x.data_ptr()), x.numel() // k,
                                    ctypes.c_void_p(y.data_ptr()), _stream(x.device)))


def prefill(handle: int, candidate: int, x: torch.Tensor) -> torch.Tensor:
    """Prefill GEMM with an explicit tile candidate (5..9); fp16 or bf16 in, the same type out."""
    _require(x.is_cuda and x.dtype in _DTYPE_CODE and x.is_contiguous(), "input must be contiguous CUDA FP16 or BF16")
    m, k = shape(handle)
    _require(x.size(-1) == k, "input shape/device mismatch")
    out_shape = list(x.shape)
    out_shape[-1] = m
    y = torch.empty(out_shape, dtype=x.dtype, device=x.device)
    x = _aligned(x)
    tokens = x.numel() // k
    ws, ws_ptr, ws_bytes = _workspace(handle, tokens, x.device)
    check(_lib.load().tx_prefill(handle, int(candidate), ctypes.c_void_p(x.data_ptr()), _DTYPE_CODE[x.dtype], tokens,
                                 ctypes.c_void_p(y.data_ptr()), ws_ptr, ws_bytes, _stream(x.device)))
    del ws
    return y


def prefill_into(handle: int, candidate: int, x: torch.Tensor, y: torch.Tensor,
                 workspace: torch.Tensor | None = None) -> None:
    """``prefill`` writing into a caller-provided ``y`` of ``[..., M]`` (x's dtype); ``workspace``
    (a CUDA tensor of at least ``workspace_bytes(handle, tokens)`` bytes) is required when that is
    nonzero."""
    m, k = shape(handle)
    if (x.dtype not in _DTYPE_CODE or y.dtype != x.dtype or not x.is_contiguous() or not y.is_contiguous()
            or x.size(-1) != k or y.size(-1) != m or x.numel() // k != y.numel() // m or x.data_ptr() % 16):
        raise TexelatorError("prefill_into: expected aligned contiguous fp16/bf16 x [..., K] and y [..., M] of x's dtype")
    ws_ptr = ctypes.c_void_p(workspace.data_ptr()) if workspace is not None else ctypes.c_void_p(None)
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    check(_lib.load().tx_prefill(handle, int(candidate), ctypes.c_void_p(x.data_ptr()), _DTYPE_CODE[x.dtype],
                                 x.numel() // k, ctypes.c_void_p(y.data_ptr()), ws_ptr, ws_bytes, _stream(x.device)))


def set_lookahead(handle: int, lookahead: int) -> None:
    check(_lib.load().tx_set_lookahead(handle, int(lookahead)))


def set_prefill(handle: int, threshold: int, tile_rows: int) -> None:
    check(_lib.load().tx_set_prefill(handle, int(threshold), int(tile_rows)))


def set_prefill_backend(handle: int, backend: int) -> None:
    check(_lib.load().tx_set_prefill_backend(handle, int(backend)))


def handle_info(handle: int) -> list[int]:
    """``[M, K, threshold, tile_rows, backend, pipelined, graphics]`` (``texelator_cuda.cu:1505-1512``)."""
    out = (ctypes.c_int64 * 7)()
    check(_lib.load().tx_handle_info(handle, out, 7))
    return [int(v) for v in out]


def gemv_plan(handle: int) -> tuple[int, bool]:
    """(K splits of the one-token GEMV, LUT mode) of a handle."""
    out = (ctypes.c_int64 * 11)()
    check(_lib.load().tx_handle_info(handle, out, 11))
    return int(out[9]), bool(out[10])


def lookahead(handle: int) -> int:
    out = (ctypes.c_int64 * 8)()
    check(_lib.load().tx_handle_info(handle, out, 8))
    return int(out[7])


def free(handle: int) -> None:
    check(_lib.load().tx_free(handle))
    _SHAPES.pop(handle, None)
    _PALETTES.pop(handle, None)


def set_palette_table(handle: int, table: torch.Tensor | None) -> None:
    """LUT-mode decode: read every block's palette from ``table`` (255 x 255 x 8 float32 on the
    handle's device, probe layout ``[e1 + 127][e0 + 127][s]``) instead of this build's defined
    palette; ``None`` restores the defined palette. The table is kept alive with the handle."""
    if table is None:
        check(_lib.load().tx_set_palette_table(handle, ctypes.c_void_p(None)))
        _PALETTES.pop(handle, None)
        return
    _require(table.is_cuda and table.dtype == torch.float32 and table.numel() == 255 * 255 * 8,
             "palette table must be a CUDA float32 tensor of 255*255*8 values")
    table = table.contiguous()
    check(_lib.load().tx_set_palette_table(handle, ctypes.c_void_p(table.data_ptr())))
    _PALETTES[handle] = table


def palette_probe() -> torch.Tensor:
    """Device-decoded palette, ``[65025, 8]`` float32 on the CPU (``texelator_cuda.cu:1551-1595``)."""
    out = torch.empty((255 * 255, 8), dtype=torch.float32)
    check(_lib.load().tx_palette_probe(ctypes.c_void_p(out.data_ptr())))
    return out


def decode_dense(handle: int, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Decoded weights as a dense ``[M, K]`` device tensor (diagnostic): bf16 (the BF16 path's
    weights) or fp16 (the FP16 path's)."""
    _require(dtype in _DTYPE_CODE, "dtype must be torch.float16 or torch.bfloat16")
    m, k = shape(handle)
    device = torch.device("cuda", torch.cuda.current_device())
    out = torch.empty((m, k), dtype=dtype, device=device)
    check(_lib.load().tx_decode_dense(handle, _DTYPE_CODE[dtype], ctypes.c_void_p(out.data_ptr()), _stream(device)))
    return out


def kernel_info(candidate: int) -> list[int]:
    """``[vgprs, static_lds, private, max_threads, tile_lds, tokens_tile, rows_tile, k_tile,
    active_workgroups_per_cu]`` -- the nine fields of the reference's ``cutlass_*_kernel_info``
    (``cutlass_texture_mainloop.cu:251-267``)."""
    out = (ctypes.c_int64 * 9)()
    check(_lib.load().tx_kernel_info(int(candidate), out, 9))
    return [int(v) for v in out]


def candidate_name(candidate: int) -> str | None:
    name = _lib.load().tx_candidate_name(int(candidate))
    return name.decode() if name else None


def cutlass_texture_kernel_info() -> list[int]:
    return kernel_info(_KERNEL_INFO_IDS["cutlass_texture_kernel_info"])


def cutlass_t1_kernel_info() -> list[int]:
    return kernel_info(_KERNEL_INFO_IDS["cutlass_t1_kernel_info"])


def cutlass_t2_kernel_info() -> list[int]:
    return kernel_info(_KERNEL_INFO_IDS["cutlass_t2_kernel_info"])


def cutlass_t3_kernel_info() -> list[int]:
    return kernel_info(_KERNEL_INFO_IDS["cutlass_t3_kernel_info"])


def cutlass_smalln_kernel_info() -> list[int]:
    return kernel_info(_KERNEL_INFO_IDS["cutlass_smalln_kernel_info"])


def _no_counterpart(name: str):
    def unsupported(*_args, **_kwargs):
        raise UnsupportedError(f"{name} has no gfx950 counterpart in this build")
    unsupported.__name__ = name
    return unsupported


# The reference's CUDA-only diagnostics (texelator_cuda.cu:1514-1536).
pipeline_kernel_info = _no_counterpart("pipeline_kernel_info")
graphics_kernel_info = _no_counterpart("graphics_kernel_info")


# FP4 hybrid staging (texelator_cuda.cu:1154-1260) in gfx950's MXFP4 format: packed E2M1 values
# uint8 [rows][K/2] (even column in the low nibble) and one E8M0 scale uint8 per 32 values
# [rows][K/32]. The reference's NVFP4 scales (E4M3 per 16, blocked) feed Blackwell's FP4 GEMM;
# these feed fp4_gemm.
def _fp4_buffers(rows: int, k: int, device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
    return (torch.empty((rows, k // 2), dtype=torch.uint8, device=device),
            torch.empty((rows, k // 32), dtype=torch.uint8, device=device))


def _check_fp4_out(packed: torch.Tensor, scales: torch.Tensor, rows: int, k: int, device: torch.device) -> None:
    _require(packed.is_cuda and packed.is_contiguous() and packed.dtype == torch.uint8 and
             tuple(packed.shape) == (rows, k // 2) and packed.device == device,
             f"packed must be contiguous CUDA uint8 [{rows}, {k // 2}]")
    _require(scales.is_cuda and scales.is_contiguous() and scales.dtype == torch.uint8 and
             tuple(scales.shape) == (rows, k // 32) and scales.device == device,
             f"scales must be contiguous CUDA uint8 [{rows}, {k // 32}]")


def quantize_activation_fp4_out(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor) -> None:
    _require(x.is_cuda and x.is_contiguous() and x.dtype == torch.bfloat16 and x.dim() == 2,
             "activation must be contiguous CUDA BF16 [tokens,K]")
    rows, k = x.shape
    _require(k % 32 == 0, "activation K must be divisible by 32")
    _check_fp4_out(packed, scales, rows, k, x.device)
    x = _aligned(x)
    check(_lib.load().tx_quantize_activation_fp4(ctypes.c_void_p(x.data_ptr()), _DTYPE_CODE[x.dtype], rows, k,
                                                  ctypes.c_void_p(packed.data_ptr()), ctypes.c_void_p(scales.data_ptr()),
                                                  x.device.index, _stream(x.device)))


def quantize_activation_fp4(x: torch.Tensor) -> list[torch.Tensor]:
    _require(x.is_cuda and x.dim() == 2, "activation must be contiguous CUDA BF16 [tokens,K]")
    packed, scales = _fp4_buffers(x.shape[0], x.shape[1], x.device)
    quantize_activation_fp4_out(x, packed, scales)
    return [packed, scales]


def decode_weight_fp4_out(handle: int, packed: torch.Tensor, scales: torch.Tensor) -> None:
    _require(bool(handle), "null Texelator handle")
    m, k = shape(handle)
    device = packed.device
    _check_fp4_out(packed, scales, m, k, device)
    check(_lib.load().tx_decode_weight_fp4(handle, ctypes.c_void_p(packed.data_ptr()),
                                           ctypes.c_void_p(scales.data_ptr()), _stream(device)))


def decode_weight_fp4(handle: int) -> list[torch.Tensor]:
    _require(bool(handle), "null Texelator handle")
    m, k = shape(handle)
    packed, scales = _fp4_buffers(m, k, torch.device("cuda", torch.cuda.current_device()))
    decode_weight_fp4_out(handle, packed, scales)
    return [packed, scales]


def fp4_gemm(x_packed: torch.Tensor, x_scales: torch.Tensor, w_packed: torch.Tensor, w_scales: torch.Tensor,
             bias: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """``y = deq(x) @ deq(w)^T`` (bf16, fp32 accumulation) ``(+ bias)``, the block-scaled GEMM the
    reference runs as ``torch._scaled_mm`` (``runtime.py:110-116``)."""
    tokens, m = x_packed.shape[0], w_packed.shape[0]
    k = 2 * x_packed.shape[1]
    device = x_packed.device
    _check_fp4_out(x_packed, x_scales, tokens, k, device)
    _check_fp4_out(w_packed, w_scales, m, k, device)
    _require(k % 64 == 0, "FP4 GEMM K must be a multiple of 64")
    if bias is not None:
        _require(bias.is_cuda and bias.dtype == torch.bfloat16 and bias.numel() == m and bias.is_contiguous(),
                 "bias must be contiguous CUDA BF16 [M]")
    y = torch.empty((tokens, m), dtype=torch.bfloat16, device=device) if out is None else out
    _require(y.dtype == torch.bfloat16 and y.is_contiguous() and tuple(y.shape) == (tokens, m),
             f"output must be contiguous BF16 [{tokens}, {m}]")
    check(_lib.load().tx_fp4_gemm(ctypes.c_void_p(x_packed.data_ptr()), ctypes.c_void_p(x_scales.data_ptr()),
                                  ctypes.c_void_p(w_packed.data_ptr()), ctypes.c_void_p(w_scales.data_ptr()),
                                  ctypes.c_void_p(None if bias is None else bias.data_ptr()), tokens, m, k,
                                  ctypes.c_void_p(y.data_ptr()), device.index, _stream(device)))
    return y
