"""ctypes binding of ``libtexelator_hip.so`` (the C ABI in ``include/texelator_hip.h``).

There is no fallback: if the library is missing or fails to load, every call raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import os

PACKAGE_ROOT = Path(__file__).resolve().parent
# TEXELATOR_HIP_LIBRARY selects another build of the same library (e.g. one compiled with
# different tile constants by texelator_amd.build); the default is the in-tree build.
LIBRARY_PATH = Path(os.environ.get("TEXELATOR_HIP_LIBRARY", PACKAGE_ROOT / "libtexelator_hip.so"))

TX_OK = 0
TX_ERR_INVALID = 1
TX_ERR_HIP = 2
TX_ERR_UNSUPPORTED = 3

TX_DTYPE_F16 = 0
TX_DTYPE_BF16 = 1
TX_DTYPE_F32 = 2

# name -> (restype, argtypes); every symbol declared in include/texelator_hip.h
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_U64 = ctypes.c_uint64
SIGNATURES = {
    "tx_last_error": (ctypes.c_char_p, []),
    "tx_pack_encoded": (_I32, [_P, _I64, _P, _I64, _P, _I32, _I32, ctypes.POINTER(_U64)]),
    "tx_pack_encoded_device": (_I32, [_P, _I64, _P, _I64, _P, _I32, _I32, ctypes.POINTER(_U64)]),
    "tx_linear": (_I32, [_U64, _P, _I32, _I64, _I64, _I32, _P, _P, _I64, _P]),
    "tx_workspace_bytes": (_I32, [_U64, _I64, ctypes.POINTER(_I64)]),
    "tx_linear_noalloc": (_I32, [_U64, _P, _I32, _I64, _I64, _I32, _P, _P]),
    "tx_noalloc_scratch_bytes": (_I32, [ctypes.POINTER(_I64)]),
    "tx_quantize_activation_fp4": (_I32, [_P, _I32, _I64, _I64, _P, _P, _I32, _P]),
    "tx_decode_weight_fp4": (_I32, [_U64, _P, _P, _P]),
    "tx_fp4_gemm": (_I32, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _I32, _P]),
    "tx_linear_f32": (_I32, [_U64, _P, _I64, _P, _P]),
    "tx_prefill": (_I32, [_U64, _I32, _P, _I32, _I64, _P, _P, _I64, _P]),
    "tx_set_lookahead": (_I32, [_U64, _I32]),
    "tx_set_prefill": (_I32, [_U64, _I32, _I32]),
    "tx_set_prefill_backend": (_I32, [_U64, _I32]),
    "tx_set_palette_table": (_I32, [_U64, _P]),
    "tx_handle_info": (_I32, [_U64, ctypes.POINTER(_I64), _I32]),
    "tx_free": (_I32, [_U64]),
    "tx_add_rmsnorm_bf16": (_I32, [_P, _P, _P, ctypes.c_float, _P, _P, _I64, _I64, _P]),
    "tx_concat_rows": (_I32, [ctypes.POINTER(_U64), _I32, ctypes.POINTER(_U64)]),
    "tx_palette_probe": (_I32, [_P]),
    "tx_decode_dense": (_I32, [_U64, _I32, _P, _P]),
    "tx_kernel_info": (_I32, [_I32, ctypes.POINTER(_I64), _I32]),
    "tx_candidate_name": (ctypes.c_char_p, [_I32]),
    "tx_add_rmsnorm": (_I32, [_P, _P, _P, ctypes.c_float, _P, _I64, _I64, _P]),
    "tx_rope_kv_cache": (_I32, [_P, _I64, _I64, _P, _P, _P, _I32, _I32, _I32, _P, _P, _P, _I64, _P]),
    "tx_decode_attention_workspace": (_I32, [_I32, _I64, ctypes.POINTER(_I64)]),
    "tx_decode_attention": (_I32, [_P, _P, _P, _P, _I64, _I32, _I32, _I32, _I64, ctypes.c_float, _P, _I64, _P, _P]),
    "tx_decode_attention_split": (_I32, [_U64, _P, _P, _I64, _I32, _I32, _I32, _P, _P, _I64, ctypes.c_float, _P, _I64,
                                         _P, _P]),
    "tx_decode_attention_o_split": (_I32, [_U64, _U64, _P, _P, _I64, _I32, _I32, _I32, _P, _P, _I64, ctypes.c_float,
                                           _P, _I64, _P]),
    "tx_swiglu": (_I32, [_P, _I64, _I64, _P, _P]),
    "tx_lm_head_argmax_workspace": (_I32, [ctypes.POINTER(ctypes.c_int64)]),
    "tx_lm_head_argmax": (_I32, [_P, _I64, _I64, _P, _P, _P, _I64, _P, _P]),
    "tx_linear_split": (_I32, [_U64, _P, _P]),
    "tx_linear_swiglu": (_I32, [_U64, _P, _P, _P]),
    "tx_linear_swiglu_pair": (_I32, [_U64, _U64, _P, _P, _P]),
    "tx_kv_cache_append": (_I32, [_P, _P, _I32, _I32, _P, _P, _I64, _P, _P]),
    "tx_rope_rotate_half": (_I32, [_P, _P, _I64, _I32, _I32, _I32, _P, _P, _P, _P, _P]),
    "tx_linear_add_bias": (_I32, [_U64, _P, _P, _P, _P]),
    "tx_linear_swiglu_prefill": (_I32, [_U64, _P, _I64, _P, _P]),
    "tx_prefill_attention": (_I32, [_P, _I64, _P, _P, _I64, _I32, _I32, _I32, _I64, ctypes.c_float, _P, _I64, _P]),
    "tx_stream_read": (_I32, [_P, _I64, _P, _P]),
    "tx_add_rmsnorm_split": (_I32, [_P, _U64, _P, ctypes.c_float, _P, _I64, _P]),
    "tx_linear_split_norm": (_I32, [_U64, _P, _P, _U64, _P, ctypes.c_float, _P]),
    "tx_linear_swiglu_norm": (_I32, [_U64, _P, _P, _U64, _P, ctypes.c_float, _P, _P]),
    "tx_linear_split_embed_norm": (_I32, [_U64, _P, _I64, _P, _P, _P, ctypes.c_float, _P]),
    "tx_rope_kv_cache_split": (_I32, [_U64, _P, _P, _P, _I32, _I32, _I32, _P, _P, _P, _I64, _P]),
    "tx_prefill_split": (_I32, [_U64, _P, _I64, _P, _I64, ctypes.POINTER(ctypes.c_int), _P]),
    "tx_add_rmsnorm_prefill_split": (_I32, [_P, _U64, _P, _I64, _P, ctypes.c_float, _P, _I64, _P]),
    "tx_rope_kv_cache_prefill_split": (_I32, [_U64, _P, _I64, _P, _P, _P, _I32, _I32, _I32, _P, _P, _P, _I64, _P]),
}

_LIB = None


class TexelatorError(RuntimeError):
    """A failed C-ABI call (the reference raises RuntimeError from TORCH_CHECK)."""


class UnsupportedError(TexelatorError):
    pass


def load() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIBRARY_PATH.exists():
            raise TexelatorError(
                f"the gfx950 BC4 library is not built ({LIBRARY_PATH}); run `python -m texelator_amd.build`")
        lib = ctypes.CDLL(str(LIBRARY_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _LIB = lib
    return _LIB


def check(status: int) -> None:
    if status == TX_OK:
        return
    message = load().tx_last_error().decode(errors="replace") or f"texelator status {status}"
    if status == TX_ERR_UNSUPPORTED:
        raise UnsupportedError(message)
    raise TexelatorError(message)
