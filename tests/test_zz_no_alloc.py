"""tx_linear_noalloc, the allocation-free tx_linear, against tx_linear through the C ABI.

The entry point keeps split-K partial sums in the library's static per-GPU scratch instead of a
caller workspace or the handle's own buffer. Its results must be bitwise those of tx_linear (same
kernels, same reduction order), call after call: each case runs two calls in a row, the second
with a smaller input, so the second reads a scratch that still holds the first call's partials.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.helpers import bf16_vector, f16_vector, lognormal_scales, random_blocks

pytestmark = pytest.mark.gpu


def _pack(ext, m, k, seed, bias=None):
    blocks = random_blocks(m, k, seed)
    scales = lognormal_scales(m, seed + 1)
    return ext.pack_encoded(torch.from_numpy(np.ascontiguousarray(blocks).reshape(-1)), torch.from_numpy(scales), bias)


def _noalloc(ext, handle, x):
    m, _ = ext.shape(handle)
    y = torch.full(list(x.shape[:-1]) + [m], float("nan"), dtype=x.dtype, device=x.device)
    ext.linear_noalloc_into(handle, x, y)
    return y


def test_scratch_size():
    from texelator_amd import _hip

    assert _hip.noalloc_scratch_bytes() == 32 << 20


# (M, K, tokens of the first call, tokens of the second, smaller, call)
PREFILL = [(1024, 5120, 512, 130), (300, 27648, 64, 32), (5120, 5120, 128, 17)]


@pytest.mark.parametrize("m,k,first,second", PREFILL)
def test_prefill_split_k_matches_linear(ext, m, k, first, second):
    handle = _pack(ext, m, k, 7 + m, bias=bf16_vector((m,), 8 + m, scale=0.1).cuda())
    try:
        assert ext.workspace_bytes(handle, first) > 0 and ext.workspace_bytes(handle, second) > 0
        for tokens in (first, second):
            x = bf16_vector((tokens, k), tokens + m).cuda()
            want = ext.linear(handle, x)
            got = _noalloc(ext, handle, x)
            torch.cuda.synchronize()
            assert torch.equal(want, got), (m, k, tokens)
    finally:
        ext.free(handle)


def test_one_token_gemv_splits_match_linear(ext):
    """Two one-token GEMVs with K splits in a row: a long-K matrix, then a smaller one."""
    big = _pack(ext, 64, 27648, 21)
    small = _pack(ext, 300, 2064, 22)
    try:
        for handle, k in ((big, 27648), (small, 2064)):
            splits, _ = ext.gemv_plan(handle)
            assert splits > 1
            x = bf16_vector((1, k), k).cuda()
            want = ext.linear(handle, x)
            got = _noalloc(ext, handle, x)
            torch.cuda.synchronize()
            assert torch.equal(want, got), k
    finally:
        ext.free(big)
        ext.free(small)


def test_fp16_bias_and_multi_token_gemv_match_linear(ext):
    """fp16 with a bias: a 40-token prefill, then 5 tokens under the threshold (the unsplit GEMV)."""
    m, k = 333, 2048
    handle = _pack(ext, m, k, 31, bias=f16_vector((m,), 32, scale=0.5).cuda())
    try:
        for tokens in (40, 5):
            x = f16_vector((tokens, k), 33 + tokens).cuda()
            want = ext.linear(handle, x)
            got = _noalloc(ext, handle, x)
            torch.cuda.synchronize()
            assert got.dtype == torch.float16 and torch.equal(want, got), tokens
    finally:
        ext.free(handle)


def test_errors_are_reported_before_any_launch(ext):
    import ctypes

    from texelator_amd import _lib

    handle = _pack(ext, 64, 256, 41)
    try:
        x = torch.zeros((1, 256), dtype=torch.bfloat16, device="cuda")
        y = torch.empty((1, 64), dtype=torch.bfloat16, device="cuda")
        lib = _lib.load()
        status = lib.tx_linear_noalloc(handle, ctypes.c_void_p(x.data_ptr()), _lib.TX_DTYPE_BF16, 256, 128, 0,
                                       ctypes.c_void_p(y.data_ptr()), None)
        assert status == _lib.TX_ERR_INVALID and b"shape" in lib.tx_last_error()
        status = lib.tx_linear_noalloc(handle, ctypes.c_void_p(x.data_ptr()), _lib.TX_DTYPE_F32, 256, 256, 0,
                                       ctypes.c_void_p(y.data_ptr()), None)
        assert status == _lib.TX_ERR_INVALID and b"FP16 or BF16" in lib.tx_last_error()
        bf_bias = _pack(ext, 64, 256, 42, bias=bf16_vector((64,), 43).cuda())
        try:
            x16 = torch.zeros((1, 256), dtype=torch.float16, device="cuda")
            with pytest.raises(RuntimeError, match="dtypes must match"):
                ext.linear_noalloc_into(bf_bias, x16, torch.empty((1, 64), dtype=torch.float16, device="cuda"))
        finally:
            ext.free(bf_bias)
    finally:
        ext.free(handle)


def test_dense_backend_is_refused_before_any_launch(ext):
    """Backend 1 (dense scratch + library GEMM) creates library state on first use, so the
    allocation-free entry point refuses its prefill-sized calls; one-token calls of the same
    handle still run the GEMV and match tx_linear."""
    from texelator_amd import _lib

    m, k = 256, 2048
    handle = _pack(ext, m, k, 51)
    try:
        ext.set_prefill(handle, 16, 128)
        ext.set_prefill_backend(handle, 1)
        x = bf16_vector((64, k), 52).cuda()
        y = torch.full((64, m), float("nan"), dtype=torch.bfloat16, device="cuda")
        with pytest.raises(_lib.UnsupportedError, match="backend 1"):
            ext.linear_noalloc_into(handle, x, y)
        torch.cuda.synchronize()
        assert torch.isnan(y.float()).all()  # nothing was launched
        x1 = bf16_vector((1, k), 53).cuda()
        assert torch.equal(ext.linear(handle, x1), _noalloc(ext, handle, x1))
    finally:
        ext.free(handle)
