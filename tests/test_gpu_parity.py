"""GPU parity of the gfx950 BC4 path against the CPU oracle, through the C ABI.

Bars: decoded weights bit-exact; GEMV fp32 output within 1e-3 relative
error of the float64 CPU matvec on the same decoded weights; prefill bf16 output within 1e-2
relative RMS of the float64 CPU GEMM; all prefill candidates bitwise equal (the reference's
autotuner gate, texelator/autotune.py:160-168).
"""
from __future__ import annotations

import hashlib

import numpy as np
import pytest
import torch

from oracle import bc4, clib
from tests.helpers import (bf16_bits, bf16_vector, f16_vector, lognormal_scales, max_rel_err_floor, random_blocks,
                           rel_err)

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-3
PREFILL_RRMS_TOL = 1e-2


def _pack(ext, blocks, scales, bias=None):
    return ext.pack_encoded(torch.from_numpy(np.ascontiguousarray(blocks).reshape(-1)),
                            torch.from_numpy(np.ascontiguousarray(scales)), bias)


def test_palette_probe_bitwise_equals_cpu_palette(ext):
    probe = ext.palette_probe().numpy()
    cpu = bc4.palette().reshape(255 * 255, 8)
    assert probe.shape == (65025, 8)
    assert np.array_equal(probe.view(np.uint32), cpu.view(np.uint32))
    assert hashlib.sha256(probe.astype("<f4").tobytes()).hexdigest() == bc4.palette_sha256()


def _every_endpoint_pair_blocks() -> np.ndarray:
    """255 rows x 255 blocks: row r has e0 = r - 127, block b has e1 = b - 127, and position p of
    every block selects palette slot p % 8, so all 65025 endpoint pairs and all eight slots occur."""
    field = sum((p % 8) << (3 * p) for p in range(16)).to_bytes(6, "little")
    blocks = np.empty((255, 255, 8), dtype=np.uint8)
    blocks[:, :, 0] = (np.arange(255) - 127).astype(np.int8).view(np.uint8)[:, None]
    blocks[:, :, 1] = (np.arange(255) - 127).astype(np.int8).view(np.uint8)[None, :]
    blocks[:, :, 2:] = np.frombuffer(field, dtype=np.uint8)
    return blocks.reshape(255, 255 * 8)


def test_every_endpoint_pair_decodes_exactly_in_gemv_and_prefill(ext, oracle_threads):
    """The decoded weights inside the GEMV and the prefill kernels, read back exactly: one-hot
    activations make every output a single decoded weight (times 1.0, plus exact zeros). Covers
    every endpoint pair and palette slot, i.e. every entry of the palette-seed tables the
    kernels copy into LDS, through the one-token and the 16-token GEMV and every prefill tile
    (identity activations over the ragged K = 4080: the prefill returns W^T)."""
    blocks = _every_endpoint_pair_blocks()
    scales = lognormal_scales(255, 901)
    m, k = 255, 255 * 16
    want = clib.decode_bf16_bits(blocks, scales).view(np.int16)
    want = torch.from_numpy(want).view(torch.bfloat16).float().numpy()
    handle = _pack(ext, blocks, scales)
    try:
        for b in range(255):  # 16-token GEMV: the 16 positions of block b
            x = torch.zeros((16, k), dtype=torch.bfloat16)
            x[torch.arange(16), 16 * b + torch.arange(16)] = 1.0
            got = ext.linear_f32(handle, x.cuda()).cpu().numpy()
            assert np.array_equal(got, want[:, 16 * b:16 * b + 16].T), f"16-token GEMV, block {b}"
        for col in (0, 7, 15, 1600, 4079):  # one-token GEMV
            x = torch.zeros((1, k), dtype=torch.bfloat16)
            x[0, col] = 1.0
            got = ext.linear_f32(handle, x.cuda()).cpu().numpy()
            assert np.array_equal(got[0], want[:, col]), f"one-token GEMV, column {col}"
        eye = torch.eye(k, dtype=torch.bfloat16).cuda()
        for candidate in range(5, 10):
            got = ext.prefill(handle, candidate, eye).float().cpu().numpy()
            assert np.array_equal(got, want.T), f"prefill candidate {candidate}"
        torch.cuda.synchronize()
    finally:
        ext.free(handle)


@pytest.mark.parametrize("m,k", [(300, 2064), (7168, 5120), (2048, 2048), (256, 2048), (11008, 2048)])
def test_fused_one_token_gemv_bitwise_equals_split_path(ext, oracle_threads, m, k):
    """Shapes whose K splits run in one workgroup (row groups spread evenly over the CUs) give
    exactly the split GEMV + reduce result. LUT mode with the defined palette decodes the same
    weights but always takes the split path, so every output is compared bit for bit: fp32, bf16
    with a bias, and the no-allocation entry point; such calls need no workspace."""
    blocks = random_blocks(m, k, 951)
    scales = lognormal_scales(m, 952)
    bias = bf16_vector((m,), 953, scale=0.5).cuda()
    x = bf16_vector((1, k), 954).cuda()
    fused = _pack(ext, blocks, scales, bias)
    split = _pack(ext, blocks, scales, bias)
    try:
        ext.set_palette_table(split, torch.from_numpy(bc4.palette()).cuda())
        assert ext.workspace_bytes(fused, 1) == 0
        assert ext.workspace_bytes(split, 1) > 0, "the shape must be split for the comparison to mean anything"
        assert torch.equal(ext.linear_f32(fused, x), ext.linear_f32(split, x))
        y = ext.linear(fused, x)
        assert torch.equal(y, ext.linear(split, x))
        y_noalloc = torch.empty_like(y)
        ext.linear_noalloc_into(fused, x, y_noalloc)
        assert torch.equal(y, y_noalloc)
        torch.cuda.synchronize()
        w = clib.decode_bf16_bits(blocks, scales)
        ref = clib.matvec_f64(w, bf16_bits(x[0].cpu()))
        got = ext.linear_f32(fused, x)[0].double().cpu().numpy()
        assert max_rel_err_floor(ref, got) <= GEMV_TOL
    finally:
        ext.free(fused)
        ext.free(split)


@pytest.mark.parametrize("m,k,seed", [(16, 128, 1), (37, 272, 2), (100, 16, 3), (64, 4096, 4), (5, 2064, 5)])
def test_decode_dense_bit_exact(ext, oracle_threads, m, k, seed):
    blocks = random_blocks(m, k, seed)
    scales = lognormal_scales(m, seed + 100)
    handle = _pack(ext, blocks, scales)
    try:
        dense = ext.decode_dense(handle)
        torch.cuda.synchronize()
        got = bf16_bits(dense.cpu())
    finally:
        ext.free(handle)
    want = clib.decode_bf16_bits(blocks, scales)
    assert got.shape == want.shape
    mismatches = int(np.count_nonzero(got != want))
    assert mismatches == 0, f"{mismatches} of {want.size} decoded weights differ"


@pytest.mark.parametrize("m,k,seed", [(16, 128, 91), (37, 272, 92), (300, 2064, 93)])
def test_device_pack_equals_host_pack(ext, oracle_threads, m, k, seed):
    """tx_pack_encoded_device (repack kernel) builds the same tiles as the host repack."""
    blocks = random_blocks(m, k, seed)
    scales = lognormal_scales(m, seed + 1)
    host = _pack(ext, blocks, scales)
    dev = ext.pack_encoded_device(torch.from_numpy(blocks.reshape(-1)).cuda(), torch.from_numpy(scales).cuda())
    x = bf16_vector((3, k), seed + 2).cuda()
    try:
        assert ext.handle_info(dev)[:2] == [m, k]
        assert torch.equal(ext.decode_dense(host), ext.decode_dense(dev))
        assert torch.equal(ext.linear_f32(host, x[:1]), ext.linear_f32(dev, x[:1]))
        assert torch.equal(ext.linear(host, x), ext.linear(dev, x))
        got = bf16_bits(ext.decode_dense(dev).cpu())
    finally:
        ext.free(host)
        ext.free(dev)
    assert np.array_equal(got, clib.decode_bf16_bits(blocks, scales))


@pytest.mark.parametrize("m,k,tokens,seed", [(16, 128, 1, 11), (37, 272, 1, 12), (1024, 5120, 1, 13),
                                             (300, 1040, 3, 14), (4096, 4096, 1, 15), (8, 27648, 1, 16)])
def test_gemv_f32_within_tolerance(ext, oracle_threads, m, k, tokens, seed):
    blocks = random_blocks(m, k, seed)
    scales = lognormal_scales(m, seed + 1)
    x = bf16_vector((tokens, k), seed + 2)
    handle = _pack(ext, blocks, scales)
    try:
        y = ext.linear_f32(handle, x.cuda()).cpu().numpy()
    finally:
        ext.free(handle)
    w = clib.decode_bf16_bits(blocks, scales)
    for t in range(tokens):
        ref = clib.matvec_f64(w, bf16_bits(x[t]))
        assert rel_err(ref, y[t]) <= GEMV_TOL
        assert max_rel_err_floor(ref, y[t]) <= GEMV_TOL


@pytest.mark.parametrize("tokens", [2, 15, 16, 17, 40])
def test_gemv_multi_token_within_tolerance(ext, oracle_threads, tokens):
    """Below the prefill threshold several tokens share one pass of the GEMV (16 per MFMA column
    block); every token must match its own float64 matvec."""
    m, k = 272, 3072
    blocks = random_blocks(m, k, 81)
    scales = lognormal_scales(m, 82)
    x = bf16_vector((tokens, k), 83)
    handle = _pack(ext, blocks, scales)
    try:
        ext.set_prefill(handle, 1 << 20, 1024)
        y32 = ext.linear_f32(handle, x.cuda()).cpu().numpy()
        y16 = ext.linear(handle, x.cuda()).float().cpu().numpy()
        single = np.stack([ext.linear_f32(handle, x[t:t + 1].cuda()).cpu().numpy()[0] for t in range(tokens)])
    finally:
        ext.free(handle)
    w = clib.decode_bf16_bits(blocks, scales)
    ref = clib.gemm_f64(bf16_bits(x), w)
    for t in range(tokens):
        assert rel_err(ref[t], y32[t]) <= GEMV_TOL
        assert max_rel_err_floor(ref[t], y32[t]) <= GEMV_TOL
        assert max_rel_err_floor(ref[t], single[t]) <= GEMV_TOL
    # the bf16 output is the fp32 sum rounded once
    assert max_rel_err_floor(ref, y16) <= 2 ** -8 + GEMV_TOL


@pytest.mark.parametrize("lookahead", [1, 2, 3, 4, 6, 8])
def test_gemv_lookahead_variants_bitwise_equal(ext, lookahead):
    m, k = 512, 5120
    blocks = random_blocks(m, k, 21)
    scales = lognormal_scales(m, 22)
    x = bf16_vector((1, k), 23).cuda()
    handle = _pack(ext, blocks, scales)
    try:
        ext.set_lookahead(handle, 1)
        base = ext.linear_f32(handle, x)
        ext.set_lookahead(handle, lookahead)
        other = ext.linear_f32(handle, x)
        again = ext.linear_f32(handle, x)
        torch.cuda.synchronize()
    finally:
        ext.free(handle)
    assert torch.equal(base, other)
    assert torch.equal(other, again)


def test_gemv_bf16_output_and_bias(ext, oracle_threads):
    m, k = 333, 2048
    blocks = random_blocks(m, k, 31)
    scales = lognormal_scales(m, 32)
    x = bf16_vector((2, k), 33)
    bias = bf16_vector((m,), 34, scale=0.5)
    handle = _pack(ext, blocks, scales, bias.cuda())
    try:
        y = ext.linear(handle, x.cuda()).float().cpu().numpy()
    finally:
        ext.free(handle)
    w = clib.decode_bf16_bits(blocks, scales)
    for t in range(2):
        ref = clib.matvec_f64(w, bf16_bits(x[t])) + bias.float().numpy()
        # one bf16 rounding of the biased sum: 2^-8 relative per element at most
        assert max_rel_err_floor(ref, y[t]) <= 2 ** -8 + GEMV_TOL


@pytest.mark.parametrize("tokens", [17, 32, 100, 128])
def test_prefill_candidates_bitwise_equal_and_within_rrms(ext, oracle_threads, tokens):
    m, k = 200, 1280
    blocks = random_blocks(m, k, 41)
    scales = lognormal_scales(m, 42)
    x = (bf16_vector((tokens, k), 43).float() * 0.125).to(torch.bfloat16)
    handle = _pack(ext, blocks, scales)
    outputs = {}
    try:
        for candidate in range(5, 10):
            outputs[candidate] = ext.prefill(handle, candidate, x.cuda())
        ext.set_prefill(handle, 1, 1024)
        via_linear = ext.linear(handle, x.cuda())
        torch.cuda.synchronize()
    finally:
        ext.free(handle)
    base = outputs[5]
    for candidate, value in outputs.items():
        assert torch.equal(base, value), f"candidate {candidate} differs from candidate 5"
    assert torch.equal(base, via_linear)
    w = clib.decode_bf16_bits(blocks, scales)
    ref = clib.gemm_f64(bf16_bits(x), w)
    got = base.float().cpu().numpy()
    assert bc4.relative_rms(ref, got) <= PREFILL_RRMS_TOL


@pytest.mark.parametrize("m", [26624, 16416, 8224])
@pytest.mark.parametrize("mode", ["bf16", "f16_bias", "lut"])
@pytest.mark.parametrize("tokens", [2, 17, 32])
def test_prefill_split_group_tile_matches_other_tiles(ext, mode, tokens, m):
    """Up to 32 tokens with exactly four K splits, candidate 9 runs the split-group tile (the four
    splits of one or two 32-row blocks in one workgroup, summed there in split order): bitwise
    equal to the tiles that write split partials for the reduce kernel, and within the prefill
    tolerance of the float64 product on sampled rows. With K = 4096 every row count here splits
    four ways on a 256-CU MI355X. 26624 rows (832 blocks) and 16416 rows (513 blocks: the last
    wave repeats its one real block, never stored) run two blocks per wave; 8224 rows (257 blocks,
    129 two-block workgroups, fewer than the CUs) run one."""
    k = 4096
    blocks = random_blocks(m, k, 611)
    scales = lognormal_scales(m, 612)
    f16 = mode == "f16_bias"
    x = f16_vector((tokens, k), 613, scale=0.125) if f16 else (bf16_vector((tokens, k), 613).float() * 0.125).to(torch.bfloat16)
    bias = f16_vector((m,), 614, scale=0.1).cuda() if f16 else None
    handle = _pack(ext, blocks, scales, bias)
    lut = None
    if mode == "lut":
        rng = np.random.default_rng(615)
        base = bc4.palette()
        lut = (base * (1 + 0.01 * rng.standard_normal(base.shape))).astype(np.float32)
        ext.set_palette_table(handle, torch.from_numpy(lut).cuda())
    try:
        mp = (m + 15) // 16 * 16
        if ext.workspace_bytes(handle, tokens) != 4 * tokens * mp * 4:
            pytest.skip("this GPU splits the shape other than four ways")
        outputs = {c: ext.prefill(handle, c, x.cuda()) for c in (9, 8, 6)}
        torch.cuda.synchronize()
    finally:
        ext.free(handle)
    for c in (8, 6):
        assert torch.equal(outputs[9], outputs[c]), f"candidate 9 differs from candidate {c}"
    rows = np.random.default_rng(616).choice(m, 512, replace=False)
    if f16:
        w = bc4.decode_f16_bits(blocks[rows], scales[rows]).view(np.float16).astype(np.float64)
        ref = x.double().numpy() @ w.T + bias.double().cpu().numpy()[rows][None, :]
        got = outputs[9].double().cpu().numpy()[:, rows]
    else:
        w = clib.decode_bf16_bits(blocks[rows], scales[rows], lut)
        ref = clib.gemm_f64(bf16_bits(x), w)
        got = outputs[9].float().cpu().numpy()[:, rows]
    assert bc4.relative_rms(ref, got) <= PREFILL_RRMS_TOL


@pytest.mark.parametrize("m,k,tokens", [(96, 4096, 20), (300, 27648, 32), (1024, 5120, 130)])
def test_prefill_split_k_matches_oracle(ext, oracle_threads, m, k, tokens):
    """Shapes whose prefill is split along K (partials in the workspace, ordered reduction):
    still bitwise equal across tiles and within the rrms bar of the float64 GEMM."""
    blocks = random_blocks(m, k, 44)
    scales = lognormal_scales(m, 45)
    x = (bf16_vector((tokens, k), 46).float() * 0.125).to(torch.bfloat16)
    bias = bf16_vector((m,), 47, scale=0.1)
    handle = _pack(ext, blocks, scales, bias.cuda())
    try:
        assert ext.workspace_bytes(handle, tokens) > 0, "shape expected to split"
        outputs = [ext.prefill(handle, c, x.cuda()) for c in range(5, 10)]
        torch.cuda.synchronize()
    finally:
        ext.free(handle)
    for c, value in zip(range(6, 10), outputs[1:]):
        assert torch.equal(outputs[0], value), f"candidate {c} differs"
    w = clib.decode_bf16_bits(blocks, scales)
    ref = clib.gemm_f64(bf16_bits(x), w) + bias.float().numpy()[None, :]
    assert bc4.relative_rms(ref, outputs[0].float().cpu().numpy()) <= PREFILL_RRMS_TOL


@pytest.mark.parametrize("m,k,tokens", [(200, 1040, 17), (200, 1040, 100), (37, 272, 40), (96, 4112, 20),
                                         (64, 16, 70), (300, 2064, 129)])
def test_prefill_ragged_k_matches_oracle(ext, oracle_threads, m, k, tokens):
    """K not a multiple of the 128-wide step (the last step's activations are staged with the
    columns past K zeroed), ragged rows and token counts, with and without K splits: every tile
    bitwise equal and within the rrms bar of the float64 GEMM."""
    blocks = random_blocks(m, k, 48)
    scales = lognormal_scales(m, 49)
    x = (bf16_vector((tokens, k), 50).float() * 0.125).to(torch.bfloat16)
    bias = bf16_vector((m,), 51, scale=0.1)
    handle = _pack(ext, blocks, scales, bias.cuda())
    try:
        outputs = [ext.prefill(handle, c, x.cuda()) for c in range(5, 10)]
        torch.cuda.synchronize()
    finally:
        ext.free(handle)
    for c, value in zip(range(6, 10), outputs[1:]):
        assert torch.equal(outputs[0], value), f"candidate {c} differs"
    w = clib.decode_bf16_bits(blocks, scales)
    ref = clib.gemm_f64(bf16_bits(x), w) + bias.float().numpy()[None, :]
    assert bc4.relative_rms(ref, outputs[0].float().cpu().numpy()) <= PREFILL_RRMS_TOL


def test_prefill_bias_double_rounding(ext):
    m, k, tokens = 64, 256, 40
    blocks = random_blocks(m, k, 51)
    scales = lognormal_scales(m, 52)
    x = bf16_vector((tokens, k), 53)
    bias = bf16_vector((m,), 54)
    plain = _pack(ext, blocks, scales)
    biased = _pack(ext, blocks, scales, bias.cuda())
    try:
        y0 = ext.prefill(plain, 6, x.cuda())
        y1 = ext.prefill(biased, 6, x.cuda())
        torch.cuda.synchronize()
    finally:
        ext.free(plain)
        ext.free(biased)
    expected = (y0.float() + bias.cuda().float()[None, :]).to(torch.bfloat16)
    assert torch.equal(y1, expected)


def test_split_k_reduction_is_deterministic(ext):
    m, k = 64, 27648  # few row groups -> many K splits
    blocks = random_blocks(m, k, 61)
    scales = lognormal_scales(m, 62)
    x = bf16_vector((1, k), 63).cuda()
    handle = _pack(ext, blocks, scales)
    try:
        first = ext.linear_f32(handle, x)
        for _ in range(20):
            assert torch.equal(first, ext.linear_f32(handle, x))
    finally:
        ext.free(handle)


def test_one_token_linear_is_reentrant_across_streams(ext):
    """One-token GEMVs with K splits on one handle from two streams at once: with the workspace
    ``linear`` passes, each call's partials are its own, so every result equals the sequential one."""
    m, k = 1024, 5120
    handle = _pack(ext, random_blocks(m, k, 95), lognormal_scales(m, 96))
    try:
        assert ext.gemv_plan(handle)[0] > 1 and ext.workspace_bytes(handle, 1) > 0
        xs = [bf16_vector((1, k), 97 + i).cuda() for i in range(2)]
        want = [ext.linear(handle, x) for x in xs]
        streams = [torch.cuda.Stream() for _ in xs]
        torch.cuda.synchronize()
        results = [[], []]
        for _ in range(20):
            for i, (stream, x) in enumerate(zip(streams, xs)):
                with torch.cuda.stream(stream):
                    results[i].append(ext.linear(handle, x))
        torch.cuda.synchronize()
    finally:
        ext.free(handle)
    for i in range(2):
        assert all(torch.equal(want[i], value) for value in results[i])


def test_kernel_info_nine_fields_and_candidate_names(ext):
    """The nine fields of the reference's ``cutlass_*_kernel_info`` (``cutlass_texture_mainloop.cu:251-267``),
    the last the occupancy (workgroups per CU), for every prefill tile and GEMV lookahead."""
    from texelator_amd import autotune

    for name, candidate in autotune.CANDIDATES.items():
        info = ext.kernel_info(candidate)
        assert len(info) == 9 and ext.candidate_name(candidate) == name
        vgprs, _, private, threads, lds, bt, bn, bk, resident = info
        assert vgprs > 0 and private == 0 and threads >= 256 and lds > 0 and resident >= 1
        assert name.startswith(("large", "medium", "small", "wide")) and f"{bt}x{bn}x{bk}" in name
    for lookahead in (1, 2, 4):
        info = ext.kernel_info(100 + lookahead)
        assert len(info) == 9 and info[5:8] == [1, 16, 128] and info[8] >= 1
    assert ext.cutlass_texture_kernel_info() == ext.kernel_info(5)


def test_handle_api_errors(ext):
    blocks = random_blocks(16, 128, 71)
    scales = lognormal_scales(16, 72)
    handle = _pack(ext, blocks, scales)
    try:
        assert ext.handle_info(handle)[:2] == [16, 128]
        with pytest.raises(RuntimeError, match="lookahead"):
            ext.set_lookahead(handle, 5)
        with pytest.raises(RuntimeError, match="threshold"):
            ext.set_prefill(handle, 0, 1024)
        with pytest.raises(RuntimeError, match="tile rows"):
            ext.set_prefill(handle, 16, 24)
        with pytest.raises(RuntimeError, match="backend") as error:
            ext.set_prefill_backend(handle, 10)
        for candidate in range(5, 10):   # the message names the real tiles
            assert f"{candidate} ({ext.candidate_name(candidate)})" in str(error.value)
        with pytest.raises(RuntimeError, match="shape"):
            ext.linear(handle, torch.zeros((1, 64), dtype=torch.bfloat16, device="cuda"))
        with pytest.raises(RuntimeError, match="FP16 or BF16"):
            ext.linear(handle, torch.zeros((1, 128), dtype=torch.float32, device="cuda"))
    finally:
        ext.free(handle)
    with pytest.raises(RuntimeError, match="uint8"):
        ext.pack_encoded(torch.zeros(16, dtype=torch.int8), torch.ones(1))
    with pytest.raises(RuntimeError, match="invalid encoded size"):
        ext.pack_encoded(torch.zeros(12, dtype=torch.uint8), torch.ones(1))


# ---- FP16 activations (the reference's FP16 GEMV and FP16 prefill, texelator_cuda.cu:94-139,
# :1004-1045): fp16 x, bias and y; the weights are fp16_rne(P * scale).

def f16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("m,k,seed", [(16, 128, 401), (37, 272, 402), (64, 4096, 403)])
def test_decode_dense_f16_bit_exact(ext, m, k, seed):
    blocks = random_blocks(m, k, seed)
    scales = lognormal_scales(m, seed + 100)
    handle = _pack(ext, blocks, scales)
    try:
        got = f16_bits(ext.decode_dense(handle, torch.float16))
    finally:
        ext.free(handle)
    want = bc4.decode_f16_bits(blocks, scales)
    mismatches = int(np.count_nonzero(got != want))
    assert mismatches == 0, f"{mismatches} of {want.size} fp16 weights differ"


@pytest.mark.parametrize("m,k,tokens,bias", [(1024, 5120, 1, False), (333, 2048, 1, True), (272, 3072, 5, True),
                                             (5120, 27648, 1, False), (64, 27648, 1, True)])
def test_gemv_f16_within_tolerance(ext, m, k, tokens, bias):
    """FP16 GEMV against the reference's arithmetic in float64: unrounded fp32 weights times the
    fp16 input, plus the bias. Our weights are rounded to fp16 (2^-11 relative each), the output
    is rounded to fp16 once (2^-11 relative per element)."""
    blocks = random_blocks(m, k, 411 + m)
    scales = lognormal_scales(m, 412 + m)
    x = f16_vector((tokens, k), 413 + m)
    b = f16_vector((m,), 414 + m, scale=0.5) if bias else None
    handle = _pack(ext, blocks, scales, b.cuda() if bias else None)
    try:
        ext.set_prefill(handle, 1 << 20, 1024)
        y = ext.linear(handle, x.cuda())
        torch.cuda.synchronize()
    finally:
        ext.free(handle)
    assert y.dtype == torch.float16
    w = bc4.decode_f32_weights(blocks, scales).astype(np.float64)
    ref = x.double().numpy() @ w.T
    if bias:
        ref = ref + b.double().numpy()[None, :]
    got = y.double().cpu().numpy()
    for t in range(tokens):
        assert rel_err(ref[t], got[t]) <= GEMV_TOL
        assert max_rel_err_floor(ref[t], got[t]) <= 2 ** -11 + GEMV_TOL


@pytest.mark.parametrize("tokens", [17, 64, 130])
def test_prefill_f16_candidates_bitwise_equal_and_within_rrms(ext, tokens):
    m, k = 200, 1280
    blocks = random_blocks(m, k, 421)
    scales = lognormal_scales(m, 422)
    x = f16_vector((tokens, k), 423, scale=0.125)
    bias = f16_vector((m,), 424, scale=0.1)
    plain = _pack(ext, blocks, scales)
    biased = _pack(ext, blocks, scales, bias.cuda())
    try:
        outputs = [ext.prefill(plain, c, x.cuda()) for c in range(5, 10)]
        with_bias = ext.prefill(biased, 6, x.cuda())
        ext.set_prefill(biased, 1, 1024)
        via_linear = ext.linear(biased, x.cuda())
        torch.cuda.synchronize()
    finally:
        ext.free(plain)
        ext.free(biased)
    for c, value in zip(range(6, 10), outputs[1:]):
        assert torch.equal(outputs[0], value), f"candidate {c} differs"
    assert outputs[0].dtype == torch.float16
    # the bias is added to the fp16 product with a second fp16 rounding (texelator_cuda.cu:630-635)
    assert torch.equal(with_bias, (outputs[0].float() + bias.cuda().float()[None, :]).to(torch.float16))
    assert torch.equal(with_bias, via_linear)
    w = bc4.decode_f16_bits(blocks, scales).view(np.float16).astype(np.float64)
    ref = x.double().numpy() @ w.T
    assert bc4.relative_rms(ref, outputs[0].double().cpu().numpy()) <= PREFILL_RRMS_TOL


def test_prefill_f16_split_k_matches_oracle(ext):
    m, k, tokens = 300, 27648, 32
    blocks = random_blocks(m, k, 431)
    scales = lognormal_scales(m, 432)
    x = f16_vector((tokens, k), 433, scale=0.125)
    handle = _pack(ext, blocks, scales)
    try:
        assert ext.workspace_bytes(handle, tokens) > 0, "shape expected to split"
        outputs = [ext.prefill(handle, c, x.cuda()) for c in (5, 9)]
        torch.cuda.synchronize()
    finally:
        ext.free(handle)
    assert torch.equal(outputs[0], outputs[1])
    w = bc4.decode_f16_bits(blocks, scales).view(np.float16).astype(np.float64)
    ref = x.double().numpy() @ w.T
    assert bc4.relative_rms(ref, outputs[0].double().cpu().numpy()) <= PREFILL_RRMS_TOL


def test_stream_read_probe(ext):
    """The streaming-read reference kernel runs over any 16-byte multiple and rejects the rest."""
    import ctypes

    from texelator_amd import _lib

    data = torch.randint(0, 256, (1 << 20,), dtype=torch.uint8, device="cuda")
    sink = torch.zeros(4096, dtype=torch.int32, device="cuda")
    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for nbytes in (16, 4096 + 16, data.numel()):
        _lib.check(lib.tx_stream_read(ctypes.c_void_p(data.data_ptr()), nbytes, ctypes.c_void_p(sink.data_ptr()), stream))
    torch.cuda.synchronize()
    with pytest.raises(_lib.TexelatorError, match="multiple of 16"):
        _lib.check(lib.tx_stream_read(ctypes.c_void_p(data.data_ptr()), 24, ctypes.c_void_p(sink.data_ptr()), stream))
