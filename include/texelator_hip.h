/*
 * texelator_hip.h -- C ABI of libtexelator_hip.so, the gfx950 BC4 weight path.
 *
 * Each entry point replaces one function of the reference's native module
 * (texelator/cuda/extension.cpp:27-48, implemented in texelator/cuda/texelator_cuda.cu).
 * Plain pointers and sizes only; no framework types. Every function returns TX_OK (0) or a
 * nonzero status; the message of the last failure on the calling thread is returned by
 * tx_last_error(). Device pointers are HIP device memory; "stream" is a hipStream_t (NULL
 * means the default stream). Launches are asynchronous on that stream.
 */
#ifndef TEXELATOR_HIP_H
#define TEXELATOR_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TX_OK 0
#define TX_ERR_INVALID 1     /* bad argument: the reference raises RuntimeError (TORCH_CHECK) */
#define TX_ERR_HIP 2         /* HIP runtime failure (reference: CUDA_CHECK) */
#define TX_ERR_UNSUPPORTED 3 /* feature of the reference with no gfx950 implementation here */

#define TX_DTYPE_F16 0
#define TX_DTYPE_BF16 1
#define TX_DTYPE_F32 2

/* Message of the last failure on this thread ("" if none). */
const char *tx_last_error(void);

/* Upload one encoded matrix and return an opaque handle.
 * Replaces texelator_pack_encoded (texelator_cuda.cu:1260-1327; extension.cpp:28).
 *   blocks       host bytes [M][bpr][8] (reference block format, encoder.py:105-117)
 *   blocks_bytes total bytes; must be a positive multiple of 8*M
 *   scales       host float32 [M]
 *   bias         optional device pointer to [M] values of bias_dtype (F16 or BF16), copied
 *   device       HIP device ordinal that will own the handle
 * K = 16 * bpr. The blocks are repacked into the gfx950 tile layout on upload. */
int tx_pack_encoded(const uint8_t *blocks, int64_t blocks_bytes, const float *scales, int64_t rows,
                    const void *bias, int bias_dtype, int device, uint64_t *handle_out);

/* Same as tx_pack_encoded, but blocks (8-byte aligned) and scales are device pointers on
 * `device`; the tile repack runs on the GPU. The reference only accepts CPU inputs
 * (texelator_cuda.cu:1262-1268); this variant serves weights encoded on the GPU. Synchronous. */
int tx_pack_encoded_device(const uint8_t *blocks, int64_t blocks_bytes, const float *scales, int64_t rows,
                           const void *bias, int bias_dtype, int device, uint64_t *handle_out);

/* A new handle holding the rows of `count` handles of one K in order (their row concatenation):
 * one GEMV launch where a caller ran one per matrix, e.g. the q, k and v projections of an
 * attention module installed as three separate modules (the reference's Hugging Face path keeps
 * them separate, texelator/runtime.py:133-145; a fused q/k/v handle has no counterpart there).
 * Every handle but the last must have a multiple of 16 rows; all or none carry a bias (one dtype);
 * one palette table or none. The lookahead and prefill settings are the first handle's. The
 * sources stay valid and independent (the new handle copies their tiles); free it with tx_free. */
int tx_concat_rows(const uint64_t *handles, int count, uint64_t *handle_out);

/* y = x W^T (+ bias). Replaces texelator_linear (texelator_cuda.cu:1329-1469; extension.cpp:30).
 *   x         device, contiguous, 16-byte aligned [tokens][K] of x_dtype (BF16 or F16). With F16
 *             the weights are rounded to fp16 before the fp32-accumulating MFMA; the reference's
 *             FP16 GEMV (texelator_cuda.cu:94-139) multiplies them unrounded (at most 2^-11
 *             relative per weight), its FP16 prefill rounds them the same way (:604-628). The
 *             bias must have x's dtype; y = round(acc + bias) on the GEMV, and
 *             round(round(acc) + bias) on the prefill path, as in the reference.
 *   x_numel   number of elements of x; tokens = x_numel / K
 *   x_last    size of x's last dimension (must equal K)
 *   y         device output [tokens][M] of x_dtype, allocated by the caller
 *   workspace device scratch of at least tx_workspace_bytes(handle, tokens) bytes, 16-byte
 *             aligned (may be NULL when that is 0), stream-ordered: the prefill path's split-K
 *             partials or backend 1's dense rows (required), or a one-token GEMV's split-K partials (optional: with NULL the
 *             handle's own buffer is used, so two such calls on one handle must not overlap)
 * tokens >= prefill threshold (and tokens > 1) uses the prefill GEMM candidate set by
 * tx_set_prefill_backend; otherwise the decode GEMV with the configured lookahead.
 * The reference allocates its prefill scratch inside the call (texelator_cuda.cu:942-957); here
 * the caller supplies it, so the library never allocates on this path. */
int tx_linear(uint64_t handle, const void *x, int x_dtype, int64_t x_numel, int64_t x_last,
              int device, void *y, void *workspace, int64_t workspace_bytes, void *stream);

/* tx_linear for callers that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. Same arguments, dispatch,
 * checks and results (bit for bit) as tx_linear, but there is no workspace argument and the
 * handle's own split-K buffer is not used: split-K partial sums go to a static 32 MiB device
 * array of the library (tx_noalloc_scratch_bytes), one per GPU, kept until the process ends.
 * No hipMalloc, hipFree or allocating library call is made. A call whose partials would exceed
 * the array fails with TX_ERR_INVALID before launching anything; a prefill-sized call on a handle
 * set to prefill backend 1 (dense scratch + library GEMM, which creates library state on first
 * use) fails with TX_ERR_UNSUPPORTED before launching anything. All calls on one GPU share the
 * array: calls that overlap on one GPU (two streams, two threads) race and must be serialised by
 * the caller; calls on one stream are ordered and safe. */
int tx_linear_noalloc(uint64_t handle, const void *x, int x_dtype, int64_t x_numel, int64_t x_last,
                      int device, void *y, void *stream);

/* FP4 hybrid prefill staging and GEMM. Replace texelator_quantize_activation_fp4[_out]
 * (texelator_cuda.cu:1154-1178, :1202-1233), texelator_decode_weight_fp4[_out] (:1179-1201,
 * :1234-1260) and the torch._scaled_mm call of texelator/runtime.py:110-116. The format is gfx950's
 * block-scaled MFMA format, MXFP4 (OCP MX v1.0): E2M1 values, two per byte with the even column in
 * the low nibble, row-major [rows][K/2]; one E8M0 scale (2^(e - 127)) per 32 values, row-major
 * [rows][K/32]. The reference writes NVFP4 (an E4M3 scale per 16 values, Blackwell's blocked scale
 * layout) for its own FP4 GEMM. Group quantization: e = floor(log2(amax)) - 2 + 127 clamped to
 * [0, 254] (0 for an all-zero group); value v -> E2M1 of v * 2^(127 - e), nearest, ties to even,
 * saturated at 6, sign bit = sign of v.
 *   tx_quantize_activation_fp4: x device bf16 [tokens][K], K a multiple of 32.
 *   tx_decode_weight_fp4: the handle's fp32 products palette * row scale (before 16-bit
 *     rounding, as the reference's quantizer; in LUT mode the palette values are the handle's
 *     table rows, as for every other kernel of that handle), M rows; K a multiple of 32.
 *   tx_fp4_gemm: y [tokens][M] bf16 = round(sum_k deq(x)[t][k] * deq(w)[m][k]) with fp32
 *     accumulation (v_mfma_scale_f32_32x32x64_f8f6f4), then + bias [M] (bf16, or NULL) with a
 *     second rounding; K a multiple of 64. Packed operands 16-byte aligned. */
int tx_quantize_activation_fp4(const void *x, int x_dtype, int64_t tokens, int64_t K, uint8_t *packed,
                               uint8_t *scales, int device, void *stream);
int tx_decode_weight_fp4(uint64_t handle, uint8_t *packed, uint8_t *scales, void *stream);
int tx_fp4_gemm(const uint8_t *x_packed, const uint8_t *x_scales, const uint8_t *w_packed, const uint8_t *w_scales,
                const void *bias, int64_t tokens, int64_t M, int64_t K, void *y, int device, void *stream);

/* Size in bytes of tx_linear_noalloc's static scratch array. */
int tx_noalloc_scratch_bytes(int64_t *bytes);

/* Workspace bytes of tx_linear and tx_prefill for `tokens` tokens: the prefill split-K partial
 * sums for tokens > 1 (with backend 1 and tokens >= the prefill threshold: the dense scratch of
 * min(tile_rows, M) decoded rows of K 16-bit weights rounded up to 256 bytes, 256 bytes of slack
 * and 8 MiB for the library GEMM, whose workspace starts at the first 256-byte boundary after the
 * rows; the caller's workspace need only be 16-byte aligned), the one-token GEMV's split-K partials for
 * tokens == 1 (0 when the shape is not split, or when one workgroup per 16-row group runs all of
 * its splits: 2 to 4 splits, row groups spreading evenly over the CUs, arithmetic palette). No
 * reference counterpart (see tx_linear). */
int tx_workspace_bytes(uint64_t handle, int64_t tokens, int64_t *bytes);

/* Decode GEMV with float32 output and no bias, for parity checks (no reference counterpart:
 * the reference only returns 16-bit outputs). x: device bf16 [tokens][K]; y: device f32. One-token
 * split-K partials use the handle's own buffer: calls on one handle must not overlap. */
int tx_linear_f32(uint64_t handle, const void *x, int64_t tokens, float *y, void *stream);

/* Prefill GEMM with an explicit candidate (5..9), x_dtype (BF16 or F16) in and out, bias
 * applied if present; same workspace rule as tx_linear. Used by the tile autotuner (reference:
 * set_prefill_backend + linear, autotune.py:144-187). */
int tx_prefill(uint64_t handle, int candidate, const void *x, int x_dtype, int64_t tokens, void *y,
               void *workspace, int64_t workspace_bytes, void *stream);

/* Replaces texelator_set_lookahead (texelator_cuda.cu:1471-1478): one of 1,2,3,4,6,8. */
int tx_set_lookahead(uint64_t handle, int lookahead);

/* Replaces texelator_set_prefill (texelator_cuda.cu:1480-1488): threshold >= 1,
 * tile_rows a positive multiple of 16: the rows backend 1 decodes per library GEMM. */
int tx_set_prefill(uint64_t handle, int threshold, int tile_rows);

/* Replaces texelator_set_prefill_backend (texelator_cuda.cu:1490-1503): 0..9. Ids 5..9 name the
 * gfx950 tile candidates. 1 is the dense-scratch path of the reference's backend 1
 * (texelator_cuda.cu:937-990): tile_rows rows at a time decoded into the workspace, one hipBLASLt
 * GEMM (fp32 accumulation) per row tile, then the bias with a second rounding; hipBLASLt is
 * opened at its first call. 0 and 2..4 (the reference's fused and CUDA-only 512-token kernels)
 * select the default tile. */
int tx_set_prefill_backend(uint64_t handle, int backend);

/* LUT-mode decode (no reference counterpart: on NVIDIA the texture unit is the palette). With a
 * non-NULL device_table -- 255*255*8 float32 in the probe layout, index ((e1+127)*255+(e0+127))*8+s,
 * 16-byte aligned, owned by the caller and kept alive while the handle uses it -- every kernel of
 * this handle reads each block's 8 palette values from the table instead of computing this
 * build's defined palette; weights are round(P[s] * scale[row]) as before. This decodes artifacts
 * encoded against another palette (e.g. the NVIDIA palette an artifact bundles as
 * hardware/common/palette.bin, packager.py:185-191) bit-exactly. NULL restores the defined palette. */
int tx_set_palette_table(uint64_t handle, const float *device_table);

/* Replaces texelator_handle_info (texelator_cuda.cu:1505-1512). Writes up to n of
 * [M, K, prefill_threshold, prefill_tile_rows, prefill_backend, pipelined(0), graphics(0),
 *  lookahead, device, decode GEMV K splits, LUT mode (0/1)]; the last four are this library's. */
int tx_handle_info(uint64_t handle, int64_t *out, int n);

/* No reference counterpart: a plain streaming read of `bytes` (multiple of 16, 16-byte aligned
 * device memory), the achievable-bandwidth reference point next to which bench.py reports the
 * GEMV. `sink` must hold 4096 uint32 (written only for a sentinel input). */
int tx_stream_read(const void *data, int64_t bytes, uint32_t *sink, void *stream);

/* Replaces texelator_free (texelator_cuda.cu:1538). Caller must ensure no work is pending. */
int tx_free(uint64_t handle);

/* Replaces texelator_palette_probe (texelator_cuda.cu:1551-1595): fills host_out with the
 * 255*255*8 float32 palette measured from the device decoder, index ((e1+127)*255+(e0+127))*8+s,
 * on the current device. Synchronous. */
int tx_palette_probe(float *host_out);

/* Decode a handle's weights to a dense device [M][K] array of dtype (BF16: bf16_rne(P*scale);
 * F16: fp16_rne(P*scale), the FP16 path's weights) -- a test-only diagnostic; no reference
 * counterpart (the reference's decode tiles write scratch, texelator_cuda.cu:604-663). */
int tx_decode_dense(uint64_t handle, int dtype, uint16_t *out, void *stream);

/* Kernel resource report for a candidate. Replaces the *_kernel_info functions
 * (texelator_cuda.cu:1514-1536, cutlass_texture_mainloop.cu:251-267). candidate 5..9: prefill
 * tiles; 100 + L: decode GEMV with lookahead L. Writes up to n of
 * [vgprs, static_lds_bytes, private_bytes, max_threads, tile_lds_bytes, tokens_tile, rows_tile, k_tile,
 *  active_workgroups_per_cu] -- the nine values of the reference's cutlass_*_kernel_info, the last
 * being its active_blocks occupancy query (cutlass_texture_mainloop.cu:251-267). For the GEMV ids the
 * LDS and occupancy figures are those of a K = 5120 split (40 tile columns of staged x). */
int tx_kernel_info(int candidate, int64_t *out, int n);

/* Name of a prefill candidate (5..9) or NULL. */
const char *tx_candidate_name(int candidate);

/* ---- Decoder-layer helpers ------------------------------------------------------------------
 * No reference counterpart: the reference runs these layers as stock Hugging Face modules
 * (docs/supported-models.md:3-5) and replaces only the linears. They let a whole BC4 decode step
 * be a short, graph-capturable kernel sequence. All device pointers; bf16 data as uint16 bits.
 * The KV caches are bf16 [kv_heads][max_context][head_dim]. */

/* residual[r] += delta[r] (delta may be NULL); out[r] = bf16(weight * bf16(residual[r] *
 * rsqrt(mean(residual[r]^2) + eps))). residual f32 [rows][hidden]; delta, out bf16; weight bf16 [hidden];
 * hidden a multiple of 4; all pointers 16-byte aligned. */
int tx_add_rmsnorm(float *residual, const void *delta, const void *weight, float eps, void *out, int64_t rows,
                   int64_t hidden, void *stream);

/* Rotate-half RoPE of the q and k heads of a packed [q | k | v] bf16 row (stride row_stride
 * elements) at positions[t]: q heads to q_out [tokens][heads][head_dim], k heads into k_cache, and
 * v heads copied into v_cache, at row positions[t]. cos/sin tables f32 [max_context][head_dim].
 * A token whose position lies outside [0, max_context) (device values, checked on the device) writes
 * nothing, neither q_out nor the caches. */
int tx_rope_kv_cache(const void *qkv, int64_t row_stride, int64_t tokens, const int64_t *positions,
                     const float *cos_table, const float *sin_table, int heads, int kv_heads, int head_dim,
                     void *q_out, void *k_cache, void *v_cache, int64_t max_context, void *stream);

/* Workspace bytes of tx_decode_attention and tx_decode_attention_split for `length` cached
 * positions (the chunk partials). */
int tx_decode_attention_workspace(int heads, int64_t length, int64_t *bytes);

/* Attention of one query token q [heads][head_dim] over cached keys 0..*position (device int64;
 * keys up to `length`, a static bound): scores from bf16 q and keys with fp32 sums, fp32
 * softmax, and the probabilities carried to 16 significant bits (bf16 hi + lo) into the fp32 sum
 * over the values; grouped-query (heads / kv_heads query heads per KV head, at most 8); head_dim
 * must be 128. out bf16 [heads][head_dim]. */
int tx_decode_attention(const void *q, const void *k_cache, const void *v_cache, const int64_t *position,
                        int64_t length, int heads, int kv_heads, int head_dim, int64_t max_context, float scale,
                        void *workspace, int64_t workspace_bytes, void *out, void *stream);

/* Causal self-attention of a prompt: query tokens 0..tokens-1 against cached keys and values
 * 0..tokens-1 (caches [kv_heads][max_context][head_dim] bf16, written for the prompt by
 * tx_rope_kv_cache), grouped-query (heads a multiple of kv_heads); head_dim must be 128. q bf16
 * rows of heads * head_dim values every q_stride elements (16-byte aligned); out bf16 rows every
 * out_stride elements. Scores from bf16 q and keys with fp32 sums, online fp32 softmax, the
 * probabilities rounded to bf16 into the fp32 sum over the values (as flash attention does). No
 * counterpart in the reference (its attention is the Hugging Face module's sdpa call). */
int tx_prefill_attention(const void *q, int64_t q_stride, const void *k_cache, const void *v_cache, int64_t tokens,
                         int heads, int kv_heads, int head_dim, int64_t max_context, float scale, void *out,
                         int64_t out_stride, void *stream);

/* tx_rope_kv_cache_split followed by tx_decode_attention, one kernel launch fewer: q and the new
 * token's key and value are the last tx_linear_split of qkv_handle ([q | k | v] rows), rotated
 * inside the attention kernel with rope_row = the RoPE tables' rows at *position (cos[head_dim]
 * then sin[head_dim], fp32, gathered by the caller once per token); the key and value are
 * written to the caches at *position (not when *position >= max_context). Bit-identical to the two calls. No counterpart in the
 * reference (its decoder layers are Hugging Face modules, docs/supported-models.md:3-5). */
int tx_decode_attention_split(uint64_t qkv_handle, const int64_t *position, const float *rope_row, int64_t length,
                              int heads, int kv_heads, int head_dim, void *k_cache, void *v_cache,
                              int64_t max_context, float scale, void *workspace, int64_t workspace_bytes, void *out,
                              void *stream);

/* tx_decode_attention_split followed by tx_linear_split of o_handle on its output, one launch fewer:
 * the attention leaves its chunk partials in `workspace` and every workgroup of the o projection's
 * one-token GEMV merges the heads of its K split from them itself (the attention's merge, done
 * where its output is consumed), so o_handle's split-K partials end bitwise as after the two calls
 * (read them with tx_add_rmsnorm_split); the key and value are written to the caches as there. The
 * attention output itself is not written. o_handle: K = heads * head_dim, BF16 bias or none.
 * TX_ERR_UNSUPPORTED, with nothing launched, where the merge does not fit the o GEMV: a LUT-mode o
 * handle, a length of more than 16 chunks of 64 positions, or more than 64 (heads of one o split) x
 * chunks. No counterpart in the reference (its decoder layers are Hugging Face modules). */
int tx_decode_attention_o_split(uint64_t qkv_handle, uint64_t o_handle, const int64_t *position, const float *rope_row,
                                int64_t length, int heads, int kv_heads, int head_dim, void *k_cache, void *v_cache,
                                int64_t max_context, float scale, void *workspace, int64_t workspace_bytes,
                                void *stream);

/* out[r][c] = bf16(silu(g) * u) for gate_up rows [g (intermediate) | u (intermediate)], fp32 math. */
int tx_swiglu(const void *gate_up, int64_t rows, int64_t intermediate, void *out, void *stream);

/* Greedy next token of a dense bf16 lm_head (no reference counterpart: the reference leaves the
 * head and the sampling to Hugging Face): *token (int64, device memory) = the first row v with the
 * largest bf16(sum_k x[k] * weight[v][k]) (fp32 sums), i.e. argmax over the bf16 logits of the
 * linear layer, in two kernel launches instead of a GEMM and an argmax. weight bf16 [vocab][hidden]
 * row-major, x bf16 [hidden] (hidden a multiple of 128, at most 16384; both 16-byte aligned); logits
 * (bf16 [vocab]) written too unless null. workspace: at least tx_lm_head_argmax_workspace bytes,
 * 16-byte aligned. NaN logits are not ranked. */
int tx_lm_head_argmax_workspace(int64_t *bytes);
int tx_lm_head_argmax(const void *weight, int64_t vocab, int64_t hidden, const void *x, void *logits, void *workspace,
                      int64_t workspace_bytes, int64_t *token, void *stream);

/* RMSNorm over a bf16 residual stream (a Hugging Face decoder layer's: no counterpart in the
 * reference's own code, whose Hugging Face path leaves the norms and residual adds to torch):
 * rows x hidden bf16. With delta: sum_out = bf16(residual + delta) (torch's bf16 add) and
 * out = bf16(weight * bf16(sum * rsqrt(mean(sum^2) + eps))) of that sum, sums of squares in fp32;
 * without (delta NULL): out = that norm of the residual, sum_out unused. One launch, one block per
 * row. Pointers 8-byte aligned; hidden a multiple of 4. */
int tx_add_rmsnorm_bf16(const void *residual, const void *delta, const void *weight, float eps, void *sum_out, void *out,
                        int64_t rows, int64_t hidden, void *stream);

/* ---- Fused single-token decode (no reference counterpart; same role as the helpers above) ----
 * tx_linear_split runs a handle's one-token decode GEMV (x bf16 [K]) but leaves its output as
 * the fp32 split-K partials in the handle's own buffer; the *_split consumers below read them,
 * sum them in split order, add the (BF16) bias and round to bf16 exactly as tx_linear would, and
 * then do their own work. A split consumer must run on the same stream after the
 * tx_linear_split of its handle and before the next one. Outputs are bit-identical to
 * tx_linear followed by the plain helper. */
int tx_linear_split(uint64_t handle, const void *x, void *stream);

/* One-token GEMV of a merged [gate (inter) | up (inter)] handle with SwiGLU applied in its
 * epilogue: out bf16 [inter] = tx_swiglu(tx_linear(handle, x)), bit for bit, in one kernel.
 * x bf16 [K]. Needs inter % 16 == 0, a BF16 bias or none, and a handle that runs its one-token
 * GEMV unsplit without LUT mode (TX_ERR_UNSUPPORTED otherwise: use tx_linear + tx_swiglu). */
int tx_linear_swiglu(uint64_t handle, const void *x, void *out, void *stream);

/* The same over two handles of one shape [inter][K], gate and up (a Hugging Face MLP's
 * gate_proj and up_proj, each a TexelatorLinear of the reference, texelator/runtime.py:133-145,
 * whose two GEMVs and activation product this call replaces): out bf16 [inter] bit for bit what
 * tx_linear_swiglu gives on the merged [gate | up] handle of the two matrices. x bf16 [K], one
 * token. TX_ERR_UNSUPPORTED for LUT-mode handles, handles with a bias or K > 16384. */
int tx_linear_swiglu_pair(uint64_t gate, uint64_t up, const void *x, void *out, void *stream);

/* One token: y bf16 [M] = bf16(bf16(x W^T) + bias), x bf16 [K], bias bf16 [M], for a handle without a
 * bias of its own: tx_linear followed by a bf16 add of a separate bias parameter (the reference's
 * TexelatorLinear with a module bias, texelator/runtime.py:141-145, y = linear(x) + bias; the
 * standalone loader's modules carry their bias that way), bit for bit, with the add done in the
 * GEMV's own epilogue or reduction. Uses the handle's split-K buffer (calls on one handle must not
 * overlap). */
int tx_linear_add_bias(uint64_t handle, const void *x, const void *bias, void *y, void *stream);

/* One token's k and v (bf16 [kv_heads][head_dim] each) into a Hugging Face static KV cache layer:
 * keys/values bf16 [kv_heads][max_len][head_dim] at row *length (a device int64, the layer's
 * cumulative length), then *length += 1, in one launch: what its update() does with an index
 * tensor, two index copies and an in-place add (no counterpart in the reference's own code, whose
 * Hugging Face path leaves the cache to transformers). A full cache is left unchanged. */
int tx_kv_cache_append(const void *k, const void *v, int kv_heads, int head_dim, void *keys, void *values,
                       int64_t max_len, int64_t *length, void *stream);

/* Rotary embedding of q bf16 [tokens][heads][head_dim] and k bf16 [tokens][kv_heads][head_dim] in
 * the "rotate half" form of a Hugging Face Llama/Qwen2 attention module (its
 * apply_rotary_pos_emb, which the reference's Hugging Face path runs as several elementwise
 * kernels; no counterpart in the reference's own code) with cos/sin bf16 [tokens][head_dim]:
 * out = bf16(bf16(x * cos) + bf16(rotate_half(x) * sin)), bit for bit torch's bf16 result, into
 * q_out and k_out (same shapes) in one launch. head_dim even, at most 512. */
int tx_rope_rotate_half(const void *q, const void *k, int64_t tokens, int heads, int kv_heads, int head_dim,
                        const void *cos, const void *sin, void *q_out, void *k_out, void *stream);

/* The prefill of a merged [gate (inter) | up (inter)] handle with SwiGLU applied in the GEMM's
 * epilogue (no reference counterpart: the reference's prefill writes the linear output and Hugging
 * Face applies the activation): out bf16 [tokens][inter] = tx_swiglu(tx_linear(handle, x)), bit
 * for bit, in one kernel and without the [tokens][2 * inter] intermediate. x bf16 [tokens][K].
 * Needs inter % 16 == 0, a BF16 bias or none, tokens at or above the handle's prefill threshold,
 * and a call whose prefill runs tile 6, 7, 8 or 9 without a K split (TX_ERR_UNSUPPORTED otherwise,
 * e.g. for the pair tile 5 or the dense backend 1: use tx_linear + tx_swiglu). */
int tx_linear_swiglu_prefill(uint64_t handle, const void *x, int64_t tokens, void *out, void *stream);

/* tx_add_rmsnorm for one row whose delta is the output of delta_handle (M == hidden). */
int tx_add_rmsnorm_split(float *residual, uint64_t delta_handle, const void *weight, float eps, void *out,
                         int64_t hidden, void *stream);

/* tx_add_rmsnorm_split(residual, delta_handle, weight, eps, x) followed by tx_linear_split(handle,
 * x), one launch fewer: every workgroup of the one-token GEMV computes the normalized x of its K
 * range itself from residual_in and delta_handle's last tx_linear_split (the same sums and roundings
 * as the separate kernel, so x and the GEMV's split partials are bitwise the same), and one of them
 * writes residual_in + delta to residual_out, which must be another buffer than residual_in (the
 * other workgroups still read it). handle K = delta_handle M = hidden; residuals fp32 [hidden],
 * weight bf16 [hidden], all 16-byte aligned. TX_ERR_UNSUPPORTED, with nothing launched, for a LUT
 * handle, hidden above 2048, a delta split more than 8 ways, or a grid whose workgroups would read
 * more than 64 MiB in all (each reads the whole row and every split of the delta): then make the
 * two calls. No counterpart
 * in the reference (its decoder layers are Hugging Face modules). */
int tx_linear_split_norm(uint64_t handle, const float *residual_in, float *residual_out, uint64_t delta_handle,
                         const void *weight, float eps, void *stream);

/* The first layer's form of tx_linear_split_norm: the residual is row *token (device int64,
 * clamped into [0, vocab)) of the bf16 embedding table embed [vocab][hidden], widened to fp32 and
 * written to residual_out; x = its RMSNorm (tx_add_rmsnorm without a delta) feeds
 * tx_linear_split(handle, x), all in one launch, bitwise as the gather, tx_add_rmsnorm and
 * tx_linear_split. hidden = handle K <= 2048; TX_ERR_UNSUPPORTED as tx_linear_split_norm. */
int tx_linear_split_embed_norm(uint64_t handle, const void *embed, int64_t vocab, const int64_t *token,
                               float *residual_out, const void *weight, float eps, void *stream);

/* The same for tx_linear_swiglu: tx_add_rmsnorm_split followed by tx_linear_swiglu(handle, x, out),
 * one launch fewer, with the requirements of both. */
int tx_linear_swiglu_norm(uint64_t handle, const float *residual_in, float *residual_out, uint64_t delta_handle,
                          const void *weight, float eps, void *out, void *stream);

/* tx_rope_kv_cache for one token whose [q | k | v] row is the output of qkv_handle. */
int tx_rope_kv_cache_split(uint64_t qkv_handle, const int64_t *positions, const float *cos_table,
                           const float *sin_table, int heads, int kv_heads, int head_dim, void *q_out,
                           void *k_cache, void *v_cache, int64_t max_context, void *stream);

/* The prefill GEMM of a call of `tokens` tokens (bf16 x [tokens][K], at or above the handle's
 * prefill threshold) that leaves its fp32 K-split partials [ks][tokens][Mp] in `workspace` (at
 * least tx_workspace_bytes for the call) instead of reducing them, for the two prefill split
 * consumers below; *splits receives ks. TX_ERR_UNSUPPORTED when the call does not split K or runs
 * the dense backend (use tx_linear). No counterpart in the reference (its prefill writes the
 * linear output and Hugging Face's modules consume it); for callers that own the layer around the
 * linears, as the decode split consumers do. */
int tx_prefill_split(uint64_t handle, const void *x, int64_t tokens, void *workspace, int64_t workspace_bytes,
                     int *splits, void *stream);

/* tx_add_rmsnorm for `tokens` rows whose delta is tx_linear's output of delta_handle (M ==
 * hidden), read from the partials tx_prefill_split left: summed in split order and rounded as the
 * prefill reduce does (the bias added with a second rounding), bit for bit. */
int tx_add_rmsnorm_prefill_split(float *residual, uint64_t delta_handle, const void *partials, int64_t tokens,
                                 const void *weight, float eps, void *out, int64_t hidden, void *stream);

/* tx_rope_kv_cache for `tokens` tokens whose [q | k | v] rows are tx_linear's output of
 * qkv_handle, read from the partials tx_prefill_split left (same rounding as the prefill reduce). */
int tx_rope_kv_cache_prefill_split(uint64_t qkv_handle, const void *partials, int64_t tokens, const int64_t *positions,
                                   const float *cos_table, const float *sin_table, int heads, int kv_heads, int head_dim,
                                   void *q_out, void *k_cache, void *v_cache, int64_t max_context, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TEXELATOR_HIP_H */
