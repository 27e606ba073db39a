// Host-side launchers of the gfx950 kernels (internal to libtexelator_hip.so).
#pragma once

#include <hip/hip_runtime.h>

#include <string>
#include <stdint.h>

namespace tx {

enum DType : int { kF16 = 0, kBF16 = 1, kF32 = 2 };

struct GemvParams {
  const uint4 *tiles;      // RG * CG tiles of 64 x 16 bytes
  const float *scales;     // [Mp], zero beyond M
  const void *x;           // [tokens][K] bf16
  const void *bias;        // [M] bf16 or nullptr
  void *y;                 // [tokens][M] bf16 or f32
  float *partials;         // [ks][tokens][Mp] when ks > 1 or force_partials
  int M, K, Mp, RG, CG, ks, tokens;
  int force_partials;      // write fp32 partials (no bias, no reduction) even when ks == 1
  int f16;                 // x, bias and y are fp16 (weights rounded to fp16) instead of bf16
  const float4 *lut;       // LUT mode: 255 x 255 x 8 fp32 palette table, or nullptr (defined palette)
  int fused;               // one token: every K split in one workgroup (gemv_fused_profitable)
  // One token, K = heads * 128 (tile column j = attention head j): x is not read; each workgroup
  // merges its heads' decode attention chunk partials (attn, attn_chunks chunks, attn_group query
  // heads per KV head) into x itself, as the attention's merge kernel would. nullptr: x is read.
  const float *attn;
  int attn_chunks, attn_group;
  // One token, K = hidden <= 2048, at most 8 producer splits: x is not read either; every workgroup
  // computes it as
  // add_rmsnorm_kernel<true> would from the residual norm_h and a producer GEMV's split partials
  // (norm_ks splits, row stride norm_Mp, bias norm_bias or nullptr), with the RMSNorm weight
  // norm_weight; workgroup 0 writes the updated residual to norm_h_out (not norm_h: the other
  // workgroups still read it). nullptr: x is read (or merged).
  // Or, with norm_embed (norm_h nullptr, no delta): the residual is row *norm_token (clamped into
  // [0, norm_vocab)) of the bf16 table norm_embed [norm_vocab][K], widened to fp32 and written to
  // norm_h_out by workgroup 0.
  const float *norm_h;
  float *norm_h_out;
  const uint16_t *norm_embed;
  const int64_t *norm_token;
  int64_t norm_vocab;
  const float *norm_partials;
  const uint16_t *norm_bias;
  const uint16_t *norm_weight;
  float norm_eps;
  int norm_ks, norm_Mp;
  // SwiGLU GEMV over two handles (gemv_swiglu_kernel): the up matrix's tiles and scales, laid out
  // as the gate matrix's (tiles/scales, RG row groups each). nullptr: one merged [gate | up] handle.
  const uint4 *tiles_up;
  const float *scales_up;
  // One token: the sum is rounded to the output type before the bias is added (then rounded again),
  // as a caller adding a separate bias to the GEMV's output would; 0: one rounding of sum + bias.
  int bias_round_first;
};

// Hidden sizes and producer splits up to which a one-token GEMV computes the add+RMSNorm of its
// input itself.
constexpr int kNormMaxHidden = 2048;
constexpr int kNormMaxSplits = 8;

// A row of the decode attention's chunk partials [kv_head][chunk][query head of the group]: the
// chunk's unnormalised output o[128], then its score maximum m and sum of exponentials l.
constexpr int kAttnRow = 130;
// Chunks (of 64 positions) up to which a one-token GEMV merges the attention's partials itself.
constexpr int kMergeMaxChunks = 16;

// Whether a one-token GEMV of RG row groups, CG tile columns and ks K splits runs all its splits in
// one workgroup per row group (no partials in memory, no reduce launch; bit-identical results):
// 2 to 4 splits, at most 8 tiles per wave, the whole x row in 56 KiB of LDS, and row groups that
// spread evenly over `cus` CUs (at most one per CU, or at least one and a half).
bool gemv_fused_profitable(int RG, int CG, int ks, int cus);

// Single-token GEMV stages the x slice of a split in LDS: at most this many tile columns
// (128 input features each) per split.
constexpr int kGemvMaxLdsColumns = 128;

struct PrefillParams {
  const uint4 *tiles;
  const float *scales;
  const void *x;           // [tokens][K] bf16
  const void *bias;        // [M] bf16 or nullptr
  void *y;                 // [tokens][M] bf16
  float *partials;         // [ks][tokens][Mp] when ks > 1 (caller's workspace)
  int M, K, Mp, RG, CG, tokens, ks;
  int f16;                 // x, bias and y are fp16 (weights rounded to fp16) instead of bf16
  const float4 *lut;       // LUT mode: 255 x 255 x 8 fp32 palette table, or nullptr (defined palette)
  int no_reduce;           // with ks > 1: leave the partials for a consumer (no reduce kernel)
};

// GEMV variants selected by the lookahead knob (number of 1 KiB tiles in flight per wave).
bool gemv_lookahead_supported(int lookahead);
hipError_t launch_gemv(const GemvParams &p, int lookahead, bool f32_out, hipStream_t stream);
hipError_t gemv_kernel_attributes(int lookahead, hipFuncAttributes *attr);
// Workgroups of the single-token bf16 GEMV with this lookahead one CU holds at once, for a split of
// `columns` tile columns (its x slice is dynamic LDS).
int gemv_resident_per_cu(int lookahead, int columns);
// One-token GEMV of a merged [gate | up] handle with a SwiGLU epilogue (p.M = 2 * inter, one
// split, bf16); p.y receives bf16 [inter].
hipError_t launch_gemv_swiglu(const GemvParams &p, int lookahead, hipStream_t stream);

// Prefill tile candidates: ids 5..9 (kept from the reference's backend numbering).
constexpr int kPrefillFirst = 5;
constexpr int kPrefillLast = 9;
bool prefill_candidate_eligible(int candidate, int M, int K);
// K splits of the prefill GEMM for a shape (the same for every candidate).
// Default tile by shape (the autotuner's profile overrides it): measured best on the 27B-class
// shapes -- small_32x128 up to 32 tokens, medium_64x128 up to 64, medium_128x128 below 256 (two
// workgroups per CU, which hide each other's LDS and decode latency), from 256 tokens
// large_256x128 (decode shared by wave pairs) when its workgroups make one round of the CUs at
// least three quarters full.
int prefill_default_candidate(int M, int K, int64_t tokens, int cus);
int prefill_splits(int M, int CG, int64_t tokens, int cus);
hipError_t launch_prefill(const PrefillParams &p, int candidate, hipStream_t stream);
// Tile `candidate` (6-9) on a merged [gate | up] matrix (p.M = 2 * inter, inter a multiple of 16,
// p.ks == 1, bf16) with a SwiGLU epilogue: p.y receives bf16 [tokens][inter], the bits of
// launch_prefill(p, candidate) followed by launch_swiglu.
bool prefill_swiglu_supported(int candidate);
hipError_t launch_prefill_swiglu(const PrefillParams &p, int candidate, hipStream_t stream);
hipError_t prefill_kernel_attributes(int candidate, hipFuncAttributes *attr, int *lds_bytes);
const char *prefill_candidate_name(int candidate);
void prefill_candidate_shape(int candidate, int *tokens, int *rows, int *k);
// Workgroups of a candidate one CU holds at once (occupancy query; 0 for an unknown id).
int prefill_resident_per_cu(int candidate);

hipError_t launch_palette_probe(float *out, hipStream_t stream);
// Streaming read of bytes (a multiple of 16) with kStreamReadBlocks workgroups; sink receives at
// most one word per workgroup (only for an input that XORs to a sentinel value).
constexpr int kStreamReadBlocks = 4096;
hipError_t launch_stream_read(const void *data, size_t bytes, uint32_t *sink, hipStream_t stream);
// Reference-layout device blocks [M][bpr][8] -> device tiles (RG x CG tiles of 1 KiB).
hipError_t launch_repack(const uint8_t *blocks, int M, int bpr, int RG, int CG, uint4 *tiles, hipStream_t stream);
hipError_t launch_decode_dense(const uint4 *tiles, const float *scales, const float4 *lut, int M, int K, int RG, int CG,
                               bool f16, uint16_t *out, hipStream_t stream);
// Rows row_begin .. row_begin + rows - 1 (row_begin a multiple of 16) decoded into the dense
// row-major out[rows][K].
hipError_t launch_decode_rows(const uint4 *tiles, const float *scales, const float4 *lut, int M, int K, int CG,
                              int row_begin, int rows, bool f16, uint16_t *out, hipStream_t stream);

// Dense-scratch prefill pieces (dense.hip). dense_gemm: y[t][m] (row-major, row stride ldy) =
// round(sum_k x[t][k] * w[m][k]) for m < rows, fp32 accumulation on hipBLASLt (loaded at first
// use); false with `error` set when the library or the call fails. add_bias: y[t][m] =
// round(y[t][m] + bias[m]) over tokens x M (the reference's second rounding).
// gemm_workspace: kDenseGemmWorkspace bytes of device scratch for the library (256-aligned).
constexpr size_t kDenseGemmWorkspace = size_t(8) << 20;
bool dense_gemm(int device, bool f16, int rows, int64_t tokens, int K, const void *w, const void *x, void *y,
                int64_t ldy, void *gemm_workspace, hipStream_t stream, std::string &error);
hipError_t launch_add_bias(void *y, const void *bias, int64_t tokens, int M, bool f16, hipStream_t stream);

// MXFP4 staging and GEMM of the FP4 hybrid prefill (fp4.hip). Groups of 32 along K (K a multiple
// of 64 for the GEMM): packed E2M1 [rows][K/2], E8M0 scales [rows][K/32].
hipError_t launch_quantize_activation_fp4(const uint16_t *x, int64_t tokens, int K, uint8_t *packed, uint8_t *scales,
                                          hipStream_t stream);
// lut: the handle's palette table in LUT mode (nullptr: the computed palette).
hipError_t launch_quantize_weight_fp4(const uint4 *tiles, const float *scales, const float4 *lut, int M, int K,
                                      int RG, int CG, uint8_t *packed, uint8_t *group_scales, hipStream_t stream);
hipError_t launch_fp4_gemm(const uint8_t *xq, const uint8_t *xs, const uint8_t *wq, const uint8_t *ws,
                           const uint16_t *bias, uint16_t *y, int tokens, int M, int K, hipStream_t stream);

// Decoder-layer helpers (decoder.hip).
struct SplitSource;
hipError_t launch_add_rmsnorm(float *h, const uint16_t *delta, const uint16_t *weight, float eps, uint16_t *out,
                              int64_t rows, int hidden, hipStream_t stream);
// The same with delta = the split-K partials of a decode GEMV (summed and rounded as the GEMV's
// own reduction does).
// bf16 residual: sum_out = bf16(residual + delta) (delta may be null: nothing written), out its norm.
hipError_t launch_add_rmsnorm_bf16(const uint16_t *residual, const uint16_t *delta, const uint16_t *weight, float eps,
                                   uint16_t *sum_out, uint16_t *out, int64_t rows, int hidden, hipStream_t stream);
hipError_t launch_add_rmsnorm_split(float *h, const SplitSource &delta, const uint16_t *weight, float eps, uint16_t *out,
                                    int64_t rows, int hidden, hipStream_t stream);
hipError_t launch_rope_cache(const uint16_t *qkv, int64_t stride, int64_t tokens, const int64_t *positions,
                             const float *cos_t, const float *sin_t, int heads, int kv_heads, int d, uint16_t *q_out,
                             uint16_t *k_cache, uint16_t *v_cache, int64_t max_ctx, hipStream_t stream);
hipError_t launch_rope_cache_split(const SplitSource &qkv, int64_t tokens, const int64_t *positions, const float *cos_t,
                                   const float *sin_t, int heads, int kv_heads, int d, uint16_t *q_out,
                                   uint16_t *k_cache, uint16_t *v_cache, int64_t max_ctx, hipStream_t stream);
int decode_attention_chunks(int64_t length);
bool decode_attention_supported(int heads, int kv_heads, int head_dim);
int64_t decode_attention_max_length();
// Decode attention workspace bytes: the chunk partials.
int64_t decode_attention_workspace(int heads, int64_t length);
hipError_t launch_decode_attention(const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                                   const int64_t *position, int64_t length, int heads, int kv_heads, int64_t max_ctx,
                                   float scale, float *partials, uint16_t *out, hipStream_t stream);
// The same with RoPE: q and the new token's key and value from the qkv GEMV's split-K partials,
// rotated with rope_row (cos[128] then sin[128] at the position); the key and value are also
// written to the caches at the position.
hipError_t launch_decode_attention_split(const SplitSource &qkv, const int64_t *position, const float *rope_row,
                                         int64_t length, int heads, int kv_heads,
                                         uint16_t *k_cache, uint16_t *v_cache, int64_t max_ctx, float scale,
                                         float *partials, uint16_t *out, hipStream_t stream);
// The same without the merge kernel: the chunk partials stay in `partials` for a one-token GEMV
// with GemvParams::attn (the o projection), which merges them itself.
hipError_t launch_decode_attention_split_partials(const SplitSource &qkv, const int64_t *position, const float *rope_row,
                                         int64_t length, int heads, int kv_heads,
                                         uint16_t *k_cache, uint16_t *v_cache, int64_t max_ctx, float scale,
                                         float *partials, hipStream_t stream);
// Causal self-attention of a prompt (queries and keys 0..tokens-1, keys and values from the
// caches [kv_heads][max_ctx][128]); q and out bf16 rows of heads * 128 with the given strides.
bool prefill_attention_supported(int heads, int kv_heads, int head_dim);
hipError_t launch_prefill_attention(const uint16_t *q, int64_t q_stride, const uint16_t *k_cache,
                                    const uint16_t *v_cache, int64_t tokens, int heads, int kv_heads, int64_t max_ctx,
                                    float scale, uint16_t *out, int64_t out_stride, hipStream_t stream);
hipError_t launch_swiglu(const uint16_t *gu, int64_t rows, int64_t inter, uint16_t *out, hipStream_t stream);
// Hugging Face's "rotate half" rotary embedding with its bf16 rounding steps: q [tokens][heads][dim]
// and k [tokens][kv_heads][dim] with cos/sin [tokens][dim], all bf16 (dim even, <= 512).
hipError_t launch_kv_append(const uint16_t *k, const uint16_t *v, int kv_heads, int dim, uint16_t *keys, uint16_t *values,
                            int64_t max_len, int64_t *length, hipStream_t stream);
hipError_t launch_rope_rotate_half(const uint16_t *q, const uint16_t *k, int64_t tokens, int heads, int kv_heads,
                                   int dim, const uint16_t *cos, const uint16_t *sin, uint16_t *q_out, uint16_t *k_out,
                                   hipStream_t stream);
// Greedy next token of a dense bf16 lm_head [vocab][hidden] (hidden a multiple of 128, at most
// 16384) for one bf16 hidden state: token[0] = the first row with the largest bf16 logit (fp32
// sums); logits (bf16 [vocab]) written too unless null. Workspace: lm_head_argmax_workspace() bytes.
int64_t lm_head_argmax_workspace();
hipError_t launch_lm_head_argmax(const uint16_t *weight, int64_t vocab, int hidden, const uint16_t *x, uint16_t *logits,
                                 void *workspace, int64_t *token, hipStream_t stream);

}  // namespace tx
