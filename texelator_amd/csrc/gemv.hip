// Decode GEMV over BC4 tiles (gfx950, wave64, MFMA accumulation).
//
// Reference: texelator_bc4_bf16_kernel<L> (texelator/cuda/texelator_cuda.cu:154-199) computes
// y[t,m] = bf16( sum_k bf16(P*scale[m]) * x[t,k] + bias[m] ) with fp32 accumulation; L is the
// number of texture requests in flight per warp. Here:
//   * a workgroup (4 waves) owns one 16-row group and one K range (a "split"); each wave streams
//     every 4th 1 KiB tile of that range with one 128-bit buffer load per lane, LOOKAHEAD tiles in
//     flight, and decodes its two blocks per tile in VGPRs (decode_block_lds);
//   * the decoded bf16 weights are the A operand of v_mfma_f32_16x16x32_bf16 (lane = row x K
//     chunk of 8), the activations the B operand with one token per column, so one pass over the
//     weights serves up to 16 tokens and the K reduction across lanes happens inside the MFMA;
//   * the four waves' accumulators are summed through LDS in wave order;
//   * with several splits each workgroup writes an fp32 partial row and a second kernel sums
//     the partials in split order, so results never depend on scheduling; where the row groups
//     spread evenly over the CUs, one workgroup instead runs every split of its row group and sums
//     them in the same order (gemv_fused_kernel: the same bits, one launch).
// Single-token calls stage x in LDS; multi-token calls read x through the cache hierarchy.
#include "bc4_device.h"
#include "elementwise.h"
#include "kernels.h"

namespace tx {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// D += A * B for 16x16x32 tiles whose operands are 8 packed 16-bit values per lane (bf16, or fp16
// with F16).
template <bool F16>
__device__ __forceinline__ f32x4 mfma(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3, uint4 b, f32x4 c) {
  const u32x4 av = {a0, a1, a2, a3};
  const u32x4 bv = {b.x, b.y, b.z, b.w};
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, av), __builtin_bit_cast(f16x8, bv), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, bv), c, 0, 0, 0);
}

// The tiles of one wave read through a buffer descriptor based at the wave's first tile: the
// tile offset is wave-uniform (a scalar register) and the lane's 16-byte slot a fixed vector
// register, so a tile load costs no vector instruction for its address. Loads are non-temporal
// (weights are read once per call). `bytes` bounds the descriptor; loads past it return zero.
struct TileStream {
  __amdgpu_buffer_rsrc_t rsrc, spare;
  int lane_offset;
  __device__ __forceinline__ TileStream(const uint4 *first, int64_t bytes, int lane)
      : rsrc(__builtin_amdgcn_make_buffer_rsrc(const_cast<uint4 *>(first), (short)0,
                                               (int)(bytes < 0x7FFFFFFF ? bytes : 0x7FFFFFFF), 0x00020000)),
        spare(__builtin_amdgcn_make_buffer_rsrc(const_cast<SeedTableImage *>(&kSeedTableImage), (short)0,
                                                kSeedTableBytes, 0x00020000)),
        lane_offset(lane * 16) {}
  // Tile j of the wave (`stride_tiles` tiles after tile j - 1) if j < n. The K loops issue one
  // load per step whatever is left, so each decode waits for its own tile only; a load past the
  // wave's n tiles reads the seed table image instead (1 KiB that every workgroup copies, so it
  // stays in L2) and its value is never used. Re-reading the wave's last tile there, as the loops
  // once did, fetched it from HBM again once the streaming loads had evicted it: ~7 MB per launch
  // of the 5120 -> 27648 shape (one tile per wave).
  __device__ __forceinline__ uint4 load(int j, int n, int stride_tiles) const {
    const bool real = j < n;
    const int offset = __builtin_amdgcn_readfirstlane(real ? j * stride_tiles * kTileBytes : 0);
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(real ? rsrc : spare, lane_offset, offset, 2 /* nt */);
    return make_uint4(v.x, v.y, v.z, v.w);
  }
};

// x of one token, 16 k-values per block: x0/x1 = block 2kg positions 0-7 / 8-15, x2/x3 = block 2kg+1.
struct XFrag {
  uint4 x0, x1, x2, x3;
};

__device__ __forceinline__ uint4 load_x8(const uint16_t *x, int k, int K) {
  return k < K ? *reinterpret_cast<const uint4 *>(x + k) : make_uint4(0, 0, 0, 0);
}

// LDS chunks (16 bytes, 8 activations) the one-token x slice of `columns` tile columns occupies:
// whole 1 KiB wave loads, so a multiple of 64.
__host__ __device__ constexpr int x_stage_chunks(int columns) { return (columns * 16 + 63) / 64 * 64; }

// One-token x slice into LDS: chunks first .. first + count - 1 of x (a K-element bf16 vector,
// 16-byte aligned) to xs[0 ..], by direct buffer-to-LDS loads (no registers, no VALU per chunk;
// wave w of `waves` issues the 1 KiB loads w, w + waves, ...). The buffer descriptor ends at K, so
// chunks at or past K read as zeros (K is a multiple of 16: a chunk is wholly in or out). Up to
// x_stage_chunks(count / 16) chunks are written. The caller waits for the loads (vmcnt) before
// the barrier that publishes them.
__device__ __forceinline__ void stage_x_lds(uint4 *xs, const uint16_t *x, int K, int first, int count, int wave,
                                            int lane, int waves = kWaves) {
  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(x), (short)0, K * 2, 0x00020000);
  for (int base = wave * 64; base < count; base += 64 * waves)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)(xs + base), 16,
                                             (first + base + lane) * 16, 0, 0, 0);
}

// x of a split whose tile columns are attention heads (GemvParams::attn): head c_begin + j (j <
// nc, one wave per head at a time) merged from the decode attention's chunk partials, exactly as
// decode_attention_combine_kernel merges a head: M = the chunks' maximum m_c, weights w_c =
// exp(m_c - M) (0 for an empty chunk), total = the sum of l_c * w_c in wave_sum's tree (lane c
// holds chunk c; with at most 16 chunks only the first 16-lane row holds any, so that is row16_sum
// of that row: the other rows add exact zeros), four fma chains acc[c % 4] over the chunks below
// the last multiple of four and the rest into acc[0], in chunk order, and x = bf16(((acc0 + acc1) +
// (acc2 + acc3)) / total) -- so x is bitwise the merge kernel's output. The weights reach every
// lane by v_readlane: no LDS round trip. Lane l produces dimensions l and l + 64 and writes them as
// stage_x_lds would place them. Every load of a head (all its chunks' values, clamped to the last
// chunk, and the lane's chunk statistics) goes out before the first wait.
__device__ __forceinline__ void merge_attention_x(uint4 *xs, const GemvParams &p, int c_begin, int nc, int wave,
                                                  int lane) {
  const int chunks = p.attn_chunks, group = p.attn_group;
  const uint32_t step = (uint32_t)group * kAttnRow;  // floats between chunks of one head
  const int main_end = chunks & ~3;
  uint16_t *xh = reinterpret_cast<uint16_t *>(xs);
  for (int j = wave; j < nc; j += kWaves) {
    const int head = c_begin + j, kv = head / group, g = head % group;
    const float *base = p.attn + ((size_t)kv * chunks * group + g) * kAttnRow;
    float o0[kMergeMaxChunks], o1[kMergeMaxChunks];
#pragma unroll
    for (int c = 0; c < kMergeMaxChunks; ++c) {
      const float *row = base + (uint32_t)min(c, chunks - 1) * step;
      o0[c] = row[lane];
      o1[c] = row[lane + 64];
    }
    const float *srow = base + (uint32_t)min(lane, chunks - 1) * step;
    const float ms = srow[kAttnRow - 2], ls = srow[kAttnRow - 1];
    const float mv = lane < chunks ? ms : -INFINITY;
    const float m = lane_value(row16_max(mv), 0);
    const float w = mv == -INFINITY ? 0.f : expf(mv - m);
    const float total = lane_value(row16_sum(lane < chunks ? __builtin_fmaf(ls, w, 0.f) : 0.f), 0);
    float a0[4] = {0.f, 0.f, 0.f, 0.f}, a1[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < kMergeMaxChunks; ++c) {
      if (c < chunks) {
        const float wc = lane_value(w, c);
        if (c < main_end) {
          a0[c & 3] = __builtin_fmaf(o0[c], wc, a0[c & 3]);
          a1[c & 3] = __builtin_fmaf(o1[c], wc, a1[c & 3]);
        } else {
          a0[0] = __builtin_fmaf(o0[c], wc, a0[0]);
          a1[0] = __builtin_fmaf(o1[c], wc, a1[0]);
        }
      }
    }
    xh[j * kTileK + lane] = to_bf(((a0[0] + a0[1]) + (a0[2] + a0[3])) / total);
    xh[j * kTileK + lane + 64] = to_bf(((a1[0] + a1[1]) + (a1[2] + a1[3])) / total);
  }
}

// x of a one-token GEMV (GemvParams::norm_h or norm_embed) as add_rmsnorm_kernel writes it, for hidden
// = p.K <= 2048 and at most 8 producer splits. That kernel's thread t handles the group of four
// columns i = t (t < 512 here); this lane stands for its threads t = 256 j + tid (j < 4; only j < 2
// hold a group). Per group: delta = bf16(partials summed in split order + bias), v = h + delta,
// the sum of squares (x^2 + y^2) + (z^2 + w^2); each of that kernel's 16 waves summed by wave_sum
// (its wave 4j + w is this wave's j-th sum; j >= 2 sum zeros) and the 16 added in order from zero;
// inv = rsqrt(total / hidden + eps); x = bf16(weight * bf16(v * inv)). So x and the updated
// residual are bitwise that kernel's. Every load (the residual, all splits clamped to the last,
// the bias and the weight of both groups) goes out before the first wait. Only the x of the
// workgroup's tile columns [c_begin, c_begin + nc) is written to xs (where stage_x_lds puts it);
// `writer` writes every updated group to norm_h_out.
constexpr int kNormStand = 1024 / kThreads;  // add_rmsnorm threads this lane stands for
constexpr int kNormSlots = 2;                 // of which hold a group (hidden <= 2048)
__device__ __forceinline__ void norm_x_lds(uint4 *xs, float *wave_sums, const GemvParams &p, int c_begin, int nc,
                                           int wave, int lane, bool writer) {
  const int hidden = p.K, groups = hidden / 4, ks = p.norm_ks;
  const int tid = wave * 64 + lane;
  const bool embed = p.norm_embed != nullptr, delta = p.norm_partials != nullptr;
  const float4 *hr = reinterpret_cast<const float4 *>(p.norm_h);
  const uint2 *er = nullptr;
  if (embed) {
    const int64_t token = min(max(*p.norm_token, (int64_t)0), p.norm_vocab - 1);
    er = reinterpret_cast<const uint2 *>(p.norm_embed + (size_t)token * hidden);
  }
  const float4 *pp = reinterpret_cast<const float4 *>(p.norm_partials);
  const int step = p.norm_Mp / 4;  // float4 between splits (one token)
  const uint2 *br = reinterpret_cast<const uint2 *>(p.norm_bias ? p.norm_bias : p.norm_weight);
  const uint2 *wr = reinterpret_cast<const uint2 *>(p.norm_weight);
  float4 hv[kNormSlots], q[kNormSlots][kNormMaxSplits];
  uint2 bv[kNormSlots], wv[kNormSlots];
#pragma unroll
  for (int j = 0; j < kNormSlots; ++j) {
    const int ic = min(j * kThreads + tid, groups - 1);
    if (embed) {
      const uint2 e = er[ic];
      hv[j] = make_float4(bf((uint16_t)(e.x & 0xFFFFu)), bf((uint16_t)(e.x >> 16)), bf((uint16_t)(e.y & 0xFFFFu)),
                          bf((uint16_t)(e.y >> 16)));
    } else {
      hv[j] = hr[ic];
    }
    if (delta) {
#pragma unroll
      for (int k = 0; k < kNormMaxSplits; ++k) q[j][k] = pp[min(k, ks - 1) * step + ic];
      bv[j] = br[ic];
    }
    wv[j] = wr[ic];
  }
  __builtin_amdgcn_sched_barrier(0);  // every load issued before the first add
  float4 v[kNormSlots];
  float ss[kNormStand] = {};
  float4 *ho = reinterpret_cast<float4 *>(p.norm_h_out);
#pragma unroll
  for (int j = 0; j < kNormSlots; ++j) {
    const int i = j * kThreads + tid;
    float4 h = hv[j];
    if (delta) {  // without a delta the residual is taken as it is (add_rmsnorm with delta NULL)
      float4 acc = q[j][0];
#pragma unroll
      for (int k = 1; k < kNormMaxSplits; ++k) {
        if (k < ks) {
          acc.x += q[j][k].x;
          acc.y += q[j][k].y;
          acc.z += q[j][k].z;
          acc.w += q[j][k].w;
        }
      }
      if (p.norm_bias) {
        acc.x += bf((uint16_t)(bv[j].x & 0xFFFFu));
        acc.y += bf((uint16_t)(bv[j].x >> 16));
        acc.z += bf((uint16_t)(bv[j].y & 0xFFFFu));
        acc.w += bf((uint16_t)(bv[j].y >> 16));
      }
      h.x += bf(to_bf(acc.x));
      h.y += bf(to_bf(acc.y));
      h.z += bf(to_bf(acc.z));
      h.w += bf(to_bf(acc.w));
    }
    v[j] = h;
    if (i < groups) {
      ss[j] = (h.x * h.x + h.y * h.y) + (h.z * h.z + h.w * h.w);
      if (writer) ho[i] = h;
    }
  }
#pragma unroll
  for (int j = 0; j < kNormStand; ++j) {
    const float s = wave_sum(ss[j]);
    if (lane == 0) wave_sums[j * kWaves + wave] = s;
  }
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < kNormStand * kWaves; ++w) total += wave_sums[w];
  const float inv = rsqrtf(total / (float)hidden + p.norm_eps);
  uint2 *xo = reinterpret_cast<uint2 *>(xs);
  const int g_begin = c_begin * (kTileK / 4), g_end = (c_begin + nc) * (kTileK / 4);
#pragma unroll
  for (int j = 0; j < kNormSlots; ++j) {
    const int i = j * kThreads + tid;
    if (i < groups && i >= g_begin && i < g_end) {
      const float4 h = v[j];
      const uint2 w = wv[j];
      const float n0 = bf(to_bf(h.x * inv)), n1 = bf(to_bf(h.y * inv)), n2 = bf(to_bf(h.z * inv)),
                  n3 = bf(to_bf(h.w * inv));
      xo[i - g_begin] = make_uint2(
          (uint32_t)to_bf(bf((uint16_t)(w.x & 0xFFFFu)) * n0) | ((uint32_t)to_bf(bf((uint16_t)(w.x >> 16)) * n1) << 16),
          (uint32_t)to_bf(bf((uint16_t)(w.y & 0xFFFFu)) * n2) | ((uint32_t)to_bf(bf((uint16_t)(w.y >> 16)) * n3) << 16));
    }
  }
}

// Single-token B operands: only output column 0 of a tile is used, so only the lanes of B column 0
// (lane % 16 == 0) read x; the other fifteen columns keep the zeros they start with
// (TX_GEMV_ZERO_COLUMNS; else every column reads x, a broadcast). Zero operands switch fewer
// multiplier bits than fifteen copies of x, the reads skipped spare LDS bandwidth, and the clock of
// this power-bound kernel follows the switching. Column 0's products and sums are the same either way.
#ifndef TX_GEMV_ZERO_COLUMNS
#define TX_GEMV_ZERO_COLUMNS 1
#endif
// x of tile column `col` into xf: one lane in sixteen, or all.
__device__ __forceinline__ void read_x_columns(XFrag &xf, const uint4 *xs, int col, int kg, int lane) {
  if (!TX_GEMV_ZERO_COLUMNS || (lane & 15) == 0) {
    const uint4 *xv = xs + col * 16 + kg * 4;
    xf.x0 = xv[0];
    xf.x1 = xv[1];
    xf.x2 = xv[2];
    xf.x3 = xv[3];
  }
}
// The same without the per-tile branch, for the two-ring SwiGLU kernel (measured faster there): the
// fifteen other columns read a zeroed 256-byte slot placed after the staged x instead of skipping
// the read.
constexpr int kZeroSlotU4 = 16;
struct XColumns {
  const uint4 *base;  // the staged x (column 0) or the zero slot
  uint32_t mask;      // keeps the tile column's offset for column 0, drops it for the others
  __device__ __forceinline__ const uint4 *at(int col, int kg) const {
    return base + (((uint32_t)col * 16u) & mask) + kg * 4;
  }
};
__device__ __forceinline__ XColumns x_columns(uint4 *xs, int zero_slot, int lane) {
  if (TX_GEMV_ZERO_COLUMNS && threadIdx.x < 16) xs[zero_slot + threadIdx.x] = make_uint4(0, 0, 0, 0);
  const bool x_lane = !TX_GEMV_ZERO_COLUMNS || (lane & 15) == 0;
  return XColumns{x_lane ? xs : xs + zero_slot, x_lane ? 0xFFFFFFFFu : 0u};
}

// One tile for one lane: decode both blocks and accumulate 4 MFMAs (block 0 into acc0, block 1
// into acc1; the two are added at the end in a fixed order).
template <bool F16>
__device__ __forceinline__ void tile_mfma(uint4 cur, const XFrag &xf, float scale, uint32_t pm,
                                          const PaletteTableStorage &t, f32x4 &acc0, f32x4 &acc1) {
  uint32_t w[8];
  decode_block_lds<F16>(cur.x, cur.y, scale, pm, t, w);
  acc0 = mfma<F16>(w[0], w[1], w[2], w[3], xf.x0, acc0);
  acc0 = mfma<F16>(w[4], w[5], w[6], w[7], xf.x1, acc0);
  decode_block_lds<F16>(cur.z, cur.w, scale, pm, t, w);
  acc1 = mfma<F16>(w[0], w[1], w[2], w[3], xf.x2, acc1);
  acc1 = mfma<F16>(w[4], w[5], w[6], w[7], xf.x3, acc1);
}

// Palette rows (8 fp32 values each) of a tile's two blocks, for LUT mode.
struct TileRows {
  float4 a03, a47, b03, b47;
};

__device__ __forceinline__ TileRows tile_rows(const float4 *lut, uint4 tile) {
  const float4 *ra = lut + 2 * (size_t)palette_row(tile.x, tile.y);
  const float4 *rb = lut + 2 * (size_t)palette_row(tile.z, tile.w);
  return TileRows{ra[0], ra[1], rb[0], rb[1]};
}

// LUT mode: the tile's weights from its palette rows.
template <bool F16>
__device__ __forceinline__ void tile_mfma_lut(uint4 cur, const TileRows &rows, const XFrag &xf, float scale,
                                              f32x4 &acc0, f32x4 &acc1) {
  uint32_t w[8];
  decode_from_palette<F16>(rows.a03, rows.a47, cur.x, cur.y, scale, w);
  acc0 = mfma<F16>(w[0], w[1], w[2], w[3], xf.x0, acc0);
  acc0 = mfma<F16>(w[4], w[5], w[6], w[7], xf.x1, acc0);
  decode_from_palette<F16>(rows.b03, rows.b47, cur.z, cur.w, scale, w);
  acc1 = mfma<F16>(w[0], w[1], w[2], w[3], xf.x2, acc1);
  acc1 = mfma<F16>(w[4], w[5], w[6], w[7], xf.x3, acc1);
}

// Wave priority from the share of a wave's tiles still to do (3 while more than three quarters
// remain, down to 0 in the last quarter). The sequencer issues the oldest ready wave first, so
// with equal priorities the first workgroups on a CU race ahead and the last ones finish alone,
// with the CU mostly idle; ranking waves by remaining work keeps them level and the CU full
// until the end of the launch.
#ifndef TX_GEMV_PRIORITY
#define TX_GEMV_PRIORITY 1
#endif
__device__ __forceinline__ void progress_priority(int remaining, int total) {
  if constexpr (!TX_GEMV_PRIORITY) return;
  if (remaining * 4 > total * 3) __builtin_amdgcn_s_setprio(3);
  else if (remaining * 2 > total) __builtin_amdgcn_s_setprio(2);
  else if (remaining * 4 > total) __builtin_amdgcn_s_setprio(1);
  else __builtin_amdgcn_s_setprio(0);
}

// Minimum waves per SIMD the register allocation must allow (7 keeps the kernel at <= 72 VGPRs
// without spills, so seven 4-wave workgroups fit on a CU).
#ifndef TX_GEMV_WAVES_PER_EU
#define TX_GEMV_WAVES_PER_EU 7
#endif

// F16: fp16 activations, bias and output with fp16-rounded weights (the reference's FP16 GEMV,
// texelator_cuda.cu:94-139, multiplies unrounded fp32 weights; the rounding costs at most 2^-11
// relative per weight).
// LUT: the palette of every block is read from a 255 x 255 x 8 table (p.lut) instead of being
// computed; the rows of tile j+1 are fetched while tile j is decoded (needs LA >= 2).
// Where a one-token GEMV's x comes from: read (staged from p.x), merged from the decode attention's
// chunk partials (merge_attention_x), or normalized from the residual and a producer's partials
// (norm_x_lds). The last two run on grids of few row groups, so their register bound is relaxed.
enum XSource : int { kXRead = 0, kXMerge = 1, kXNorm = 2 };

template <bool F16, int LA, bool MULTI, bool F32OUT, bool LUT, int XSRC = kXRead>
__global__ __launch_bounds__(kThreads, LUT || XSRC != kXRead ? 4 : TX_GEMV_WAVES_PER_EU) void gemv_kernel(GemvParams p) {
  static_assert(XSRC == kXRead || (!MULTI && !LUT), "a merged or normalized x feeds one token's staged x");
  constexpr bool MERGE = XSRC == kXMerge;
  static_assert(!LUT || LA >= 2, "LUT mode prefetches the palette rows of the next tile");
  extern __shared__ uint4 xs[];  // single token: x slice, 16 uint4 (128 bf16) per tile column
  __shared__ __attribute__((aligned(16))) PaletteTableStorage tables;
  constexpr int kRedTokens = MULTI ? 16 : 1;  // one token: 256 bytes of LDS instead of 4 KiB
  __shared__ float red[kWaves][kRedTokens][16];  // [wave][token][row]

  const int g = blockIdx.x;
  const int split = blockIdx.y;
  const int t0 = blockIdx.z * 16;
  const int tc = min(16, p.tokens - t0);
  // Tile columns of this split. The host keeps ks * CG below 2^31, so 32-bit products are exact;
  // an unsplit launch needs no division at all (a 64-bit one cost ~300 scalar instructions per
  // wave before the first tile load could issue).
  int c_begin = 0, c_end = p.CG;
  if (p.ks > 1) {
    c_begin = (int)((uint32_t)split * (uint32_t)p.CG / (uint32_t)p.ks);
    c_end = (int)((uint32_t)(split + 1) * (uint32_t)p.CG / (uint32_t)p.ks);
  }
  const int nc = c_end - c_begin;
  const uint16_t *x = static_cast<const uint16_t *>(p.x);

  const int lane = threadIdx.x & 63;
  // The wave index is uniform across the wave: keep it (and everything derived from it, the
  // tile loop included) in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nt = nc > wave ? (nc - wave + kWaves - 1) / kWaves : 0;
  // Tile j of this wave is tile column c_begin + j*kWaves + wave of row group g. A wave with no
  // tile (nc < kWaves) still issues its prefetch loads (TileStream::load sends them to the spare).
  const int64_t first_tile = (int64_t)g * p.CG + c_begin + min(wave, nc - 1);
  const TileStream stream(p.tiles + first_tile * 64, ((int64_t)p.RG * p.CG - first_tile) * kTileBytes, lane);

  // Ring of LA+1 tile slots: while tile j is decoded, tiles j+1..j+LA are in flight. The first
  // loads are issued before the LDS set-up so that they overlap it.
  constexpr int R = LA + 1;
  uint4 ring[R];
#pragma unroll
  for (int u = 0; u < LA; ++u) ring[u] = stream.load(u, nt, kWaves);

  const int i = lane & 15;   // weight row within the group; token column of the B operand
  const int kg = lane >> 4;  // K chunk: blocks 2kg and 2kg+1 of each tile
  const int row = g * kTileRows + i;
  const float scale = p.scales[row];  // loaded with the tiles and x, not after the barrier

  if constexpr (MERGE) {
    copy_seed_tables(tables, wave, lane, kWaves);  // in flight while the heads are merged
    merge_attention_x(xs, p, c_begin, nc, wave, lane);
  } else if constexpr (XSRC == kXNorm) {
    __shared__ float norm_sums[kNormStand * kWaves];
    copy_seed_tables(tables, wave, lane, kWaves);  // in flight while x is normalized
    norm_x_lds(xs, norm_sums, p, c_begin, nc, wave, lane, blockIdx.x == 0 && blockIdx.y == 0);
  } else {
    if constexpr (!MULTI) stage_x_lds(xs, x, p.K, c_begin * 16, nc * 16, wave, lane);
    if constexpr (!LUT) copy_seed_tables(tables, wave, lane, kWaves);
  }
  if constexpr (!MULTI || !LUT) __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): x and the tables have landed
  __syncthreads();

  const uint32_t pm = pm_scale_pair<F16>(scale);
  // Multi-token: this lane's token column (duplicates the last token past the end).
  const uint16_t *xrow = x + (size_t)(t0 + min(i, tc - 1)) * p.K;

  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  // Single token: B column 0 gets x (read_x_columns), the others zeros or x; only output column 0
  // is read.
  XFrag xf{};
  auto load_xf = [&](int j) {
    const int col = j * kWaves + wave;  // tile column within this split
    if constexpr (MULTI) {
      const int k = (c_begin + col) * kTileK + kg * 32;
      xf.x0 = load_x8(xrow, k, p.K);
      xf.x1 = load_x8(xrow, k + 8, p.K);
      xf.x2 = load_x8(xrow, k + 16, p.K);
      xf.x3 = load_x8(xrow, k + 24, p.K);
    } else {
      read_x_columns(xf, xs, col, kg, lane);
    }
  };

  // Main loop over whole ring turns, branch-free: every step issues exactly one load (clamped to
  // the wave's last tile near the end), so each decode waits only for its own tile.
  int j0 = 0;
  if constexpr (LUT) {
    const float4 *lut = p.lut;
    TileRows cur = tile_rows(lut, ring[0]);
    for (; j0 + R <= nt; j0 += R) {
      progress_priority(nt - j0, nt);
#pragma unroll
      for (int u = 0; u < R; ++u) {
        ring[(u + LA) % R] = stream.load(j0 + u + LA, nt, kWaves);
        const TileRows next = tile_rows(lut, ring[(u + 1) % R]);  // tile j+1 (clamped near the end)
        load_xf(j0 + u);
        tile_mfma_lut<F16>(ring[u], cur, xf, scale, acc0, acc1);
        cur = next;
      }
    }
#pragma unroll
    for (int u = 0; u < LA; ++u) {
      const TileRows next = tile_rows(lut, ring[(u + 1) % R]);
      if (j0 + u < nt) {
        load_xf(j0 + u);
        tile_mfma_lut<F16>(ring[u], cur, xf, scale, acc0, acc1);
      }
      cur = next;
    }
  } else {
    for (; j0 + R <= nt; j0 += R) {
      progress_priority(nt - j0, nt);
#pragma unroll
      for (int u = 0; u < R; ++u) {
        ring[(u + LA) % R] = stream.load(j0 + u + LA, nt, kWaves);
        load_xf(j0 + u);
        tile_mfma<F16>(ring[u], xf, scale, pm, tables, acc0, acc1);
      }
    }
    // Tail: at most LA tiles, already in slots 0..LA-1.
#pragma unroll
    for (int u = 0; u < LA; ++u)
      if (j0 + u < nt) {
        load_xf(j0 + u);
        tile_mfma<F16>(ring[u], xf, scale, pm, tables, acc0, acc1);
      }
  }

  // acc[r] = partial y[token i][row 4kg + r] of this wave.
  const f32x4 acc = acc0 + acc1;
  if (i < tc) {
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][MULTI ? i : 0][kg * 4 + r] = acc[r];
  }
  __syncthreads();

  if (threadIdx.x < tc * 16) {
    const int n = threadIdx.x >> 4;
    const int rr = threadIdx.x & 15;
    const int nn = MULTI ? n : 0;
    float total = red[0][nn][rr];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) total += red[w][nn][rr];
    const int out_row = g * kTileRows + rr;
    const int token = t0 + n;
    if (p.ks > 1 || p.force_partials) {
      p.partials[((size_t)split * p.tokens + token) * p.Mp + out_row] = total;
    } else if (out_row < p.M) {
      if constexpr (F32OUT) {
        static_cast<float *>(p.y)[(size_t)token * p.M + out_row] = total;
      } else {
        if (p.bias) {
          if (p.bias_round_first) total = F16 ? (float)(_Float16)total : bf(to_bf(total));
          total += half_bits_to_float<F16>(static_cast<const uint16_t *>(p.bias)[out_row]);
        }
        if constexpr (F16) static_cast<_Float16 *>(p.y)[(size_t)token * p.M + out_row] = (_Float16)total;
        else static_cast<__bf16 *>(p.y)[(size_t)token * p.M + out_row] = (__bf16)total;
      }
    }
  }
}

// One token, every K split in one workgroup: 4 * ks waves (ks <= kFusedMaxSplits) for one 16-row
// group, wave w doing exactly what wave w % 4 of split w / 4 does in gemv_kernel (same tile columns
// and order, same MFMA chains, same acc0 + acc1), so each split's sum over its four waves (in wave
// order) is gemv_kernel's partial, and the splits are then summed in split order, bias added and
// the result cast as splitk_reduce_kernel does: bit-identical to gemv_kernel + the reduce, in one
// launch and without partials in memory. The whole x row is staged in LDS once.
constexpr int kFusedMaxSplits = 4;

template <bool F16, int LA, bool F32OUT>
__global__ __launch_bounds__(kThreads * kFusedMaxSplits, TX_GEMV_WAVES_PER_EU) void gemv_fused_kernel(GemvParams p) {
  extern __shared__ uint4 xs[];  // the whole x row: 16 uint4 per tile column
  __shared__ __attribute__((aligned(16))) PaletteTableStorage tables;
  __shared__ float red[kWaves * kFusedMaxSplits][16];  // [wave][row]

  const int g = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int waves = kWaves * p.ks;
  const int split = wave / kWaves, wq = wave % kWaves;  // split, and the wave's place within it
  int c_begin = 0, c_end = p.CG;
  if (p.ks > 1) {
    c_begin = (int)((uint32_t)split * (uint32_t)p.CG / (uint32_t)p.ks);
    c_end = (int)((uint32_t)(split + 1) * (uint32_t)p.CG / (uint32_t)p.ks);
  }
  const int nc = c_end - c_begin;
  const int nt = nc > wq ? (nc - wq + kWaves - 1) / kWaves : 0;
  const int64_t first_tile = (int64_t)g * p.CG + c_begin + min(wq, nc - 1);
  const TileStream stream(p.tiles + first_tile * 64, ((int64_t)p.RG * p.CG - first_tile) * kTileBytes, lane);

  constexpr int R = LA + 1;
  uint4 ring[R];
#pragma unroll
  for (int u = 0; u < LA; ++u) ring[u] = stream.load(u, nt, kWaves);

  const int i = lane & 15;
  const int kg = lane >> 4;
  const float scale = p.scales[g * kTileRows + i];
  stage_x_lds(xs, static_cast<const uint16_t *>(p.x), p.K, 0, p.CG * 16, wave, lane, waves);
  copy_seed_tables(tables, wave, lane, waves);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): x and the tables have landed
  __syncthreads();

  const uint32_t pm = pm_scale_pair<F16>(scale);
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  XFrag xf{};
  auto load_xf = [&](int j) { read_x_columns(xf, xs, c_begin + j * kWaves + wq, kg, lane); };
  int j0 = 0;
  for (; j0 + R <= nt; j0 += R) {
    progress_priority(nt - j0, nt);
#pragma unroll
    for (int u = 0; u < R; ++u) {
      ring[(u + LA) % R] = stream.load(j0 + u + LA, nt, kWaves);
      load_xf(j0 + u);
      tile_mfma<F16>(ring[u], xf, scale, pm, tables, acc0, acc1);
    }
  }
#pragma unroll
  for (int u = 0; u < LA; ++u)
    if (j0 + u < nt) {
      load_xf(j0 + u);
      tile_mfma<F16>(ring[u], xf, scale, pm, tables, acc0, acc1);
    }

  const f32x4 acc = acc0 + acc1;  // partial y[row 4kg + r] of this wave
  if (i == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][kg * 4 + r] = acc[r];
  }
  __syncthreads();

  if (threadIdx.x < 16) {
    const int rr = threadIdx.x;
    float total = 0.f;
    for (int s = 0; s < p.ks; ++s) {
      float part = red[kWaves * s][rr];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) part += red[kWaves * s + w][rr];
      total = s == 0 ? part : total + part;
    }
    const int out_row = g * kTileRows + rr;
    if (out_row < p.M) {
      if constexpr (F32OUT) {
        static_cast<float *>(p.y)[out_row] = total;
      } else {
        if (p.bias) {
          if (p.bias_round_first) total = F16 ? (float)(_Float16)total : bf(to_bf(total));
          total += half_bits_to_float<F16>(static_cast<const uint16_t *>(p.bias)[out_row]);
        }
        if constexpr (F16) static_cast<_Float16 *>(p.y)[out_row] = (_Float16)total;
        else static_cast<__bf16 *>(p.y)[out_row] = (__bf16)total;
      }
    }
  }
}

// One-token GEMV of a merged [gate | up] handle (M = 2 * inter, inter a multiple of 16, one K
// split) whose epilogue applies SwiGLU: out[r] = bf16(silu(bf16(gate_r)) * bf16(up_r)), exactly the
// values tx_linear followed by tx_swiglu produce. Workgroup g computes gate row group g and up row
// group g + RG/2 with the same four-wave K split, tile order and MFMA chains as gemv_kernel, so
// each of the two row groups' sums is bit-identical to the plain GEMV's. Two rings of LA + 1 tiles
// are in flight, so the occupancy bound falls with LA (no spills).
// NORM: x computed by norm_x_lds (GemvParams::norm_h) instead of read.
// With GemvParams::tiles_up the up rows come from a second handle of the same shape (row group g
// of each; RG row groups, M = 2 * inter): the same sums, bit for bit, as the merged handle of the
// two matrices.
template <int LA, bool NORM = false>
__global__ __launch_bounds__(kThreads, NORM ? 4 : (LA == 1 ? 6 : (LA == 2 ? 5 : 4))) void gemv_swiglu_kernel(GemvParams p) {
  extern __shared__ uint4 xs[];
  __shared__ __attribute__((aligned(16))) PaletteTableStorage tables;
  __shared__ float red[2][kWaves][16];  // [gate|up][wave][row]

  const int g = blockIdx.x;
  const bool pair = p.tiles_up != nullptr;
  const int half = pair ? 0 : p.RG / 2;  // up row group of g: g + half of tiles, or g of tiles_up
  const int nc = p.CG;
  const uint16_t *x = static_cast<const uint16_t *>(p.x);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nt = nc > wave ? (nc - wave + kWaves - 1) / kWaves : 0;
  const int first = min(wave, nc - 1);
  const int64_t gate_first = (int64_t)g * p.CG + first, up_first = (int64_t)(g + half) * p.CG + first;
  const int64_t total = (int64_t)p.RG * p.CG;
  const uint4 *up_base = pair ? p.tiles_up : p.tiles;
  const float *up_scales = pair ? p.scales_up : p.scales;
  const TileStream gate_tiles(p.tiles + gate_first * 64, (total - gate_first) * kTileBytes, lane);
  const TileStream up_tiles(up_base + up_first * 64, (total - up_first) * kTileBytes, lane);

  constexpr int R = LA + 1;
  uint4 ring_g[R], ring_u[R];
#pragma unroll
  for (int u = 0; u < LA; ++u) {
    ring_g[u] = gate_tiles.load(u, nt, kWaves);
    ring_u[u] = up_tiles.load(u, nt, kWaves);
  }
  const int i = lane & 15;
  const int kg = lane >> 4;
  const float scale_g = p.scales[g * kTileRows + i];  // loaded with the tiles and x
  const float scale_u = up_scales[(g + half) * kTileRows + i];
  if constexpr (NORM) {
    __shared__ float norm_sums[kNormStand * kWaves];
    copy_seed_tables(tables, wave, lane, kWaves);  // in flight while x is normalized
    norm_x_lds(xs, norm_sums, p, 0, nc, wave, lane, blockIdx.x == 0);
  } else {
    stage_x_lds(xs, x, p.K, 0, nc * 16, wave, lane);
    copy_seed_tables(tables, wave, lane, kWaves);
  }
  const XColumns xcols = x_columns(xs, x_stage_chunks(p.CG), lane);  // zeroes the slot before the barrier
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): x and the tables have landed
  __syncthreads();

  const uint32_t pm_g = pm_scale_pair<false>(scale_g);
  const uint32_t pm_u = pm_scale_pair<false>(scale_u);
  f32x4 ga0 = {0.f, 0.f, 0.f, 0.f}, ga1 = ga0, ua0 = ga0, ua1 = ga0;
  XFrag xf;  // B column 0 gets x, the others zeros (x_columns); only output column 0 is read
  auto consume = [&](int u, int j) {
    {
      const uint4 *xv = xcols.at(j * kWaves + wave, kg);
      xf.x0 = xv[0];
      xf.x1 = xv[1];
      xf.x2 = xv[2];
      xf.x3 = xv[3];
    }
    tile_mfma<false>(ring_g[u], xf, scale_g, pm_g, tables, ga0, ga1);
    tile_mfma<false>(ring_u[u], xf, scale_u, pm_u, tables, ua0, ua1);
  };
  int j0 = 0;
  for (; j0 + R <= nt; j0 += R) {
    progress_priority(nt - j0, nt);
#pragma unroll
    for (int u = 0; u < R; ++u) {
      ring_g[(u + LA) % R] = gate_tiles.load(j0 + u + LA, nt, kWaves);
      ring_u[(u + LA) % R] = up_tiles.load(j0 + u + LA, nt, kWaves);
      consume(u, j0 + u);
    }
  }
#pragma unroll
  for (int u = 0; u < LA; ++u)
    if (j0 + u < nt) consume(u, j0 + u);

  const f32x4 gacc = ga0 + ga1, uacc = ua0 + ua1;
  if (i == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      red[0][wave][kg * 4 + r] = gacc[r];
      red[1][wave][kg * 4 + r] = uacc[r];
    }
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    const int rr = threadIdx.x;
    float gate = red[0][0][rr], up = red[1][0][rr];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
      gate += red[0][w][rr];
      up += red[1][w][rr];
    }
    const int row = g * kTileRows + rr;  // output index = gate row
    const int inter = p.M / 2;
    if (row < inter) {
      const uint16_t *bias = static_cast<const uint16_t *>(p.bias);
      if (bias) {
        gate += bf(bias[row]);
        up += bf(bias[inter + row]);
      }
      const float act = swiglu_value(bf(to_bf(gate)), bf(to_bf(up)));
      static_cast<uint16_t *>(p.y)[row] = to_bf(act);
    }
  }
}

// y[t][m] = sum over splits s (in order) of partials[s][t][m], then bias and output cast
// (split_sums, which fused consumers of the partials use as well). KS > 0: exactly KS splits,
// all loaded before the first add; KS = 0: any count, four at a time.
constexpr int kReduceMaxKS = 16;
template <bool F16, bool F32OUT, int KS>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemvParams p) {
  const int m = blockIdx.x * 256 + threadIdx.x;
  const int token = blockIdx.y;
  if (m >= p.M) return;
  const SplitSource src{p.partials, F32OUT ? nullptr : static_cast<const uint16_t *>(p.bias), p.ks, p.Mp, p.tokens,
                        F32OUT ? 0 : p.bias_round_first};
  const int64_t cols[1] = {m};
  float sums[1];
  split_sums<1, F16, KS>(src, token, cols, sums);
  const float total = sums[0];
  if constexpr (F32OUT) {
    static_cast<float *>(p.y)[(size_t)token * p.M + m] = total;
  } else if constexpr (F16) {
    static_cast<_Float16 *>(p.y)[(size_t)token * p.M + m] = (_Float16)total;
  } else {
    static_cast<__bf16 *>(p.y)[(size_t)token * p.M + m] = (__bf16)total;
  }
}

template <bool F16, bool F32OUT, int KS = 1>
void launch_splitk_reduce(const GemvParams &p, hipStream_t stream) {
  const dim3 grid((p.M + 255) / 256, p.tokens);
  if constexpr (KS <= kReduceMaxKS) {
    if (p.ks == KS) hipLaunchKernelGGL((splitk_reduce_kernel<F16, F32OUT, KS>), grid, dim3(256), 0, stream, p);
    else launch_splitk_reduce<F16, F32OUT, KS + 1>(p, stream);
  } else {
    hipLaunchKernelGGL((splitk_reduce_kernel<F16, F32OUT, 0>), grid, dim3(256), 0, stream, p);
  }
}

// Tile columns up to which the fused kernel stages the whole x row (56 KiB of LDS: two workgroups
// per CU with the seed tables).
constexpr int kFusedMaxColumns = 224;

bool fused_eligible(const GemvParams &p) {
  return p.fused && p.tokens == 1 && !p.lut && !p.force_partials && !p.attn && !p.norm_h && !p.norm_embed && p.ks > 1 &&
         p.ks <= kFusedMaxSplits &&
         p.CG <= kFusedMaxColumns;
}

template <bool F16, int LA, bool MULTI, bool F32OUT>
hipError_t launch_variant(const GemvParams &p, hipStream_t stream) {
  if constexpr (!MULTI) {
    if (fused_eligible(p)) {
      const size_t lds = (size_t)x_stage_chunks(p.CG) * sizeof(uint4);
      hipLaunchKernelGGL((gemv_fused_kernel<F16, LA, F32OUT>), dim3(p.RG), dim3(kThreads * p.ks), lds, stream, p);
      return hipGetLastError();
    }
  }
  const int max_cols = (p.CG + p.ks - 1) / p.ks;
  const size_t lds = MULTI ? 0 : (size_t)x_stage_chunks(max_cols) * sizeof(uint4);
  dim3 grid(p.RG, p.ks, (p.tokens + 15) / 16);
  if constexpr (!MULTI && !F16 && F32OUT) {
    if (p.attn) {  // the caller checked: one token, force_partials, no LUT, K = heads * 128
      hipLaunchKernelGGL((gemv_kernel<false, LA, false, true, false, kXMerge>), grid, dim3(kThreads), lds, stream, p);
      return hipGetLastError();
    }
    if (p.norm_h || p.norm_embed) {  // the caller checked: one token, force_partials, no LUT, K <= 2048
      hipLaunchKernelGGL((gemv_kernel<false, LA, false, true, false, kXNorm>), grid, dim3(kThreads), lds, stream, p);
      return hipGetLastError();
    }
  }
  if (p.lut) {
    constexpr int kLutLA = LA < 2 ? 2 : LA;  // the palette-row prefetch needs a second tile in flight
    hipLaunchKernelGGL((gemv_kernel<F16, kLutLA, MULTI, F32OUT, true>), grid, dim3(kThreads), lds, stream, p);
  } else {
    hipLaunchKernelGGL((gemv_kernel<F16, LA, MULTI, F32OUT, false>), grid, dim3(kThreads), lds, stream, p);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.ks == 1 || p.force_partials) return e;
  launch_splitk_reduce<F16, F32OUT>(p, stream);
  return hipGetLastError();
}

// The fp32-output variants (parity and split consumers) exist for bf16 activations only.
template <int LA>
hipError_t launch_la(const GemvParams &p, bool f32_out, hipStream_t stream) {
  const bool multi = p.tokens > 1;
  if (p.f16) {
    if (f32_out) return hipErrorInvalidValue;
    return multi ? launch_variant<true, LA, true, false>(p, stream) : launch_variant<true, LA, false, false>(p, stream);
  }
  if (multi) return f32_out ? launch_variant<false, LA, true, true>(p, stream) : launch_variant<false, LA, true, false>(p, stream);
  return f32_out ? launch_variant<false, LA, false, true>(p, stream) : launch_variant<false, LA, false, false>(p, stream);
}

}  // namespace

hipError_t launch_gemv_swiglu(const GemvParams &p, int lookahead, hipStream_t stream) {
  const size_t lds = (size_t)(x_stage_chunks(p.CG) + kZeroSlotU4) * sizeof(uint4);
  const dim3 grid(p.tiles_up ? p.RG : p.RG / 2);
  if (p.norm_h || p.norm_embed) {
    switch (lookahead) {
      case 1: hipLaunchKernelGGL((gemv_swiglu_kernel<1, true>), grid, dim3(kThreads), lds, stream, p); break;
      case 2: hipLaunchKernelGGL((gemv_swiglu_kernel<2, true>), grid, dim3(kThreads), lds, stream, p); break;
      default: hipLaunchKernelGGL((gemv_swiglu_kernel<4, true>), grid, dim3(kThreads), lds, stream, p); break;
    }
    return hipGetLastError();
  }
  switch (lookahead) {
    case 1: hipLaunchKernelGGL(gemv_swiglu_kernel<1>, grid, dim3(kThreads), lds, stream, p); break;
    case 2: hipLaunchKernelGGL(gemv_swiglu_kernel<2>, grid, dim3(kThreads), lds, stream, p); break;
    default: hipLaunchKernelGGL(gemv_swiglu_kernel<4>, grid, dim3(kThreads), lds, stream, p); break;
  }
  return hipGetLastError();
}

bool gemv_fused_profitable(int RG, int CG, int ks, int cus) {
  if (ks < 2 || ks > kFusedMaxSplits || CG > kFusedMaxColumns) return false;
  const int tiles_per_wave = ((CG + ks - 1) / ks + kWaves - 1) / kWaves;
  return tiles_per_wave <= 8 && (RG <= cus || 2 * RG >= 3 * cus);
}

bool gemv_lookahead_supported(int la) { return la == 1 || la == 2 || la == 3 || la == 4 || la == 6 || la == 8; }

hipError_t launch_gemv(const GemvParams &p, int lookahead, bool f32_out, hipStream_t stream) {
  switch (lookahead) {
    case 1: return launch_la<1>(p, f32_out, stream);
    case 2: return launch_la<2>(p, f32_out, stream);
    case 3: return launch_la<3>(p, f32_out, stream);
    case 4: return launch_la<4>(p, f32_out, stream);
    case 6: return launch_la<6>(p, f32_out, stream);
    case 8: return launch_la<8>(p, f32_out, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t gemv_kernel_attributes(int lookahead, hipFuncAttributes *attr) {
  switch (lookahead) {
    case 1: return hipFuncGetAttributes(attr, reinterpret_cast<const void *>(&gemv_kernel<false, 1, false, false, false>));
    case 2: return hipFuncGetAttributes(attr, reinterpret_cast<const void *>(&gemv_kernel<false, 2, false, false, false>));
    case 3: return hipFuncGetAttributes(attr, reinterpret_cast<const void *>(&gemv_kernel<false, 3, false, false, false>));
    case 4: return hipFuncGetAttributes(attr, reinterpret_cast<const void *>(&gemv_kernel<false, 4, false, false, false>));
    case 6: return hipFuncGetAttributes(attr, reinterpret_cast<const void *>(&gemv_kernel<false, 6, false, false, false>));
    case 8: return hipFuncGetAttributes(attr, reinterpret_cast<const void *>(&gemv_kernel<false, 8, false, false, false>));
    default: return hipErrorInvalidValue;
  }
}

int gemv_resident_per_cu(int lookahead, int columns) {
  const void *fn = nullptr;
  switch (lookahead) {
    case 1: fn = reinterpret_cast<const void *>(&gemv_kernel<false, 1, false, false, false>); break;
    case 2: fn = reinterpret_cast<const void *>(&gemv_kernel<false, 2, false, false, false>); break;
    case 3: fn = reinterpret_cast<const void *>(&gemv_kernel<false, 3, false, false, false>); break;
    case 4: fn = reinterpret_cast<const void *>(&gemv_kernel<false, 4, false, false, false>); break;
    case 6: fn = reinterpret_cast<const void *>(&gemv_kernel<false, 6, false, false, false>); break;
    case 8: fn = reinterpret_cast<const void *>(&gemv_kernel<false, 8, false, false, false>); break;
    default: return 0;
  }
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, kThreads, (size_t)x_stage_chunks(columns) * sizeof(uint4)) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

}  // namespace tx
