// Decoder-layer helpers around the BC4 linears (gfx950): fused residual add + RMSNorm, RoPE +
// KV-cache write, split-length decode attention and SwiGLU.
//
// No reference counterpart: the reference runs these layers as stock Hugging Face modules
// (docs/supported-models.md:3-5) and only replaces the linears. Here they exist so that a whole
// decode step is a short, graph-capturable sequence of kernels.
//
// Layouts: activations row-major bf16 [rows][width]; the residual stream fp32; the KV caches
// bf16 [kv_head][position][head_dim].
#include <math.h>

#include <type_traits>

#include "elementwise.h"
#include "kernels.h"

namespace tx {

namespace {

// Calls f with std::integral_constant<int, ks> for split counts 1-4 (the kernels' loop-free
// variants) and with 0 (the generic loop) for more.
template <typename F>
void with_split_count(int ks, F &&f) {
  switch (ks) {
    case 1: f(std::integral_constant<int, 1>{}); break;
    case 2: f(std::integral_constant<int, 2>{}); break;
    case 3: f(std::integral_constant<int, 3>{}); break;
    case 4: f(std::integral_constant<int, 4>{}); break;
    default: f(std::integral_constant<int, 0>{}); break;
  }
}

// h[row] += delta[row] (if given); out[row] = bf16(weight * bf16(h * rsqrt(mean(h^2) + eps))).
// One block per row; each thread owns groups of 4 columns (4 * t + 4096 * i), all of whose
// loads are issued before the reduction. hidden must be a multiple of 4.
// With SPLIT, delta is the fp32 split-K partials of a decode GEMV: each group's partials are read
// as float4 per split (four splits of every group in flight together; KS > 0 means ks == KS, read
// without a loop) and summed in split order plus the bias, exactly as split_sum does. Both variants reduce in the same order, so their outputs
// are bit-identical; a row gets 1024 threads (a decode step has a single row).
constexpr int kNormThreads = 1024;

template <bool SPLIT, int KS>
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(float *h, const uint16_t *delta, SplitSource split,
                                                                   const uint16_t *weight, float eps, uint16_t *out,
                                                                   int hidden) {
  constexpr int kThreads = kNormThreads;
  constexpr int kUnroll = 2;  // register-resident groups per thread per pass (covers 8192 columns)
  __shared__ float partial[kThreads / 64];
  float4 *hr = reinterpret_cast<float4 *>(h + (size_t)blockIdx.x * hidden);
  const uint2 *dr = !SPLIT && delta ? reinterpret_cast<const uint2 *>(delta + (size_t)blockIdx.x * hidden) : nullptr;
  uint2 *orow = reinterpret_cast<uint2 *>(out + (size_t)blockIdx.x * hidden);
  const uint2 *wr = reinterpret_cast<const uint2 *>(weight);
  const int groups = hidden / 4;
  // One pass covers every group (hidden <= 8192): the values stay in registers for the output,
  // and the norm weight is loaded with them.
  const bool one_pass = groups <= kThreads * kUnroll;
  float4 v[kUnroll];
  uint2 wv[kUnroll];
  float ss = 0.f;
  for (int base = 0; base < groups; base += kThreads * kUnroll) {
    // load phase: every load of this pass in flight at once (indices clamped, then masked)
    uint2 d[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int i = min(base + u * kThreads + (int)threadIdx.x, groups - 1);
      v[u] = hr[i];
      if (!SPLIT && dr) d[u] = dr[i];
      if (one_pass) wv[u] = wr[i];
    }
    if constexpr (SPLIT) {
      // The bias (from a valid address whether or not there is one) and four splits of partials
      // go out before the first add; with KS (ks == KS) there is no loop, select or branch.
      const float4 *pp = reinterpret_cast<const float4 *>(split.partials + (size_t)blockIdx.x * split.Mp);
      const size_t step = (size_t)split.tokens * split.Mp / 4;
      const uint2 *bp = reinterpret_cast<const uint2 *>(split.bias ? split.bias : reinterpret_cast<const uint16_t *>(split.partials));
      int col[kUnroll];
      uint2 b[kUnroll];
      float4 acc[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        col[u] = min(base + u * kThreads + (int)threadIdx.x, groups - 1);
        b[u] = bp[col[u]];
      }
      if constexpr (KS > 0) {
        float4 q[KS][kUnroll];
#pragma unroll
        for (int k = 0; k < KS; ++k)
#pragma unroll
          for (int u = 0; u < kUnroll; ++u) q[k][u] = pp[(size_t)k * step + col[u]];
        __builtin_amdgcn_sched_barrier(0);  // every load issued before the first add
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          acc[u] = q[0][u];
#pragma unroll
          for (int k = 1; k < KS; ++k) {
            acc[u].x += q[k][u].x;
            acc[u].y += q[k][u].y;
            acc[u].z += q[k][u].z;
            acc[u].w += q[k][u].w;
          }
        }
      } else {
        constexpr int kGroup = 4;
        for (int k0 = 0; k0 < split.ks; k0 += kGroup) {
          float4 q[kGroup][kUnroll];
#pragma unroll
          for (int g = 0; g < kGroup; ++g)
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) q[g][u] = pp[(size_t)min(k0 + g, split.ks - 1) * step + col[u]];
#pragma unroll
          for (int g = 0; g < kGroup; ++g) {
            const int k = k0 + g;
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
              const float4 a = acc[u], x = q[g][u];
              acc[u] = k == 0 ? x : (k < split.ks ? make_float4(a.x + x.x, a.y + x.y, a.z + x.z, a.w + x.w) : a);
            }
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        if (split.round_first && split.bias) {  // the prefill epilogue: the bias with a second rounding
          acc[u].x = bf(to_bf(acc[u].x));
          acc[u].y = bf(to_bf(acc[u].y));
          acc[u].z = bf(to_bf(acc[u].z));
          acc[u].w = bf(to_bf(acc[u].w));
        }
        if (split.bias) {
          acc[u].x += bf((uint16_t)(b[u].x & 0xFFFFu));
          acc[u].y += bf((uint16_t)(b[u].x >> 16));
          acc[u].z += bf((uint16_t)(b[u].y & 0xFFFFu));
          acc[u].w += bf((uint16_t)(b[u].y >> 16));
        }
        d[u].x = (uint32_t)to_bf(acc[u].x) | ((uint32_t)to_bf(acc[u].y) << 16);
        d[u].y = (uint32_t)to_bf(acc[u].z) | ((uint32_t)to_bf(acc[u].w) << 16);
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int i = base + u * kThreads + (int)threadIdx.x;
      if (i >= groups) continue;
      if (SPLIT || dr) {
        v[u].x += bf((uint16_t)(d[u].x & 0xFFFFu));
        v[u].y += bf((uint16_t)(d[u].x >> 16));
        v[u].z += bf((uint16_t)(d[u].y & 0xFFFFu));
        v[u].w += bf((uint16_t)(d[u].y >> 16));
        hr[i] = v[u];
      }
      ss += (v[u].x * v[u].x + v[u].y * v[u].y) + (v[u].z * v[u].z + v[u].w * v[u].w);
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) total += partial[w];
  const float inv = rsqrtf(total / (float)hidden + eps);
  auto normalize = [&](const float4 &h4, const uint2 &w) {
    const float n0 = bf(to_bf(h4.x * inv)), n1 = bf(to_bf(h4.y * inv)), n2 = bf(to_bf(h4.z * inv)), n3 = bf(to_bf(h4.w * inv));
    const uint32_t lo = (uint32_t)to_bf(bf((uint16_t)(w.x & 0xFFFFu)) * n0) | ((uint32_t)to_bf(bf((uint16_t)(w.x >> 16)) * n1) << 16);
    const uint32_t hi = (uint32_t)to_bf(bf((uint16_t)(w.y & 0xFFFFu)) * n2) | ((uint32_t)to_bf(bf((uint16_t)(w.y >> 16)) * n3) << 16);
    return make_uint2(lo, hi);
  };
  if (one_pass) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int i = u * kThreads + (int)threadIdx.x;
      if (i < groups) orow[i] = normalize(v[u], wv[u]);
    }
    return;
  }
  for (int i = threadIdx.x; i < groups; i += kThreads) orow[i] = normalize(hr[i], wr[i]);
}

// The same normalization over a bf16 residual kept in bf16, as a Hugging Face decoder layer keeps it:
// v = bf16(residual + delta) (torch's bf16 add: the fp32 sum rounded once) written to sum_out, or
// v = residual when delta is null (nothing written); out = bf16(weight * bf16(v * rsqrt(mean(v^2) +
// eps))). Thread t owns the groups of four columns 4 * (t + 1024 * i) and sums their squares in the
// order add_rmsnorm_kernel does, so for the same v both kernels give the same bits.
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_bf16_kernel(const uint16_t *residual, const uint16_t *delta,
                                                                        const uint16_t *weight, float eps,
                                                                        uint16_t *sum_out, uint16_t *out, int hidden) {
  constexpr int kThreads = kNormThreads;
  constexpr int kUnroll = 2;
  __shared__ float partial[kThreads / 64];
  const size_t row = (size_t)blockIdx.x * hidden;
  const uint2 *rr = reinterpret_cast<const uint2 *>(residual + row);
  const uint2 *dr = delta ? reinterpret_cast<const uint2 *>(delta + row) : nullptr;
  uint2 *sr = delta ? reinterpret_cast<uint2 *>(sum_out + row) : nullptr;
  uint2 *orow = reinterpret_cast<uint2 *>(out + row);
  const uint2 *wr = reinterpret_cast<const uint2 *>(weight);
  const int groups = hidden / 4;
  const bool one_pass = groups <= kThreads * kUnroll;
  auto value = [&](int i) {
    const uint2 r = rr[i];
    float4 v = make_float4(bf((uint16_t)(r.x & 0xFFFFu)), bf((uint16_t)(r.x >> 16)), bf((uint16_t)(r.y & 0xFFFFu)),
                           bf((uint16_t)(r.y >> 16)));
    if (dr) {
      const uint2 d = dr[i];
      v.x = bf(to_bf(v.x + bf((uint16_t)(d.x & 0xFFFFu))));
      v.y = bf(to_bf(v.y + bf((uint16_t)(d.x >> 16))));
      v.z = bf(to_bf(v.z + bf((uint16_t)(d.y & 0xFFFFu))));
      v.w = bf(to_bf(v.w + bf((uint16_t)(d.y >> 16))));
    }
    return v;
  };
  float4 v[kUnroll];
  uint2 wv[kUnroll];
  float ss = 0.f;
  for (int base = 0; base < groups; base += kThreads * kUnroll) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int i = base + u * kThreads + (int)threadIdx.x;
      if (i >= groups) continue;
      v[u] = value(i);
      if (one_pass) wv[u] = wr[i];
      if (sr) {
        sr[i] = make_uint2((uint32_t)to_bf(v[u].x) | ((uint32_t)to_bf(v[u].y) << 16),
                           (uint32_t)to_bf(v[u].z) | ((uint32_t)to_bf(v[u].w) << 16));
      }
      ss += (v[u].x * v[u].x + v[u].y * v[u].y) + (v[u].z * v[u].z + v[u].w * v[u].w);
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) total += partial[w];
  const float inv = rsqrtf(total / (float)hidden + eps);
  auto normalize = [&](const float4 &h4, const uint2 &w) {
    const float n0 = bf(to_bf(h4.x * inv)), n1 = bf(to_bf(h4.y * inv)), n2 = bf(to_bf(h4.z * inv)), n3 = bf(to_bf(h4.w * inv));
    const uint32_t lo = (uint32_t)to_bf(bf((uint16_t)(w.x & 0xFFFFu)) * n0) | ((uint32_t)to_bf(bf((uint16_t)(w.x >> 16)) * n1) << 16);
    const uint32_t hi = (uint32_t)to_bf(bf((uint16_t)(w.y & 0xFFFFu)) * n2) | ((uint32_t)to_bf(bf((uint16_t)(w.y >> 16)) * n3) << 16);
    return make_uint2(lo, hi);
  };
  if (one_pass) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int i = u * kThreads + (int)threadIdx.x;
      if (i < groups) orow[i] = normalize(v[u], wv[u]);
    }
    return;
  }
  // wider rows: v again from the inputs (the residual and delta are unchanged; sum_out is not read)
  for (int i = threadIdx.x; i < groups; i += kThreads) orow[i] = normalize(value(i), wr[i]);
}


// One block per (token, head); thread j rotates the pair (j, j + d/2) of rotate-half RoPE.
// q heads are written to q_out; k heads are rotated into the K cache; v heads are copied.
// With SPLIT, the [q | k | v] row is the fp32 split-K partials of the qkv decode GEMV.
template <bool SPLIT>
__global__ void rope_cache_kernel(const uint16_t *qkv, SplitSource split, int64_t stride, const int64_t *positions,
                                  const float *cos_t, const float *sin_t, int heads, int kv_heads, int d, uint16_t *q_out,
                                  uint16_t *k_cache, uint16_t *v_cache, int64_t max_ctx) {
  const int t = blockIdx.x;
  const int head = blockIdx.y;
  const int j = threadIdx.x;
  const int half = d / 2;
  const int64_t pos = positions[t];
  // A position outside the cache (and the RoPE tables, which have max_ctx rows) writes nothing:
  // the host cannot see the value, so the bound is checked here.
  if (pos < 0 || pos >= max_ctx) return;
  const uint16_t *row = qkv + (size_t)t * stride;
  auto value = [&](int64_t col) { return SPLIT ? split_value(split, t, col) : bf(row[col]); };
  if (head < heads + kv_heads) {
    const float x1 = value((int64_t)head * d + j), x2 = value((int64_t)head * d + j + half);
    const float c1 = cos_t[pos * d + j], c2 = cos_t[pos * d + j + half];
    const float s1 = sin_t[pos * d + j], s2 = sin_t[pos * d + j + half];
    const uint16_t o1 = to_bf(x1 * c1 - x2 * s1);
    const uint16_t o2 = to_bf(x2 * c2 + x1 * s2);
    uint16_t *dst = head < heads ? q_out + ((size_t)t * heads + head) * d
                                 : k_cache + ((size_t)(head - heads) * max_ctx + pos) * d;
    dst[j] = o1;
    dst[j + half] = o2;
  } else {
    const int kv = head - heads - kv_heads;
    const int64_t col = (int64_t)(heads + kv_heads + kv) * d;
    uint16_t *dst = v_cache + ((size_t)kv * max_ctx + pos) * d;
    dst[j] = to_bf(value(col + j));
    dst[j + half] = to_bf(value(col + j + half));
  }
}

constexpr int kChunk = 64;      // keys per attention block
constexpr int kHeadDim = 128;   // head_dim handled by the decode attention kernels
constexpr int kMaxGroup = 8;    // query heads per KV head
constexpr int kRowU4 = kHeadDim * 2 / 16;  // uint4 per cached key or value row (16)
// LDS row stride of the key tile in uint4: one uint4 of padding, so the 16 keys a wave scores at
// once (256 bytes apart unpadded) fall into different LDS banks.
constexpr int kKeyStrideU4 = kRowU4 + 1;
// 16 bytes as a native vector (a uint4 struct copy goes through private memory when it is
// held across the kernel's other loads)
typedef uint32_t dwordx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
constexpr int kPRow = kChunk + 8;  // bf16 per row of the probability operands (144 bytes: no conflicts)

// D += A * B on a 16x16x32 bf16 tile: lane l holds A row l % 16 and B column l % 16, each with
// k = 8 (l / 16) .. + 7; D column l % 16, rows 4 (l / 16) .. + 3.
__device__ __forceinline__ f32x4_t mfma_bf16(dwordx4 a, dwordx4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// bf16 index of value (dimension d, key) in the transposed value tile [128][64]: each row is
// eight 16-byte slots of 8 keys, slot (key / 8) stored at (key / 8) ^ ((d + d / 8) % 8), so that
// the PV operand reads (8 keys of 16 dimensions) and the transposing writes (16 dimensions of
// one key) spread over the LDS banks.
__device__ __forceinline__ int vt_index(int d, int key) {
  return d * kChunk + 8 * ((key >> 3) ^ ((d + (d >> 3)) & 7)) + (key & 7);
}

// Split-length decode attention for one query token. Block (kv, chunk) loads the chunk's keys and
// values (those <= position) into LDS in one burst (values transposed), scores the group's query
// heads against them on the matrix cores (bf16 q and keys, exact products, fp32 sums), takes the
// softmax statistics in fp32, multiplies the probabilities (as bf16 hi + lo, 16 significant
// bits) by the values on the matrix cores, and writes the chunk's max m, sum of exp l and
// unnormalised output o to partials[kv][chunk][g][130].
// ROPE: q and the new token's key and value come from the qkv decode GEMV's split-K partials
// (summed, rounded and rotated exactly as rope_cache_kernel<true> does, with the RoPE table rows
// of the position gathered by the caller, so no load waits for the position); the block whose
// chunk holds the position writes the key and value into the caches and into its own tiles.
// Every load of a block (chunk rows, partials, RoPE row, position) goes out before the first wait:
// the kernel's time is one memory latency plus the arithmetic, not a chain of latencies.
// (Merging the chunks in the same launch -- each block publishing its partials behind a device
// fence and the last one to take a ticket merging -- measured slower on MI355X: every such fence
// writes back the XCD's L2, 64 times per XCD and layer at 4096 positions.)

struct AttnInput {
  const uint16_t *q;  // bf16 [heads][128] (without ROPE)
  SplitSource split;  // [q | k | v] split-K partials (with ROPE)
  const float *rope_row;  // cos[128] then sin[128] at the token's position (with ROPE)
  int heads, kv_heads;
};

// KS > 0 (with ROPE): the qkv GEMV has exactly KS splits, read without a loop.
template <bool ROPE, int KS>
__global__ __launch_bounds__(256) void decode_attention_kernel(AttnInput in, uint16_t *k_cache, uint16_t *v_cache,
                                                               const int64_t *position, int group, int64_t max_ctx,
                                                               float scale, int chunks, float *partials) {
  __shared__ uint4 ks[kChunk * kKeyStrideU4];       // keys [key][128] bf16, padded rows
  __shared__ __align__(16) uint16_t vt[kHeadDim * kChunk];     // values [dim][key] bf16 (vt_index)
  __shared__ uint4 qs[16 * kKeyStrideU4];             // q [head][128] bf16, padded rows, heads >= group zero
  __shared__ float probs[kMaxGroup][kChunk];          // scores, then probabilities (fp32)
  __shared__ __align__(16) uint16_t pb[2][16][kPRow];          // probabilities as bf16 hi + lo, heads >= group zero
  __shared__ float stats[kMaxGroup][2];
  const int kv = blockIdx.x;
  const int chunk = blockIdx.y;
  const int tid = threadIdx.x;
  const int j0 = chunk * kChunk;
  float *out = partials + ((size_t)kv * chunks + chunk) * group * (kHeadDim + 2);
  const int64_t pos = *position;
  // Issue the chunk's K/V rows (clamped into the cache) and q before the position arrives:
  // nothing waits for a load whose result only masks.
  // (32-bit byte offsets from the head's base: a head's cache is well under 4 GiB)
  const char *kg = reinterpret_cast<const char *>(k_cache + (size_t)kv * max_ctx * kHeadDim);
  const char *vg = reinterpret_cast<const char *>(v_cache + (size_t)kv * max_ctx * kHeadDim);
  dwordx4 kr[4], vr[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int idx = u * 256 + tid;
    const uint32_t row = (uint32_t)min((int64_t)(j0 + idx / kRowU4), max_ctx - 1);
    const uint32_t off = (row * kRowU4 + idx % kRowU4) * 16u;
    kr[u] = *reinterpret_cast<const dwordx4 *>(kg + off);
    vr[u] = *reinterpret_cast<const dwordx4 *>(vg + off);
  }
  __builtin_amdgcn_sched_barrier(0);  // the tile loads go out first, all eight of them
  constexpr int kHalf = kHeadDim / 2;
  // Without ROPE: q element u * 256 + tid of the group. With ROPE: the rotate-half pair
  // (j, j + 64) of head g for p = u * 256 + tid = 64 g + j (u < 2 covers 8 heads), as the
  // unrotated sums x1, x2, and the new token's key pair (j, j + 64) (tid < 64) or value element
  // tid - 64 (tid < 192). Every block loads the new token's partials and the RoPE row with the
  // rest, so no load waits for the position or for another load.
  constexpr int kQ = ROPE ? 2 : kMaxGroup * kHeadDim / 256;
  float qv[kQ], qw[kQ], nk[2] = {0.f, 0.f};
  float c1 = 0.f, c2 = 0.f, s1 = 0.f, s2 = 0.f;
  if constexpr (ROPE) {
    const int j = tid % kHalf;
    int64_t cols[2 * kQ + 2];
#pragma unroll
    for (int u = 0; u < kQ; ++u) {
      const int i = u * 256 + tid;
      const int64_t col = i < group * kHalf ? (int64_t)(kv * group + i / kHalf) * kHeadDim + j : 0;
      cols[2 * u] = col;
      cols[2 * u + 1] = col + kHalf;
    }
    const int64_t kcol = (int64_t)(in.heads + kv) * kHeadDim + j;
    const int64_t vcol = (int64_t)(in.heads + in.kv_heads + kv) * kHeadDim + min(max(tid - kHalf, 0), kHeadDim - 1);
    cols[2 * kQ] = tid < kHalf ? kcol : vcol;
    cols[2 * kQ + 1] = kcol + kHalf;
    c1 = in.rope_row[j];
    c2 = in.rope_row[j + kHalf];
    s1 = in.rope_row[kHeadDim + j];
    s2 = in.rope_row[kHeadDim + j + kHalf];
    float sums[2 * kQ + 2];
    split_sums<2 * kQ + 2, false, KS>(in.split, 0, cols, sums);
#pragma unroll
    for (int u = 0; u < kQ; ++u) {
      qv[u] = bf(to_bf(sums[2 * u]));
      qw[u] = bf(to_bf(sums[2 * u + 1]));
    }
    nk[0] = bf(to_bf(sums[2 * kQ]));
    nk[1] = bf(to_bf(sums[2 * kQ + 1]));
  } else {
#pragma unroll
    for (int u = 0; u < kQ; ++u) {
      const int i = u * 256 + tid;
      qv[u] = i < group * kHeadDim ? bf(in.q[(size_t)kv * group * kHeadDim + i]) : 0.f;
    }
  }
  // The tiles, in every block and without a branch, so the compiler keeps the tile loads where
  // they were issued: keys as loaded, values zeroed past the position.
  const int count = (int)min((int64_t)kChunk, max(pos - j0 + 1, (int64_t)0));  // valid keys in this chunk
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int idx = u * 256 + tid;
    const int key = idx / kRowU4, c = idx % kRowU4;
    reinterpret_cast<dwordx4 *>(ks)[key * kKeyStrideU4 + c] = kr[u];
    const dwordx4 v = key < count ? vr[u] : dwordx4{0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 8; ++e) vt[vt_index(8 * c + e, key)] = (uint16_t)(v[e / 2] >> (16 * (e & 1)));
  }
  const bool active = count > 0;
  if (active) {
    // With ROPE the chunk that holds the position takes that row from the partials, not from the
    // cache (which this block writes).
    // (A position at or past the end of the cache is never written.)
    const int fresh = ROPE && pos - j0 < kChunk && pos < max_ctx ? (int)(pos - j0) : -1;
    uint16_t *qh = reinterpret_cast<uint16_t *>(qs);
    constexpr int kQRow = kKeyStrideU4 * 8;  // bf16 per padded q row
#pragma unroll
    for (int u = 0; u < kQ; ++u) {
      const int i = u * 256 + tid;
      if constexpr (ROPE) {
        if (i < group * kHalf) {
          const int g = i / kHalf, j = i % kHalf;
          const float x1 = qv[u], x2 = qw[u];
          qh[g * kQRow + j] = to_bf(x1 * c1 - x2 * s1);
          qh[g * kQRow + j + kHalf] = to_bf(x2 * c2 + x1 * s2);
        }
      } else {
        if (i < group * kHeadDim) qh[(i / kHeadDim) * kQRow + i % kHeadDim] = to_bf(qv[u]);
      }
    }
    // the MFMA operand rows of heads past the group: zero
    for (int i = tid; i < (16 - group) * kQRow / 2; i += 256)
      reinterpret_cast<uint32_t *>(qh + group * kQRow)[i] = 0u;
    for (int i = tid; i < 2 * (16 - group) * kPRow / 2; i += 256) {
      const int h = i / (kPRow / 2), r = i % (kPRow / 2);
      reinterpret_cast<uint32_t *>(&pb[h / (16 - group)][group + h % (16 - group)][0])[r] = 0u;
    }
    if (fresh >= 0) {
      // This chunk holds the new token: rotate its key, take its value, write both to the caches
      // and over the tiles' row of the position (after the barrier that orders the tile stores).
      __syncthreads();
      uint16_t *krow = reinterpret_cast<uint16_t *>(ks + fresh * kKeyStrideU4);
      if (tid < kHalf) {
        const float x1 = nk[0], x2 = nk[1];
        const uint16_t o1 = to_bf(x1 * c1 - x2 * s1), o2 = to_bf(x2 * c2 + x1 * s2);
        uint16_t *dst = k_cache + ((size_t)kv * max_ctx + pos) * kHeadDim;
        dst[tid] = o1;
        dst[tid + kHalf] = o2;
        krow[tid] = o1;
        krow[tid + kHalf] = o2;
      } else if (tid < kHalf + kHeadDim) {
        const int e = tid - kHalf;
        const uint16_t v = to_bf(nk[0]);
        v_cache[((size_t)kv * max_ctx + pos) * kHeadDim + e] = v;
        vt[vt_index(e, fresh)] = v;
      }
    }
    __syncthreads();

    const int wave = tid >> 6, lane = tid & 63;
    const int n = lane & 15, q4 = lane >> 4;
    // scores on the matrix cores: wave w takes keys 16w..16w+15; A = q (16 head rows, zero past
    // the group), B = the keys, K = the 128 dimensions in four steps. bf16 products are exact in
    // the fp32 accumulator.
    {
      const int key = 16 * wave + n;
      const uint4 *qrow = qs + n * kKeyStrideU4;
      const uint4 *krow = ks + key * kKeyStrideU4;
      f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < kHeadDim / 32; ++st) {
        const uint4 a = qrow[4 * st + q4], b = krow[4 * st + q4];
        sc = mfma_bf16(dwordx4{a.x, a.y, a.z, a.w}, dwordx4{b.x, b.y, b.z, b.w}, sc);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int h = 4 * q4 + r;
        if (h < group) probs[h][key] = key < count ? sc[r] * scale : -INFINITY;
      }
    }
    __syncthreads();

    // per query head: max, exp, sum (one wave per head, one lane per key); the probabilities are
    // kept as bf16 hi + lo (hi + lo = p to 16 significant bits) for the PV product
    for (int g = wave; g < group; g += 4) {
      const float a = probs[g][lane];
      const float m = wave_max(a);
      const float pa = expf(a - m);
      const uint16_t hi = to_bf(pa);
      pb[0][g][lane] = hi;
      pb[1][g][lane] = to_bf(pa - bf(hi));
      const float l = wave_sum(pa);
      if (lane == 0) {
        stats[g][0] = m;
        stats[g][1] = l;
      }
    }
    __syncthreads();

    // o[g][d] = sum_j p[g][j] v[j][d] on the matrix cores: wave w takes dimensions 32w..32w+31
    // (two 16-wide tiles); A = p as hi and lo (16 head rows), B = the transposed values, K = the
    // 64 keys in two steps. Keys past the position have p = 0 and zeroed values.
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int d = 32 * wave + 16 * t + n;
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < kChunk / 32; ++st) {
        const int k0 = 32 * st + 8 * q4;
        const uint4 b = *reinterpret_cast<const uint4 *>(&vt[vt_index(d, k0)]);
        const uint4 ah = *reinterpret_cast<const uint4 *>(&pb[0][n][k0]);
        const uint4 al = *reinterpret_cast<const uint4 *>(&pb[1][n][k0]);
        const dwordx4 bv = {b.x, b.y, b.z, b.w};
        acc = mfma_bf16(dwordx4{ah.x, ah.y, ah.z, ah.w}, bv, acc);
        acc = mfma_bf16(dwordx4{al.x, al.y, al.z, al.w}, bv, acc);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int h = 4 * q4 + r;
        if (h < group) out[(size_t)h * (kHeadDim + 2) + d] = acc[r];
      }
    }
    if (tid < group) {
      out[(size_t)tid * (kHeadDim + 2) + kHeadDim] = stats[tid][0];
      out[(size_t)tid * (kHeadDim + 2) + kHeadDim + 1] = stats[tid][1];
    }
  } else {
    // chunk past the position: an empty partial for the merge kernel
    for (int i = tid; i < group * (kHeadDim + 2); i += 256) out[i] = (i % (kHeadDim + 2)) == kHeadDim ? -INFINITY : 0.f;
  }
}

// Merge the chunks of one query head (block = head, thread = dimension) into bf16 output.
// The loads of the common case go out at once -- this thread's chunk statistics and its
// dimension's output of the first kHeld chunks (4096 positions) -- so the merge waits for memory
// once; chunks past kHeld are read eight at a time. The sums run over the chunks in the same
// order either way: acc[c % 4] for the chunks below the last multiple of four, the rest into
// acc[0], then ((acc0 + acc1) + (acc2 + acc3)) / total.
constexpr int kMaxChunks = 1024;
__global__ __launch_bounds__(128) void decode_attention_combine_kernel(const float *partials, int group, int chunks,
                                                                       uint16_t *out) {
  constexpr int kHeld = 64;
  constexpr int kPerThread = kMaxChunks / 128;
  __shared__ float weight[kMaxChunks];
  __shared__ float red[2];
  const int head = blockIdx.x;
  const int kv = head / group, g = head % group;
  const int dd = threadIdx.x;
  const float *base = partials + ((size_t)kv * chunks * group + g) * (kHeadDim + 2);
  const uint32_t step = (uint32_t)group * (kHeadDim + 2);  // floats between chunks
  auto at = [&](int c, int e) { return base[(uint32_t)min(c, chunks - 1) * step + e]; };
  float o[kHeld];
#pragma unroll
  for (int i = 0; i < kHeld; ++i) o[i] = at(i, dd);
  float mv[kPerThread], lv[kPerThread];
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    mv[u] = at(dd + 128 * u, kHeadDim);
    lv[u] = at(dd + 128 * u, kHeadDim + 1);
  }
  float m = -INFINITY;
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) m = dd + 128 * u < chunks ? fmaxf(m, mv[u]) : m;
  m = wave_max(m);
  if ((dd & 63) == 0) red[dd >> 6] = m;
  __syncthreads();
  m = fmaxf(red[0], red[1]);
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    const int c = dd + 128 * u;
    if (c < chunks) {
      const float w = mv[u] == -INFINITY ? 0.f : expf(mv[u] - m);
      weight[c] = w;
      total = __builtin_fmaf(lv[u], w, total);
    }
  }
  total = wave_sum(total);
  if ((dd & 63) == 0) red[dd >> 6] = total;
  __syncthreads();
  total = red[0] + red[1];
  const int main_end = chunks & ~3;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  auto add = [&](int c, float v) {
    const float w = weight[min(c, chunks - 1)];
    if (c < main_end) acc[c & 3] = __builtin_fmaf(v, w, acc[c & 3]);
    else if (c < chunks) acc[0] = __builtin_fmaf(v, w, acc[0]);
  };
#pragma unroll
  for (int i = 0; i < kHeld; ++i) add(i, o[i]);
  for (int c0 = kHeld; c0 < chunks; c0 += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = at(c0 + u, dd);
#pragma unroll
    for (int u = 0; u < 8; ++u) add(c0 + u, v[u]);
  }
  out[(size_t)head * kHeadDim + dd] = to_bf(((acc[0] + acc[1]) + (acc[2] + acc[3])) / total);
}

// Causal self-attention of a prompt: query tokens 0..T-1 against keys 0..T-1 (the prompt's own
// cache rows), grouped-query, head_dim 128. Block (query block of 64, head), heaviest query blocks
// first, HALVES sets of 4 waves: the waves of half hf take the key blocks kb = hf, hf + HALVES, ...
// up to the diagonal (with two halves a query block's chain of dependent key blocks is half as
// long, for grids too small to fill the GPU); wave w of a half owns queries 64*qb + 16w .. +15.
// For each of its key blocks of 64 keys: the block's keys (padded rows) and values (transposed:
// lane l loads dimensions 2l, 2l+1 of eight consecutive keys, one coalesced 256-byte key row per
// load, and writes them as two 8-key runs) go to the half's LDS tiles, staged through registers
// one of the half's blocks ahead; scores S = q k^T on the matrix cores (bf16 products, fp32 sums),
// scaled by scale*log2(e) and masked causally on the diagonal block; an online softmax in fp32 with
// exp2 (running max m and sum l per query; row reductions over the 16 lanes of a DPP row), the
// output rescaled by exp2(m_old - m_new); the probabilities rounded to bf16 (their rounded values
// summed into l) and multiplied by the values on the matrix cores (fp32 sums). With two halves
// their (m, l, O) meet in LDS at the end: O = O0 exp2(m0 - M) + O1 exp2(m1 - M) and likewise l,
// M = max(m0, m1). out = bf16(O / l). Values of keys past the prompt are zeroed, so stale cache
// rows never reach the sums.
constexpr int kPromptQueries = 64;


constexpr int kKeyTileBytes = kChunk * kKeyStrideU4 * 16;   // keys [key][128] bf16, padded rows
constexpr int kValueTileBytes = kHeadDim * kChunk * 2;      // values [dim][key] bf16 (vt_index)
constexpr int kMergeFloats = 4 + 4 + 32;                    // m[4], l[4], O[8][4] of a lane

template <int HALVES>
__global__ __launch_bounds__(256 * HALVES, HALVES == 1 ? 2 : 1) void prefill_attention_kernel(
    const uint16_t *q, int64_t q_stride, const uint16_t *k_cache, const uint16_t *v_cache, int tokens, int group,
    int64_t max_ctx, float scale, uint16_t *out, int64_t out_stride) {
  // Per half: a key tile and a value tile; after the K loop the same bytes carry half 1's (m, l, O).
  __shared__ __align__(16) char tiles[HALVES * (kKeyTileBytes + kValueTileBytes)];
  __shared__ __align__(16) uint16_t ps[4 * HALVES][16][kPRow];  // per wave: probabilities [query][key] bf16
  static_assert(HALVES == 1 || 4 * kMergeFloats * 64 * 4 <= HALVES * (kKeyTileBytes + kValueTileBytes), "merge area");
  const int qb = (int)gridDim.x - 1 - (int)blockIdx.x, head = blockIdx.y, kv = head / group;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  // half, wave within it, thread within it (compile-time constants with one half)
  const int hf = HALVES == 1 ? 0 : wave >> 2, wq = HALVES == 1 ? wave : wave & 3, ht = HALVES == 1 ? tid : tid & 255;
  uint4 *ks = reinterpret_cast<uint4 *>(tiles + hf * (kKeyTileBytes + kValueTileBytes));
  uint16_t *vt = reinterpret_cast<uint16_t *>(tiles + hf * (kKeyTileBytes + kValueTileBytes) + kKeyTileBytes);
  const int n = lane & 15, q4 = lane >> 4;
  const int q0 = qb * kPromptQueries + 16 * wq;  // this wave's first query
  const float sl2 = scale * 1.44269504088896340736f;  // scores in log2 units
  // q as MFMA A operands: row n = query q0 + n (clamped into the prompt), dimensions 32 st + 8 q4 ..
  dwordx4 qa[4];
  {
    const uint16_t *qr = q + (size_t)min(q0 + n, tokens - 1) * q_stride + (size_t)head * kHeadDim;
#pragma unroll
    for (int st = 0; st < 4; ++st) qa[st] = *reinterpret_cast<const dwordx4 *>(qr + 32 * st + 8 * q4);
  }
  // (32-bit byte offsets from the head's base: a head's cache is well under 4 GiB)
  const char *kg = reinterpret_cast<const char *>(k_cache + (size_t)kv * max_ctx * kHeadDim);
  const char *vg = reinterpret_cast<const char *>(v_cache + (size_t)kv * max_ctx * kHeadDim);
  struct Block {
    dwordx4 k[4];      // keys: 16-byte pieces idx = u * 256 + ht (key idx / 16, dimensions 8 (idx % 16) ..)
    uint32_t v[16];    // values: dimensions 2 lane, 2 lane + 1 of keys 8 (2 wq + j / 8) + j % 8
  };
  // Blocks past the diagonal are never loaded (the clamp keeps every address inside the cache).
  auto load_block = [&](Block &b, int kb) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int idx = u * 256 + ht;
      const uint32_t row = (uint32_t)min((int64_t)(kb * kChunk + idx / kRowU4), max_ctx - 1);
      b.k[u] = *reinterpret_cast<const dwordx4 *>(kg + (row * kRowU4 + idx % kRowU4) * 16u);
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t row = (uint32_t)min((int64_t)(kb * kChunk + 16 * wq + j), max_ctx - 1);
      b.v[j] = *reinterpret_cast<const uint32_t *>(vg + (row * kHeadDim + 2 * lane) * 2u);
    }
  };
  float m[4], l[4];  // running max (log2 units) and sum of the lane's rows, queries q0 + 4 q4 + r
  f32x4_t o[8];      // o[dt][r] = O[query q0 + 4 q4 + r][dimension 16 dt + n]
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.f;
  }
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // One turn: the half's block kb = HALVES * it + hf from `blk`, whose registers then take the
  // half's next block (loaded while this one is multiplied). Every half runs every turn (the
  // barriers are workgroup-wide); a half whose blocks have run out idles through it.
  auto turn = [&](int it, Block &blk) __attribute__((always_inline)) {
    const int kb = HALVES * it + hf;
    const bool active = HALVES == 1 || kb <= qb;  // one half runs every block up to the diagonal
    __syncthreads();  // the previous block's tiles are no longer read
    if (active) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int idx = u * 256 + ht;
        reinterpret_cast<dwordx4 *>(ks)[(idx / kRowU4) * kKeyStrideU4 + idx % kRowU4] = blk.k[u];
      }
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int key0 = 16 * wq + 8 * half;  // eight keys of this thread's run
        uint32_t w[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) w[j] = kb * kChunk + key0 + j < tokens ? blk.v[8 * half + j] : 0u;
        const uint4 lo = make_uint4(__builtin_amdgcn_perm(w[1], w[0], 0x05040100u), __builtin_amdgcn_perm(w[3], w[2], 0x05040100u),
                                    __builtin_amdgcn_perm(w[5], w[4], 0x05040100u), __builtin_amdgcn_perm(w[7], w[6], 0x05040100u));
        const uint4 hi = make_uint4(__builtin_amdgcn_perm(w[1], w[0], 0x07060302u), __builtin_amdgcn_perm(w[3], w[2], 0x07060302u),
                                    __builtin_amdgcn_perm(w[5], w[4], 0x07060302u), __builtin_amdgcn_perm(w[7], w[6], 0x07060302u));
        *reinterpret_cast<uint4 *>(&vt[vt_index(2 * lane, key0)]) = lo;
        *reinterpret_cast<uint4 *>(&vt[vt_index(2 * lane + 1, key0)]) = hi;
      }
    }
    __syncthreads();
    if (active && kb + HALVES <= qb) load_block(blk, kb + HALVES);  // in flight while this block is multiplied
    float alpha[4];
    if (active) {
      // scores of sub-tile s (keys 16 s .. 16 s + 15 of the block): sc[s][r] = S[query q0+4q4+r][key 16s+n]
      f32x4_t sc[4];
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const uint4 *krow = ks + (16 * s4 + n) * kKeyStrideU4;
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const uint4 b = krow[4 * st + q4];
          acc = mfma_bf16(qa[st], dwordx4{b.x, b.y, b.z, b.w}, acc);
        }
        sc[s4] = acc;
      }
      const bool diagonal = kb == qb;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float mx = -INFINITY;
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
          const int key = kb * kChunk + 16 * s4 + n, query = q0 + 4 * q4 + r;
          float v = sc[s4][r] * sl2;
          if (diagonal && (key > query || key >= tokens)) v = -INFINITY;
          sc[s4][r] = v;
          mx = fmaxf(mx, v);
        }
        // Every row has an unmasked key in every block up to the diagonal (key 64 kb <= query), so
        // the running max is finite from a half's first block on.
        const float mnew = fmaxf(m[r], row16_max(mx));
        alpha[r] = __builtin_amdgcn_exp2f(m[r] - mnew);
        m[r] = mnew;
        float rs = 0.f;
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
          const uint16_t pb = to_bf(__builtin_amdgcn_exp2f(sc[s4][r] - mnew));
          ps[wave][4 * q4 + r][16 * s4 + n] = pb;
          rs += bf(pb);
        }
        l[r] = l[r] * alpha[r] + row16_sum(rs);
      }
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) o[dt][r] *= alpha[r];
    }
    __syncthreads();  // the probabilities are in LDS
    if (active) {
      // O += P V: A = the probabilities (row n, keys 32 kst + 8 q4 ..), B = the transposed values
#pragma unroll
      for (int kst = 0; kst < kChunk / 32; ++kst) {
        const uint4 a = *reinterpret_cast<const uint4 *>(&ps[wave][n][32 * kst + 8 * q4]);
        const dwordx4 av = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const uint4 b = *reinterpret_cast<const uint4 *>(&vt[vt_index(16 * dt + n, 32 * kst + 8 * q4)]);
          o[dt] = mfma_bf16(av, dwordx4{b.x, b.y, b.z, b.w}, o[dt]);
        }
      }
    }
  };
  const int turns = (qb + HALVES) / HALVES;
  Block cur;
  if (hf <= qb) load_block(cur, hf);
  for (int it = 0; it < turns; ++it) turn(it, cur);

  if constexpr (HALVES == 2) {
    // Half 1 hands its (m, l, O) to half 0 through the tile bytes ([wq][item][lane] floats); a half
    // that processed no block hands m = -inf, l = 0, O = 0, which the merge weighs by zero.
    __syncthreads();  // every tile read is done
    float *mg = reinterpret_cast<float *>(tiles) + wq * kMergeFloats * 64 + lane;
    if (hf == 1) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        mg[r * 64] = m[r];
        mg[(4 + r) * 64] = l[r];
      }
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) mg[(8 + 4 * dt + r) * 64] = o[dt][r];
    }
    __syncthreads();
    if (hf == 1) return;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float m1 = mg[r * 64], l1 = mg[(4 + r) * 64];
      const float mm = fmaxf(m[r], m1);  // m[r] is finite: half 0 processed key block 0
      const float a0 = __builtin_amdgcn_exp2f(m[r] - mm), a1 = __builtin_amdgcn_exp2f(m1 - mm);
      l[r] = l[r] * a0 + l1 * a1;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) o[dt][r] = o[dt][r] * a0 + mg[(8 + 4 * dt + r) * 64] * a1;
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int query = q0 + 4 * q4 + r;
    if (query >= tokens) continue;
    const float inv = 1.0f / l[r];
    uint16_t *dst = out + (size_t)query * out_stride + (size_t)head * kHeadDim + n;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) dst[16 * dt] = to_bf(o[dt][r] * inv);
  }
}

// Greedy next token of a dense bf16 lm_head W [vocab][hidden] for one hidden state x [hidden]:
// token = the first v with the largest bf16(sum_k x[k] W[v][k]) (fp32 sums), as argmax over the
// bf16 logits of a linear layer picks it. First pass: workgroup b takes a contiguous range of
// rows; its waves take four rows at a time, sixteen lanes per row streaming the row in 16-byte
// chunks (chunk 16c + lane of the row; x as fp32 in LDS), four accumulators per lane summed in a
// fixed order, then over the row's sixteen lanes by DPP. Each lane group keeps its best (value,
// row); the workgroup's best goes to the partials. Second pass: one workgroup reduces those. The
// order (larger value, then smaller row) is total, so the result does not depend on the
// reduction order. NaN logits are not ranked. Optionally the bf16 logits are written too.
constexpr int kHeadThreads = 256;
constexpr int kHeadBlocks = 1024;  // first-pass workgroups: partials of kHeadBlocks (value, row)

__device__ __forceinline__ bool head_better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

__global__ __launch_bounds__(kHeadThreads) void lm_head_argmax_kernel(const uint16_t *w, int64_t vocab, int hidden,
                                                                      const uint16_t *x, uint16_t *logits,
                                                                      float *part_val, int *part_idx) {
  extern __shared__ float xs[];  // x as fp32 [hidden]
  __shared__ float wave_val[kHeadThreads / 64];
  __shared__ int wave_idx[kHeadThreads / 64];
  for (int i = threadIdx.x; i < hidden / 8; i += kHeadThreads) {
    const uint4 v = reinterpret_cast<const uint4 *>(x)[i];
    reinterpret_cast<float4 *>(xs)[2 * i] = make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xFFFF0000u),
                                                        __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xFFFF0000u));
    reinterpret_cast<float4 *>(xs)[2 * i + 1] = make_float4(__uint_as_float(v.z << 16), __uint_as_float(v.z & 0xFFFF0000u),
                                                            __uint_as_float(v.w << 16), __uint_as_float(v.w & 0xFFFF0000u));
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, grp = lane >> 4, l16 = lane & 15;
  const int64_t per = (vocab + gridDim.x - 1) / gridDim.x;
  const int64_t v0 = (int64_t)blockIdx.x * per, v1 = min(vocab, v0 + per);
  const int chunks = hidden / 128;  // 16-byte chunks of a row per lane (hidden % 128 == 0)
  float best = -INFINITY;
  int best_row = 0x7FFFFFFF;
  for (int64_t base = v0; base < v1; base += 16) {
    const int64_t row = base + 4 * wave + grp;
    const bool valid = row < v1;
    const dwordx4 *wr = reinterpret_cast<const dwordx4 *>(w + (size_t)min(row, v1 - 1) * hidden) + l16;
    const float4 *xr = reinterpret_cast<const float4 *>(xs) + 2 * l16;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    auto madd = [&](const dwordx4 &q, int c) {
      const float4 a = xr[32 * c], b = xr[32 * c + 1];
      const uint32_t wq[4] = {q[0], q[1], q[2], q[3]};
      const float xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[e] = __builtin_fmaf(__uint_as_float(wq[e] << 16), xv[2 * e], acc[e]);
        acc[e] = __builtin_fmaf(__uint_as_float(wq[e] & 0xFFFF0000u), xv[2 * e + 1], acc[e]);
      }
    };
    constexpr int kBatch = 8;  // loads in flight per lane, issued before the first multiply
    int c0 = 0;
    for (; c0 + kBatch <= chunks; c0 += kBatch) {
      dwordx4 q[kBatch];  // streamed once: nontemporal
#pragma unroll
      for (int u = 0; u < kBatch; ++u) q[u] = __builtin_nontemporal_load(wr + 16 * (c0 + u));
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < kBatch; ++u) madd(q[u], c0 + u);
    }
    for (; c0 < chunks; ++c0) madd(__builtin_nontemporal_load(wr + 16 * c0), c0);
    const float total = row16_sum((acc[0] + acc[1]) + (acc[2] + acc[3]));
    const uint16_t bits = to_bf(total);
    if (valid) {
      if (logits && l16 == 0) logits[row] = bits;
      const float value = bf(bits);
      if (head_better(value, (int)row, best, best_row)) {
        best = value;
        best_row = (int)row;
      }
    }
  }
  // The wave's four lane groups, then the workgroup's waves.
#pragma unroll
  for (int off = 16; off < 64; off <<= 1) {
    const float ov = __shfl_xor(best, off);
    const int oi = __shfl_xor(best_row, off);
    if (head_better(ov, oi, best, best_row)) {
      best = ov;
      best_row = oi;
    }
  }
  if (lane == 0) {
    wave_val[wave] = best;
    wave_idx[wave] = best_row;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < kHeadThreads / 64; ++i)
      if (head_better(wave_val[i], wave_idx[i], best, best_row)) {
        best = wave_val[i];
        best_row = wave_idx[i];
      }
    part_val[blockIdx.x] = best;
    part_idx[blockIdx.x] = best_row;
  }
}

__global__ __launch_bounds__(kHeadThreads) void lm_head_argmax_final_kernel(const float *part_val, const int *part_idx,
                                                                            int parts, int64_t *token) {
  __shared__ float wave_val[kHeadThreads / 64];
  __shared__ int wave_idx[kHeadThreads / 64];
  float best = -INFINITY;
  int best_row = 0x7FFFFFFF;
  for (int i = threadIdx.x; i < parts; i += kHeadThreads)
    if (head_better(part_val[i], part_idx[i], best, best_row)) {
      best = part_val[i];
      best_row = part_idx[i];
    }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float ov = __shfl_xor(best, off);
    const int oi = __shfl_xor(best_row, off);
    if (head_better(ov, oi, best, best_row)) {
      best = ov;
      best_row = oi;
    }
  }
  if ((threadIdx.x & 63) == 0) {
    wave_val[threadIdx.x >> 6] = best;
    wave_idx[threadIdx.x >> 6] = best_row;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < kHeadThreads / 64; ++i)
      if (head_better(wave_val[i], wave_idx[i], best, best_row)) {
        best = wave_val[i];
        best_row = wave_idx[i];
      }
    // every row's logit was NaN: row 0
    token[0] = best_row == 0x7FFFFFFF ? 0 : (int64_t)best_row;
  }
}

// out[r][c] = bf16(silu(g) * u) with g = gu[r][c], u = gu[r][inter + c], in fp32.
__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t *gu, int64_t rows, int64_t inter, uint16_t *out) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;   // one group of 8 columns
  const int64_t groups = inter / 8;
  if (idx >= rows * groups) return;
  const int64_t r = idx / groups, c = (idx % groups) * 8;
  const uint4 gv = *reinterpret_cast<const uint4 *>(gu + r * 2 * inter + c);
  const uint4 uv = *reinterpret_cast<const uint4 *>(gu + r * 2 * inter + inter + c);
  *reinterpret_cast<uint4 *>(out + r * inter + c) = swiglu8(gv, uv);
}

// Rotary embedding in the "rotate half" form of Hugging Face's Llama/Qwen2 models, with their
// bf16 rounding steps: for the head row x of token t (halves x1 = x[:d/2], x2 = x[d/2:]) and that
// token's cos/sin rows, out = bf16(bf16(x * cos) + bf16(rotate_half(x) * sin)), rotate_half(x) =
// [-x2, x1]: each bf16 product exact in fp32 then rounded, the sum in fp32 then rounded, which is
// what torch's bf16 elementwise kernels compute for q * cos + rotate_half(q) * sin. Block (t, r):
// row r of token t, query heads then key heads; thread i handles positions i and i + d/2.
__global__ __launch_bounds__(256) void rope_rotate_half_kernel(const uint16_t *q, const uint16_t *k, int heads,
                                                               int kv_heads, int dim, const uint16_t *cos,
                                                               const uint16_t *sin, uint16_t *q_out,
                                                               uint16_t *k_out) {
  const int64_t t = blockIdx.x;
  const int r = blockIdx.y;
  const int i = threadIdx.x, half = dim / 2;
  const bool is_q = r < heads;
  const int64_t row = is_q ? t * heads + r : t * kv_heads + (r - heads);
  const uint16_t *x = (is_q ? q : k) + row * dim;
  uint16_t *o = (is_q ? q_out : k_out) + row * dim;
  const uint16_t *c = cos + t * dim, *s = sin + t * dim;
  const float x1 = bf(x[i]), x2 = bf(x[i + half]);
  const float lo = bf(to_bf(x1 * bf(c[i]))) + bf(to_bf(-x2 * bf(s[i])));
  const float hi = bf(to_bf(x2 * bf(c[i + half]))) + bf(to_bf(x1 * bf(s[i + half])));
  o[i] = to_bf(lo);
  o[i + half] = to_bf(hi);
}

// One token's k and v rows (kv_heads x dim bf16 each) into a Hugging Face static cache [kv_heads][max_len][dim]
// at row *length, then *length += 1: the index copies and the length update of its update() in one
// block. Every thread reads the length before thread 0 advances it (the barrier orders the two). A
// full cache (length >= max_len) is left as it is, length included.
__global__ __launch_bounds__(256) void kv_append_kernel(const uint16_t *k, const uint16_t *v, int kv_heads, int dim,
                                                        uint16_t *keys, uint16_t *values, int64_t max_len,
                                                        int64_t *length) {
  const int64_t pos = *length;
  __syncthreads();
  if (pos < 0 || pos >= max_len) return;
  for (int i = threadIdx.x; i < kv_heads * dim; i += blockDim.x) {
    const int h = i / dim, j = i - h * dim;
    const size_t at = ((size_t)h * max_len + pos) * dim + j;
    keys[at] = k[i];
    values[at] = v[i];
  }
  if (threadIdx.x == 0) *length = pos + 1;
}

}  // namespace

hipError_t launch_add_rmsnorm(float *h, const uint16_t *delta, const uint16_t *weight, float eps, uint16_t *out,
                              int64_t rows, int hidden, hipStream_t stream) {
  hipLaunchKernelGGL((add_rmsnorm_kernel<false, 0>), dim3((unsigned)rows), dim3(kNormThreads), 0, stream, h, delta, SplitSource{},
                     weight, eps, out, hidden);
  return hipGetLastError();
}

hipError_t launch_add_rmsnorm_bf16(const uint16_t *residual, const uint16_t *delta, const uint16_t *weight, float eps,
                                   uint16_t *sum_out, uint16_t *out, int64_t rows, int hidden, hipStream_t stream) {
  hipLaunchKernelGGL(add_rmsnorm_bf16_kernel, dim3((unsigned)rows), dim3(kNormThreads), 0, stream, residual, delta, weight,
                     eps, sum_out, out, hidden);
  return hipGetLastError();
}

hipError_t launch_add_rmsnorm_split(float *h, const SplitSource &delta, const uint16_t *weight, float eps, uint16_t *out,
                                    int64_t rows, int hidden, hipStream_t stream) {
  auto launch = [&](auto ks) {
    hipLaunchKernelGGL((add_rmsnorm_kernel<true, decltype(ks)::value>), dim3((unsigned)rows), dim3(kNormThreads), 0, stream,
                       h, nullptr, delta, weight, eps, out, hidden);
  };
  // Eight splits (the 3B-class down GEMV, one token or a 512-token prompt) also read loop-free.
  if (delta.ks == 8) launch(std::integral_constant<int, 8>{});
  else with_split_count(delta.ks, launch);
  return hipGetLastError();
}

hipError_t launch_rope_cache(const uint16_t *qkv, int64_t stride, int64_t tokens, const int64_t *positions,
                             const float *cos_t, const float *sin_t, int heads, int kv_heads, int d, uint16_t *q_out,
                             uint16_t *k_cache, uint16_t *v_cache, int64_t max_ctx, hipStream_t stream) {
  hipLaunchKernelGGL(rope_cache_kernel<false>, dim3((unsigned)tokens, heads + 2 * kv_heads), dim3(d / 2), 0, stream, qkv,
                     SplitSource{}, stride, positions, cos_t, sin_t, heads, kv_heads, d, q_out, k_cache, v_cache, max_ctx);
  return hipGetLastError();
}

hipError_t launch_rope_cache_split(const SplitSource &qkv, int64_t tokens, const int64_t *positions, const float *cos_t,
                                   const float *sin_t, int heads, int kv_heads, int d, uint16_t *q_out,
                                   uint16_t *k_cache, uint16_t *v_cache, int64_t max_ctx, hipStream_t stream) {
  hipLaunchKernelGGL(rope_cache_kernel<true>, dim3((unsigned)tokens, heads + 2 * kv_heads), dim3(d / 2), 0, stream,
                     nullptr, qkv, 0, positions, cos_t, sin_t, heads, kv_heads, d, q_out, k_cache, v_cache, max_ctx);
  return hipGetLastError();
}

int decode_attention_chunks(int64_t length) { return (int)((length + kChunk - 1) / kChunk); }

bool decode_attention_supported(int heads, int kv_heads, int head_dim) {
  return head_dim == kHeadDim && kv_heads > 0 && heads % kv_heads == 0 && heads / kv_heads <= kMaxGroup;
}

int64_t decode_attention_max_length() { return (int64_t)kMaxChunks * kChunk; }

int64_t decode_attention_workspace(int heads, int64_t length) {
  return (int64_t)decode_attention_chunks(length) * heads * (kHeadDim + 2) * (int64_t)sizeof(float);
}

namespace {
// combine false: the chunk partials are left for a GEMV that merges them (GemvParams::attn).
template <bool ROPE>
hipError_t launch_attention(const AttnInput &in, uint16_t *k_cache, uint16_t *v_cache, const int64_t *position,
                            int64_t length, int64_t max_ctx, float scale, float *partials, uint16_t *out,
                            hipStream_t stream, bool combine = true) {
  const int chunks = decode_attention_chunks(length);
  const int group = in.heads / in.kv_heads;
  auto launch = [&](auto ks) {
    hipLaunchKernelGGL((decode_attention_kernel<ROPE, decltype(ks)::value>), dim3(in.kv_heads, chunks), dim3(256), 0,
                       stream, in, k_cache, v_cache, position, group, max_ctx, scale, chunks, partials);
  };
  if constexpr (ROPE) with_split_count(in.split.ks, launch);
  else launch(std::integral_constant<int, 0>{});
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !combine) return e;
  hipLaunchKernelGGL(decode_attention_combine_kernel, dim3(in.heads), dim3(kHeadDim), 0, stream, partials, group, chunks, out);
  return hipGetLastError();
}
}  // namespace

bool prefill_attention_supported(int heads, int kv_heads, int head_dim) {
  return head_dim == kHeadDim && kv_heads > 0 && heads % kv_heads == 0;
}

hipError_t launch_prefill_attention(const uint16_t *q, int64_t q_stride, const uint16_t *k_cache,
                                    const uint16_t *v_cache, int64_t tokens, int heads, int kv_heads, int64_t max_ctx,
                                    float scale, uint16_t *out, int64_t out_stride, hipStream_t stream) {
  const dim3 grid((unsigned)((tokens + kPromptQueries - 1) / kPromptQueries), (unsigned)heads);
  // Two halves per query block where the 4-wave blocks would not give every CU one (16 heads at
  // 512 tokens: 18.8 -> 16.3 us); otherwise 4-wave blocks, two per CU (40 heads: 25.5 vs 32.6 us).
  int device = 0, cus = 0;
  if (hipGetDevice(&device) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
    return hipGetLastError();
  if ((int64_t)grid.x * grid.y <= cus)
    hipLaunchKernelGGL(prefill_attention_kernel<2>, grid, dim3(512), 0, stream, q, q_stride, k_cache, v_cache, (int)tokens,
                       heads / kv_heads, max_ctx, scale, out, out_stride);
  else
    hipLaunchKernelGGL(prefill_attention_kernel<1>, grid, dim3(256), 0, stream, q, q_stride, k_cache, v_cache, (int)tokens,
                       heads / kv_heads, max_ctx, scale, out, out_stride);
  return hipGetLastError();
}

hipError_t launch_decode_attention(const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                                   const int64_t *position, int64_t length, int heads, int kv_heads, int64_t max_ctx,
                                   float scale, float *partials, uint16_t *out, hipStream_t stream) {
  AttnInput in{};
  in.q = q;
  in.heads = heads;
  in.kv_heads = kv_heads;
  return launch_attention<false>(in, const_cast<uint16_t *>(k_cache), const_cast<uint16_t *>(v_cache), position, length,
                                 max_ctx, scale, partials, out, stream);
}

hipError_t launch_decode_attention_split(const SplitSource &qkv, const int64_t *position, const float *rope_row,
                                         int64_t length, int heads, int kv_heads,
                                         uint16_t *k_cache, uint16_t *v_cache, int64_t max_ctx, float scale,
                                         float *partials, uint16_t *out, hipStream_t stream) {
  AttnInput in{};
  in.split = qkv;
  in.rope_row = rope_row;
  in.heads = heads;
  in.kv_heads = kv_heads;
  return launch_attention<true>(in, k_cache, v_cache, position, length, max_ctx, scale, partials, out, stream);
}

hipError_t launch_decode_attention_split_partials(const SplitSource &qkv, const int64_t *position, const float *rope_row,
                                                  int64_t length, int heads, int kv_heads, uint16_t *k_cache,
                                                  uint16_t *v_cache, int64_t max_ctx, float scale, float *partials,
                                                  hipStream_t stream) {
  static_assert(kAttnRow == kHeadDim + 2 && kMergeMaxChunks <= 64, "the partials layout the GEMV merge reads");
  AttnInput in{};
  in.split = qkv;
  in.rope_row = rope_row;
  in.heads = heads;
  in.kv_heads = kv_heads;
  return launch_attention<true>(in, k_cache, v_cache, position, length, max_ctx, scale, partials, nullptr, stream,
                                false);
}

int64_t lm_head_argmax_workspace() { return (int64_t)kHeadBlocks * (int64_t)(sizeof(float) + sizeof(int)); }

hipError_t launch_lm_head_argmax(const uint16_t *weight, int64_t vocab, int hidden, const uint16_t *x, uint16_t *logits,
                                 void *workspace, int64_t *token, hipStream_t stream) {
  float *part_val = static_cast<float *>(workspace);
  int *part_idx = reinterpret_cast<int *>(part_val + kHeadBlocks);
  const int blocks = (int)std::min<int64_t>(kHeadBlocks, (vocab + 15) / 16);
  hipLaunchKernelGGL(lm_head_argmax_kernel, dim3(blocks), dim3(kHeadThreads), (size_t)hidden * sizeof(float), stream, weight,
                     vocab, hidden, x, logits, part_val, part_idx);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(lm_head_argmax_final_kernel, dim3(1), dim3(kHeadThreads), 0, stream, part_val, part_idx, blocks, token);
  return hipGetLastError();
}

hipError_t launch_rope_rotate_half(const uint16_t *q, const uint16_t *k, int64_t tokens, int heads, int kv_heads,
                                   int dim, const uint16_t *cos, const uint16_t *sin, uint16_t *q_out, uint16_t *k_out,
                                   hipStream_t stream) {
  hipLaunchKernelGGL(rope_rotate_half_kernel, dim3((unsigned)tokens, (unsigned)(heads + kv_heads)), dim3(dim / 2), 0,
                     stream, q, k, heads, kv_heads, dim, cos, sin, q_out, k_out);
  return hipGetLastError();
}

hipError_t launch_kv_append(const uint16_t *k, const uint16_t *v, int kv_heads, int dim, uint16_t *keys, uint16_t *values,
                            int64_t max_len, int64_t *length, hipStream_t stream) {
  hipLaunchKernelGGL(kv_append_kernel, dim3(1), dim3(256), 0, stream, k, v, kv_heads, dim, keys, values, max_len, length);
  return hipGetLastError();
}

hipError_t launch_swiglu(const uint16_t *gu, int64_t rows, int64_t inter, uint16_t *out, hipStream_t stream) {
  const int64_t threads = rows * (inter / 8);
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, gu, rows, inter, out);
  return hipGetLastError();
}

}  // namespace tx
