// Elementwise device helpers shared by the decoder-layer kernels and the decode GEMV, so that a
// value computed in a fused kernel is bit-identical to the one a standalone kernel writes.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace tx {

__device__ __forceinline__ float bf(uint16_t v) { return __builtin_bit_cast(float, (uint32_t)v << 16); }

__device__ __forceinline__ float hf(uint16_t v) { return (float)__builtin_bit_cast(_Float16, v); }

// A 16-bit value (fp16 with F16, else bf16) widened to fp32.
template <bool F16>
__device__ __forceinline__ float half_bits_to_float(uint16_t v) {
  if constexpr (F16) return hf(v);
  else return bf(v);
}

// Round to bf16, nearest-even.
__device__ __forceinline__ uint16_t to_bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// Reductions over the 16 lanes of a DPP row (xor 1, xor 2, half-row mirror, row mirror): every
// lane of the row ends with the same value.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_mov<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_mov<0x141>(v));  // row_half_mirror
  return fmaxf(v, dpp_mov<0x140>(v));  // row_mirror
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x141>(v);
  return v + dpp_mov<0x140>(v);
}
__device__ __forceinline__ float lane_value(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
// Sum over the 64 lanes of a wave in one fixed tree: each 16-lane row by row16_sum, then the rows
// as (r0 + r1) + (r2 + r3). Every lane gets the result; no LDS round trip. A wave whose rows 1-3
// hold zeros gets row 0's sum exactly (adding +0 changes nothing for a sum of non-negative values).
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}
// Maximum over the 64 lanes of a wave (exact in any order).
__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

// SwiGLU of one pair in fp32: silu(g) * u.
__device__ __forceinline__ float swiglu_value(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// bf16(silu(g) * u) for 8 packed bf16 pairs.
__device__ __forceinline__ uint4 swiglu8(uint4 gv, uint4 uv) {
  const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
  uint32_t ow[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float a0 = swiglu_value(bf((uint16_t)(gw[e] & 0xFFFFu)), bf((uint16_t)(uw[e] & 0xFFFFu)));
    const float a1 = swiglu_value(bf((uint16_t)(gw[e] >> 16)), bf((uint16_t)(uw[e] >> 16)));
    ow[e] = (uint32_t)to_bf(a0) | ((uint32_t)to_bf(a1) << 16);
  }
  return make_uint4(ow[0], ow[1], ow[2], ow[3]);
}

// Output m of token t of a split-K GEMV: the fp32 partials [ks][tokens][Mp] summed in split
// order starting from split 0, plus the bf16 bias, rounded to bf16 (returned widened to fp32).
// The decode GEMV's own reduction uses this, so fused consumers reproduce its output bits.
// round_first: the prefill GEMM's epilogue instead -- the sum rounded to bf16 first, the bias
// added with a second rounding (prefill_reduce_kernel), so consumers of prefill partials
// reproduce its output bits.
struct SplitSource {
  const float *partials;
  const uint16_t *bias;  // [M] of the activation type (bf16, or fp16 with F16), or nullptr
  int ks, Mp, tokens;
  int round_first;
};

// split_sum for N columns m[i] of one token at once. The loads go out four splits at a time for
// every column (split index clamped to the last one, extra values unused) before the first add,
// so a consumer pays the memory latency once per four splits instead of once per split and
// column. The bias is read from a valid address whether or not there is one, and added last.
// KS > 0: the caller guarantees ks == KS, and the code has no loop, select or branch at all, so
// the compiler keeps the caller's own earlier loads where they were issued.
template <int N, bool F16 = false, int KS = 0>
__device__ __forceinline__ void split_sums(const SplitSource &s, int64_t token, const int64_t (&m)[N], float (&total)[N]) {
  const float *p = s.partials + (size_t)token * s.Mp;
  const size_t stride = (size_t)s.tokens * s.Mp;
  const uint16_t *bias = s.bias ? s.bias : reinterpret_cast<const uint16_t *>(s.partials);
  // 32-bit byte offsets from a uniform base (columns < 2^30), so each load needs one VGPR of
  // address instead of two
  uint32_t off4[N];
  uint16_t b[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    off4[i] = (uint32_t)m[i] * 4u;
    b[i] = *reinterpret_cast<const uint16_t *>(reinterpret_cast<const char *>(bias) + off4[i] / 2u);
    total[i] = 0.f;
  }
  auto load = [&](int k, int i) { return *reinterpret_cast<const float *>(reinterpret_cast<const char *>(p + (size_t)k * stride) + off4[i]); };
  if constexpr (KS > 0) {
    float v[KS][N];
#pragma unroll
    for (int k = 0; k < KS; ++k)
#pragma unroll
      for (int i = 0; i < N; ++i) v[k][i] = load(k, i);
    __builtin_amdgcn_sched_barrier(0);  // every load issued before the first add
#pragma unroll
    for (int i = 0; i < N; ++i) {
      total[i] = v[0][i];
#pragma unroll
      for (int k = 1; k < KS; ++k) total[i] += v[k][i];
    }
  } else {
    constexpr int kGroup = 4;
    for (int k0 = 0; k0 < s.ks; k0 += kGroup) {
      float v[kGroup][N];
#pragma unroll
      for (int u = 0; u < kGroup; ++u)
#pragma unroll
        for (int i = 0; i < N; ++i) v[u][i] = load(min(k0 + u, s.ks - 1), i);
#pragma unroll
      for (int u = 0; u < kGroup; ++u) {
        const int k = k0 + u;
#pragma unroll
        for (int i = 0; i < N; ++i) total[i] = k == 0 ? v[u][i] : (k < s.ks ? total[i] + v[u][i] : total[i]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    if (s.round_first) total[i] = F16 ? (float)(_Float16)total[i] : bf(to_bf(total[i]));
    total[i] = s.bias ? total[i] + half_bits_to_float<F16>(b[i]) : total[i];
  }
}

template <bool F16 = false>
__device__ __forceinline__ float split_sum(const SplitSource &s, int64_t token, int64_t m) {
  const int64_t cols[1] = {m};
  float total[1];
  split_sums<1, F16>(s, token, cols, total);
  return total[0];
}

__device__ __forceinline__ float split_value(const SplitSource &s, int64_t token, int64_t m) {
  return bf(to_bf(split_sum(s, token, m)));
}

}  // namespace tx
