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
struct SplitSource {
  const float *partials;
  const uint16_t *bias;  // [M] of the activation type (bf16, or fp16 with F16), or nullptr
  int ks, Mp, tokens;
};

template <bool F16 = false>
__device__ __forceinline__ float split_sum(const SplitSource &s, int64_t token, int64_t m) {
  const float *p = s.partials + (size_t)token * s.Mp + m;
  const size_t stride = (size_t)s.tokens * s.Mp;
  float total = p[0];
  for (int k = 1; k < s.ks; ++k) total += p[k * stride];
  if (s.bias) total += half_bits_to_float<F16>(s.bias[m]);
  return total;
}

__device__ __forceinline__ float split_value(const SplitSource &s, int64_t token, int64_t m) {
  return bf(to_bf(split_sum(s, token, m)));
}

}  // namespace tx
