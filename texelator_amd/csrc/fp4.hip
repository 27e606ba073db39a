// MXFP4 staging and the block-scaled GEMM of the opt-in FP4 hybrid prefill (gfx950).
//
// Reference: texelator/runtime.py:66-131 (at 512 tokens, for the MLP shapes, quantize the
// activation and the decoded BC4 weight to FP4 and multiply them with torch._scaled_mm, bf16
// output) and its quantizers texelator/cuda/texelator_cuda.cu:1046-1152 (E2M1 values with the sign
// in bit 3, two per byte, low nibble first; one scale per group; the weight quantizer starts from
// the fp32 products palette * row scale). The reference's groups are NVFP4 (16 values, E4M3 scale
// max/6, a Blackwell-blocked scale layout). gfx950's block-scaled MFMA takes the OCP MX format
// instead, so this build quantizes to MXFP4: groups of 32 along K with one E8M0 scale
// 2^(e - 127), e = floor(log2(amax)) - 2 + 127 (clamped to [0, 254], 0 for an all-zero group), each
// value v * 2^(127 - e) rounded to E2M1 to nearest with ties to even and saturated at 6. Scales are
// stored row-major [rows][K/32]; packed values [rows][K/2].
//
// The GEMM, y[t][m] = bf16(sum_k deq(x)[t][k] deq(w)[m][k]) (+ the bf16 bias with a second
// rounding), runs v_mfma_scale_f32_32x32x64_f8f6f4 with both operands E2M1 (format 4): lane l of
// an operand holds row (or token) l % 32 and K elements 32*(l/32) .. +31 of the 64-wide step, 16
// bytes, and the E8M0 scale of exactly that group; fp32 accumulation.
#include "bc4_device.h"
#include "elementwise.h"
#include "kernels.h"

namespace tx {

namespace {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// E2M1 code of v (already scaled by the group's 2^(127 - e)): nearest magnitude of
// {0, 0.5, 1, 1.5, 2, 3, 4, 6}, ties to the even code, saturating at 6; bit 3 is v's sign.
__device__ __forceinline__ uint32_t e2m1(float v) {
  const float m = fabsf(v);
  const uint32_t code = (uint32_t)(m > 0.25f) + (uint32_t)(m >= 0.75f) + (uint32_t)(m > 1.25f) +
                        (uint32_t)(m >= 1.75f) + (uint32_t)(m > 2.5f) + (uint32_t)(m >= 3.5f) + (uint32_t)(m > 5.0f);
  return code | ((__float_as_uint(v) >> 31) << 3);
}

// E8M0 exponent of a group whose largest magnitude is amax: floor(log2(amax)) - 2 + 127 from
// amax's exponent field (0 for zero and subnormal maxima, as clamping gives).
__device__ __forceinline__ uint32_t group_exponent(float amax) {
  return (uint32_t)max((int)((__float_as_uint(amax) >> 23) & 0xFFu) - 2, 0);
}

// Quantize 32 values: 16 packed bytes (as four words) and the E8M0 exponent.
__device__ __forceinline__ uint32_t quantize32(const float (&v)[32], uint32_t (&packed)[4]) {
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
  const uint32_t e = group_exponent(amax);
  const float inv = __uint_as_float((254u - e) << 23);  // 2^(127 - e), exact
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) word |= e2m1(v[8 * w + j] * inv) << (4 * j);
    packed[w] = word;
  }
  return e;
}

// One thread per group of 32 activations (bf16, row-major [tokens][K]).
__global__ __launch_bounds__(256) void quantize_activation_kernel(const uint16_t *x, int64_t tokens, int K,
                                                                  uint8_t *packed, uint8_t *scales) {
  const int groups = K / 32;
  const int64_t index = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (index >= tokens * groups) return;
  const uint4 *src = reinterpret_cast<const uint4 *>(x + index * 32);
  float v[32];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint4 u = src[q];
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[8 * q + 2 * j] = bf((uint16_t)(w[j] & 0xFFFFu));
      v[8 * q + 2 * j + 1] = bf((uint16_t)(w[j] >> 16));
    }
  }
  uint32_t out[4];
  scales[index] = (uint8_t)quantize32(v, out);
  reinterpret_cast<uint4 *>(packed)[index] = make_uint4(out[0], out[1], out[2], out[3]);
}

// The 16 fp32 products palette * scale of one device block, in position order.
__device__ __forceinline__ void block_products(uint32_t a, uint32_t b, float scale, float *out) {
  const Palette pal = palette8(a, b);
#pragma unroll
  for (int p = 0; p < 16; ++p) {
    const uint32_t word = p < 8 ? a : b;
    const int c = p & 3;
    const uint32_t sel = (p & 4) ? (word >> (8 * c)) & 7u : (word >> (8 * c + 5)) & 7u;
    float value = pal.p[0];
#pragma unroll
    for (int s = 1; s < 8; ++s) value = sel == (uint32_t)s ? pal.p[s] : value;
    out[p] = value * scale;
  }
}

// One thread per 16-byte tile slot: two consecutive blocks of one row = one group of 32.
__global__ __launch_bounds__(256) void quantize_weight_kernel(const uint4 *tiles, const float *row_scales, int M, int K,
                                                              int RG, int CG, uint8_t *packed, uint8_t *scales) {
  const size_t slot = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (slot >= (size_t)RG * CG * 64) return;
  const int lane = slot & 63;
  const size_t tile = slot >> 6;
  const int g = (int)(tile / CG), c = (int)(tile % CG);
  const int row = g * kTileRows + (lane & 15);
  const int group = 4 * c + (lane >> 4);  // blocks 2*group, 2*group + 1
  const int groups = K / 32;
  if (row >= M || group >= groups) return;
  const uint4 cur = tiles[slot];
  const float scale = row_scales[row];
  float v[32];
  block_products(cur.x, cur.y, scale, v);
  block_products(cur.z, cur.w, scale, v + 16);
  uint32_t out[4];
  scales[(size_t)row * groups + group] = (uint8_t)quantize32(v, out);
  reinterpret_cast<uint4 *>(packed + (size_t)row * (K / 2))[group] = make_uint4(out[0], out[1], out[2], out[3]);
}

// Workgroup tile: 128 rows (wave w: rows 32w..32w+31) x 128 tokens (four 32-token blocks per
// wave), K in steps of 64. Rows and tokens past the matrix are clamped (computed, never stored).
__global__ __launch_bounds__(256) void fp4_gemm_kernel(const uint8_t *xq, const uint8_t *xs, const uint8_t *wq,
                                                       const uint8_t *ws, const uint16_t *bias, uint16_t *y,
                                                       int tokens, int M, int K) {
  constexpr int TB = 4;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r32 = lane & 31, h = lane >> 5;
  const int n0 = blockIdx.x * 128 + 32 * wave, t0 = blockIdx.y * 128;
  const int groups = K / 32;
  const size_t row_bytes = (size_t)K / 2;
  const int row = min(n0 + r32, M - 1);
  const uint8_t *wrow = wq + row * row_bytes + 16 * h;
  const uint8_t *wsc = ws + (size_t)row * groups + h;
  const uint8_t *xrow[TB];
  const uint8_t *xsc[TB];
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) {
    const int t = min(t0 + 32 * tb + r32, tokens - 1);
    xrow[tb] = xq + t * row_bytes + 16 * h;
    xsc[tb] = xs + (size_t)t * groups + h;
  }
  f32x16 acc[TB];
#pragma unroll
  for (int tb = 0; tb < TB; ++tb)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[tb][r] = 0.f;
  auto load = [&](int step, u32x4 &a, int &sa, u32x4 (&b)[TB], int (&sb)[TB]) {
    a = *reinterpret_cast<const u32x4 *>(wrow + 32 * (size_t)step);
    sa = wsc[2 * step];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      b[tb] = *reinterpret_cast<const u32x4 *>(xrow[tb] + 32 * (size_t)step);
      sb[tb] = xsc[tb][2 * step];
    }
  };
  const int steps = K / 64;
  u32x4 a, b[TB];
  int sa, sb[TB];
  load(0, a, sa, b, sb);
  for (int step = 0; step < steps; ++step) {
    u32x4 an, bn[TB];
    int san, sbn[TB];
    load(min(step + 1, steps - 1), an, san, bn, sbn);
    const i32x8 av = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0};
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      const i32x8 bv = {(int)b[tb].x, (int)b[tb].y, (int)b[tb].z, (int)b[tb].w, 0, 0, 0, 0};
      acc[tb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, acc[tb], 4, 4, 0, sa, 0, sb[tb]);
    }
    a = an;
    sa = san;
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      b[tb] = bn[tb];
      sb[tb] = sbn[tb];
    }
  }
  // acc[tb][r] = D[row 8(r/4) + 4h + r%4 of the wave's 32][token 32 tb + r32]
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) {
    const int t = t0 + 32 * tb + r32;
    if (t >= tokens) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int n = n0 + 8 * (r / 4) + 4 * h + (r % 4);
      if (n >= M) continue;
      float out = bf(to_bf(acc[tb][r]));
      if (bias) out += bf(bias[n]);
      y[(size_t)t * M + n] = to_bf(out);
    }
  }
}

}  // namespace

hipError_t launch_quantize_activation_fp4(const uint16_t *x, int64_t tokens, int K, uint8_t *packed, uint8_t *scales,
                                          hipStream_t stream) {
  const int64_t groups = tokens * (K / 32);
  hipLaunchKernelGGL(quantize_activation_kernel, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, stream, x,
                     tokens, K, packed, scales);
  return hipGetLastError();
}

hipError_t launch_quantize_weight_fp4(const uint4 *tiles, const float *scales, int M, int K, int RG, int CG,
                                      uint8_t *packed, uint8_t *group_scales, hipStream_t stream) {
  const size_t slots = (size_t)RG * CG * 64;
  hipLaunchKernelGGL(quantize_weight_kernel, dim3((unsigned)((slots + 255) / 256)), dim3(256), 0, stream, tiles,
                     scales, M, K, RG, CG, packed, group_scales);
  return hipGetLastError();
}

hipError_t launch_fp4_gemm(const uint8_t *xq, const uint8_t *xs, const uint8_t *wq, const uint8_t *ws,
                           const uint16_t *bias, uint16_t *y, int tokens, int M, int K, hipStream_t stream) {
  const dim3 grid((unsigned)((M + 127) / 128), (unsigned)((tokens + 127) / 128));
  hipLaunchKernelGGL(fp4_gemm_kernel, grid, dim3(256), 0, stream, xq, xs, wq, ws, bias, y, tokens, M, K);
  return hipGetLastError();
}

}  // namespace tx
