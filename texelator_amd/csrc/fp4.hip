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
#include <type_traits>

#include "bc4_device.h"
#include "elementwise.h"
#include "kernels.h"

namespace tx {

namespace {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// E8M0 exponent of a group whose largest magnitude is amax: floor(log2(amax)) - 2 + 127 from
// amax's exponent field (0 for zero and subnormal maxima, as clamping gives).
__device__ __forceinline__ uint32_t group_exponent(float amax) {
  return (uint32_t)max((int)((__float_as_uint(amax) >> 23) & 0xFFu) - 2, 0);
}

// Two E2M1 codes (a in the low nibble, b in the high one) written into byte SEL of `word`. The
// E2M1 code of v (already multiplied by the group's 2^(127 - e)) is the nearest magnitude of
// {0, 0.5, 1, 1.5, 2, 3, 4, 6} with ties to the even code, saturating at 6, with v's sign in bit 3.
// v_cvt_scalef32_pk_fp4_f32 computes exactly that for v / scale (called here with scale 1):
// checked against the rule on ties, saturation, signed zeros, subnormals and random values under
// power-of-two scales, and the quantizer tests compare every code with the oracle.
template <int SEL>
__device__ __forceinline__ uint32_t e2m1_pair(uint32_t word, float a, float b) {
  return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, a, b, 1.0f, SEL);
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
    word = e2m1_pair<0>(word, v[8 * w] * inv, v[8 * w + 1] * inv);
    word = e2m1_pair<1>(word, v[8 * w + 2] * inv, v[8 * w + 3] * inv);
    word = e2m1_pair<2>(word, v[8 * w + 4] * inv, v[8 * w + 5] * inv);
    word = e2m1_pair<3>(word, v[8 * w + 6] * inv, v[8 * w + 7] * inv);
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

// One device block for the weight quantizer: its 8 palette products P[s] * scale (the fp32 values
// the 16 weights take), which of them the selectors use, and the selector words of positions
// 0-3, 4-7, 8-11, 12-15 (byte c = the position's palette slot).
struct BlockEntries {
  float q[8];
  uint32_t used;  // bit s: some position selects slot s
  uint32_t sel[4];
};

// With a palette table (LUT mode, probe layout) the 8 values come from the block's table row,
// as every other kernel of a LUT-mode handle reads them; otherwise they are computed.
__device__ __forceinline__ BlockEntries block_entries(uint32_t a, uint32_t b, float scale, const float4 *lut) {
  BlockEntries out;
  if (lut) {
    const float4 *r = lut + 2 * (size_t)palette_row(a, b);
    const float4 p03 = r[0], p47 = r[1];
    const float p[8] = {p03.x, p03.y, p03.z, p03.w, p47.x, p47.y, p47.z, p47.w};
#pragma unroll
    for (int s = 0; s < 8; ++s) out.q[s] = p[s] * scale;
  } else {
    const Palette pal = palette8(a, b);
#pragma unroll
    for (int s = 0; s < 8; ++s) out.q[s] = pal.p[s] * scale;
  }
  out.sel[0] = (a >> 5) & 0x07070707u;
  out.sel[1] = a & 0x07070707u;
  out.sel[2] = (b >> 5) & 0x07070707u;
  out.sel[3] = b & 0x07070707u;
  // one-hot byte per position (1 << slot, from the byte table 1, 2, 4, ..., 128), OR-folded
  uint32_t oh = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) oh |= perm(0x80402010u, 0x08040201u, out.sel[i]);
  oh |= oh >> 16;
  out.used = (oh | (oh >> 8)) & 0xFFu;
  return out;
}

// Largest magnitude among the used slots (the largest |weight| of the block), as float bits:
// for non-negative floats integer order is float order.
__device__ __forceinline__ uint32_t used_amax_bits(const BlockEntries &e) {
  uint32_t m = 0;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const uint32_t bits = __float_as_uint(e.q[s]) & 0x7FFFFFFFu;
    m = max(m, (e.used >> s) & 1u ? bits : 0u);
  }
  return m;
}

// The block's 16 weights as E2M1 nibbles (positions 0-15 -> bytes 0-7, even position in the low
// nibble): the 8 slot codes E2M1(q[s] * inv) from four paired conversions, then each position's
// code picked by byte permutes with its selector.
__device__ __forceinline__ void block_codes(const BlockEntries &e, float inv, uint32_t &lo, uint32_t &hi) {
  uint32_t t = 0;  // nibble s = code of slot s
  t = e2m1_pair<0>(t, e.q[0] * inv, e.q[1] * inv);
  t = e2m1_pair<1>(t, e.q[2] * inv, e.q[3] * inv);
  t = e2m1_pair<2>(t, e.q[4] * inv, e.q[5] * inv);
  t = e2m1_pair<3>(t, e.q[6] * inv, e.q[7] * inv);
  const uint32_t even = t & 0x0F0F0F0Fu;         // bytes: codes of slots 0, 2, 4, 6
  const uint32_t odd = (t >> 4) & 0x0F0F0F0Fu;   // bytes: codes of slots 1, 3, 5, 7
  const uint32_t t03 = perm(odd, even, 0x05010400u);  // byte s: code of slot s, s = 0..3
  const uint32_t t47 = perm(odd, even, 0x07030602u);  // slots 4..7
  uint32_t y[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t x = perm(t47, t03, e.sel[i]);  // codes of the four positions, one per byte
    y[i] = x | (x >> 4);                            // bytes 0 and 2: two positions each
  }
  lo = perm(y[1], y[0], 0x06040200u);
  hi = perm(y[3], y[2], 0x06040200u);
}

// One thread per 16-byte tile slot: two consecutive blocks of one row = one group of 32.
__global__ __launch_bounds__(256) void quantize_weight_kernel(const uint4 *tiles, const float *row_scales, const float4 *lut,
                                                              int M, int K, int RG, int CG, uint8_t *packed,
                                                              uint8_t *scales) {
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
  const BlockEntries b0 = block_entries(cur.x, cur.y, scale, lut);
  const BlockEntries b1 = block_entries(cur.z, cur.w, scale, lut);
  const uint32_t e = group_exponent(__uint_as_float(max(used_amax_bits(b0), used_amax_bits(b1))));
  const float inv = __uint_as_float((254u - e) << 23);  // 2^(127 - e), exact
  uint4 out;
  block_codes(b0, inv, out.x, out.y);
  block_codes(b1, inv, out.z, out.w);
  scales[(size_t)row * groups + group] = (uint8_t)e;
  reinterpret_cast<uint4 *>(packed + (size_t)row * (K / 2))[group] = out;
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

// Staged GEMM (K a multiple of 128): the same workgroup tile (128 rows x 128 tokens, wave w rows
// 32w..32w+31, four 32-token blocks per wave) and the same MFMAs in the same K order as
// fp4_gemm_kernel, so the same results, with the operands moved the way the matrix cores need:
//   * K runs in steps of 128 (MFMA chunks kc = 0, 1 of 64);
//   * the step's activations (128 tokens x 64 bytes) and their four scale bytes per token are
//     loaded once per workgroup (two 16-byte chunks and, for threads < 128, one token's scale
//     word per thread) and written to LDS at the end of the previous step; LDS row = token,
//     16-byte chunk c stored at c ^ ((token >> 2) & 3) so that the eight tokens of an LDS pass
//     fall on distinct banks;
//   * each wave's own weight rows go straight to registers (no sharing to gain);
//   * every load is issued kFp4Ahead steps before its use into a ring of register stages
//     (ordinary loads only, so the compiler's wait counts are exact) and the loop is unrolled over
//     the ring, so no stage is copied between registers.
constexpr int kFp4Step = 128;   // K per step
constexpr int kFp4Ahead = 3;    // steps between a load and the step that uses it
constexpr int kFp4Ring = 4;     // register stages (kFp4Ahead + 1)

template <int XC>
struct Fp4Stage {
  u32x4 w[2];    // this lane's weight operand of chunks 0 and 1
  uint32_t ws;   // the four scale bytes of this lane's weight row in the step
  u32x4 x[XC];   // the activation chunks this thread stages
  uint32_t xs;   // the scale word of the token this thread stages (threads < BT)
};

// TB token blocks of 32 per workgroup (every wave multiplies its 32 rows by all of them).
template <int TB>
__global__ __launch_bounds__(256) void fp4_gemm_staged_kernel(const uint8_t *xq, const uint8_t *xs, const uint8_t *wq,
                                                              const uint8_t *ws, const uint16_t *bias, uint16_t *y,
                                                              int tokens, int M, int K) {
  constexpr int BT = 32 * TB;
  constexpr int XC = BT * 4 / 256;  // 16-byte activation chunks staged per thread and step
  __shared__ __attribute__((aligned(16))) uint8_t xl0[BT * 64];
  __shared__ __attribute__((aligned(16))) uint8_t xl1[BT * 64];
  __shared__ uint32_t sl0[BT];
  __shared__ uint32_t sl1[BT];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r32 = lane & 31, h = lane >> 5;
  const int n0 = blockIdx.x * 128 + 32 * wave, t0 = blockIdx.y * BT;
  const int groups = K / 32;
  const size_t row_bytes = (size_t)K / 2;
  const int steps = K / kFp4Step;
  // This lane's weight row, and the two activation chunks (q = tid, tid + 256 of the 512 chunks
  // of a step) and the token scale word this thread stages.
  const int row = min(n0 + r32, M - 1);
  const uint8_t *wrow = wq + (size_t)row * row_bytes + 16 * h;
  const uint32_t *wsrow = reinterpret_cast<const uint32_t *>(ws + (size_t)row * groups);
  const uint8_t *xsrc[XC];
  int xdst[XC];
#pragma unroll
  for (int i = 0; i < XC; ++i) {
    const int q = (int)threadIdx.x + 256 * i;
    const int tok = q >> 2, c = q & 3;
    xsrc[i] = xq + (size_t)min(t0 + tok, tokens - 1) * row_bytes + 16 * c;
    xdst[i] = tok * 64 + 16 * (c ^ ((tok >> 2) & 3));
  }
  const uint32_t *xssrc =
      reinterpret_cast<const uint32_t *>(xs + (size_t)min(t0 + (int)(threadIdx.x % BT), tokens - 1) * groups);

  auto load = [&](Fp4Stage<XC> &st, int s) {
    s = min(s, steps - 1);
    st.w[0] = *reinterpret_cast<const u32x4 *>(wrow + 64 * (size_t)s);
    st.w[1] = *reinterpret_cast<const u32x4 *>(wrow + 64 * (size_t)s + 32);
    st.ws = wsrow[s];
#pragma unroll
    for (int i = 0; i < XC; ++i) st.x[i] = *reinterpret_cast<const u32x4 *>(xsrc[i] + 64 * (size_t)s);
    st.xs = threadIdx.x < BT ? xssrc[s] : 0u;
  };
  auto write = [&](uint8_t *xl, uint32_t *sl, const Fp4Stage<XC> &st) {
#pragma unroll
    for (int i = 0; i < XC; ++i) *reinterpret_cast<u32x4 *>(xl + xdst[i]) = st.x[i];
    if (threadIdx.x < BT) sl[threadIdx.x] = st.xs;
  };

  f32x16 acc[TB];
#pragma unroll
  for (int tb = 0; tb < TB; ++tb)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[tb][r] = 0.f;

  auto compute = [&](const uint8_t *xl, const uint32_t *sl, const Fp4Stage<XC> &st) {
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      const int tok = 32 * tb + r32;
      const uint32_t sw = sl[tok];
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const u32x4 b = *reinterpret_cast<const u32x4 *>(xl + tok * 64 + 16 * ((2 * kc + h) ^ ((tok >> 2) & 3)));
        const i32x8 av = {(int)st.w[kc].x, (int)st.w[kc].y, (int)st.w[kc].z, (int)st.w[kc].w, 0, 0, 0, 0};
        const i32x8 bv = {(int)b.x, (int)b.y, (int)b.z, (int)b.w, 0, 0, 0, 0};
        const int sa = (int)((st.ws >> (8 * (2 * kc + h))) & 0xFFu);
        const int sb = (int)((sw >> (8 * (2 * kc + h))) & 0xFFu);
        acc[tb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, acc[tb], 4, 4, 0, sa, 0, sb);
      }
    }
  };

  Fp4Stage<XC> ring[kFp4Ring];
#pragma unroll
  for (int u = 0; u < kFp4Ahead; ++u) load(ring[u], u);
  write(xl0, sl0, ring[0]);
  __syncthreads();
  // Step s uses stage s % 4 (its weights) and LDS buffer s % 2, loads step s + 3 into stage
  // (s + 3) % 4 (the one step s - 1 used) and writes step s + 1's activations (stage (s + 1) % 4)
  // to buffer (s + 1) % 2, which step s - 1 read before its barrier.
  auto step = [&](int s, auto u) {
    constexpr int U = decltype(u)::value;
    load(ring[(U + kFp4Ahead) % kFp4Ring], s + kFp4Ahead);
    compute(U % 2 ? xl1 : xl0, U % 2 ? sl1 : sl0, ring[U]);
    if (s + 1 < steps) write(U % 2 ? xl0 : xl1, U % 2 ? sl0 : sl1, ring[(U + 1) % kFp4Ring]);
    __syncthreads();
  };
  for (int s0 = 0; s0 < steps; s0 += kFp4Ring) {
    step(s0, std::integral_constant<int, 0>{});
    if (s0 + 1 < steps) step(s0 + 1, std::integral_constant<int, 1>{});
    if (s0 + 2 < steps) step(s0 + 2, std::integral_constant<int, 2>{});
    if (s0 + 3 < steps) step(s0 + 3, std::integral_constant<int, 3>{});
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

hipError_t launch_quantize_weight_fp4(const uint4 *tiles, const float *scales, const float4 *lut, int M, int K,
                                      int RG, int CG, uint8_t *packed, uint8_t *group_scales, hipStream_t stream) {
  const size_t slots = (size_t)RG * CG * 64;
  hipLaunchKernelGGL(quantize_weight_kernel, dim3((unsigned)((slots + 255) / 256)), dim3(256), 0, stream, tiles,
                     scales, lut, M, K, RG, CG, packed, group_scales);
  return hipGetLastError();
}

hipError_t launch_fp4_gemm(const uint8_t *xq, const uint8_t *xs, const uint8_t *wq, const uint8_t *ws,
                           const uint16_t *bias, uint16_t *y, int tokens, int M, int K, hipStream_t stream) {
  const dim3 grid((unsigned)((M + 127) / 128), (unsigned)((tokens + 127) / 128));
  // The staged kernel reads the scales as 4-byte words (4 groups per 128-wide step).
  const bool staged = K % kFp4Step == 0 && reinterpret_cast<uintptr_t>(xs) % 4 == 0 &&
                      reinterpret_cast<uintptr_t>(ws) % 4 == 0;
  // 128 tokens per workgroup: 256 halves the grid (272 workgroups at 17408 rows) and measured
  // 9-40% slower at 512 tokens.
  constexpr int TB = 4;
  if (staged)
    hipLaunchKernelGGL(fp4_gemm_staged_kernel<TB>, dim3(grid.x, (unsigned)((tokens + 32 * TB - 1) / (32 * TB))), dim3(256),
                       0, stream, xq, xs, wq, ws, bias, y, tokens, M, K);
  else
    hipLaunchKernelGGL(fp4_gemm_kernel, grid, dim3(256), 0, stream, xq, xs, wq, ws, bias, y, tokens, M, K);
  return hipGetLastError();
}

}  // namespace tx
