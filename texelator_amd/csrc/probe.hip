// Exhaustive palette probe and dense decode (diagnostics).
//
// Reference: texelator_palette_probe / texelator_dump_palette
// (texelator/cuda/texelator_cuda.cu:1542-1595) sample every endpoint pair (e0, e1) in
// [-127,127]^2 and write out[(y*255 + x)*8 + s] with x = e0+127, y = e1+127. Here the same
// table is produced by the register decoder (palette8 in bc4_device.h) run on probe blocks built
// in the device layout, so its SHA-256 can be compared with the CPU palette.
#include "bc4_device.h"
#include "kernels.h"

namespace tx {

namespace {

// Device-layout word for endpoint byte eb (biased, 0..254) with selector bits zero.
__device__ __forceinline__ uint32_t endpoint_word(uint32_t eb) {
  uint32_t w = 0;
#pragma unroll
  for (int c = 0; c < 4; ++c) w |= ((eb >> (2 * c)) & 3u) << (8 * c + 3);
  return w;
}

__global__ void palette_probe_kernel(float *out) {
  const int index = blockIdx.x * blockDim.x + threadIdx.x;
  if (index >= 255 * 255) return;
  const uint32_t x = index % 255;
  const uint32_t y = index / 255;
  Palette pal = palette8(endpoint_word(x), endpoint_word(y));
  float4 *dst = reinterpret_cast<float4 *>(out + (size_t)index * 8);
  dst[0] = make_float4(pal.p[0], pal.p[1], pal.p[2], pal.p[3]);
  dst[1] = make_float4(pal.p[4], pal.p[5], pal.p[6], pal.p[7]);
}

// One thread per lane-slot of a tile of row groups g_begin .. g_begin + groups - 1: decodes two
// blocks of row `row` into out[row - row_begin][K] for rows below row_end (bf16 bits, or fp16 bits
// with F16).
template <bool F16>
__global__ void decode_dense_kernel(const uint4 *tiles, const float *scales, const float4 *lut, int M, int K, int CG,
                                    int g_begin, int groups, int row_end, uint16_t *out) {
  const size_t local = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (local >= (size_t)groups * CG * 64) return;
  const int lane = local & 63;
  const size_t tile = local >> 6;
  const int g = g_begin + (int)(tile / CG);
  const int c = (int)(tile % CG);
  const int row = g * kTileRows + (lane & 15);
  if (row >= M || row >= row_end) return;
  const size_t slot = (size_t)g_begin * CG * 64 + local;
  const uint4 cur = tiles[slot];
  const float scale = scales[row];
  const uint32_t pm = pm_scale_pair<F16>(scale);
  uint32_t w[2][8];
  if (lut) {  // LUT mode: the palette rows come from the table
    const float4 *ra = lut + 2 * (size_t)palette_row(cur.x, cur.y);
    const float4 *rb = lut + 2 * (size_t)palette_row(cur.z, cur.w);
    decode_from_palette<F16>(ra[0], ra[1], cur.x, cur.y, scale, w[0]);
    decode_from_palette<F16>(rb[0], rb[1], cur.z, cur.w, scale, w[1]);
  } else {
    decode_block<F16>(cur.x, cur.y, scale, pm, w[0]);
    decode_block<F16>(cur.z, cur.w, scale, pm, w[1]);
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int k0 = (c * kTileBlocks + 2 * (lane >> 4) + h) * 16;
    if (k0 >= K) continue;
    uint16_t *dst = out + (size_t)(row - g_begin * kTileRows) * K + k0;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      dst[2 * q] = (uint16_t)(w[h][q] & 0xFFFFu);
      dst[2 * q + 1] = (uint16_t)(w[h][q] >> 16);
    }
  }
}

// Plain streaming read (the measurement's reference point for the GEMV): every lane XORs a
// grid-strided range of 16-byte words with 8 loads in flight; a word equal to a value no input
// holds is written, so the loads cannot be dropped.
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4 *data, size_t words, uint32_t *sink) {
  constexpr int kUnroll = 8;
  const size_t stride = (size_t)gridDim.x * 256;
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  uint32_t h = 0;
  for (; i + (kUnroll - 1) * stride < words; i += kUnroll * stride) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = __builtin_nontemporal_load(data + i + u * stride);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) h ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < words; i += stride) {
    const u32x4 v = __builtin_nontemporal_load(data + i);
    h ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (h == 0x9E3779B9u) sink[blockIdx.x] = h;
}

}  // namespace

hipError_t launch_stream_read(const void *data, size_t bytes, uint32_t *sink, hipStream_t stream) {
  hipLaunchKernelGGL(stream_read_kernel, dim3(kStreamReadBlocks), dim3(256), 0, stream, static_cast<const u32x4 *>(data),
                     bytes / 16, sink);
  return hipGetLastError();
}

hipError_t launch_palette_probe(float *out, hipStream_t stream) {
  hipLaunchKernelGGL(palette_probe_kernel, dim3((255 * 255 + 255) / 256), dim3(256), 0, stream, out);
  return hipGetLastError();
}

hipError_t launch_decode_rows(const uint4 *tiles, const float *scales, const float4 *lut, int M, int K, int CG,
                              int row_begin, int rows, bool f16, uint16_t *out, hipStream_t stream) {
  const int g_begin = row_begin / kTileRows;
  const int row_end = row_begin + rows;
  const int groups = (row_end + kTileRows - 1) / kTileRows - g_begin;
  const size_t slots = (size_t)groups * CG * 64;
  const dim3 grid((unsigned)((slots + 255) / 256));
  if (f16)
    hipLaunchKernelGGL(decode_dense_kernel<true>, grid, dim3(256), 0, stream, tiles, scales, lut, M, K, CG, g_begin,
                       groups, row_end, out);
  else
    hipLaunchKernelGGL(decode_dense_kernel<false>, grid, dim3(256), 0, stream, tiles, scales, lut, M, K, CG, g_begin,
                       groups, row_end, out);
  return hipGetLastError();
}

hipError_t launch_decode_dense(const uint4 *tiles, const float *scales, const float4 *lut, int M, int K, int RG, int CG,
                               bool f16, uint16_t *out, hipStream_t stream) {
  (void)RG;
  return launch_decode_rows(tiles, scales, lut, M, K, CG, 0, M, f16, out, stream);
}

}  // namespace tx
