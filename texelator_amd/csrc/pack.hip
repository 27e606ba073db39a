// Device-side repack of reference-layout BC4 blocks into gfx950 tiles.
//
// The reference uploads CPU blocks into a texture (texelator_cuda.cu:1296-1312). Blocks that are
// already in device memory (e.g. encoded on the GPU) are repacked here without a host round
// trip; the per-block encoding is the same function the host repack uses (bc4_device.h).
#include "bc4_device.h"
#include "kernels.h"

namespace tx {

namespace {

// One thread per lane slot of a tile: two reference blocks -> 16 bytes of the tile.
__global__ void repack_kernel(const uint8_t *blocks, int M, int bpr, int RG, int CG, uint4 *tiles) {
  const size_t slot = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (slot >= (size_t)RG * CG * 64) return;
  const int lane = (int)(slot & 63);
  const size_t tile = slot >> 6;
  const int g = (int)(tile / CG);
  const int c = (int)(tile % CG);
  const int m = g * kTileRows + (lane & 15);
  uint32_t w[4];
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int blk = c * kTileBlocks + 2 * (lane >> 4) + half;
    uint32_t a = kZeroBlockWord, b = kZeroBlockWord;
    if (m < M && blk < bpr) {
      const uint2 raw = *reinterpret_cast<const uint2 *>(blocks + ((size_t)m * bpr + blk) * 8);
      uint8_t bytes[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bytes[i] = (uint8_t)(raw.x >> (8 * i));
        bytes[4 + i] = (uint8_t)(raw.y >> (8 * i));
      }
      encode_device_block(bytes, a, b);
    }
    w[2 * half] = a;
    w[2 * half + 1] = b;
  }
  tiles[slot] = make_uint4(w[0], w[1], w[2], w[3]);
}

}  // namespace

hipError_t launch_repack(const uint8_t *blocks, int M, int bpr, int RG, int CG, uint4 *tiles, hipStream_t stream) {
  const size_t slots = (size_t)RG * CG * 64;
  hipLaunchKernelGGL(repack_kernel, dim3((unsigned)((slots + 255) / 256)), dim3(256), 0, stream, blocks, M, bpr, RG,
                     CG, tiles);
  return hipGetLastError();
}

}  // namespace tx
