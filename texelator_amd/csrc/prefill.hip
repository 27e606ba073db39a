// BF16 prefill GEMM over BC4 tiles (gfx950 MFMA).
//
// Reference: the CUTLASS MmaPipelined prefill whose operand-B iterator rebuilds BC4 weights
// (texelator/cuda/cutlass_texture_mainloop.cu:58-188, launcher :203-249) computes
// D[T x M] = X[T x K] * W^T with W = bf16(P*scale[row]), fp32 accumulation and a bf16 output;
// the bias is added afterwards with a second bf16 rounding (:190-199). Its five tile shapes
// (tokens x rows x K) 256x128x32, 128x128x32, 128x64x32, 64x128x32, 32x32x64 are backends 5..9.
//
// Here a workgroup (4 waves) owns a BT x BN output tile and walks K in steps of 128 columns
// (one column of BC4 tiles):
//   * the BT x 128 activation tile is copied to LDS;
//   * the BN x 128 weight tile is decoded from BC4 straight into LDS as bf16 (no dense copy in
//     global memory ever exists), each lane decoding two blocks with the register decoder;
//   * each wave multiplies its (BT/WT) x (BN/WN) sub-tile with v_mfma_f32_16x16x32_bf16.
// Every candidate accumulates each output in the same order (32-column MFMA steps from k = 0
// upward into one fp32 accumulator), so all candidates give bitwise-identical results.
#include "bc4_device.h"
#include "kernels.h"

namespace tx {

namespace {

constexpr int kThreads = 256;
constexpr int kStride = 136;  // LDS row stride in bf16 elements (128 + 8 padding)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_bits_to_float(uint16_t v) {
  return __builtin_bit_cast(float, (uint32_t)v << 16);
}

template <int BT, int BN, int WT, int WN>
__global__ __launch_bounds__(kThreads) void prefill_kernel(PrefillParams p) {
  static_assert(WT * WN == 4, "four waves per workgroup");
  constexpr int TW = BT / WT;  // tokens per wave
  constexpr int NW = BN / WN;  // rows per wave
  constexpr int MT = TW / 16;
  constexpr int NT = NW / 16;
  static_assert(MT >= 1 && NT >= 1, "wave tile must cover at least one 16x16 MFMA tile");
  __shared__ __attribute__((aligned(16))) uint16_t xs[BT * kStride];
  __shared__ __attribute__((aligned(16))) uint16_t ws[BN * kStride];

  const int n0 = blockIdx.x * BN;
  const int t0 = blockIdx.y * BT;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wt = wave / WN;
  const int wn = wave % WN;
  const uint16_t *x = static_cast<const uint16_t *>(p.x);

  f32x4 acc[MT][NT];
#pragma unroll
  for (int a = 0; a < MT; ++a)
#pragma unroll
    for (int b = 0; b < NT; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int i = lane & 15;
  const int kg = lane >> 4;

  for (int c = 0; c < p.CG; ++c) {
    // Activation tile: BT rows x 128 columns, 16 bytes per thread per pass.
    for (int idx = threadIdx.x; idx < BT * 16; idx += kThreads) {
      const int r = idx >> 4;
      const int q = idx & 15;
      const int t = t0 + r;
      const int k = c * kTileK + q * 8;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (t < p.tokens) {
        const uint16_t *src = x + (size_t)t * p.K + k;
        if (k + 8 <= p.K) {
          v = *reinterpret_cast<const uint4 *>(src);
        } else {
          uint16_t e[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) e[u] = (k + u < p.K) ? src[u] : (uint16_t)0;
          v.x = e[0] | ((uint32_t)e[1] << 16);
          v.y = e[2] | ((uint32_t)e[3] << 16);
          v.z = e[4] | ((uint32_t)e[5] << 16);
          v.w = e[6] | ((uint32_t)e[7] << 16);
        }
      }
      *reinterpret_cast<uint4 *>(xs + r * kStride + q * 8) = v;
    }
    // Weight tile: BN/16 BC4 tiles, decoded by lanes of the four waves.
    for (int d = wave; d < BN / kTileRows; d += 4) {
      const int g = n0 / kTileRows + d;
      uint32_t w0[8], w1[8];
      if (g < p.RG) {
        const uint4 cur = load_stream(p.tiles + ((size_t)g * p.CG + c) * 64 + lane);
        const float scale = p.scales[g * kTileRows + i];
        const uint32_t pm = pm_scale_pair(scale);
        decode_block(cur.x, cur.y, scale, pm, w0);
        decode_block(cur.z, cur.w, scale, pm, w1);
      } else {
#pragma unroll
        for (int u = 0; u < 8; ++u) w0[u] = w1[u] = 0u;
      }
      uint4 *dst = reinterpret_cast<uint4 *>(ws + (d * kTileRows + i) * kStride + kg * 32);
      dst[0] = make_uint4(w0[0], w0[1], w0[2], w0[3]);
      dst[1] = make_uint4(w0[4], w0[5], w0[6], w0[7]);
      dst[2] = make_uint4(w1[0], w1[1], w1[2], w1[3]);
      dst[3] = make_uint4(w1[4], w1[5], w1[6], w1[7]);
    }
    __syncthreads();

#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      bf16x8 a[MT], b[NT];
#pragma unroll
      for (int u = 0; u < MT; ++u)
        a[u] = *reinterpret_cast<const bf16x8 *>(xs + (wt * TW + u * 16 + i) * kStride + kk * 32 + kg * 8);
#pragma unroll
      for (int u = 0; u < NT; ++u)
        b[u] = *reinterpret_cast<const bf16x8 *>(ws + (wn * NW + u * 16 + i) * kStride + kk * 32 + kg * 8);
#pragma unroll
      for (int u = 0; u < MT; ++u)
#pragma unroll
        for (int v = 0; v < NT; ++v) acc[u][v] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[u], b[v], acc[u][v], 0, 0, 0);
    }
    __syncthreads();
  }

  // acc[u][v][r] = D[token 4*kg + r][row i] of the 16x16 sub-tile (u, v).
  __bf16 *y = static_cast<__bf16 *>(p.y);
  const uint16_t *bias = static_cast<const uint16_t *>(p.bias);
#pragma unroll
  for (int v = 0; v < NT; ++v) {
    const int n = n0 + wn * NW + v * 16 + i;
    if (n >= p.M) continue;
    const float bv = bias ? bf16_bits_to_float(bias[n]) : 0.f;
#pragma unroll
    for (int u = 0; u < MT; ++u) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = t0 + wt * TW + u * 16 + kg * 4 + r;
        if (t < p.tokens) {
          __bf16 out = (__bf16)acc[u][v][r];
          if (bias) out = (__bf16)((float)out + bv);
          y[(size_t)t * p.M + n] = out;
        }
      }
    }
  }
}

struct Candidate {
  const char *name;
  int bt, bn;
  const void *fn;
  hipError_t (*launch)(const PrefillParams &, hipStream_t);
  int lds;
};

template <int BT, int BN, int WT, int WN>
hipError_t launch_tile(const PrefillParams &p, hipStream_t stream) {
  dim3 grid((p.M + BN - 1) / BN, (p.tokens + BT - 1) / BT);
  hipLaunchKernelGGL((prefill_kernel<BT, BN, WT, WN>), grid, dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

#define TX_CANDIDATE(NAME, BT, BN, WT, WN)                                                              \
  Candidate {                                                                                          \
    NAME, BT, BN, reinterpret_cast<const void *>(&prefill_kernel<BT, BN, WT, WN>),                     \
        &launch_tile<BT, BN, WT, WN>, (BT + BN) * kStride * 2                                          \
  }

const Candidate kCandidates[] = {
    TX_CANDIDATE("large_256x128x128", 256, 128, 2, 2),
    TX_CANDIDATE("medium_128x128x128", 128, 128, 2, 2),
    TX_CANDIDATE("medium_128x64x128", 128, 64, 2, 2),
    TX_CANDIDATE("medium_64x128x128", 64, 128, 2, 2),
    TX_CANDIDATE("small_32x64x128", 32, 64, 2, 2),
};

const Candidate *find(int candidate) {
  if (candidate < kPrefillFirst || candidate > kPrefillLast) return nullptr;
  return &kCandidates[candidate - kPrefillFirst];
}

}  // namespace

bool prefill_candidate_eligible(int candidate, int M, int K) {
  return find(candidate) != nullptr && M > 0 && K > 0 && K % 16 == 0;
}

hipError_t launch_prefill(const PrefillParams &p, int candidate, hipStream_t stream) {
  const Candidate *c = find(candidate);
  if (!c) return hipErrorInvalidValue;
  return c->launch(p, stream);
}

hipError_t prefill_kernel_attributes(int candidate, hipFuncAttributes *attr, int *lds_bytes) {
  const Candidate *c = find(candidate);
  if (!c) return hipErrorInvalidValue;
  if (lds_bytes) *lds_bytes = c->lds;
  return hipFuncGetAttributes(attr, c->fn);
}

const char *prefill_candidate_name(int candidate) {
  const Candidate *c = find(candidate);
  return c ? c->name : nullptr;
}

void prefill_candidate_shape(int candidate, int *tokens, int *rows, int *k) {
  const Candidate *c = find(candidate);
  *tokens = c ? c->bt : 0;
  *rows = c ? c->bn : 0;
  *k = c ? kTileK : 0;
}

}  // namespace tx
