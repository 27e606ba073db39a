// BF16 prefill GEMM over BC4 tiles (gfx950 MFMA, weight-stationary).
//
// Reference: the CUTLASS MmaPipelined prefill whose operand-B iterator rebuilds BC4 weights
// (texelator/cuda/cutlass_texture_mainloop.cu:58-188, launcher :203-249) computes
// D[T x M] = X[T x K] * W^T with W = bf16(P*scale[row]), fp32 accumulation and a bf16 output;
// the bias is added afterwards with a second bf16 rounding (:190-199). Its five tile shapes are
// backends 5..9; here ids 5..9 name this build's own tile candidates.
//
// A workgroup (4 waves) owns BT = 16*MT tokens x BN = 64*NT output rows x one K range (split):
//   * each wave owns NT 16-row groups; it streams their BC4 tiles (one 1 KiB tile per group and
//     128-wide K step, LA steps ahead) and decodes them (palette seeds from LDS tables) straight
//     into MFMA A operands in registers -- weights never pass through LDS, and no dense 16-bit
//     copy exists anywhere;
//   * the activations of a K step (BT x 128 bf16) are double-buffered in LDS and shared by the
//     four waves; lane (token, kg) reads the 8 values matching the decoded weights' K chunk;
//   * v_mfma_f32_16x16x32_bf16 with rows as M and tokens as N: acc[u][v] = D[rows][tokens].
// Every candidate uses the same MFMA K grouping and order, and the K splits depend only on the
// shape, so all candidates give bitwise-identical results. With several splits the partial sums
// are written to the caller's workspace and reduced in split order by a second kernel.
// Workgroups are mapped so that each XCD (workgroups arrive round-robin) works on few
// (token tile, split) pairs: their activations stay in that XCD's L2.
#include <algorithm>

#include "bc4_device.h"
#include "elementwise.h"
#include "kernels.h"

namespace tx {

namespace {

constexpr int kThreads = 256;
constexpr int kStride = 136;  // LDS row stride of the activation tile in bf16 (128 + 8 padding)
constexpr int kXcds = 8;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// D += A * B on 16x16x32 tiles of packed 16-bit operands (bf16, or fp16 with F16).
template <bool F16>
__device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Round to the output type and widen back (bf16, or fp16 with F16).
template <bool F16>
__device__ __forceinline__ float round_out(float v) {
  if constexpr (F16) return (float)(_Float16)v;
  else return (float)(__bf16)v;
}

template <bool F16>
__device__ __forceinline__ void store_out(void *y, size_t index, float v) {
  if constexpr (F16) static_cast<_Float16 *>(y)[index] = (_Float16)v;
  else static_cast<__bf16 *>(y)[index] = (__bf16)v;
}

struct WorkItem {
  int t0, n0, c_begin, nc, split;
};

// Token-tile-major, then split, then row tile; contiguous ranges go to one XCD.
__device__ __forceinline__ bool work_item(const PrefillParams &p, int BT, int BN, WorkItem &w) {
  const int n_rows = (p.M + BN - 1) / BN;
  const int n_tok = (p.tokens + BT - 1) / BT;
  const int items = n_rows * n_tok * p.ks;
  const int per_xcd = (items + kXcds - 1) / kXcds;
  const int q = (int)(blockIdx.x % kXcds) * per_xcd + (int)(blockIdx.x / kXcds);
  if (q >= items) return false;
  const int row_tile = q % n_rows;
  const int rest = q / n_rows;
  w.split = rest % p.ks;
  w.t0 = (rest / p.ks) * BT;
  w.n0 = row_tile * BN;
  w.c_begin = (int)((int64_t)w.split * p.CG / p.ks);
  w.nc = (int)((int64_t)(w.split + 1) * p.CG / p.ks) - w.c_begin;
  return true;
}

// F16: fp16 activations, bias and output, weights rounded to fp16 (the reference's FP16 prefill
// decodes __float2half(P*scale) into its scratch matrix, texelator_cuda.cu:604-628, and adds
// the bias with a second fp16 rounding, :630-635).
// PIPE: software-pipelined K loop (see the step below). LUT: palettes read from p.lut (a
// 255 x 255 x 8 fp32 table) instead of computed.
template <bool F16, int MT, int NT, int LA, bool PIPE, bool LUT>
__global__ __launch_bounds__(kThreads) void prefill_kernel(PrefillParams p) {
  static_assert(!PIPE || LA >= 2, "the pipelined K loop needs two weight tiles in flight");
  constexpr int BT = 16 * MT;
  constexpr int BN = 64 * NT;
  constexpr int R = LA + 1;
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][BT * kStride];
  __shared__ PaletteTableStorage tables;

  WorkItem w;
  if (!work_item(p, BT, BN, w)) return;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int i = lane & 15;
  const int kg = lane >> 4;
  const uint16_t *x = static_cast<const uint16_t *>(p.x);

  // Row groups of this wave (clamped into the matrix; rows past M are computed, never stored).
  const uint4 *gtiles[NT];
  float scale[NT];
  uint32_t pm[NT];
#pragma unroll
  for (int v = 0; v < NT; ++v) {
    const int g = min(w.n0 / kTileRows + wave * NT + v, p.RG - 1);
    gtiles[v] = p.tiles + ((size_t)g * p.CG + w.c_begin) * 64 + lane;
    scale[v] = p.scales[g * kTileRows + i];
    pm[v] = pm_scale_pair<F16>(scale[v]);
  }

  // Weight ring: slot s holds the NT tiles of one K step.
  uint4 ring[R][NT];
#pragma unroll
  for (int u = 0; u < LA; ++u)
#pragma unroll
    for (int v = 0; v < NT; ++v) ring[u][v] = load_stream(gtiles[v] + (size_t)min(u, w.nc - 1) * 64);

  // Activation staging: MT uint4 per thread per K step (16 uint4 per token row).
  uint4 xr[MT];
  auto load_x = [&](int j) {
    const int c = w.c_begin + min(j, w.nc - 1);
#pragma unroll
    for (int v = 0; v < MT; ++v) {
      const int idx = v * kThreads + threadIdx.x;
      const int t = w.t0 + (idx >> 4);
      const int k = c * kTileK + (idx & 15) * 8;
      xr[v] = (t < p.tokens && k < p.K) ? *reinterpret_cast<const uint4 *>(x + (size_t)t * p.K + k)
                                        : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_x = [&](int buf) {
#pragma unroll
    for (int v = 0; v < MT; ++v) {
      const int idx = v * kThreads + threadIdx.x;
      *reinterpret_cast<uint4 *>(&xs[buf][(idx >> 4) * kStride + (idx & 15) * 8]) = xr[v];
    }
  };
  load_x(0);
  store_x(0);
  load_x(1);
  if constexpr (!LUT) build_palette_tables(tables, threadIdx.x, kThreads);
  __syncthreads();

  f32x4 acc[MT][NT];
#pragma unroll
  for (int a = 0; a < MT; ++a)
#pragma unroll
    for (int b = 0; b < NT; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Decode one K step's NT tiles into A operands: a[v][q] covers block 2kg + (q >> 1), positions
  // 8*(q & 1) .. +7, i.e. K offset 32kg + 8q within the step.
  auto decode_step = [&](const uint4 (&tiles)[NT], u32x4 (&a)[NT][4]) {
    if constexpr (LUT) {
      float4 rows[NT][4];  // all palette rows of the step in flight together
#pragma unroll
      for (int v = 0; v < NT; ++v) {
        const float4 *ra = p.lut + 2 * (size_t)palette_row(tiles[v].x, tiles[v].y);
        const float4 *rb = p.lut + 2 * (size_t)palette_row(tiles[v].z, tiles[v].w);
        rows[v][0] = ra[0];
        rows[v][1] = ra[1];
        rows[v][2] = rb[0];
        rows[v][3] = rb[1];
      }
#pragma unroll
      for (int v = 0; v < NT; ++v) {
        uint32_t d[8];
        decode_from_palette<F16>(rows[v][0], rows[v][1], tiles[v].x, tiles[v].y, scale[v], d);
        a[v][0] = u32x4{d[0], d[1], d[2], d[3]};
        a[v][1] = u32x4{d[4], d[5], d[6], d[7]};
        decode_from_palette<F16>(rows[v][2], rows[v][3], tiles[v].z, tiles[v].w, scale[v], d);
        a[v][2] = u32x4{d[0], d[1], d[2], d[3]};
        a[v][3] = u32x4{d[4], d[5], d[6], d[7]};
      }
    } else {
#pragma unroll
      for (int v = 0; v < NT; ++v) {
        uint32_t d[8];
        decode_block_lds<F16>(tiles[v].x, tiles[v].y, scale[v], pm[v], tables, d);
        a[v][0] = u32x4{d[0], d[1], d[2], d[3]};
        a[v][1] = u32x4{d[4], d[5], d[6], d[7]};
        decode_block_lds<F16>(tiles[v].z, tiles[v].w, scale[v], pm[v], tables, d);
        a[v][2] = u32x4{d[0], d[1], d[2], d[3]};
        a[v][3] = u32x4{d[4], d[5], d[6], d[7]};
      }
    }
  };
  auto mfma_step = [&](int j, const u32x4 (&a)[NT][4]) {
    const uint16_t *xb = xs[j & 1];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int mu = 0; mu < MT; ++mu) {
        const u32x4 b = *reinterpret_cast<const u32x4 *>(xb + (mu * 16 + i) * kStride + kg * 32 + q * 8);
#pragma unroll
        for (int v = 0; v < NT; ++v) acc[mu][v] = mfma<F16>(a[v][q], b, acc[mu][v]);
      }
    }
  };

  // Whole ring turns, then at most LA tail steps (each step issues the same loads, clamped).
  auto run_steps = [&](auto &&step) {
    int j0 = 0;
    for (; j0 + R <= w.nc; j0 += R) {
#pragma unroll
      for (int u = 0; u < R; ++u) step(j0 + u, u);
    }
#pragma unroll
    for (int u = 0; u < LA; ++u)
      if (j0 + u < w.nc) step(j0 + u, u);
  };

  if constexpr (PIPE) {
    // Software-pipelined: step j multiplies the tiles decoded during step j-1 while decoding tile
    // j+1 (already in the ring), so the decode's VALU work and the MFMAs interleave in one
    // instruction stream. Tile j+1 was requested a step earlier (LA >= 2).
    u32x4 acur[NT][4];
    decode_step(ring[0], acur);
    run_steps([&](int j, int u) {
      const int jn = min(j + LA, w.nc - 1);
#pragma unroll
      for (int v = 0; v < NT; ++v) ring[(u + LA) % R][v] = load_stream(gtiles[v] + (size_t)jn * 64);
      u32x4 anext[NT][4];
      decode_step(ring[(u + 1) % R], anext);  // tile j+1 (past the end: the clamped last tile, unused)
      mfma_step(j, acur);
      store_x((j + 1) & 1);  // the next step's activations, into the buffer read two steps ago
      load_x(j + 2);
      __syncthreads();
#pragma unroll
      for (int v = 0; v < NT; ++v)
#pragma unroll
        for (int q = 0; q < 4; ++q) acur[v][q] = anext[v][q];
    });
  } else {
    run_steps([&](int j, int u) {
      const int jn = min(j + LA, w.nc - 1);
#pragma unroll
      for (int v = 0; v < NT; ++v) ring[(u + LA) % R][v] = load_stream(gtiles[v] + (size_t)jn * 64);
      u32x4 a[NT][4];
      decode_step(ring[u], a);
      mfma_step(j, a);
      store_x((j + 1) & 1);  // the next step's activations, into the buffer read two steps ago
      load_x(j + 2);
      __syncthreads();
    });
  }

  // acc[mu][v][r] = D[row 4kg + r of group v][token mu*16 + i].
  const uint16_t *bias = static_cast<const uint16_t *>(p.bias);
#pragma unroll
  for (int mu = 0; mu < MT; ++mu) {
    const int t = w.t0 + mu * 16 + i;
    if (t >= p.tokens) continue;
#pragma unroll
    for (int v = 0; v < NT; ++v) {
      const int row0 = w.n0 + (wave * NT + v) * kTileRows + kg * 4;
      if (p.ks > 1) {
        float *dst = p.partials + ((size_t)w.split * p.tokens + t) * p.Mp + row0;
        if (row0 < p.Mp) *reinterpret_cast<float4 *>(dst) = make_float4(acc[mu][v][0], acc[mu][v][1], acc[mu][v][2], acc[mu][v][3]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int n = row0 + r;
          if (n < p.M) {
            float out = round_out<F16>(acc[mu][v][r]);
            if (bias) out += half_bits_to_float<F16>(bias[n]);
            store_out<F16>(p.y, (size_t)t * p.M + n, out);
          }
        }
      }
    }
  }
}

// y[t][m] = round(sum over splits in order of partials[s][t][m]), then the bias with a second
// rounding (the reference's epilogue order); bf16, or fp16 with F16.
template <bool F16>
__global__ __launch_bounds__(256) void prefill_reduce_kernel(PrefillParams p) {
  const int m = blockIdx.x * 256 + threadIdx.x;
  const int t = blockIdx.y;
  if (m >= p.M) return;
  float total = 0.f;
  for (int s = 0; s < p.ks; ++s) total += p.partials[((size_t)s * p.tokens + t) * p.Mp + m];
  float out = round_out<F16>(total);
  if (p.bias) out += half_bits_to_float<F16>(static_cast<const uint16_t *>(p.bias)[m]);
  store_out<F16>(p.y, (size_t)t * p.M + m, out);
}

struct Candidate {
  const char *name;
  int bt, bn;
  const void *fn;
  hipError_t (*launch)(const PrefillParams &, hipStream_t);
  int lds;
};

template <int MT, int NT, int LA, bool PIPE>
hipError_t launch_tile(const PrefillParams &p, hipStream_t stream) {
  constexpr int BT = 16 * MT, BN = 64 * NT;
  const int items = ((p.M + BN - 1) / BN) * ((p.tokens + BT - 1) / BT) * p.ks;
  const int grid = ((items + kXcds - 1) / kXcds) * kXcds;
  if (p.lut) {
    if (p.f16)
      hipLaunchKernelGGL((prefill_kernel<true, MT, NT, LA, PIPE, true>), dim3(grid), dim3(kThreads), 0, stream, p);
    else
      hipLaunchKernelGGL((prefill_kernel<false, MT, NT, LA, PIPE, true>), dim3(grid), dim3(kThreads), 0, stream, p);
  } else if (p.f16) {
    hipLaunchKernelGGL((prefill_kernel<true, MT, NT, LA, PIPE, false>), dim3(grid), dim3(kThreads), 0, stream, p);
  } else {
    hipLaunchKernelGGL((prefill_kernel<false, MT, NT, LA, PIPE, false>), dim3(grid), dim3(kThreads), 0, stream, p);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.ks == 1) return e;
  if (p.f16)
    hipLaunchKernelGGL(prefill_reduce_kernel<true>, dim3((p.M + 255) / 256, p.tokens), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(prefill_reduce_kernel<false>, dim3((p.M + 255) / 256, p.tokens), dim3(256), 0, stream, p);
  return hipGetLastError();
}

#define TX_CANDIDATE(NAME, MT, NT, LA, PIPE)                                                            \
  Candidate {                                                                                          \
    NAME, 16 * (MT), 64 * (NT), reinterpret_cast<const void *>(&prefill_kernel<false, MT, NT, LA, PIPE, false>), \
        &launch_tile<MT, NT, LA, PIPE>, 2 * 16 * (MT) * kStride * 2                                    \
  }

// Weight tiles in flight per wave, in K steps.
#ifndef TX_PREFILL_LA
#define TX_PREFILL_LA 2
#endif

// The two 128-token tiles pipeline their K loop (4-5% faster at T >= 128 on the 27B shapes); the
// smaller tiles run it plainly (pipelining cost them up to 12% at T = 32).
const Candidate kCandidates[] = {
    TX_CANDIDATE("large_128x256x128", 8, 4, TX_PREFILL_LA, true),
    TX_CANDIDATE("medium_128x128x128", 8, 2, TX_PREFILL_LA, true),
    TX_CANDIDATE("medium_64x256x128", 4, 4, TX_PREFILL_LA, false),
    TX_CANDIDATE("medium_64x128x128", 4, 2, TX_PREFILL_LA, false),
    TX_CANDIDATE("small_32x128x128", 2, 2, TX_PREFILL_LA, false),
};

const Candidate *find(int candidate) {
  if (candidate < kPrefillFirst || candidate > kPrefillLast) return nullptr;
  return &kCandidates[candidate - kPrefillFirst];
}

}  // namespace

int prefill_splits(int M, int CG, int64_t tokens, int cus) {
  // Candidate-independent so that every tile gives the same sums: about two workgroups of the
  // largest tile per CU, each split at least 8 tile columns long, partials at most 32 MiB.
  const int64_t items = ((M + 255) / 256) * ((tokens + 127) / 128);
  const int64_t target = 2 * (int64_t)cus;
  if (items >= target) return 1;
  int64_t ks = (target + items - 1) / items;
  ks = std::min<int64_t>(ks, std::max(1, CG / 8));
  const int64_t cap = std::max<int64_t>(1, (int64_t(32) << 20) / (tokens * (int64_t)((M + 15) / 16 * 16) * 4));
  ks = std::min(ks, cap);
  return (int)std::max<int64_t>(1, ks);
}

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
