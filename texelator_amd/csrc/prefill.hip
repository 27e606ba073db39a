// BF16 prefill GEMM over BC4 tiles (gfx950 MFMA, weight-stationary).
//
// Reference: the CUTLASS MmaPipelined prefill whose operand-B iterator rebuilds BC4 weights
// (texelator/cuda/cutlass_texture_mainloop.cu:58-188, launcher :203-249) computes
// D[T x M] = X[T x K] * W^T with W = bf16(P*scale[row]), fp32 accumulation and a bf16 output;
// the bias is added afterwards with a second bf16 rounding (:190-199). Its five tile shapes are
// backends 5..9; here ids 5..9 name this build's own tile candidates.
//
// A workgroup (4 waves) owns BT = 32*TB tokens x BN = 128*RB output rows x one K range (split):
//   * each wave owns RB blocks of 32 rows (two 16-row tile groups each). Per 128-wide K step it
//     streams the two groups' 1 KiB tiles (LA steps ahead): lane l gathers the 32 bytes holding
//     blocks 2h, 2h+1, 4+2h, 5+2h (h = l / 32) of row l % 32, and decodes them (palette seeds from
//     LDS tables) straight into MFMA A operands -- weights never pass through LDS, and no dense
//     16-bit copy exists anywhere;
//   * v_mfma_f32_32x32x16_bf16 (twice the rate of the 16x16x32 form on gfx950): MFMA
//     s = 4*h2 + 2j + e of a step (h2 = which 64-wide half of the step) takes positions 8e..8e+7 of
//     block 4*h2 + j from lanes 0-31 and of block 4*h2 + 2 + j from lanes 32-63, i.e.
//     K = {64*h2 + 16j + 8e ..+7} u {64*h2 + 32 + 16j + 8e ..+7}: every MFMA's K set lies in one
//     64-wide half. The activations of the step (BT x 128 bf16) are double-buffered in LDS, shared
//     by the four waves, and read with the same K sets; they are staged by direct global-to-LDS
//     loads (no registers) one step ahead, in rows of 256 bytes whose 16-byte slots are
//     XOR-swizzled by row;
//   * acc[tb][rb] = D[32 rows of block rb][32 tokens of block tb].
// Candidate 5 (prefill_pair_kernel) is the 8-wave 256-token x 128-row variant in which wave pairs
// split each step's decode by K half and hand the operands to each other through LDS.
// Every candidate uses the same MFMA K grouping and order, and the K splits depend only on the
// shape, so all candidates give bitwise-identical results. With several splits the partial sums
// are written to the caller's workspace and reduced in split order by a second kernel.
// Workgroups are mapped so that each XCD (workgroups arrive round-robin) works on few
// (token tile, split) pairs: their activations stay in that XCD's L2.
#include <algorithm>
#include <array>
#include <type_traits>

#include "bc4_device.h"
#include "elementwise.h"
#include "kernels.h"

namespace tx {

namespace {

constexpr int kThreads = 256;
constexpr int kXcds = 8;

// Weight tiles in flight per wave, in K steps: the pipelined 128-token tiles, the plain tiles.
#ifndef TX_PREFILL_LA
#define TX_PREFILL_LA 3
#endif
#ifndef TX_PREFILL_LA_PLAIN
#define TX_PREFILL_LA_PLAIN 2
#endif
// When a pipelined step issues the direct loads of the next step's activations: 0 before its
// weight loads, 1 after them, 2 spread over the woven regions. Plain steps issue them after
// their weight loads.
#ifndef TX_PREFILL_STAGE
#define TX_PREFILL_STAGE 2
#endif
constexpr int kStage = TX_PREFILL_STAGE;
// Scheduling regions per K step of the woven loop (each holds 8/NR MFMA groups and its share of
// the next tile's block decodes).
#ifndef TX_PREFILL_REGIONS
#define TX_PREFILL_REGIONS 8
#endif
constexpr int NR = TX_PREFILL_REGIONS;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// D += A * B on 32x32x16 tiles of packed 16-bit operands (bf16, or fp16 with F16).
template <bool F16>
__device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
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

// Token-tile-major, then split, then row tile; contiguous ranges go to one XCD. `rows` rows are
// tiled (p.M unless given).
__device__ __forceinline__ bool work_item(const PrefillParams &p, int BT, int BN, WorkItem &w, int rows = -1) {
  const int n_rows = ((rows < 0 ? p.M : rows) + BN - 1) / BN;
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
  // ks * CG < 2^31 (prefill_splits), so the 32-bit products are exact.
  w.c_begin = (int)((uint32_t)w.split * (uint32_t)p.CG / (uint32_t)p.ks);
  w.nc = (int)((uint32_t)(w.split + 1) * (uint32_t)p.CG / (uint32_t)p.ks) - w.c_begin;
  return true;
}

// Buffer descriptor over `bytes` bytes from `base` (records clamped to 2^31 - 1; loads past the
// end return zeros, direct-to-LDS loads past it write zeros). The tile kernels read weights and
// stage activations through descriptors: with only buffer loads in flight the compiler counts
// them exactly and waits for just the loads a use needs (vmcnt(N)); global_load_lds in flight
// beside global loads made it wait for every load (vmcnt(0)), so a step's fresh loads were waited
// for as soon as an older one was used.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0,
                                           (int)(bytes < 0x7FFFFFFF ? bytes : 0x7FFFFFFF), 0x00020000);
}

// 16 bytes at voffset + soffset of a weight descriptor (streaming: weights are read once).
__device__ __forceinline__ uint4 load_weights16(__amdgpu_buffer_rsrc_t r, uint32_t voffset, int soffset) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voffset, soffset, 2 /* nt */);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Descriptor over the tiles from tile (g, c) to the end of the matrix.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const PrefillParams &p, int g, int c) {
  const int64_t first = (int64_t)g * p.CG + c;
  return buffer_rsrc(p.tiles + first * 64, ((int64_t)p.RG * p.CG - first) * kTileBytes);
}

// Output staging through LDS for tiles of 128 rows. In the accumulators each lane holds four
// consecutive rows of one token, so direct stores are 2-byte (16-bit outputs) or 16-byte (fp32
// partials) writes to a different token row per lane; staged, a token's outputs are contiguous and
// every store writes a whole 16-byte chunk. A staged token row is 256 bytes (16 chunks), chunk c
// stored at c ^ (token % 16): 16-bit outputs keep all 128 rows in one buffer (chunk = 8 rows);
// fp32 partials keep rows 0-63 in one buffer and rows 64-127 in another (chunk = 4 rows).
__device__ __forceinline__ void stage_out16(uint16_t *buf, int token, int row, uint32_t lo, uint32_t hi) {
  *reinterpret_cast<uint2 *>(buf + token * 128 + 8 * ((row >> 3) ^ (token & 15)) + (row & 7)) = make_uint2(lo, hi);
}
__device__ __forceinline__ void stage_out32(uint16_t *buf, int token, int row, float4 v) {
  *reinterpret_cast<float4 *>(buf + token * 128 + 8 * (((row & 63) >> 2) ^ (token & 15))) = v;
}
// 16-bit value of an output (the plain epilogue's rounding, bias with a second rounding).
template <bool F16>
__device__ __forceinline__ uint16_t out_bits(float acc, const uint16_t *bias, int n) {
  float out = round_out<F16>(acc);
  if (bias) out += half_bits_to_float<F16>(bias[n]);
  return F16 ? __builtin_bit_cast(uint16_t, (_Float16)out) : __builtin_bit_cast(uint16_t, (__bf16)out);
}
// Copy a staged tile of `bt` tokens out with `threads` threads (after a barrier): 16-bit outputs
// to y [tokens][M] (M % 8 == 0, y 16-byte aligned), or fp32 partials to the split's [tokens][Mp].
template <bool F32>
__device__ __forceinline__ void store_staged(const PrefillParams &p, const WorkItem &w, const uint16_t *buf0,
                                             const uint16_t *buf1, int bt, int threads) {
  const int chunks = bt * (F32 ? 32 : 16);
  for (int id = (int)threadIdx.x; id < chunks; id += threads) {
    const int c = id & 15, t = (id >> 4) % bt, half = F32 ? (id >> 4) / bt : 0;
    const uint4 v = *reinterpret_cast<const uint4 *>((half ? buf1 : buf0) + t * 128 + 8 * (c ^ (t & 15)));
    const int token = w.t0 + t;
    if (token >= p.tokens) continue;
    if constexpr (F32) {
      const int row = w.n0 + 64 * half + 4 * c;
      if (row < p.Mp) *reinterpret_cast<uint4 *>(p.partials + ((size_t)w.split * p.tokens + token) * p.Mp + row) = v;
    } else {
      const int n = w.n0 + 8 * c;
      if (n < p.M) *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(p.y) + (size_t)token * p.M + n) = v;
    }
  }
}

// F16: fp16 activations, bias and output, weights rounded to fp16 (the reference's FP16 prefill
// decodes __float2half(P*scale) into its scratch matrix, texelator_cuda.cu:604-628, and adds
// the bias with a second fp16 rounding, :630-635).
// PIPE: software-pipelined K loop (tile j+1 decoded while tile j is multiplied). LUT: palettes
// read from p.lut (a 255 x 255 x 8 fp32 table) instead of computed.
// SWIGLU (RB = 1, bf16, one K split): p holds a merged [gate | up] matrix (M = 2 * inter, inter a
// multiple of 16); wave w owns gate rows n0 + 32 * (w / 2) .. + 31 (w even) or the matching up rows
// (w odd), and the epilogue writes y[t][n] = bf16(silu(G) * U) for inter columns, G and U being
// the bf16 outputs the plain epilogue would store: each up wave hands its accumulators to its gate
// partner through LDS. The bits of the GEMM followed by the SwiGLU kernel.
template <bool F16, int TB, int RB, int LA, bool PIPE, bool LUT, bool SWIGLU = false>
__global__ __launch_bounds__(kThreads) void prefill_kernel(PrefillParams p) {
  static_assert(!PIPE || LA >= 2, "the pipelined K loop needs two weight tiles in flight");
  static_assert(!SWIGLU || (RB == 1 && !F16), "the SwiGLU epilogue pairs the waves' row blocks (bf16)");
  constexpr int BT = 32 * TB;
  constexpr int BN = 128 * RB;
  constexpr int XC = BT * 16 / kThreads;  // 16-byte activation chunks staged per thread per step
  constexpr int D = PIPE ? 1 : 0;         // step j decodes weight tile j + D
  constexpr int NS = LA - D;              // weight tiles held between steps
  // The two activation buffers are separate LDS objects, so the compiler can tell the reads of
  // one from the direct-to-LDS loads that fill the other and does not make them wait.
  __shared__ __attribute__((aligned(16))) uint16_t xs0[BT * kTileK];
  __shared__ __attribute__((aligned(16))) uint16_t xs1[BT * kTileK];
  __shared__ __attribute__((aligned(16))) PaletteTableStorage tables;

  WorkItem w;
  if (!work_item(p, BT, SWIGLU ? BN / 2 : BN, w, SWIGLU ? p.M / 2 : -1)) return;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r32 = lane & 31;  // row of the 32-row block (A), token of the 32-token block (B)
  const int h = lane >> 5;    // which four blocks of the step this lane holds
  const uint16_t *x = static_cast<const uint16_t *>(p.x);
  // K offset within the step of this lane's 8 activations for MFMA s (s = 4*h2 + 2*j + e).
  auto k_offset = [&](int s) { return 64 * (s >> 2) + 32 * h + 16 * ((s >> 1) & 1) + 8 * (s & 1); };

  // Row blocks of this wave: 32 rows = tile groups 2b and 2b+1 (clamped into the matrix; rows
  // past M are computed, never stored). Lane slot (row & 15) + 16h of a tile holds blocks
  // 2h, 2h+1 of that row; slot + 32 holds blocks 4+2h, 5+2h.
  // The wave's tiles are read through a descriptor based at its first tile group g0 (wave-uniform;
  // every g of the wave is at or above it), lane offsets in bytes.
  int g0;
  if constexpr (SWIGLU) {
    const int half_rg = p.RG / 2;
    g0 = min(w.n0 / kTileRows + (wave >> 1) * 2, half_rg - 1) + ((wave & 1) ? half_rg : 0);
  } else {
    g0 = min(w.n0 / kTileRows + wave * RB * 2, p.RG - 1);
  }
  const __amdgpu_buffer_rsrc_t trsrc = tile_rsrc(p, g0, w.c_begin);
  uint32_t tlane[RB];
  float scale[RB];
  uint32_t pm[RB];
#pragma unroll
  for (int b = 0; b < RB; ++b) {
    int g;
    if constexpr (SWIGLU) {
      const int half_rg = p.RG / 2;
      g = min(w.n0 / kTileRows + (wave >> 1) * 2 + (r32 >> 4), half_rg - 1) + ((wave & 1) ? half_rg : 0);
    } else {
      g = min(w.n0 / kTileRows + (wave * RB + b) * 2 + (r32 >> 4), p.RG - 1);
    }
    tlane[b] = (uint32_t)(((g - g0) * p.CG * 64 + (lane & 15) + 16 * h) * 16);
    scale[b] = p.scales[g * kTileRows + (lane & 15)];
    pm[b] = pm_scale_pair<F16>(scale[b]);
  }
  // The two 16-byte pieces of each row block for one K step (past the end: the last step's).
  auto load_tiles = [&](uint4 (&slot)[RB][2], int j) {
    const int off = __builtin_amdgcn_readfirstlane(min(j, w.nc - 1) * kTileBytes);
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      slot[b][0] = load_weights16(trsrc, tlane[b], off);
      slot[b][1] = load_weights16(trsrc, tlane[b], off + 512);
    }
  };

  // Activation tile of a step in LDS: token row r takes 256 bytes, and its 16-byte slot q holds
  // columns 8*(q ^ (r % 16))..+7 of the step (XOR swizzle: the 16 rows one MFMA operand read
  // serves per LDS pass fall on distinct banks). Thread i stages row 16v + i/16 (v < XC) into
  // slot i % 16; with a direct load, lane l of a wave lands in slot l of the wave's 1 KiB.
  const int srow = threadIdx.x >> 4;                 // = row % 16 for every v
  const int scol = ((threadIdx.x & 15) ^ srow) * 8;  // step column of the chunk this thread stages
  const bool tile_full = w.t0 + BT <= p.tokens;      // uniform: no row past the tokens
  const uint32_t lane_off = (uint32_t)(srow * p.K + scol) * 2;  // bytes from row 16v, column 0
  // Activations of the token tile through a descriptor based at its first row.
  const __amdgpu_buffer_rsrc_t xrsrc =
      buffer_rsrc(x + (size_t)w.t0 * p.K, (int64_t)min(BT, p.tokens - w.t0) * p.K * 2);
  auto stage_part = [&](uint16_t *buf, int j, int v0, int v1) {
    const int c = w.c_begin + j;
    if ((c + 1) * kTileK <= p.K) {
      // Direct loads: a uniform offset (row 16v of the tile, the step's first column) plus a
      // 32-bit lane offset. Rows past the tokens repeat the last token; their outputs are never
      // stored. The base row is clamped too, so the offset is never negative.
#pragma unroll
      for (int v = v0; v < v1; ++v) {
        const int row0 = tile_full ? w.t0 + 16 * v : min(w.t0 + 16 * v, p.tokens - 1);
        const int base = __builtin_amdgcn_readfirstlane(((row0 - w.t0) * p.K + c * kTileK) * 2);
        uint32_t off = lane_off;
        if (!tile_full) off = (uint32_t)((min(w.t0 + 16 * v + srow, p.tokens - 1) - row0) * p.K + scol) * 2;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            xrsrc, (__attribute__((address_space(3))) void *)(buf + (16 * v + 4 * wave) * kTileK), 16, off, base, 0, 0);
      }
    } else if (v0 == 0) {
      // The matrix's last, partial K tile: columns past K are staged as zeros (read from an
      // offset past the descriptor's end, which returns zeros).
      const int k = c * kTileK + scol;
#pragma unroll 2
      for (int v = 0; v < XC; ++v) {
        const int t = min(w.t0 + 16 * v + srow, p.tokens - 1);
        const uint32_t off = k < p.K ? (uint32_t)((t - w.t0) * p.K + k) * 2 : 0x7FFFFFF0u;
        const u32x4 value = __builtin_amdgcn_raw_buffer_load_b128(xrsrc, off, 0, 0);
        *reinterpret_cast<u32x4 *>(buf + (16 * v + srow) * kTileK + (threadIdx.x & 15) * 8) = value;
      }
    }
  };
  auto stage_x = [&](uint16_t *buf, int j) { stage_part(buf, j, 0, XC); };
  // Element offset of this lane's B operand of MFMA s in token block 0 of a staged tile.
  const int sw = r32 & 15;
  auto b_off = [&](int s) { return r32 * kTileK + 8 * ((k_offset(s) >> 3) ^ sw); };
  // End of a step: this wave's direct loads have landed (with kStage 0 on a pipelined tile at most
  // the 2*RB weight loads issued after them are outstanding, and loads complete in order), its
  // LDS stores are done, then the workgroup barrier. A fence would also wait for weight loads
  // that may stay in flight across the barrier; the memory clobber keeps the compiler from moving
  // LDS accesses across it.
  auto step_barrier = [&]() {
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(PIPE && kStage == 0 ? 2 * RB : 0) : "memory");
  };

  // Prologue: step 0's activations, the palette tables, the first weight tiles.
  stage_x(xs0, 0);
  __builtin_amdgcn_sched_barrier(0);
  uint4 ring[NS > 0 ? NS : 1][RB][2];
  uint4 first[RB][2];
  if constexpr (PIPE) load_tiles(first, 0);
#pragma unroll
  for (int u = 0; u < NS; ++u) load_tiles(ring[u], u + D);
  if constexpr (!LUT) copy_seed_tables(tables, wave, lane, kThreads / 64);
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();

  f32x16 acc[TB][RB];
#pragma unroll
  for (int a = 0; a < TB; ++a)
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

  // Decode one K step into A operands: a[b][2j + e] = positions 8e..8e+7 of this lane's block j.
  auto decode_step = [&](const uint4 (&slot)[RB][2], u32x4 (&a)[RB][8]) {
#pragma unroll
    for (int b = 0; b < RB; ++b) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 &piece = slot[b][j >> 1];
        const uint32_t wa = (j & 1) ? piece.z : piece.x;
        const uint32_t wb = (j & 1) ? piece.w : piece.y;
        uint32_t d[8];
        if constexpr (LUT) {
          const float4 *row = p.lut + 2 * (size_t)palette_row(wa, wb);
          decode_from_palette<F16>(row[0], row[1], wa, wb, scale[b], d);
        } else {
          decode_block_lds<F16>(wa, wb, scale[b], pm[b], tables, d);
        }
        a[b][2 * j] = u32x4{d[0], d[1], d[2], d[3]};
        a[b][2 * j + 1] = u32x4{d[4], d[5], d[6], d[7]};
      }
    }
  };
  auto mfma_step = [&](const uint16_t *xb, const u32x4 (&a)[RB][8]) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) {
        const u32x4 bv = *reinterpret_cast<const u32x4 *>(xb + tb * 32 * kTileK + b_off(s));
#pragma unroll
        for (int b = 0; b < RB; ++b) acc[tb][b] = mfma<F16>(a[b][s], bv, acc[tb][b]);
      }
    }
  };
  // Step j reads buffer j & 1 while the direct loads fill the other one (last read in step j-1,
  // which ended with a barrier) with step j+1's activations. The K loop runs two steps per turn,
  // so that which buffer a step reads is known at compile time.
  auto run_steps = [&](auto &&step) {
    int j0 = 0;
    for (; j0 + 2 <= w.nc; j0 += 2) {
      step(j0, xs0, xs1);
      step(j0 + 1, xs1, xs0);
    }
    if (j0 < w.nc) step(j0, xs0, xs1);
  };
  // Shift the held weight tiles by one step; `fresh` is the tile loaded this step.
  auto shift_ring = [&](const uint4 (&fresh)[RB][2]) {
#pragma unroll
    for (int u = 0; u + 1 < NS; ++u)
#pragma unroll
      for (int b = 0; b < RB; ++b) {
        ring[u][b][0] = ring[u + 1][b][0];
        ring[u][b][1] = ring[u + 1][b][1];
      }
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      ring[NS - 1][b][0] = fresh[b][0];
      ring[NS - 1][b][1] = fresh[b][1];
    }
  };

  if constexpr (PIPE) {
    // Software-pipelined: step j multiplies the tiles decoded during step j-1 while decoding tile
    // j+1 (held since step j-1, LA >= 2). The step is woven: each of its eight MFMA groups (one
    // per K set s) carries the decode of one block of tile j+1 and the activation reads of the
    // next group, in a scheduling region of its own (the decoded block is pinned to it), so the
    // matrix core and the VALU work side by side instead of in turn.
    u32x4 acur[RB][8];
    decode_step(first, acur);
    run_steps([&](int j, const uint16_t *xb, uint16_t *xn) {
      const bool more = j + 1 < w.nc;
      if (kStage == 0 && more) stage_x(xn, j + 1);
      __builtin_amdgcn_sched_barrier(0);
      uint4 fresh[RB][2];
      load_tiles(fresh, j + LA);
      __builtin_amdgcn_sched_barrier(0);
      if ((kStage == 1 || (kStage == 2 && LUT)) && more) stage_x(xn, j + 1);
      const uint4(&next)[RB][2] = ring[0];  // tile j+1 (past the end: the clamped last tile)
      u32x4 anext[RB][8];
      if constexpr (LUT) {
        decode_step(next, anext);  // the palette-row gathers of a step stay together
        mfma_step(xb, acur);
      } else {
        auto read_b = [&](int tb, int sg) {
          return *reinterpret_cast<const u32x4 *>(xb + tb * 32 * kTileK + b_off(sg));
        };
        constexpr int kBlocks = 4 * RB;                  // blocks per lane and step
        constexpr int kRegions = kBlocks < NR ? kBlocks : NR;  // regions per step
        constexpr int kGroups = 8 / kRegions;             // MFMA groups (K sets) per region
        constexpr int kPer = kBlocks / kRegions;          // block decodes per region
        static_assert(8 % kRegions == 0 && kBlocks % kRegions == 0, "regions must split the step evenly");
        auto block_words = [&](int q, uint32_t &wa, uint32_t &wb) {
          const uint4 &piece = next[q >> 2][(q & 3) >> 1];
          wa = (q & 1) ? piece.z : piece.x;
          wb = (q & 1) ? piece.w : piece.y;
        };
        u32x4 bcur[kGroups][TB];
#pragma unroll
        for (int g = 0; g < kGroups; ++g)
#pragma unroll
          for (int tb = 0; tb < TB; ++tb) bcur[g][tb] = read_b(tb, g);
        // The palette seeds of each region's blocks are read one region ahead, so their LDS
        // latency is not on the decode's critical path.
        Seeds seeds[kPer];
#pragma unroll
        for (int e = 0; e < kPer; ++e) {
          uint32_t wa, wb;
          block_words(e, wa, wb);
          seeds[e] = read_seeds(wa, wb, tables);
        }
#pragma unroll
        for (int rg = 0; rg < kRegions; ++rg) {
          if (kStage == 2 && more) stage_part(xn, j + 1, rg * XC / kRegions, (rg + 1) * XC / kRegions);
          u32x4 bnext[kGroups][TB];
          if (rg + 1 < kRegions) {
#pragma unroll
            for (int g = 0; g < kGroups; ++g)
#pragma unroll
              for (int tb = 0; tb < TB; ++tb) bnext[g][tb] = read_b(tb, (rg + 1) * kGroups + g);
          }
          Seeds cur[kPer];
#pragma unroll
          for (int e = 0; e < kPer; ++e) cur[e] = seeds[e];
          if (rg + 1 < kRegions) {
#pragma unroll
            for (int e = 0; e < kPer; ++e) {
              uint32_t na, nb;
              block_words((rg + 1) * kPer + e, na, nb);
              seeds[e] = read_seeds(na, nb, tables);
            }
          }
#pragma unroll
          for (int e = 0; e < kPer; ++e) {
            const int q = rg * kPer + e, b = q >> 2, jj = q & 3;
            uint32_t wa, wb;
            block_words(q, wa, wb);
            uint32_t d[8];
            decode_from_seeds_mode<F16>(cur[e].base, cur[e].end, cur[e].step, cur[e].mode, wa, wb, scale[b], pm[b], d);
            anext[b][2 * jj] = u32x4{d[0], d[1], d[2], d[3]};
            anext[b][2 * jj + 1] = u32x4{d[4], d[5], d[6], d[7]};
          }
#pragma unroll
          for (int g = 0; g < kGroups; ++g)
#pragma unroll
            for (int tb = 0; tb < TB; ++tb)
#pragma unroll
              for (int rb = 0; rb < RB; ++rb)
                acc[tb][rb] = mfma<F16>(acur[rb][rg * kGroups + g], bcur[g][tb], acc[tb][rb]);
#pragma unroll
          for (int e = 0; e < kPer; ++e) {
            const int q = rg * kPer + e, b = q >> 2, jj = q & 3;
            asm volatile("" : "+v"(anext[b][2 * jj]), "+v"(anext[b][2 * jj + 1]));
          }
          __builtin_amdgcn_sched_barrier(0);
          if (rg + 1 < kRegions) {
#pragma unroll
            for (int g = 0; g < kGroups; ++g)
#pragma unroll
              for (int tb = 0; tb < TB; ++tb) bcur[g][tb] = bnext[g][tb];
          }
        }
      }
      step_barrier();
#pragma unroll
      for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int s = 0; s < 8; ++s) acur[b][s] = anext[b][s];
      shift_ring(fresh);
    });
  } else {
    run_steps([&](int j, const uint16_t *xb, uint16_t *xn) {
      uint4 fresh[RB][2];
      load_tiles(fresh, j + LA);
      __builtin_amdgcn_sched_barrier(0);
      if (j + 1 < w.nc) stage_x(xn, j + 1);
      u32x4 a[RB][8];
      decode_step(ring[0], a);
      mfma_step(xb, a);
      step_barrier();
      shift_ring(fresh);
    });
  }

  // acc[tb][b][r] = D[row 8(r/4) + 4h + r%4 of row block b][token tb*32 + r32].
  const uint16_t *bias = static_cast<const uint16_t *>(p.bias);
  if constexpr (SWIGLU) {
    // Each wave pair (gate wave 2q, up wave 2q + 1, the same rows and tokens) splits the SwiGLU
    // work: the gate wave takes accumulator groups e = 4*tb + rq < 2*TB, the up wave the rest. Each
    // hands the groups its partner takes through the first activation buffer ([wave][e'][r][lane],
    // e' counting the handed groups; every LDS access of the K loop ended at its last barrier). The
    // outputs are staged in the second buffer as [BT tokens][64 columns] (128-byte token rows, chunk
    // c at c ^ (token % 8)) and leave in 16-byte chunks.
    float *xch = reinterpret_cast<float *>(xs0);
    const int pair = wave >> 1;
    const bool up = wave & 1;
    constexpr int G = 4 * TB;  // accumulator groups of four rows
#pragma unroll
    for (int e = 0; e < G; ++e) {
      const bool mine = up ? e >= G / 2 : e < G / 2;
      if (!mine) {
        const int slot = up ? e : e - G / 2;
#pragma unroll
        for (int r = 0; r < 4; ++r) xch[((wave * (G / 2) + slot) * 4 + r) * 64 + lane] = acc[e >> 2][0][4 * (e & 3) + r];
      }
    }
    __syncthreads();
    const int inter = p.M / 2;
    const int partner = wave ^ 1;
    const bool staged = (inter & 7) == 0 && (reinterpret_cast<uintptr_t>(p.y) & 15) == 0;
#pragma unroll
    for (int e = 0; e < G; ++e) {
      const bool mine = up ? e >= G / 2 : e < G / 2;
      if (!mine) continue;
      const int tb = e >> 2, rq = e & 3;
      const int slot = up ? e - G / 2 : e;  // where the partner put this group
      const int tl = tb * 32 + r32;
      const int col = 32 * pair + 8 * rq + 4 * h;  // column within the workgroup's 64
      uint16_t outv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float other = xch[((partner * (G / 2) + slot) * 4 + r) * 64 + lane];
        const float own = acc[tb][0][4 * rq + r];
        const int n = min(w.n0 + col + r, inter - 1);
        float gv = round_out<false>(up ? other : own), uv = round_out<false>(up ? own : other);
        if (bias) {
          gv = round_out<false>(gv + bf(bias[n]));
          uv = round_out<false>(uv + bf(bias[inter + n]));
        }
        outv[r] = to_bf(swiglu_value(gv, uv));
      }
      if (staged) {
        *reinterpret_cast<uint2 *>(xs1 + tl * 64 + 8 * ((col >> 3) ^ (tl & 7)) + (col & 7)) =
            make_uint2((uint32_t)outv[0] | ((uint32_t)outv[1] << 16), (uint32_t)outv[2] | ((uint32_t)outv[3] << 16));
      } else {
        const int t = w.t0 + tl;
        if (t < p.tokens) {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (w.n0 + col + r < inter) static_cast<uint16_t *>(p.y)[(size_t)t * inter + w.n0 + col + r] = outv[r];
        }
      }
    }
    if (!staged) return;
    __syncthreads();
#pragma unroll
    for (int it = 0; it < BT * 8 / kThreads; ++it) {
      const int id = it * kThreads + (int)threadIdx.x;
      const int tl = id >> 3, c = id & 7;
      const int t = w.t0 + tl, n = w.n0 + 8 * c;
      if (t < p.tokens && n < inter)
        *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(p.y) + (size_t)t * inter + n) =
            *reinterpret_cast<const uint4 *>(xs1 + tl * 64 + 8 * (c ^ (tl & 7)));
    }
    return;
  }
  if constexpr (RB == 1) {
    const bool f32 = p.ks > 1;
    if (f32 || ((p.M & 7) == 0 && (reinterpret_cast<uintptr_t>(p.y) & 15) == 0)) {
      __syncthreads();  // the activation tiles are free
      uint16_t *buf = f32 && wave >= 2 ? xs1 : xs0;
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) {
        const int tl = tb * 32 + r32;
        const f32x16 &v = acc[tb][0];
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const int row = wave * 32 + 8 * rq + 4 * h;
          if (f32) {
            stage_out32(buf, tl, row, make_float4(v[4 * rq], v[4 * rq + 1], v[4 * rq + 2], v[4 * rq + 3]));
          } else {
            const int n = min(w.n0 + row, p.M - 4);
            stage_out16(buf, tl, row,
                        (uint32_t)out_bits<F16>(v[4 * rq], bias, n) | ((uint32_t)out_bits<F16>(v[4 * rq + 1], bias, n + 1) << 16),
                        (uint32_t)out_bits<F16>(v[4 * rq + 2], bias, n + 2) | ((uint32_t)out_bits<F16>(v[4 * rq + 3], bias, n + 3) << 16));
          }
        }
      }
      __syncthreads();
      if (f32) store_staged<true>(p, w, xs0, xs1, BT, kThreads);
      else store_staged<false>(p, w, xs0, xs1, BT, kThreads);
      return;
    }
  }
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) {
    const int t = w.t0 + tb * 32 + r32;
    if (t >= p.tokens) continue;
#pragma unroll
    for (int b = 0; b < RB; ++b) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int row0 = w.n0 + (wave * RB + b) * 32 + 8 * rq + 4 * h;
        const f32x16 &v = acc[tb][b];
        if (p.ks > 1) {
          float *dst = p.partials + ((size_t)w.split * p.tokens + t) * p.Mp + row0;
          if (row0 < p.Mp) *reinterpret_cast<float4 *>(dst) = make_float4(v[4 * rq], v[4 * rq + 1], v[4 * rq + 2], v[4 * rq + 3]);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int n = row0 + r;
            if (n < p.M) {
              float out = round_out<F16>(v[4 * rq + r]);
              if (bias) out += half_bits_to_float<F16>(bias[n]);
              store_out<F16>(p.y, (size_t)t * p.M + n, out);
            }
          }
        }
      }
    }
  }
}

// Split-group tile (candidate 9 with exactly four K splits, up to 32 tokens, K a multiple of
// 128): a workgroup holds the four splits of one (32-token tile, RBW x 32-row blocks), one per
// wave, and each wave runs its split on its own -- weights decoded in registers as in
// prefill_kernel, activations staged by the wave itself into its own LDS buffers (direct
// buffer-to-LDS loads, 1 KiB contiguous per load) half a step at a time -- so the K loop has no
// workgroup barrier. With RBW = 2 a wave multiplies one staged activation slice by two row blocks
// (two independent MFMA chains): the activations are read from L2 once per 64 rows instead of once
// per 32, which was the kernel's bound (per K column, 32 tokens of bf16 activations are 64 bytes
// against 16 bytes of weights in a 32-row block). At the end the four splits are summed in split order
// through LDS, as prefill_reduce_kernel sums them: no partials leave the workgroup and no reduce
// kernel runs. Same lane layouts, K sets and order as prefill_kernel, hence the same bits.
#ifndef TX_SMALL_WAVE
#define TX_SMALL_WAVE 1
#endif
#ifndef TX_WAVE_RBW2_MIN_WGS
#define TX_WAVE_RBW2_MIN_WGS 256
#endif

template <bool F16, bool LUT, int RBW>
__global__ __launch_bounds__(kThreads) void prefill_wave_kernel(PrefillParams p) {
  static_assert(RBW == 1 || RBW == 2, "one or two 32-row blocks per wave");
  // Per wave, K columns 0-63 (xlo) and 64-127 (xhi) of a step for its 32 tokens: token row r takes
  // 128 bytes, its 16-byte slot q holds columns 8*(q ^ ((r >> 1) % 8)).. +7 of the half (the 16
  // rows one operand read serves per LDS pass then fall on distinct banks: even and odd rows sit in
  // opposite halves of the banks). The two halves are separate LDS objects, so the compiler can
  // tell reads of one from loads into the other.
  __shared__ __attribute__((aligned(16))) uint16_t xlo[4][32 * 64];
  __shared__ __attribute__((aligned(16))) uint16_t xhi[4][32 * 64];
  __shared__ __attribute__((aligned(16))) PaletteTableStorage tables;

  const int lane = threadIdx.x & 63;
  const int split = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // = wave
  const int r32 = lane & 31;
  const int h = lane >> 5;
  const int row_blocks = (p.M + 31) / 32;
  const int row_groups = (row_blocks + RBW - 1) / RBW;
  const int wgs = row_groups * ((p.tokens + 31) / 32);
  const int per_xcd = (wgs + kXcds - 1) / kXcds;
  const int q = (int)(blockIdx.x % kXcds) * per_xcd + (int)(blockIdx.x / kXcds);
  if (q >= wgs) return;
  if constexpr (!LUT) copy_seed_tables(tables, split, lane, kThreads / 64);
  const int rg = q % row_groups;
  const int t0 = (q / row_groups) * 32;
  const int c_begin = (int)((uint32_t)split * (uint32_t)p.CG / 4u);
  const int nc = (int)((uint32_t)(split + 1) * (uint32_t)p.CG / 4u) - c_begin;

  // A operands of row block rb_b = RBW*rg + b (clamped to the last block; a duplicate block is
  // computed, never stored): lane slot (row & 15) + 16h of tile group 2rb_b + (r32 >> 4) (clamped
  // into the matrix; rows past M are computed, never stored), as in prefill_kernel.
  int n0[RBW];
  float scale[RBW];
  uint32_t pm[RBW], tlane[RBW];
  // Weights and activations are read through buffer descriptors (wave-uniform base and step
  // offset, per-lane offset). With only buffer loads in flight the compiler waits for exactly the
  // loads a use needs (vmcnt(N)); global_load_lds in flight beside global loads made it wait for
  // every load (vmcnt(0)) before each use of a weight tile. The tile descriptor starts at tile
  // (gbase, c_begin), gbase = the first group of the wave's first block (<= RG - 1).
  const int gbase = 2 * RBW * rg;
#pragma unroll
  for (int b = 0; b < RBW; ++b) {
    const int rb = min(RBW * rg + b, row_blocks - 1);
    n0[b] = (RBW * rg + b) * 32;
    const int g = min(2 * rb + (r32 >> 4), p.RG - 1);
    scale[b] = p.scales[g * kTileRows + (lane & 15)];
    pm[b] = pm_scale_pair<F16>(scale[b]);
    tlane[b] = (uint32_t)(((g - gbase) * p.CG * 64 + (lane & 15) + 16 * h) * 16);
  }
  const int64_t first_tile = (int64_t)gbase * p.CG + c_begin;
  const int64_t tile_bytes = ((int64_t)p.RG * p.CG - first_tile) * kTileBytes;
  const __amdgpu_buffer_rsrc_t trsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint4 *>(p.tiles + first_tile * 64), (short)0, (int)(tile_bytes < 0x7FFFFFFF ? tile_bytes : 0x7FFFFFFF),
      0x00020000);
  typedef uint4 Tiles[RBW][2];
  // Tiles of step j; past the split's last step (the K loop loads one step ahead whatever is
  // left) through an empty descriptor, whose loads return zeros without touching memory, instead
  // of re-reading the last tiles from HBM once the streaming loads have evicted them.
  const __amdgpu_buffer_rsrc_t none = buffer_rsrc(p.tiles, 0);
  auto load_tiles = [&](Tiles &slot, int j) {
    const bool real = j < nc;
    const int off = __builtin_amdgcn_readfirstlane(real ? j * kTileBytes : 0);
#pragma unroll
    for (int b = 0; b < RBW; ++b) {
      const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(real ? trsrc : none, tlane[b], off, 2 /* nt */);
      const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(real ? trsrc : none, tlane[b], off + 512, 2 /* nt */);
      slot[b][0] = make_uint4(v0.x, v0.y, v0.z, v0.w);
      slot[b][1] = make_uint4(v1.x, v1.y, v1.z, v1.w);
    }
  };

  // Staging of half `hf` of step j (K is a multiple of 128 here): load v brings token rows
  // 8v .. 8v + 7, lane l landing in slot l % 8 of row 8v + l / 8, so it fetches the half's chunk
  // (l % 8) ^ (((8v + l / 8) >> 1) % 8). Rows past the tokens repeat the last token (never stored).
  const uint16_t *x = static_cast<const uint16_t *>(p.x);
  const int srow = lane >> 3;  // row within the load's eight
  uint32_t row_off[4];         // byte offsets of this lane's four token rows and chunks
#pragma unroll
  for (int v = 0; v < 4; ++v)
    row_off[v] = 2u * ((uint32_t)min(t0 + 8 * v + srow, p.tokens - 1) * (uint32_t)p.K +
                       8u * (uint32_t)((lane & 7) ^ ((4 * v + (srow >> 1)) & 7)));
  const int64_t x_bytes = ((int64_t)p.tokens * p.K - (int64_t)c_begin * kTileK) * 2;
  const __amdgpu_buffer_rsrc_t xrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(x + (size_t)c_begin * kTileK), (short)0, (int)(x_bytes < 0x7FFFFFFF ? x_bytes : 0x7FFFFFFF),
      0x00020000);
  auto stage = [&](uint16_t *buf, int j, int hf) {
    const int off = __builtin_amdgcn_readfirstlane((j * kTileK + 64 * hf) * 2);
#pragma unroll
    for (int v = 0; v < 4; ++v)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xrsrc, (__attribute__((address_space(3))) void *)(buf + 8 * v * 64), 16,
                                               row_off[v], off, 0, 0);
  };
  // B operand of MFMA 4*hf + s (s < 4): columns 32h + 16*(s>>1) + 8*(s&1) .. +7 of half hf.
  auto read_b = [&](const uint16_t *buf, int s) {
    return *reinterpret_cast<const u32x4 *>(buf + r32 * 64 + 8 * ((4 * h + s) ^ ((r32 >> 1) & 7)));
  };

  uint16_t *mylo = xlo[split];
  uint16_t *myhi = xhi[split];
  Tiles ta, tb;  // weight tiles of the even and the odd steps
  stage(mylo, 0, 0);
  load_tiles(ta, 0);
  stage(myhi, 0, 1);
  if constexpr (!LUT) {
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();  // the seed tables
  }

  f32x16 acc[RBW];
#pragma unroll
  for (int b = 0; b < RBW; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[b][r] = 0.f;

  // Block jj of row block b's weight tile into that block's MFMAs 2jj, 2jj + 1.
  auto words = [](const Tiles &tile, int b, int jj, uint32_t &wa, uint32_t &wb) {
    const uint4 &piece = tile[b][jj >> 1];
    wa = (jj & 1) ? piece.z : piece.x;
    wb = (jj & 1) ? piece.w : piece.y;
  };
  // Block jj of row block b's weight tile into that block's MFMAs 2jj, 2jj + 1 (palette seeds
  // already read from the LDS tables, or the palette row from p.lut).
  auto block = [&](const Tiles &tile, int b, int jj, const Seeds &sd, const u32x4 &b0, const u32x4 &b1) {
    uint32_t wa, wb, d[8];
    words(tile, b, jj, wa, wb);
    if constexpr (LUT) {
      const float4 *row = p.lut + 2 * (size_t)palette_row(wa, wb);
      decode_from_palette<F16>(row[0], row[1], wa, wb, scale[b], d);
    } else {
      decode_from_seeds_mode<F16>(sd.base, sd.end, sd.step, sd.mode, wa, wb, scale[b], pm[b], d);
    }
    acc[b] = mfma<F16>(u32x4{d[0], d[1], d[2], d[3]}, b0, acc[b]);
    acc[b] = mfma<F16>(u32x4{d[4], d[5], d[6], d[7]}, b1, acc[b]);
  };
  // Step j multiplies weight tiles `cur` (loaded during step j - 1) and loads tiles j + 1 into
  // `next`. Each half buffer is read into registers together with the palette seeds of the half's
  // blocks (one LDS wait for both, so no seed read waits inside a decode), then refilled with the
  // next step's half while this step's blocks are decoded and multiplied. Loads are issued low
  // half (4), weights (2 RBW), high half (4): 4 + 2 RBW later loads stay in flight at each half
  // buffer's wait.
  constexpr int kLaterLoads = 4 + 2 * RBW;
  constexpr int kHalfWait = 0x0F70 | kLaterLoads;  // vmcnt(kLaterLoads), lgkmcnt and expcnt free
  auto half = [&](int jn, int jt, int hf, uint16_t *buf, const Tiles &cur, Tiles &next) {
    u32x4 bv[4];
    Seeds sd[2][RBW];
    __builtin_amdgcn_s_waitcnt(kHalfWait);  // this half of step j has landed
#pragma unroll
    for (int s = 0; s < 4; ++s) bv[s] = read_b(buf, s);
    if constexpr (!LUT) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
#pragma unroll
        for (int b = 0; b < RBW; ++b) {
          uint32_t wa, wb;
          words(cur, b, 2 * hf + jj, wa, wb);
          sd[jj][b] = read_seeds(wa, wb, tables);
        }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the reads are done before the refill
    __builtin_amdgcn_sched_barrier(0);
    stage(buf, jn, hf);
    if (hf == 0) load_tiles(next, jt);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int b = 0; b < RBW; ++b) block(cur, b, 2 * hf + jj, sd[jj][b], bv[2 * jj], bv[2 * jj + 1]);
  };
  auto step = [&](int j, const Tiles &cur, Tiles &next) {
    const int jn = min(j + 1, nc - 1);
    half(jn, j + 1, 0, mylo, cur, next);
    half(jn, j + 1, 1, myhi, cur, next);
  };
  int j = 0;
  for (; j + 2 <= nc; j += 2) {
    step(j, ta, tb);
    step(j + 1, tb, ta);
  }
  if (j < nc) step(j, ta, tb);

  // acc[b][r] = D[row 8(r/4) + 4h + r%4 of block b][token t0 + r32]. The four splits are summed in
  // split order from zero through each wave's buffers (after its last refill has landed), two
  // blocks at a time (block 2i in the low buffer, 2i + 1 in the high one); wave w finishes rows
  // 8w + 4h .. + 3 of each block.
  const int t = t0 + r32;
  const uint16_t *bias = static_cast<const uint16_t *>(p.bias);
  uint16_t *y = static_cast<uint16_t *>(p.y) + (size_t)min(t, p.tokens - 1) * p.M;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
  for (int b0 = 0; b0 < RBW; b0 += 2) {
    if (b0 > 0) __syncthreads();  // the previous pair's sums are read
#pragma unroll
    for (int b = b0; b < b0 + 2 && b < RBW; ++b) {
      float *mine = reinterpret_cast<float *>(b == b0 ? mylo : myhi);
#pragma unroll
      for (int r = 0; r < 16; ++r) mine[r * 64 + lane] = acc[b][r];
    }
    __syncthreads();
    if (t < p.tokens) {
#pragma unroll
      for (int b = b0; b < b0 + 2 && b < RBW; ++b) {
        const int n = n0[b] + 8 * split + 4 * h;
        uint32_t out[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float total = 0.f;
#pragma unroll
          for (int s = 0; s < 4; ++s)
            total += reinterpret_cast<const float *>(b == b0 ? xlo[s] : xhi[s])[(4 * split + r) * 64 + lane];
          out[r] = n + r < p.M ? out_bits<F16>(total, bias, n + r) : 0u;
        }
        if (n + 3 < p.M && ((reinterpret_cast<uintptr_t>(y + n) & 7) == 0)) {
          *reinterpret_cast<uint2 *>(y + n) = make_uint2(out[0] | (out[1] << 16), out[2] | (out[3] << 16));
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < p.M) y[n + r] = (uint16_t)out[r];
        }
      }
    }
  }
}

// Pair-shared tile: 8 waves, 256 tokens x 128 rows. Waves w and w + 4 own the same 32-row block
// (rb = w % 4) for token halves 0 and 1. Per K step each of the two decodes only the blocks of
// one 64-wide half of the step (h2 = its token half, MFMAs s = 4*h2 .. 4*h2 + 3) and hands the
// operands to its partner through LDS, so a weight is decoded once per 256 tokens while every
// SIMD keeps two waves. MFMA order per accumulator is the other tiles' (s = 0..7 per step), so
// the results are bitwise equal to theirs. Palette seeds are computed in registers: the two
// activation buffers (64 KiB each) and the operand exchange (32 KiB) fill the 160 KiB of LDS.
constexpr int kPairThreads = 512;
// Scheduling regions per K step of the pair-shared tile (each 8/kPairRegions MFMA groups; the two
// block decodes go to the first region of each half of the step).
#ifndef TX_PAIR_REGIONS
#define TX_PAIR_REGIONS 4
#endif
constexpr int kPairRegions = TX_PAIR_REGIONS;
#ifndef TX_PAIR_LA
#define TX_PAIR_LA TX_PREFILL_LA
#endif

template <bool F16, int LA, bool LUT>
__global__ __launch_bounds__(kPairThreads) void prefill_pair_kernel(PrefillParams p) {
  static_assert(LA >= 2, "the pipelined K loop needs two weight tiles in flight");
  constexpr int BT = 256, BN = 128, TBH = 4;  // tokens, rows, 32-token blocks per wave
  constexpr int XC = BT * 16 / kPairThreads;  // 16-byte activation chunks staged per thread per step
  constexpr int NS = LA - 1;                  // weight pieces held between steps
  __shared__ __attribute__((aligned(16))) uint16_t xs0[BT * kTileK];
  __shared__ __attribute__((aligned(16))) uint16_t xs1[BT * kTileK];
  __shared__ u32x4 xch[4][2][4][64];  // [row block][K half][MFMA of the half][lane]

  WorkItem w;
  if (!work_item(p, BT, BN, w)) return;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rb = wave & 3;
  const int half = wave >> 2;
  const int r32 = lane & 31;
  const int h = lane >> 5;
  const uint16_t *x = static_cast<const uint16_t *>(p.x);
  auto k_offset = [&](int s) { return 64 * (s >> 2) + 32 * h + 16 * ((s >> 1) & 1) + 8 * (s & 1); };

  // This wave's piece of each step: lane slot (row & 15) + 16h + 32*half of the row block's tiles,
  // i.e. blocks 4*half + 2h (words x, y) and 4*half + 2h + 1 (words z, w) of row l % 32.
  const int g = min(w.n0 / kTileRows + rb * 2 + (r32 >> 4), p.RG - 1);
  const int g0 = min(w.n0 / kTileRows + rb * 2, p.RG - 1);  // wave-uniform, <= g
  const __amdgpu_buffer_rsrc_t trsrc = tile_rsrc(p, g0, w.c_begin);
  const uint32_t tlane = (uint32_t)(((g - g0) * p.CG * 64 + (lane & 15) + 16 * h + 32 * half) * 16);
  const float scale = p.scales[g * kTileRows + (lane & 15)];
  const uint32_t pm = pm_scale_pair<F16>(scale);
  auto load_piece = [&](int j) {
    return load_weights16(trsrc, tlane, __builtin_amdgcn_readfirstlane(min(j, w.nc - 1) * kTileBytes));
  };
  // Operands a[2jj + e] = positions 8e..8e+7 of local block jj (MFMA s = 4*half + 2jj + e).
  auto decode_one = [&](const uint4 &piece, int jj, u32x4 (&a)[4]) {
    const uint32_t wa = jj ? piece.z : piece.x;
    const uint32_t wb = jj ? piece.w : piece.y;
    uint32_t d[8];
    if constexpr (LUT) {
      const float4 *row = p.lut + 2 * (size_t)palette_row(wa, wb);
      decode_from_palette<F16>(row[0], row[1], wa, wb, scale, d);
    } else {
      decode_block<F16>(wa, wb, scale, pm, d);
    }
    a[2 * jj] = u32x4{d[0], d[1], d[2], d[3]};
    a[2 * jj + 1] = u32x4{d[4], d[5], d[6], d[7]};
  };

  // Activation staging as in prefill_kernel, 512 threads: thread i stages row 32v + i/16 into
  // slot i % 16 (row % 16 = (i/16) % 16).
  const int srow = threadIdx.x >> 4;
  const int scol = ((threadIdx.x & 15) ^ (srow & 15)) * 8;
  const bool tile_full = w.t0 + BT <= p.tokens;
  const uint32_t lane_off = (uint32_t)(srow * p.K + scol) * 2;
  const __amdgpu_buffer_rsrc_t xrsrc =
      buffer_rsrc(x + (size_t)w.t0 * p.K, (int64_t)min(BT, p.tokens - w.t0) * p.K * 2);
  auto stage_part = [&](uint16_t *buf, int j, int v0, int v1) {
    const int c = w.c_begin + j;
    if ((c + 1) * kTileK <= p.K) {
#pragma unroll
      for (int v = v0; v < v1; ++v) {
        const int row0 = tile_full ? w.t0 + 32 * v : min(w.t0 + 32 * v, p.tokens - 1);
        const int base = __builtin_amdgcn_readfirstlane(((row0 - w.t0) * p.K + c * kTileK) * 2);
        uint32_t off = lane_off;
        if (!tile_full) off = (uint32_t)((min(w.t0 + 32 * v + srow, p.tokens - 1) - row0) * p.K + scol) * 2;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            xrsrc, (__attribute__((address_space(3))) void *)(buf + (32 * v + 4 * wave) * kTileK), 16, off, base, 0, 0);
      }
    } else if (v0 == 0) {
      // Columns past K are staged as zeros (an offset past the descriptor's end reads zeros).
      const int k = c * kTileK + scol;
#pragma unroll 2
      for (int v = 0; v < XC; ++v) {
        const int t = min(w.t0 + 32 * v + srow, p.tokens - 1);
        const uint32_t off = k < p.K ? (uint32_t)((t - w.t0) * p.K + k) * 2 : 0x7FFFFFF0u;
        const u32x4 value = __builtin_amdgcn_raw_buffer_load_b128(xrsrc, off, 0, 0);
        *reinterpret_cast<u32x4 *>(buf + (32 * v + srow) * kTileK + (threadIdx.x & 15) * 8) = value;
      }
    }
  };
  auto full_barrier = [&]() { asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };
  auto lds_barrier = [&]() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

  // Prologue: step 0's activations and the first weight pieces.
  stage_part(xs0, 0, 0, XC);
  __builtin_amdgcn_sched_barrier(0);
  const uint4 first = load_piece(0);
  uint4 ring[NS];
#pragma unroll
  for (int u = 0; u < NS; ++u) ring[u] = load_piece(u + 1);
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();

  auto run = [&](auto half_c) {
    constexpr int HALF = decltype(half_c)::value;
    f32x16 acc[TBH];
#pragma unroll
    for (int tb = 0; tb < TBH; ++tb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[tb][r] = 0.f;
    // Operands of the step being multiplied: this wave's half and its partner's.
    u32x4 aown[4], apar[4];
    decode_one(first, 0, aown);
    decode_one(first, 1, aown);
#pragma unroll
    for (int sl = 0; sl < 4; ++sl) xch[rb][HALF][sl][lane] = aown[sl];
    full_barrier();
#pragma unroll
    for (int sl = 0; sl < 4; ++sl) apar[sl] = xch[rb][1 - HALF][sl][lane];
    lds_barrier();
    auto operand = [&](int s) -> const u32x4 & { return (s >> 2) == HALF ? aown[s & 3] : apar[s & 3]; };

    auto step = [&](int j, const uint16_t *xb, uint16_t *xn) {
      const bool more = j + 1 < w.nc;
      const uint4 fresh = load_piece(j + LA);
      __builtin_amdgcn_sched_barrier(0);
      const uint4 next = ring[0];  // piece of step j+1 (past the end: the clamped last piece)
      auto read_b = [&](int tb, int s) {
        return *reinterpret_cast<const u32x4 *>(xb + (128 * HALF + 32 * tb + r32) * kTileK +
                                                8 * ((k_offset(s) >> 3) ^ (r32 & 15)));
      };
      constexpr int NRG = kPairRegions, SG = 8 / NRG;  // regions, MFMA groups per region
      u32x4 anext[4];
      u32x4 bcur[SG][TBH];
#pragma unroll
      for (int e = 0; e < SG; ++e)
#pragma unroll
        for (int tb = 0; tb < TBH; ++tb) bcur[e][tb] = read_b(tb, e);
#pragma unroll
      for (int rg = 0; rg < NRG; ++rg) {
        if (more) stage_part(xn, j + 1, rg * XC / NRG, (rg + 1) * XC / NRG);
        u32x4 bnext[SG][TBH];
        if (rg + 1 < NRG) {
#pragma unroll
          for (int e = 0; e < SG; ++e)
#pragma unroll
            for (int tb = 0; tb < TBH; ++tb) bnext[e][tb] = read_b(tb, SG * (rg + 1) + e);
        }
        const bool dec = rg % (NRG / 2) == 0;  // first region of each half of the step
        const int jj = rg / (NRG / 2);
        if (dec) decode_one(next, jj, anext);
#pragma unroll
        for (int e = 0; e < SG; ++e)
#pragma unroll
          for (int tb = 0; tb < TBH; ++tb) acc[tb] = mfma<F16>(operand(SG * rg + e), bcur[e][tb], acc[tb]);
        if (dec) asm volatile("" : "+v"(anext[2 * jj]), "+v"(anext[2 * jj + 1]));
        __builtin_amdgcn_sched_barrier(0);
        if (rg + 1 < NRG) {
#pragma unroll
          for (int e = 0; e < SG; ++e)
#pragma unroll
            for (int tb = 0; tb < TBH; ++tb) bcur[e][tb] = bnext[e][tb];
        }
      }
      // Hand over the next step's operands: written before the step's barrier, read after it, and
      // a second barrier before they are overwritten a step later.
#pragma unroll
      for (int sl = 0; sl < 4; ++sl) xch[rb][HALF][sl][lane] = anext[sl];
      full_barrier();
#pragma unroll
      for (int sl = 0; sl < 4; ++sl) {
        aown[sl] = anext[sl];
        apar[sl] = xch[rb][1 - HALF][sl][lane];
      }
      lds_barrier();
#pragma unroll
      for (int u = 0; u + 1 < NS; ++u) ring[u] = ring[u + 1];
      ring[NS - 1] = fresh;
    };
    int j0 = 0;
    for (; j0 + 2 <= w.nc; j0 += 2) {
      step(j0, xs0, xs1);
      step(j0 + 1, xs1, xs0);
    }
    if (j0 < w.nc) step(j0, xs0, xs1);

    // acc[tb][r] = D[row 8(r/4) + 4h + r%4 of row block rb][token 128*HALF + 32*tb + r32].
    const uint16_t *bias = static_cast<const uint16_t *>(p.bias);
    const bool f32 = p.ks > 1;
    if (f32 || ((p.M & 7) == 0 && (reinterpret_cast<uintptr_t>(p.y) & 15) == 0)) {
      __syncthreads();  // the activation tiles are free
      uint16_t *buf = f32 && rb >= 2 ? xs1 : xs0;
#pragma unroll
      for (int tb = 0; tb < TBH; ++tb) {
        const int tl = 128 * HALF + 32 * tb + r32;
        const f32x16 &v = acc[tb];
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const int row = rb * 32 + 8 * rq + 4 * h;
          if (f32) {
            stage_out32(buf, tl, row, make_float4(v[4 * rq], v[4 * rq + 1], v[4 * rq + 2], v[4 * rq + 3]));
          } else {
            const int n = min(w.n0 + row, p.M - 4);
            stage_out16(buf, tl, row,
                        (uint32_t)out_bits<F16>(v[4 * rq], bias, n) | ((uint32_t)out_bits<F16>(v[4 * rq + 1], bias, n + 1) << 16),
                        (uint32_t)out_bits<F16>(v[4 * rq + 2], bias, n + 2) | ((uint32_t)out_bits<F16>(v[4 * rq + 3], bias, n + 3) << 16));
          }
        }
      }
      __syncthreads();
      if (f32) store_staged<true>(p, w, xs0, xs1, BT, kPairThreads);
      else store_staged<false>(p, w, xs0, xs1, BT, kPairThreads);
      return;
    }
#pragma unroll
    for (int tb = 0; tb < TBH; ++tb) {
      const int t = w.t0 + 128 * HALF + tb * 32 + r32;
      if (t >= p.tokens) continue;
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int row0 = w.n0 + rb * 32 + 8 * rq + 4 * h;
        const f32x16 &v = acc[tb];
        if (p.ks > 1) {
          float *dst = p.partials + ((size_t)w.split * p.tokens + t) * p.Mp + row0;
          if (row0 < p.Mp) *reinterpret_cast<float4 *>(dst) = make_float4(v[4 * rq], v[4 * rq + 1], v[4 * rq + 2], v[4 * rq + 3]);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int n = row0 + r;
            if (n < p.M) {
              float out = round_out<F16>(v[4 * rq + r]);
              if (bias) out += half_bits_to_float<F16>(bias[n]);
              store_out<F16>(p.y, (size_t)t * p.M + n, out);
            }
          }
        }
      }
    }
  };
  if (half == 0) run(std::integral_constant<int, 0>{});
  else run(std::integral_constant<int, 1>{});
}

// Wide tile: 512 tokens x 128 rows, so that at 512 tokens every weight is decoded once. K runs in
// half steps of 64 columns (MFMAs s = 4q .. 4q + 3 of step column c, q = 0, 1: the other tiles'
// K sets and order, so the results are bitwise equal to theirs).
//   * decode: the workgroup's threads share the 512 blocks of a half step (2 or 1 each, seeds in
//     registers) and write the 16-bit weights to an LDS tile [128 rows][64 columns];
//   * activations: [512 tokens][64 columns] staged by direct global-to-LDS loads (a 1 KiB wave
//     load covers 8 tokens x 128 bytes);
//   * each wave multiplies its row blocks (A from the weight tile) by its 128 tokens (4 token
//     blocks, B from the activation tile), so each LDS operand read feeds several MFMAs.
// Both LDS tiles store the 16-byte chunk c of row (or token) r at chunk c ^ ((r >> 1) & 7) of the
// 128-byte row: the 16 lanes one LDS pass serves then hit distinct banks.
// Weight and activation tiles are double-buffered (160 KiB); one barrier per half step, before
// which every load issued during the previous half step completes.
// Waves per workgroup of the wide tile: 4 (one per SIMD, each wave all 128 rows x 128 tokens)
// or 8 (two per SIMD, each wave 64 rows x 128 tokens).
#ifndef TX_WIDE_WAVES
#define TX_WIDE_WAVES 8
#endif
constexpr int kWideWaves = TX_WIDE_WAVES;
constexpr int kWideThreads = 64 * kWideWaves;
constexpr int kHalfK = kTileK / 2;

// KFULL: K is a multiple of 128 (no staging of columns past K).
// SWIGLU: p holds a merged [gate | up] matrix (M = 2 * inter, inter a multiple of 16, one K
// split, bf16): the workgroup's 128 rows are gate rows n0..n0+63 and the matching up rows, as row
// blocks [gate 0-31 | up 0-31 | gate 32-63 | up 32-63], so each wave holds a gate accumulator and
// the up accumulator of the same rows and tokens; the epilogue writes
// y[t][n] = bf16(silu(G) * U) for inter columns, with G and U the bf16 outputs the plain epilogue
// would store (bias added with its second rounding) -- the bits of the GEMM followed by the
// SwiGLU kernel, without the [tokens][2 * inter] intermediate.
template <bool F16, bool LUT, bool KFULL, bool SWIGLU = false>
__global__ __launch_bounds__(kWideThreads) void prefill_wide_kernel(PrefillParams p) {
  static_assert(!SWIGLU || !F16, "the SwiGLU epilogue is bf16");
  constexpr int WV = kWideWaves;
  static_assert(WV == 4 || WV == 8, "4 or 8 waves");
  constexpr int BT = 512, BN = 128;
  constexpr int TW = 4, RW = 16 / WV;   // token and row blocks (of 32) per wave
  constexpr int NRG = 4 / RW;           // row groups: wave w owns row group w % NRG, tokens w / NRG
  constexpr int DEC = 512 / (64 * WV);  // blocks each thread decodes per half step (2 or 1)
  constexpr int XV = BT * kHalfK * 2 / (kWideThreads * 16);  // direct loads per thread per half step
  constexpr int NMF = TW * RW;          // MFMAs per slice
  constexpr int NRD = TW + RW;          // operand reads per slice
  using Piece = std::conditional_t<DEC == 2, u32x4, u32x2>;
  __shared__ __attribute__((aligned(128))) uint16_t ws0[BN * kHalfK];
  __shared__ __attribute__((aligned(128))) uint16_t ws1[BN * kHalfK];
  __shared__ __attribute__((aligned(128))) uint16_t xs0[BT * kHalfK];
  __shared__ __attribute__((aligned(128))) uint16_t xs1[BT * kHalfK];

  WorkItem w;
  if (!work_item(p, BT, SWIGLU ? BN / 2 : BN, w, SWIGLU ? p.M / 2 : -1)) return;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rg = wave % NRG, tg = wave / NRG;
  const int r32 = lane & 31;
  const int h = lane >> 5;
  const int sw = (r32 >> 1) & 7;  // swizzle of every row and token this lane reads
  const uint16_t *x = static_cast<const uint16_t *>(p.x);
  const int nh = 2 * w.nc;  // half steps

  // Decode assignment. A half step of the 128 rows is 8 tiles x 32 slots of 16 bytes (slot
  // (row % 16) + 16*sub of tile column c's half q holds blocks 2*sub, 2*sub + 1 of that half of
  // the row). With 4 waves thread i owns slot i (both blocks); with 8 waves threads 2j and 2j + 1
  // own block 0 and 1 of slot j. Rows past M are clamped into the matrix (computed, never stored).
  const int slot = DEC == 2 ? (int)threadIdx.x : (int)(threadIdx.x >> 1);
  const int sub = (slot >> 4) & 1;
  const int drow = 16 * (slot >> 5) + (slot & 15);  // row within the 128
  int g;
  if constexpr (SWIGLU) {
    // 16-row group q of the workgroup: row block q / 2 (gate if even, up if odd) of pair q / 4
    const int q = slot >> 5, half_rg = p.RG / 2;
    const int gate_rg = min(w.n0 / kTileRows + 2 * (q >> 2) + (q & 1), half_rg - 1);
    g = gate_rg + (((q >> 1) & 1) ? half_rg : 0);
  } else {
    g = min(w.n0 / kTileRows + (slot >> 5), p.RG - 1);
  }
  const uint4 *gt = p.tiles + ((size_t)g * p.CG + w.c_begin) * 64 + (slot & 15) + 16 * sub;
  const float scale = p.scales[g * kTileRows + (slot & 15)];
  const uint32_t pm = pm_scale_pair<F16>(scale);
  auto load_piece = [&](int u) {
    const int v = min(u, nh - 1);
    const uint4 *ptr = gt + (size_t)(v >> 1) * 64 + 32 * (v & 1);
    if constexpr (DEC == 2) return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(ptr));
    else return __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(ptr) + (threadIdx.x & 1));
  };
  // Decode block jj (0, 1) of the slot: the 16-bit weights of its two 16-byte chunks of the weight
  // tile (chunk 4*sub + 2*jj + e holds positions 8e..8e+7).
  auto decode_piece = [&](const Piece &piece, int jj, u32x4 (&out)[2]) __attribute__((always_inline)) {
    const uint32_t wa = DEC == 2 && jj ? piece[2] : piece[0];
    const uint32_t wb = DEC == 2 && jj ? piece[3] : piece[1];
    uint32_t d[8];
    if constexpr (LUT) {
      const float4 *row = p.lut + 2 * (size_t)palette_row(wa, wb);
      decode_from_palette<F16>(row[0], row[1], wa, wb, scale, d);
    } else {
      decode_block<F16>(wa, wb, scale, pm, d);
    }
    out[0] = u32x4{d[0], d[1], d[2], d[3]};
    out[1] = u32x4{d[4], d[5], d[6], d[7]};
  };
  // Byte offset of this thread's chunk 4*sub (swizzled) in a weight buffer; chunk 4*sub + 2*jj + e
  // is at that offset ^ 16*(2*jj + e) (the buffers are 128-byte aligned, so the XOR only touches
  // the chunk index bits).
  const uint32_t wrow = (uint32_t)(drow * kHalfK * 2 + 16 * ((4 * sub) ^ ((drow >> 1) & 7)));
  auto lds_addr = [](const uint16_t *ptr) { return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint16_t *)ptr; };
  // The weight stores are inline assembly: the compiler cannot tell them apart from the direct
  // loads in flight to the activation buffer and would wait for those loads before each store.
  // The barrier of the half step waits for them (lgkmcnt(0)). The offset is made opaque here so
  // that the four addresses are derived at each store instead of being held (or spilled) across
  // the K loop.
  auto store_chunks = [&](uint16_t *wn, int jj, const u32x4 (&v)[2]) __attribute__((always_inline)) {
    uint32_t o = wrow;
    asm volatile("" : "+v"(o));
    const uint32_t base = lds_addr(wn);
    asm volatile("ds_write_b128 %0, %1" ::"v"(base + (o ^ (32u * jj))), "v"(v[0]));
    asm volatile("ds_write_b128 %0, %1" ::"v"(base + (o ^ (32u * jj + 16u))), "v"(v[1]));
  };
  // The blocks this thread decodes per half step, and where: slice 2*i for block i.
  auto my_block = [&](int i) { return DEC == 2 ? i : (int)(threadIdx.x & 1); };

  // Direct load v of this wave fills tokens 8*(WV*v + wave) .. +7 of the activation tile; lane l
  // lands in physical chunk l%8 of token l/8 there, so it fetches logical chunk
  // (l%8) ^ ((token >> 1) & 7) = (l%8) ^ (4*(wave%2) + l/16).
  const int xl_tok = lane >> 3;
  const int xl_chunk = (lane & 7) ^ (4 * (wave & 1) + (lane >> 4));
  const bool tile_full = w.t0 + BT <= p.tokens;  // uniform: no token past the input
  const uint32_t lane_off = (uint32_t)(xl_tok * p.K + 8 * xl_chunk) * 2;
  auto stage = [&](uint16_t *xn, int u) __attribute__((always_inline)) {
    const int c = w.c_begin + (u >> 1);
    const int k0 = c * kTileK + kHalfK * (u & 1);
    if (KFULL || k0 + kHalfK <= p.K) {
#pragma unroll
      for (int v = 0; v < XV; ++v) {
        const int tok0 = 8 * (WV * v + wave);
        const int row0 = tile_full ? w.t0 + tok0 : min(w.t0 + tok0, p.tokens - 1);
        const char *base = reinterpret_cast<const char *>(x + ((size_t)row0 * p.K + k0));
        uint32_t off = lane_off;
        if (!tile_full) off = (uint32_t)((min(w.t0 + tok0 + xl_tok, p.tokens - 1) - row0) * p.K + 8 * xl_chunk) * 2;
        __builtin_amdgcn_global_load_lds((const void *)(base + off),
                                         (__attribute__((address_space(3))) void *)(xn + tok0 * kHalfK), 16, 0, 0);
      }
    } else {
      // The matrix's last K columns: chunks past K are staged as zeros (K is a multiple of 16,
      // so a chunk of 8 columns is wholly inside or outside).
      const int k = k0 + 8 * xl_chunk;
#pragma unroll 2
      for (int v = 0; v < XV; ++v) {
        const int tok = 8 * (WV * v + wave) + xl_tok;
        const int t = min(w.t0 + tok, p.tokens - 1);
        uint4 value = make_uint4(0u, 0u, 0u, 0u);
        if (k < p.K) value = *reinterpret_cast<const uint4 *>(x + (size_t)t * p.K + k);
        *reinterpret_cast<uint4 *>(xn + tok * kHalfK + 8 * (lane & 7)) = value;
      }
    }
  };

  // Prologue: half step 0's activations and weights, half step 1's activations and the pieces
  // of half steps 1 and 2.
  stage(xs0, 0);
  __builtin_amdgcn_sched_barrier(0);
  const Piece first = load_piece(0);
  Piece next = load_piece(1);
  stage(xs1, 1);  // nh >= 2: every split has at least one tile column
  __builtin_amdgcn_sched_barrier(0);
  Piece fresh = load_piece(2);
#pragma unroll
  for (int i = 0; i < DEC; ++i) {
    u32x4 v[2];
    decode_piece(first, my_block(i), v);
    store_chunks(ws0, my_block(i), v);
  }
  asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" : "+v"(next), "+v"(fresh) : : "memory");

  f32x16 acc[TW][RW];
#pragma unroll
  for (int tb = 0; tb < TW; ++tb)
#pragma unroll
    for (int rb = 0; rb < RW; ++rb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[tb][rb][r] = 0.f;

  // Operand reads of slice sl (0..3) of a half step.
  auto read_a = [&](const uint16_t *wb, int rb, int sl) {
    return *reinterpret_cast<const u32x4 *>(wb + (32 * (RW * rg + rb) + r32) * kHalfK + 8 * ((4 * h + sl) ^ sw));
  };
  auto read_b = [&](const uint16_t *xb, int tb, int sl) {
    return *reinterpret_cast<const u32x4 *>(xb + (128 * tg + 32 * tb + r32) * kHalfK + 8 * ((4 * h + sl) ^ sw));
  };

  // Operands of the slice being multiplied; slice 0 of half step 0 first.
  u32x4 a[RW], b[TW];
#pragma unroll
  for (int rb = 0; rb < RW; ++rb) a[rb] = read_a(ws0, rb, 0);
#pragma unroll
  for (int tb = 0; tb < TW; ++tb) b[tb] = read_b(xs0, tb, 0);

  // One half step u, multiplying buffers (wb, xb) while the weights of half step u + 1 are
  // decoded into wn: four regions, one per slice, each holding the slice's MFMAs, the next
  // slice's LDS reads (in the region's first MFMAs, so they land before the region ends) and, in
  // slice 2i, the decode of this thread's block i of `next` (the piece of half step u + 1),
  // interleaved by scheduling groups; the decoded chunks are stored after the region's MFMAs.
  // The barrier sits halfway through slice 3: it waits for every load and LDS access issued
  // before it. Then, while the rest of slice 3's MFMAs run, the operands of half step u + 1's
  // slice 0 are read, the direct loads of half step u + 2 go to the buffer just released (xb)
  // and the piece of half step u + 3 is loaded: each load has a whole half step to land.
  // Empty statements right after the barrier redefine `fresh` (the piece of half step u + 2) and
  // the slice-3 operands still to be used, so the compiler does not wait for the loads and reads
  // issued after the barrier before it uses them.
  auto half_step = [&](int u, const uint16_t *wb, uint16_t *xb, uint16_t *wn, const uint16_t *xn) __attribute__((always_inline)) {
#pragma unroll
    for (int sl = 0; sl < 3; ++sl) {
      u32x4 an[RW], bn[TW];
#pragma unroll
      for (int rb = 0; rb < RW; ++rb) an[rb] = read_a(wb, rb, sl + 1);
#pragma unroll
      for (int tb = 0; tb < TW; ++tb) bn[tb] = read_b(xb, tb, sl + 1);
      const bool dec = (sl & 1) == 0 && (sl >> 1) < DEC;
      u32x4 dv[2];
      if (dec) decode_piece(next, my_block(sl >> 1), dv);
#pragma unroll
      for (int tb = 0; tb < TW; ++tb)
#pragma unroll
        for (int rb = 0; rb < RW; ++rb) acc[tb][rb] = mfma<F16>(a[rb], b[tb], acc[tb][rb]);
      // The reads two per MFMA from the first MFMA on; a decode's VALU spread over the MFMAs.
#pragma unroll
      for (int i = 0; i < NMF; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (2 * i < NRD) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        if (dec && 2 * i < NRD) __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
        if (dec && 2 * i >= NRD) __builtin_amdgcn_sched_group_barrier(0x002, WV == 4 ? 5 : 8, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (dec) store_chunks(wn, my_block(sl >> 1), dv);
#pragma unroll
      for (int rb = 0; rb < RW; ++rb) a[rb] = an[rb];
#pragma unroll
      for (int tb = 0; tb < TW; ++tb) b[tb] = bn[tb];
    }
    // Slice 3: token blocks 0-1, the barrier, the next half step's loads, token blocks 2-3.
#pragma unroll
    for (int tb = 0; tb < TW / 2; ++tb)
#pragma unroll
      for (int rb = 0; rb < RW; ++rb) acc[tb][rb] = mfma<F16>(a[rb], b[tb], acc[tb][rb]);
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    asm volatile("" : "+v"(fresh));
#pragma unroll
    for (int rb = 0; rb < RW; ++rb) asm volatile("" : "+v"(a[rb]));
#pragma unroll
    for (int tb = TW / 2; tb < TW; ++tb) asm volatile("" : "+v"(b[tb]));
    next = fresh;
    __builtin_amdgcn_sched_barrier(0);
    // Past the end the reads take buffers that were never staged (unused), and the staging
    // repeats the last half step into the released buffer (never read again).
    u32x4 an[RW], bn[TW];
#pragma unroll
    for (int rb = 0; rb < RW; ++rb) an[rb] = read_a(wn, rb, 0);
#pragma unroll
    for (int tb = 0; tb < TW; ++tb) bn[tb] = read_b(xn, tb, 0);
    stage(xb, min(u + 2, nh - 1));
    fresh = load_piece(u + 3);
#pragma unroll
    for (int tb = TW / 2; tb < TW; ++tb)
#pragma unroll
      for (int rb = 0; rb < RW; ++rb) acc[tb][rb] = mfma<F16>(a[rb], b[tb], acc[tb][rb]);
    // (MFMA, 2 reads, loads) from the first MFMA on; the reads land while the last MFMAs run.
#pragma unroll
    for (int i = 0; i < NMF / 2; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (2 * i < NRD) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x010, (XV + 1 + NMF / 2 - 1) / (NMF / 2), 0);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int rb = 0; rb < RW; ++rb) a[rb] = an[rb];
#pragma unroll
    for (int tb = 0; tb < TW; ++tb) b[tb] = bn[tb];
  };
  for (int u = 0; u < nh; u += 2) {
    half_step(u, ws0, xs0, ws1, xs1);
    half_step(u + 1, ws1, xs1, ws0, xs0);
  }
  // The last half step's repeated staging lands before the workgroup's LDS is released.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // acc[tb][rb][r] = D[row 8(r/4) + 4h + r%4 of row block RW*rg + rb][token 128*tg + 32*tb + r32].
  const uint16_t *bias = static_cast<const uint16_t *>(p.bias);
  // 16-bit outputs leave through LDS where whole 16-byte chunks can be stored: each lane holds four
  // consecutive rows of one token, so direct stores would be 2-byte writes to a different token row
  // per lane. Staged, a token's outputs are contiguous and every store covers 8 columns.
  const bool staged = p.ks == 1 && ((SWIGLU ? p.M / 2 : p.M) & 7) == 0 && (reinterpret_cast<uintptr_t>(p.y) & 15) == 0;
  if (staged) __syncthreads();  // every operand read of the K loop is done: the activation tiles are free
  if constexpr (SWIGLU) {
    // Row blocks RW*rg + 2i (gate) and + 1 (up) cover gate-space rows 32*(RW/2*rg + i) of the 64.
    const int inter = p.M / 2;
    if (staged) {
      // Tile [512 tokens][64 columns] in xs0: token row of 128 bytes, chunk c (8 columns) at c ^ (token % 8).
#pragma unroll
      for (int tb = 0; tb < TW; ++tb) {
        const int tl = 128 * tg + 32 * tb + r32;
#pragma unroll
        for (int i = 0; i < RW / 2; ++i) {
          __builtin_amdgcn_sched_barrier(0);
          const f32x16 &vg = acc[tb][2 * i], &vu = acc[tb][2 * i + 1];
#pragma unroll
          for (int rq = 0; rq < 4; ++rq) {
            const int col = 32 * (RW / 2 * rg + i) + 8 * rq + 4 * h;  // column within the 64
            uint32_t packed[2];
#pragma unroll
            for (int r = 0; r < 4; r += 2) {
              uint16_t pair[2];
#pragma unroll
              for (int e = 0; e < 2; ++e) {
                const int n = min(w.n0 + col + r + e, inter - 1);
                float gv = round_out<false>(vg[4 * rq + r + e]), uv = round_out<false>(vu[4 * rq + r + e]);
                if (bias) {
                  gv = round_out<false>(gv + bf(bias[n]));
                  uv = round_out<false>(uv + bf(bias[inter + n]));
                }
                pair[e] = to_bf(swiglu_value(gv, uv));
              }
              packed[r / 2] = (uint32_t)pair[0] | ((uint32_t)pair[1] << 16);
            }
            *reinterpret_cast<uint2 *>(xs0 + tl * 64 + 8 * ((col >> 3) ^ (tl & 7)) + (col & 7)) =
                make_uint2(packed[0], packed[1]);
          }
        }
      }
      __syncthreads();
#pragma unroll
      for (int it = 0; it < BT * 8 / kWideThreads; ++it) {
        const int id = it * kWideThreads + (int)threadIdx.x;
        const int tl = id >> 3, c = id & 7;
        const int t = w.t0 + tl, n = w.n0 + 8 * c;
        if (t < p.tokens && n < inter)
          *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(p.y) + (size_t)t * inter + n) =
              *reinterpret_cast<const uint4 *>(xs0 + tl * 64 + 8 * (c ^ (tl & 7)));
      }
      return;
    }
#pragma unroll
    for (int tb = 0; tb < TW; ++tb) {
      const int t = w.t0 + 128 * tg + tb * 32 + r32;
      if (t >= p.tokens) continue;
#pragma unroll
      for (int i = 0; i < RW / 2; ++i) {
        __builtin_amdgcn_sched_barrier(0);
        const f32x16 &vg = acc[tb][2 * i], &vu = acc[tb][2 * i + 1];
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int n = w.n0 + 32 * (RW / 2 * rg + i) + 8 * rq + 4 * h + r;
            if (n < inter) {
              float gv = round_out<false>(vg[4 * rq + r]), uv = round_out<false>(vu[4 * rq + r]);
              if (bias) {
                gv = round_out<false>(gv + bf(bias[n]));
                uv = round_out<false>(uv + bf(bias[inter + n]));
              }
              static_cast<uint16_t *>(p.y)[(size_t)t * inter + n] = to_bf(swiglu_value(gv, uv));
            }
          }
        }
      }
    }
    return;
  }
  if (staged) {
    // Tile [512 tokens][128 rows]: tokens 0-255 in xs0, 256-511 in xs1 (which one is uniform per
    // wave); a token row of 256 bytes, chunk c (rows 8c..8c+7) at c ^ (token % 16).
    uint16_t *half_tile = tg < 2 ? xs0 : xs1;
#pragma unroll
    for (int tb = 0; tb < TW; ++tb) {
      const int tl = (128 * tg + 32 * tb + r32) & 255;
#pragma unroll
      for (int rb = 0; rb < RW; ++rb) {
        __builtin_amdgcn_sched_barrier(0);
        const f32x16 &v = acc[tb][rb];
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const int row = 32 * (RW * rg + rb) + 8 * rq + 4 * h;  // row within the 128
          uint32_t packed[2];
#pragma unroll
          for (int r = 0; r < 4; r += 2) {
            uint16_t pair[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              float out = round_out<F16>(v[4 * rq + r + e]);
              if (bias) out += half_bits_to_float<F16>(bias[min(w.n0 + row + r + e, p.M - 1)]);
              pair[e] = F16 ? __builtin_bit_cast(uint16_t, (_Float16)out) : to_bf(out);
            }
            packed[r / 2] = (uint32_t)pair[0] | ((uint32_t)pair[1] << 16);
          }
          *reinterpret_cast<uint2 *>(half_tile + tl * 128 + 8 * ((row >> 3) ^ (tl & 15)) + (row & 7)) =
              make_uint2(packed[0], packed[1]);
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < BT * 16 / kWideThreads; ++it) {
      const int id = it * kWideThreads + (int)threadIdx.x;
      const int tl = id >> 4, c = id & 15;
      const int t = w.t0 + tl, n = w.n0 + 8 * c;
      if (t < p.tokens && n < p.M)
        *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(p.y) + (size_t)t * p.M + n) =
            *reinterpret_cast<const uint4 *>((tl < 256 ? xs0 : xs1) + (tl & 255) * 128 + 8 * (c ^ (tl & 15)));
    }
    return;
  }
#pragma unroll
  for (int tb = 0; tb < TW; ++tb) {
    const int t = w.t0 + 128 * tg + tb * 32 + r32;
    if (t >= p.tokens) continue;
#pragma unroll
    for (int rb = 0; rb < RW; ++rb) {
      __builtin_amdgcn_sched_barrier(0);  // one accumulator at a time: no spills
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int row0 = w.n0 + 32 * (RW * rg + rb) + 8 * rq + 4 * h;
        const f32x16 &v = acc[tb][rb];
        if (p.ks > 1) {
          float *dst = p.partials + ((size_t)w.split * p.tokens + t) * p.Mp + row0;
          if (row0 < p.Mp) *reinterpret_cast<float4 *>(dst) = make_float4(v[4 * rq], v[4 * rq + 1], v[4 * rq + 2], v[4 * rq + 3]);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int n = row0 + r;
            if (n < p.M) {
              float out = round_out<F16>(v[4 * rq + r]);
              if (bias) out += half_bits_to_float<F16>(bias[n]);
              store_out<F16>(p.y, (size_t)t * p.M + n, out);
            }
          }
        }
      }
    }
  }
}

// y[t][m] = round(sum over splits in order of partials[s][t][m]), then the bias with a second
// rounding (the reference's epilogue order); bf16, or fp16 with F16.
// KS > 0: exactly KS splits, every partial loaded before the first add (a runtime loop waited
// for memory once per split); KS = 0: any count.
template <bool F16, int KS>
__global__ __launch_bounds__(256) void prefill_reduce_kernel(PrefillParams p) {
  const int m = blockIdx.x * 256 + threadIdx.x;
  const int t = blockIdx.y;
  if (m >= p.M) return;
  // the bias goes out with the partials (from a valid address whether or not there is one)
  const uint16_t b = (p.bias ? static_cast<const uint16_t *>(p.bias) : reinterpret_cast<const uint16_t *>(p.partials))[m];
  float total = 0.f;
  const float *src = p.partials + (size_t)t * p.Mp + m;
  const size_t stride = (size_t)p.tokens * p.Mp;
  if constexpr (KS > 0) {
    float v[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) v[s] = src[s * stride];
#pragma unroll
    for (int s = 0; s < KS; ++s) total += v[s];
  } else {
    for (int s = 0; s < p.ks; ++s) total += src[s * stride];
  }
  float out = round_out<F16>(total);
  if (p.bias) out += half_bits_to_float<F16>(b);
  store_out<F16>(p.y, (size_t)t * p.M + m, out);
}

struct Candidate {
  const char *name;
  int bt, bn, bk;
  const void *fn;
  hipError_t (*launch)(const PrefillParams &, hipStream_t);
  int lds;
  int threads;
};

// The ordered reduction of the split-K partials, after the tile kernel.
template <bool F16>
void launch_reduce_as(const PrefillParams &p, hipStream_t stream) {
  const dim3 grid((p.M + 255) / 256, p.tokens);
  switch (p.ks) {
    case 2: hipLaunchKernelGGL((prefill_reduce_kernel<F16, 2>), grid, dim3(256), 0, stream, p); break;
    case 3: hipLaunchKernelGGL((prefill_reduce_kernel<F16, 3>), grid, dim3(256), 0, stream, p); break;
    case 4: hipLaunchKernelGGL((prefill_reduce_kernel<F16, 4>), grid, dim3(256), 0, stream, p); break;
    default: hipLaunchKernelGGL((prefill_reduce_kernel<F16, 0>), grid, dim3(256), 0, stream, p); break;
  }
}

hipError_t launch_reduce(const PrefillParams &p, hipStream_t stream) {
  if (p.f16) launch_reduce_as<true>(p, stream);
  else launch_reduce_as<false>(p, stream);
  return hipGetLastError();
}

template <int LA>
hipError_t launch_pair(const PrefillParams &p, hipStream_t stream) {
  const int items = ((p.M + 127) / 128) * ((p.tokens + 255) / 256) * p.ks;
  const int grid = ((items + kXcds - 1) / kXcds) * kXcds;
  if (p.lut) {
    if (p.f16)
      hipLaunchKernelGGL((prefill_pair_kernel<true, LA, true>), dim3(grid), dim3(kPairThreads), 0, stream, p);
    else
      hipLaunchKernelGGL((prefill_pair_kernel<false, LA, true>), dim3(grid), dim3(kPairThreads), 0, stream, p);
  } else if (p.f16) {
    hipLaunchKernelGGL((prefill_pair_kernel<true, LA, false>), dim3(grid), dim3(kPairThreads), 0, stream, p);
  } else {
    hipLaunchKernelGGL((prefill_pair_kernel<false, LA, false>), dim3(grid), dim3(kPairThreads), 0, stream, p);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.ks == 1 || p.no_reduce) return e;
  return launch_reduce(p, stream);
}

template <bool F16, bool LUT>
void launch_wide_as(const PrefillParams &p, int grid, hipStream_t stream) {
  if (p.K % kTileK == 0)
    hipLaunchKernelGGL((prefill_wide_kernel<F16, LUT, true>), dim3(grid), dim3(kWideThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((prefill_wide_kernel<F16, LUT, false>), dim3(grid), dim3(kWideThreads), 0, stream, p);
}

hipError_t launch_wide(const PrefillParams &p, hipStream_t stream) {
  const int items = ((p.M + 127) / 128) * ((p.tokens + 511) / 512) * p.ks;
  const int grid = ((items + kXcds - 1) / kXcds) * kXcds;
  if (p.lut) {
    if (p.f16) launch_wide_as<true, true>(p, grid, stream);
    else launch_wide_as<false, true>(p, grid, stream);
  } else if (p.f16) {
    launch_wide_as<true, false>(p, grid, stream);
  } else {
    launch_wide_as<false, false>(p, grid, stream);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.ks == 1 || p.no_reduce) return e;
  return launch_reduce(p, stream);
}

template <bool LUT>
void launch_wide_swiglu_as(const PrefillParams &p, int grid, hipStream_t stream) {
  if (p.K % kTileK == 0)
    hipLaunchKernelGGL((prefill_wide_kernel<false, LUT, true, true>), dim3(grid), dim3(kWideThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((prefill_wide_kernel<false, LUT, false, true>), dim3(grid), dim3(kWideThreads), 0, stream, p);
}

template <int TB, int RB, int LA, bool PIPE>
hipError_t launch_tile(const PrefillParams &p, hipStream_t stream) {
  constexpr int BT = 32 * TB, BN = 128 * RB;
  const int items = ((p.M + BN - 1) / BN) * ((p.tokens + BT - 1) / BT) * p.ks;
  const int grid = ((items + kXcds - 1) / kXcds) * kXcds;
  if (p.lut) {
    if (p.f16)
      hipLaunchKernelGGL((prefill_kernel<true, TB, RB, LA, PIPE, true>), dim3(grid), dim3(kThreads), 0, stream, p);
    else
      hipLaunchKernelGGL((prefill_kernel<false, TB, RB, LA, PIPE, true>), dim3(grid), dim3(kThreads), 0, stream, p);
  } else if (p.f16) {
    hipLaunchKernelGGL((prefill_kernel<true, TB, RB, LA, PIPE, false>), dim3(grid), dim3(kThreads), 0, stream, p);
  } else {
    hipLaunchKernelGGL((prefill_kernel<false, TB, RB, LA, PIPE, false>), dim3(grid), dim3(kThreads), 0, stream, p);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.ks == 1 || p.no_reduce) return e;
  return launch_reduce(p, stream);
}

template <bool F16, bool LUT>
void launch_wave_as(const PrefillParams &p, hipStream_t stream) {
  // Two row blocks per wave when that still gives every CU of the MI355X (256) a workgroup
  // (measured: gate 5120 -> 27648 at 32 tokens 35.0 -> 27.6 us; three blocks per wave, 288
  // workgroups, 35.9 us; four, 216 workgroups, 31.5 us).
  const int row_blocks = (p.M + 31) / 32, token_tiles = (p.tokens + 31) / 32;
  const int wide = (row_blocks + 1) / 2 * token_tiles;
  if (wide >= TX_WAVE_RBW2_MIN_WGS) {
    hipLaunchKernelGGL((prefill_wave_kernel<F16, LUT, 2>), dim3((wide + kXcds - 1) / kXcds * kXcds), dim3(kThreads), 0,
                       stream, p);
  } else {
    const int wgs = row_blocks * token_tiles;
    hipLaunchKernelGGL((prefill_wave_kernel<F16, LUT, 1>), dim3((wgs + kXcds - 1) / kXcds * kXcds), dim3(kThreads), 0,
                       stream, p);
  }
}

// Candidate 9: the split-group tile where a workgroup holds all four K splits of a 32- or 64-row
// block (exactly four splits, up to 32 tokens, K a multiple of 128, partials not wanted by the
// caller): no reduce launch. Elsewhere the register-decoding 32-token tile, which was faster with
// split partials (down 27648 -> 5120 at 32 tokens: 40.1 vs 42.0 us). Both give the same bits.
hipError_t launch_small(const PrefillParams &p, hipStream_t stream) {
  if (!TX_SMALL_WAVE || p.ks != 4 || p.tokens > 32 || p.K % kTileK != 0 || p.no_reduce)
    return launch_tile<1, 1, TX_PREFILL_LA_PLAIN, false>(p, stream);
  if (p.lut) {
    if (p.f16) launch_wave_as<true, true>(p, stream);
    else launch_wave_as<false, true>(p, stream);
  } else if (p.f16) {
    launch_wave_as<true, false>(p, stream);
  } else {
    launch_wave_as<false, false>(p, stream);
  }
  return hipGetLastError();  // the four splits are summed in the tile
}

#define TX_CANDIDATE(NAME, TB, RB, LA, PIPE)                                                            \
  Candidate {                                                                                          \
    NAME, 32 * (TB), 128 * (RB), kTileK, reinterpret_cast<const void *>(&prefill_kernel<false, TB, RB, LA, PIPE, false>), \
        &launch_tile<TB, RB, LA, PIPE>, 2 * 32 * (TB) * kTileK * 2, kThreads                          \
  }

// The 256- and 128-token tiles pipeline their K loop; the smaller tiles run it plainly.
const Candidate kCandidates[] = {
    Candidate{"large_256x128x128", 256, 128, kTileK,
              reinterpret_cast<const void *>(&prefill_pair_kernel<false, TX_PAIR_LA, false>),
              &launch_pair<TX_PAIR_LA>, 2 * 256 * kTileK * 2 + 4 * 2 * 4 * 64 * 16, kPairThreads},
    TX_CANDIDATE("medium_128x128x128", 4, 1, TX_PREFILL_LA, true),
    Candidate{"wide_512x128x64", 512, 128, kHalfK,
              reinterpret_cast<const void *>(&prefill_wide_kernel<false, false, true>),
              &launch_wide, 2 * (512 + 128) * kHalfK * 2, kWideThreads},
    TX_CANDIDATE("medium_64x128x128", 2, 1, TX_PREFILL_LA_PLAIN, false),
    Candidate{"small_32x128x128", 32, 128, kTileK,
              reinterpret_cast<const void *>(&prefill_kernel<false, 1, 1, TX_PREFILL_LA_PLAIN, false, false>),
              &launch_small, 2 * 32 * kTileK * 2, kThreads},
};

const Candidate *find(int candidate) {
  if (candidate < kPrefillFirst || candidate > kPrefillLast) return nullptr;
  return &kCandidates[candidate - kPrefillFirst];
}

// Workgroups of each candidate that one CU holds at once (its compiled registers and LDS), queried
// once; 1 if the runtime cannot say.
const std::array<int, kPrefillLast - kPrefillFirst + 1> &resident_per_cu() {
  static const std::array<int, kPrefillLast - kPrefillFirst + 1> table = [] {
    std::array<int, kPrefillLast - kPrefillFirst + 1> out{};
    for (size_t i = 0; i < out.size(); ++i) {
      int n = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kCandidates[i].fn, kCandidates[i].threads, 0) != hipSuccess ||
          n < 1) {
        (void)hipGetLastError();
        n = 1;
      }
      out[i] = n;
    }
    return out;
  }();
  return table;
}

}  // namespace

int prefill_default_candidate(int M, int K, int64_t tokens, int cus) {
  if (tokens <= 32) return 9;   // small_32x128x128
  if (tokens <= 64) return 8;   // medium_64x128x128
  if (tokens < 256) return 6;   // medium_128x128x128
  const int CG = (K + kTileK - 1) / kTileK;
  // K splits of a one-workgroup-per-CU tile with `items` workgroups per split (the rule of
  // prefill_splits).
  auto splits = [&](int64_t items) {
    int64_t ks = std::max<int64_t>(1, cus / items);
    ks = std::min<int64_t>(ks, std::max(1, CG / 8));
    return std::min(ks, std::max<int64_t>(1, (int64_t(32) << 20) / (tokens * (int64_t)((M + 15) / 16 * 16) * 4)));
  };
  // The 512-token wide tile from 384 tokens (at most a quarter of its MFMA work past the
  // tokens) when its workgroups make one round of the CUs at least three quarters full, or
  // several rounds at least four fifths full on average.
  if (tokens >= 384) {
    const int64_t wi = (int64_t)((M + 127) / 128) * ((tokens + 511) / 512);
    if (wi > (int64_t)cus) {
      if (5 * wi >= 4 * (int64_t)cus * ((wi + cus - 1) / cus)) return 7;
    } else if (4 * wi * splits(wi) >= 3 * (int64_t)cus) {
      return 7;
    }
  }
  // The pair-shared 256x128 tile (one workgroup per CU) when its workgroups, K splits included,
  // make one round of the CUs at least three quarters full; otherwise the 128x128 tile, whose
  // finer grain fills sparse grids and the last of several rounds better.
  const int64_t items = (int64_t)((M + 127) / 128) * ((tokens + 255) / 256);
  if (items > (int64_t)cus) return 6;
  return 4 * items * splits(items) >= 3 * (int64_t)cus ? 5 : 6;
}

int prefill_splits(int M, int CG, int64_t tokens, int cus) {
  // Candidate-independent, so that every tile gives the same sums, and sized for the default tile
  // of this shape: as many splits as keep all of its workgroups resident at once, each split at
  // least 8 tile columns long, partials at most 32 MiB.
  const int dc = prefill_default_candidate(M, CG * kTileK, tokens, cus);
  const Candidate *c = find(dc);
  const int64_t items = ((M + c->bn - 1) / c->bn) * ((tokens + c->bt - 1) / c->bt);
  const int64_t slots = (int64_t)resident_per_cu()[dc - kPrefillFirst] * cus;
  int64_t ks = std::max<int64_t>(1, slots / items);
  ks = std::min<int64_t>(ks, std::max(1, CG / 8));
  const int64_t cap = std::max<int64_t>(1, (int64_t(32) << 20) / (tokens * (int64_t)((M + 15) / 16 * 16) * 4));
  ks = std::min(ks, cap);
  ks = std::min<int64_t>(ks, std::max(1, 0x7FFFFFFF / std::max(CG, 1)));  // the kernels' 32-bit split arithmetic
  return (int)std::max<int64_t>(1, ks);
}

bool prefill_candidate_eligible(int candidate, int M, int K) {
  return find(candidate) != nullptr && M > 0 && K > 0 && K % 16 == 0;
}

template <int TB, int LA, bool PIPE>
hipError_t launch_tile_swiglu(const PrefillParams &p, hipStream_t stream) {
  const int items = ((p.M / 2 + 63) / 64) * ((p.tokens + 32 * TB - 1) / (32 * TB));
  const int grid = ((items + kXcds - 1) / kXcds) * kXcds;
  if (p.lut)
    hipLaunchKernelGGL((prefill_kernel<false, TB, 1, LA, PIPE, true, true>), dim3(grid), dim3(kThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((prefill_kernel<false, TB, 1, LA, PIPE, false, true>), dim3(grid), dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

bool prefill_swiglu_supported(int candidate) { return candidate >= 6 && candidate <= 9; }

hipError_t launch_prefill_swiglu(const PrefillParams &p, int candidate, hipStream_t stream) {
  if (p.f16 || p.ks != 1 || p.M % 32 != 0) return hipErrorInvalidValue;
  switch (candidate) {
    case 6: return launch_tile_swiglu<4, TX_PREFILL_LA, true>(p, stream);
    case 8: return launch_tile_swiglu<2, TX_PREFILL_LA_PLAIN, false>(p, stream);
    case 9: return launch_tile_swiglu<1, TX_PREFILL_LA_PLAIN, false>(p, stream);
    case 7: {
      const int items = ((p.M / 2 + 63) / 64) * ((p.tokens + 511) / 512);
      const int grid = ((items + kXcds - 1) / kXcds) * kXcds;
      if (p.lut) launch_wide_swiglu_as<true>(p, grid, stream);
      else launch_wide_swiglu_as<false>(p, grid, stream);
      return hipGetLastError();
    }
    default: return hipErrorInvalidValue;
  }
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

int prefill_resident_per_cu(int candidate) {
  return find(candidate) ? resident_per_cu()[candidate - kPrefillFirst] : 0;
}

void prefill_candidate_shape(int candidate, int *tokens, int *rows, int *k) {
  const Candidate *c = find(candidate);
  *tokens = c ? c->bt : 0;
  *rows = c ? c->bn : 0;
  *k = c ? c->bk : 0;
}

}  // namespace tx
