// BC4 device layout and ALU decoder for gfx950.
//
// Reference semantics (paths in the reference checkout):
//   block format  texelator/encoder.py:105-117 -- [e0:i8][e1:i8][48-bit selectors, 3 bits each,
//                 position p at bits 3p..3p+2]; position p of block b is input column 16b+p
//                 (texelator/cuda/texelator_cuda.cu:127-131).
//   decoded value texelator/cuda/texelator_cuda.cu:141-152 -- bf16_rne(palette * scale[row]),
//                 fp32 product.
//
// The palette is computed in registers instead of sampled from texture hardware:
//   endpoints clamped to [-127,127]; base = RN(e0/127), end = RN(e1/127);
//   e0 > e1 : step = RN((e1-e0)/889); P[s] = fma(s-1, step, base), s = 2..7
//   e0 <= e1: step = RN((e1-e0)/635); P[s] = fma(s-1, step, base), s = 2..5; P[6] = -1, P[7] = +1.
// Correctly rounded quotients use q = fma(n, RHI, n*RLO) with RHI = RN(1/d), RLO = RN(1/d - RHI);
// this is exact-rounded for every |n| <= 889 and d in {127, 635, 889} (checked exhaustively).
//
// Device block (8 bytes, two little-endian dwords A, B), written by the host repack:
//   A byte c (c = 0..3): bits 0-2 = sel[4+c],  bits 3-4 = bits 2c..2c+1 of eb0,  bits 5-7 = sel[c]
//   B byte c:            bits 0-2 = sel[12+c], bits 3-4 = bits 2c..2c+1 of eb1,  bits 5-7 = sel[8+c]
// with eb = clamp(e, -127, 127) + 127. Selector groups ((A>>5) & 0x07070707, A & 0x07070707, ...)
// are then ready-made v_perm_b32 byte selectors for four positions each, and one v_dot4 of
// A & 0x18181818 with weights 1,4,16,64 gives 8*eb0: a byte offset into a table of 8-byte entries.
//
// Tile layout: rows padded to a multiple of 16, blocks per row padded to a multiple of 8. A tile
// is 16 rows x 8 blocks = 1 KiB; tile (g, c) sits at ((g * CG) + c) * 1 KiB. Inside a tile, lane
// l (0..63) owns 16 contiguous bytes: row 16g + (l & 15), blocks 8c + 2(l >> 4) and +1. One
// wave-wide 128-bit load therefore reads one whole contiguous tile.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tx {

constexpr int kTileRows = 16;
constexpr int kTileBlocks = 8;
constexpr int kTileBytes = 1024;
constexpr int kTileK = kTileBlocks * 16;  // 128 input columns per tile

// Reciprocal pairs (hi = RN(1/d), lo = RN(1/d - hi)) for the correctly rounded quotients.
constexpr float kInv127Hi = 0x1.020408p-7f;
constexpr float kInv127Lo = 0x1.020408p-35f;
constexpr float kInv889Hi = 0x1.26e00ap-10f;
constexpr float kInv889Lo = -0x1.91ff6cp-35f;
constexpr float kInv635Hi = 0x1.9cd34p-10f;
constexpr float kInv635Lo = 0x1.9cd34p-38f;
// The same pairs pre-divided by 8, because the register endpoint extraction yields 8*e (the
// scaling by 2^3 is exact, so results are unchanged).
constexpr float kR127Hi = kInv127Hi / 8.0f;
constexpr float kR127Lo = kInv127Lo / 8.0f;
constexpr float kR889Hi = kInv889Hi / 8.0f;
constexpr float kR889Lo = kInv889Lo / 8.0f;
constexpr float kR635Hi = kInv635Hi / 8.0f;
constexpr float kR635Lo = kInv635Lo / 8.0f;

// Device block whose endpoints are 0/0 and selectors 0: decodes to zero weights (padding).
constexpr uint32_t kZeroBlockWord = 0x08181818u;

// One reference block (8 bytes: e0, e1, 48-bit little-endian selector field) -> device words
// A, B (layout above). Endpoint byte -128 is clamped to -127 as the decoder does. Used by the
// host repack and by the device repack kernel, so both produce identical tiles.
__host__ __device__ inline void encode_device_block(const uint8_t *blk, uint32_t &a, uint32_t &b) {
  int e0 = (int)(int8_t)blk[0];
  int e1 = (int)(int8_t)blk[1];
  e0 = e0 < -127 ? -127 : e0;
  e1 = e1 < -127 ? -127 : e1;
  const uint32_t eb0 = (uint32_t)(e0 + 127);
  const uint32_t eb1 = (uint32_t)(e1 + 127);
  uint64_t bits = 0;
  for (int i = 0; i < 6; ++i) bits |= (uint64_t)blk[2 + i] << (8 * i);
  a = 0;
  b = 0;
  for (int c = 0; c < 4; ++c) {
    const uint32_t s0 = (uint32_t)(bits >> (3 * c)) & 7u;
    const uint32_t s1 = (uint32_t)(bits >> (3 * (4 + c))) & 7u;
    const uint32_t s2 = (uint32_t)(bits >> (3 * (8 + c))) & 7u;
    const uint32_t s3 = (uint32_t)(bits >> (3 * (12 + c))) & 7u;
    a |= (s1 | (((eb0 >> (2 * c)) & 3u) << 3) | (s0 << 5)) << (8 * c);
    b |= (s3 | (((eb1 >> (2 * c)) & 3u) << 3) | (s2 << 5)) << (8 * c);
  }
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Streaming 128-bit load of one lane's tile slot (weights are read once per call).
__device__ __forceinline__ uint4 load_stream(const uint4 *ptr) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(ptr));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2 v = {(__bf16)a, (__bf16)b};  // v_cvt_pk_bf16_f32, round-to-nearest-even
  return __builtin_bit_cast(uint32_t, v);
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  f16x2 v = {(_Float16)a, (_Float16)b};  // v_cvt_pk_f16_f32, round-to-nearest-even
  return __builtin_bit_cast(uint32_t, v);
}

// Two fp32 weights rounded to the 16-bit weight type: bf16 (the BF16 path) or fp16 (the FP16
// path, texelator_cuda.cu:624).
template <bool F16>
__device__ __forceinline__ uint32_t pack_weights(float a, float b) {
  if constexpr (F16) return pack_f16x2(a, b);
  else return pack_bf16x2(a, b);
}

// 8*e from the 2-bit fields in bits 3-4 of each byte (dot4 with weights 1,4,16,64 and a
// wrapping bias of -127*8).
__device__ __forceinline__ float endpoint_x8(uint32_t word) {
  return (float)(int)__builtin_amdgcn_udot4(word & 0x18181818u, 0x40100401u, 0xFFFFFC08u, false);
}

struct Palette {
  float p[8];
  bool eight;
};

// The fp32 palette of one block (the values a LUT row holds).
__device__ __forceinline__ Palette palette8(uint32_t a, uint32_t b) {
  Palette out;
  float f0 = endpoint_x8(a);
  float f1 = endpoint_x8(b);
  float d = f1 - f0;
  out.eight = f0 > f1;
  float rhi = out.eight ? kR889Hi : kR635Hi;
  float rlo = out.eight ? kR889Lo : kR635Lo;
  float step = __builtin_fmaf(d, rhi, d * rlo);
  float base = __builtin_fmaf(f0, kR127Hi, f0 * kR127Lo);
  float end = __builtin_fmaf(f1, kR127Hi, f1 * kR127Lo);
  out.p[0] = base;
  out.p[1] = end;
  out.p[2] = base + step;
  out.p[3] = __builtin_fmaf(2.0f, step, base);
  out.p[4] = __builtin_fmaf(3.0f, step, base);
  out.p[5] = __builtin_fmaf(4.0f, step, base);
  out.p[6] = out.eight ? __builtin_fmaf(5.0f, step, base) : -1.0f;
  out.p[7] = out.eight ? __builtin_fmaf(6.0f, step, base) : 1.0f;
  return out;
}

// Packed 16-bit pair (-scale, +scale): slots 6 and 7 of a 6-value block.
template <bool F16 = false>
__device__ __forceinline__ uint32_t pm_scale_pair(float scale) { return pack_weights<F16>(-scale, scale); }

// The 16 packed weights of one block from its 8 scaled palette values packed in pairs (pk01 =
// values 0 and 1, ...). w[j] holds positions 2j (low half) and 2j+1 (high half).
__device__ __forceinline__ void select_weights(uint32_t pk01, uint32_t pk23, uint32_t pk45, uint32_t pk67, uint32_t a,
                                               uint32_t b, uint32_t w[8]) {
  // Byte tables: low and high bytes of the eight 16-bit values.
  uint32_t lo0 = perm(pk23, pk01, 0x06040200u);
  uint32_t hi0 = perm(pk23, pk01, 0x07050301u);
  uint32_t lo1 = perm(pk67, pk45, 0x06040200u);
  uint32_t hi1 = perm(pk67, pk45, 0x07050301u);
  uint32_t sel[4] = {(a >> 5) & 0x07070707u, a & 0x07070707u, (b >> 5) & 0x07070707u,
                     b & 0x07070707u};
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    uint32_t l = perm(lo1, lo0, sel[g]);
    uint32_t h = perm(hi1, hi0, sel[g]);
    w[2 * g] = perm(h, l, 0x05010400u);
    w[2 * g + 1] = perm(h, l, 0x07030602u);
  }
}

// Packed 16-bit weights (bf16, or fp16 with F16) of one block from its fp32 palette seeds.
// mode: all ones in 8-value mode (e0 > e1), zero in 6-value mode; pm: the 6-value mode's slots 6
// and 7 (pm_scale_pair of the same type), merged in with one bitfield insert.
template <bool F16 = false>
__device__ __forceinline__ void decode_from_seeds_mode(float base, float end, float step, uint32_t mode, uint32_t a,
                                                       uint32_t b, float scale, uint32_t pm, uint32_t w[8]) {
  float p2 = base + step;
  float p3 = __builtin_fmaf(2.0f, step, base);
  float p4 = __builtin_fmaf(3.0f, step, base);
  float p5 = __builtin_fmaf(4.0f, step, base);
  float p6 = __builtin_fmaf(5.0f, step, base);
  float p7 = __builtin_fmaf(6.0f, step, base);
  uint32_t pk01 = pack_weights<F16>(base * scale, end * scale);
  uint32_t pk23 = pack_weights<F16>(p2 * scale, p3 * scale);
  uint32_t pk45 = pack_weights<F16>(p4 * scale, p5 * scale);
  uint32_t pk67 = pack_weights<F16>(p6 * scale, p7 * scale);
  pk67 = (pk67 & mode) | (pm & ~mode);  // v_bfi_b32
  select_weights(pk01, pk23, pk45, pk67, a, b, w);
}

// The same with the mode as a flag (seeds computed in registers).
template <bool F16 = false>
__device__ __forceinline__ void decode_from_seeds(float base, float end, float step, bool eight, uint32_t a,
                                                  uint32_t b, float scale, uint32_t pm, uint32_t w[8]) {
  float p2 = base + step;
  float p3 = __builtin_fmaf(2.0f, step, base);
  float p4 = __builtin_fmaf(3.0f, step, base);
  float p5 = __builtin_fmaf(4.0f, step, base);
  float p6 = __builtin_fmaf(5.0f, step, base);
  float p7 = __builtin_fmaf(6.0f, step, base);
  uint32_t pk01 = pack_weights<F16>(base * scale, end * scale);
  uint32_t pk23 = pack_weights<F16>(p2 * scale, p3 * scale);
  uint32_t pk45 = pack_weights<F16>(p4 * scale, p5 * scale);
  uint32_t pk67 = pack_weights<F16>(p6 * scale, p7 * scale);
  pk67 = eight ? pk67 : pm;
  select_weights(pk01, pk23, pk45, pk67, a, b, w);
}

// Packed 16-bit weights of one block whose 8 palette values come from a table row (LUT mode:
// any palette, e.g. one measured from another GPU's texture unit): round(P[s] * scale).
template <bool F16 = false>
__device__ __forceinline__ void decode_from_palette(float4 p03, float4 p47, uint32_t a, uint32_t b, float scale,
                                                    uint32_t w[8]) {
  select_weights(pack_weights<F16>(p03.x * scale, p03.y * scale), pack_weights<F16>(p03.z * scale, p03.w * scale),
                 pack_weights<F16>(p47.x * scale, p47.y * scale), pack_weights<F16>(p47.z * scale, p47.w * scale), a, b, w);
}

// Row of a block's endpoint pair in a 255 x 255 x 8 palette table, (e1 + 127) * 255 + (e0 + 127)
// (the probe layout), from the device words' 2-bit endpoint fields.
__device__ __forceinline__ uint32_t palette_row(uint32_t a, uint32_t b) {
  const uint32_t eb0 = __builtin_amdgcn_udot4(a & 0x18181818u, 0x40100401u, 0u, false) >> 3;
  const uint32_t eb1 = __builtin_amdgcn_udot4(b & 0x18181818u, 0x40100401u, 0u, false) >> 3;
  return eb1 * 255u + eb0;
}

// Decode one device block to 16 weights (bf16, or fp16 with F16), palette seeds computed in
// registers.
template <bool F16 = false>
__device__ __forceinline__ void decode_block(uint32_t a, uint32_t b, float scale, uint32_t pm,
                                             uint32_t w[8]) {
  float f0 = endpoint_x8(a);
  float f1 = endpoint_x8(b);
  float d = f1 - f0;
  bool eight = f0 > f1;
  float rhi = eight ? kR889Hi : kR635Hi;
  float rlo = eight ? kR889Lo : kR635Lo;
  float step = __builtin_fmaf(d, rhi, d * rlo);
  float base = __builtin_fmaf(f0, kR127Hi, f0 * kR127Lo);
  float end = __builtin_fmaf(f1, kR127Hi, f1 * kR127Lo);
  decode_from_seeds<F16>(base, end, step, eight, a, b, scale, pm, w);
}

// LDS tables of the palette seeds, shared by a workgroup:
//   base[i].x = RN((i - 127) / 127)                                   i = 0..254  (.y unused)
//   step[j]   = {RN(d / 889) if d < 0 else RN(d / 635), mode},  d = j - 254,   j = 0..508
// with mode = 0xFFFFFFFF for d < 0 (e1 < e0, exactly the 8-value mode) and 0 otherwise. Same
// arithmetic as decode_block. Both tables have 8-byte entries addressed by 8 * index, which is
// what the endpoint extraction yields; a step entry and its mode are read by one 64-bit load.
struct PaletteTableStorage {
  float2 base[255];
  uint2 step[509];
  uint2 pad[4];  // 6144 bytes: six whole 1 KiB wave loads (copy_seed_tables)
};
constexpr int kSeedTableBytes = 6144;

// The same tables as a compile-time image in device memory (words in LDS order), so that a
// workgroup copies them instead of computing them. Each quotient is the correctly rounded float
// RN(n/d); double division rounded to float gives exactly that for every entry here (n and d
// below 2^10: checked exhaustively against exact rational rounding), which is also what
// decode_block's fma with a split reciprocal yields for every numerator here.
struct SeedTableImage {
  uint32_t words[kSeedTableBytes / 4];
};

constexpr SeedTableImage make_seed_table_image() {
  SeedTableImage t{};
  for (int i = 0; i < 255; ++i) t.words[2 * i] = __builtin_bit_cast(uint32_t, (float)((double)(i - 127) / 127.0));
  for (int j = 0; j < 509; ++j) {
    const int d = j - 254;
    const double q = d < 0 ? (double)d / 889.0 : (double)d / 635.0;
    t.words[510 + 2 * j] = __builtin_bit_cast(uint32_t, (float)q);
    t.words[511 + 2 * j] = d < 0 ? 0xFFFFFFFFu : 0u;
  }
  return t;
}

static __device__ const SeedTableImage kSeedTableImage = make_seed_table_image();

// Copy the seed tables into LDS with direct buffer-to-LDS loads (1 KiB per wave load, waves
// 0..nwaves-1 of the workgroup). The caller waits for them (vmcnt) before the barrier that
// publishes them.
__device__ __forceinline__ void copy_seed_tables(PaletteTableStorage &t, int wave, int lane, int nwaves) {
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<SeedTableImage *>(&kSeedTableImage), (short)0, kSeedTableBytes, 0x00020000);
  for (int q = wave; q < kSeedTableBytes / 1024; q += nwaves)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rsrc, (__attribute__((address_space(3))) void *)(reinterpret_cast<char *>(&t) + 1024 * q), 16,
        1024 * q + 16 * lane, 0, 0, 0);
}

// 8 * eb from the 2-bit endpoint fields in bits 3-4 of each byte: a byte offset into the tables.
__device__ __forceinline__ uint32_t endpoint_offset(uint32_t word) {
  return __builtin_amdgcn_udot4(word & 0x18181818u, 0x40100401u, 0u, false);
}

// The palette seeds of one device block, read from the LDS tables.
struct Seeds {
  float base, end, step;
  uint32_t mode;  // all ones in 8-value mode
};

__device__ __forceinline__ Seeds read_seeds(uint32_t a, uint32_t b, const PaletteTableStorage &t) {
  const uint32_t o0 = endpoint_offset(a);
  const uint32_t o1 = endpoint_offset(b);
  const int od = (int)o1 - (int)o0;  // 8 * (e1 - e0)
  const char *base_bytes = reinterpret_cast<const char *>(t.base);
  const char *step_bytes = reinterpret_cast<const char *>(&t.step[254]);
  const uint2 sm = *reinterpret_cast<const uint2 *>(step_bytes + od);
  return Seeds{*reinterpret_cast<const float *>(base_bytes + o0), *reinterpret_cast<const float *>(base_bytes + o1),
               __uint_as_float(sm.x), sm.y};
}

// Decode one device block with the palette seeds read from LDS tables.
template <bool F16 = false>
__device__ __forceinline__ void decode_block_lds(uint32_t a, uint32_t b, float scale, uint32_t pm,
                                                 const PaletteTableStorage &t, uint32_t w[8]) {
  const Seeds s = read_seeds(a, b, t);
  decode_from_seeds_mode<F16>(s.base, s.end, s.step, s.mode, a, b, scale, pm, w);
}

}  // namespace tx
