// Batch-1 decode GEMV over BC4 tiles (gfx950, wave64).
//
// Reference: texelator_bc4_bf16_kernel<L> (texelator/cuda/texelator_cuda.cu:154-199) computes
// y[t,m] = bf16( sum_k bf16(P*scale[m]) * x[t,k] + bias[m] ) with fp32 accumulation; L is the
// number of texture requests in flight. Here the same sum is formed from streamed BC4 tiles:
//   * one workgroup = 4 waves = one 16-row group x one K-slice; the x slice is staged in LDS;
//   * each wave streams every 4th 1 KiB tile of the slice with one 128-bit load per lane
//     (LOOKAHEAD tiles in flight), decodes its two blocks in VGPRs (bc4_device.h) and
//     accumulates with v_dot2_f32_bf16;
//   * lanes of one row are combined with cross-lane shuffles, waves through LDS (fixed order);
//   * when the K range is split over workgroups, each writes an fp32 partial and the last one
//     to arrive (agent-scope counter) sums the partials in split order, so the result does not
//     depend on scheduling. The counter is reset by that last workgroup.
#include "bc4_device.h"
#include "kernels.h"

namespace tx {

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float dot2(uint32_t w, uint32_t x, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), __builtin_bit_cast(bf16x2, x),
                                        acc, false);
}

__device__ __forceinline__ float bf16_bits_to_float(uint16_t v) {
  return __builtin_bit_cast(float, (uint32_t)v << 16);
}

template <int LA, bool F32OUT>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvParams p) {
  extern __shared__ uint4 xs[];  // x slice, 16 uint4 (128 bf16) per tile column
  __shared__ float red[4][16];
  __shared__ int last_flag;

  const int g = blockIdx.x;
  const int split = blockIdx.y;
  const int token = blockIdx.z;
  const int c_begin = (int)((int64_t)split * p.CG / p.ks);
  const int c_end = (int)((int64_t)(split + 1) * p.CG / p.ks);
  const int nc = c_end - c_begin;

  const uint16_t *x = static_cast<const uint16_t *>(p.x) + (size_t)token * p.K;
  for (int idx = threadIdx.x; idx < nc * 16; idx += kThreads) {
    const int k0 = (c_begin * 16 + idx) * 8;
    uint4 v;
    if (k0 + 8 <= p.K) {
      v = *reinterpret_cast<const uint4 *>(x + k0);
    } else {
      uint16_t e[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) e[q] = (k0 + q < p.K) ? x[k0 + q] : (uint16_t)0;
      v.x = e[0] | ((uint32_t)e[1] << 16);
      v.y = e[2] | ((uint32_t)e[3] << 16);
      v.z = e[4] | ((uint32_t)e[5] << 16);
      v.w = e[6] | ((uint32_t)e[7] << 16);
    }
    xs[idx] = v;
  }
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int i = lane & 15;
  const int kg = lane >> 4;
  const int row = g * kTileRows + i;
  const float scale = p.scales[row];
  const uint32_t pm = pm_scale_pair(scale);
  const uint4 *tile_ptr = p.tiles + ((size_t)g * p.CG + c_begin) * 64 + lane;
  const int nt = nc > wave ? (nc - wave + 3) / 4 : 0;

  float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f, acc3 = 0.f;
  uint4 buf[LA];
#pragma unroll
  for (int u = 0; u < LA; ++u)
    if (u < nt) buf[u] = load_stream(tile_ptr + (size_t)(u * 4 + wave) * 64);

  for (int j0 = 0; j0 < nt; j0 += LA) {
#pragma unroll
    for (int u = 0; u < LA; ++u) {
      const int j = j0 + u;
      if (j < nt) {
        const uint4 cur = buf[u];
        if (j + LA < nt) buf[u] = load_stream(tile_ptr + (size_t)((j + LA) * 4 + wave) * 64);
        const uint4 *xv = xs + (j * 4 + wave) * 16 + kg * 4;
        const uint4 x0 = xv[0], x1 = xv[1], x2 = xv[2], x3 = xv[3];
        uint32_t w[8];
        decode_block(cur.x, cur.y, scale, pm, w);
        acc0 = dot2(w[0], x0.x, acc0);
        acc1 = dot2(w[1], x0.y, acc1);
        acc0 = dot2(w[2], x0.z, acc0);
        acc1 = dot2(w[3], x0.w, acc1);
        acc0 = dot2(w[4], x1.x, acc0);
        acc1 = dot2(w[5], x1.y, acc1);
        acc0 = dot2(w[6], x1.z, acc0);
        acc1 = dot2(w[7], x1.w, acc1);
        decode_block(cur.z, cur.w, scale, pm, w);
        acc2 = dot2(w[0], x2.x, acc2);
        acc3 = dot2(w[1], x2.y, acc3);
        acc2 = dot2(w[2], x2.z, acc2);
        acc3 = dot2(w[3], x2.w, acc3);
        acc2 = dot2(w[4], x3.x, acc2);
        acc3 = dot2(w[5], x3.y, acc3);
        acc2 = dot2(w[6], x3.z, acc2);
        acc3 = dot2(w[7], x3.w, acc3);
      }
    }
  }

  float acc = (acc0 + acc1) + (acc2 + acc3);
  acc += __shfl_xor(acc, 16);
  acc += __shfl_xor(acc, 32);
  if (lane < 16) red[wave][lane] = acc;
  __syncthreads();

  float total = 0.f;
  if (threadIdx.x < 16) total = ((red[0][threadIdx.x] + red[1][threadIdx.x]) + red[2][threadIdx.x]) + red[3][threadIdx.x];

  if (p.ks > 1) {
    if (threadIdx.x < 16) {
      p.partials[(size_t)split * p.Mp + g * kTileRows + threadIdx.x] = total;
      __threadfence();
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      const uint32_t prior = __hip_atomic_fetch_add(p.counters + g, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
      last_flag = (prior == (uint32_t)(p.ks - 1));
    }
    __syncthreads();
    if (!last_flag) return;
    __threadfence();
    if (threadIdx.x < 16) {
      total = 0.f;
      for (int s = 0; s < p.ks; ++s)
        total += __hip_atomic_load(p.partials + (size_t)s * p.Mp + g * kTileRows + threadIdx.x, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
    if (threadIdx.x == 0)
      __hip_atomic_store(p.counters + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  if (threadIdx.x < 16) {
    const int out_row = g * kTileRows + threadIdx.x;
    if (out_row < p.M) {
      if constexpr (F32OUT) {
        static_cast<float *>(p.y)[(size_t)token * p.M + out_row] = total;
      } else {
        float value = total;
        if (p.bias) value += bf16_bits_to_float(static_cast<const uint16_t *>(p.bias)[out_row]);
        static_cast<__bf16 *>(p.y)[(size_t)token * p.M + out_row] = (__bf16)value;
      }
    }
  }
}

template <int LA>
hipError_t launch_la(const GemvParams &p, bool f32_out, hipStream_t stream) {
  const int max_cols = (p.CG + p.ks - 1) / p.ks;
  const size_t lds = (size_t)max_cols * 16 * sizeof(uint4);
  dim3 grid(p.RG, p.ks, p.tokens);
  if (f32_out)
    hipLaunchKernelGGL((gemv_kernel<LA, true>), grid, dim3(kThreads), lds, stream, p);
  else
    hipLaunchKernelGGL((gemv_kernel<LA, false>), grid, dim3(kThreads), lds, stream, p);
  return hipGetLastError();
}

}  // namespace

bool gemv_lookahead_supported(int la) { return la == 1 || la == 2 || la == 3 || la == 4 || la == 6 || la == 8; }

hipError_t launch_gemv(const GemvParams &p, int lookahead, bool f32_out, hipStream_t stream) {
  switch (lookahead) {
    case 1: return launch_la<1>(p, f32_out, stream);
    case 2: return launch_la<2>(p, f32_out, stream);
    case 3: return launch_la<3>(p, f32_out, stream);
    case 4: return launch_la<4>(p, f32_out, stream);
    case 6: return launch_la<6>(p, f32_out, stream);
    case 8: return launch_la<8>(p, f32_out, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t gemv_kernel_attributes(int lookahead, hipFuncAttributes *attr) {
  switch (lookahead) {
    case 1: return hipFuncGetAttributes(attr, reinterpret_cast<const void *>(&gemv_kernel<1, false>));
    case 2: return hipFuncGetAttributes(attr, reinterpret_cast<const void *>(&gemv_kernel<2, false>));
    case 3: return hipFuncGetAttributes(attr, reinterpret_cast<const void *>(&gemv_kernel<3, false>));
    case 4: return hipFuncGetAttributes(attr, reinterpret_cast<const void *>(&gemv_kernel<4, false>));
    case 6: return hipFuncGetAttributes(attr, reinterpret_cast<const void *>(&gemv_kernel<6, false>));
    case 8: return hipFuncGetAttributes(attr, reinterpret_cast<const void *>(&gemv_kernel<8, false>));
    default: return hipErrorInvalidValue;
  }
}

}  // namespace tx
