/*
 * Plain-C restatement of the BC4 weight path -- TEST INFRASTRUCTURE ONLY.
 *
 * Built to oracle/liboracle.so by oracle/Makefile. Used by tests/ (as an independent
 * second restatement next to oracle/bc4.py) and by bench.py's cpu_baseline leg.
 *
 * Reference anchors (reference checkout paths):
 *   block format      texelator/encoder.py:105-117, texelator/cuda/texelator_cuda.cu:127-131
 *   palette layout    texelator/encoder.py:11-20, texelator/cuda/texelator_cuda.cu:1542-1595
 *   decoded weight    texelator/cuda/texelator_cuda.cu:141-152  (bf16_rne(P * scale), fp32 product)
 *   matvec            texelator/cuda/texelator_cuda.cu:154-199  (sum over K of w * x)
 *   prefill GEMM      texelator/cuda/cutlass_texture_mainloop.cu:203-249 (D[T,M] = X W^T)
 *
 * Palette definition (this build's): endpoints clamped to [-127,127]; base = RN(e0/127),
 * end = RN(e1/127); e0 > e1: step = RN((e1-e0)/889), P[s] = fma(s-1, step, base), s=2..7;
 * else step = RN((e1-e0)/635), P[s] = fma(s-1, step, base), s=2..5, P[6] = -1, P[7] = +1.
 * Compiled with -ffp-contract=off so that the only fused operations are the explicit fmaf.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static float crdiv(int n, int d) {
  /* The double quotient is correctly rounded and never lands on a float midpoint for these
   * operands (|n| <= 889, odd d in {127,635,889}), so the conversion is a single correct
   * rounding of n/d. */
  return (float)((double)n / (double)d);
}

static void palette_row(int e0, int e1, float out[8]) {
  int eight = e0 > e1;
  float base = crdiv(e0, 127);
  float end = crdiv(e1, 127);
  float step = crdiv(e1 - e0, eight ? 889 : 635);
  out[0] = base;
  out[1] = end;
  for (int s = 2; s < 8; ++s) out[s] = fmaf((float)(s - 1), step, base);
  if (!eight) {
    out[6] = -1.0f;
    out[7] = 1.0f;
  }
}

/* out: 255*255*8 floats, index ((e1+127)*255 + (e0+127))*8 + s */
void oracle_palette(float *out) {
  for (int y = 0; y < 255; ++y)
    for (int x = 0; x < 255; ++x) palette_row(x - 127, y - 127, out + ((size_t)y * 255 + x) * 8);
}

static uint16_t bf16_rne(float v) {
  uint32_t u;
  memcpy(&u, &v, 4);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static int clamp_endpoint(uint8_t byte) {
  int e = (int)(int8_t)byte;
  return e < -127 ? -127 : e;
}

/* blocks: [M][bpr][8] bytes; scales: [M]; lut: 255*255*8 floats or NULL for the built-in
 * palette; out: [M][16*bpr] bf16 bit patterns. */
void oracle_decode_bf16(const uint8_t *blocks, const float *scales, int64_t M, int64_t bpr,
                        const float *lut, uint16_t *out) {
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    float scale = scales[m];
    for (int64_t b = 0; b < bpr; ++b) {
      const uint8_t *blk = blocks + ((size_t)m * bpr + b) * 8;
      int e0 = clamp_endpoint(blk[0]);
      int e1 = clamp_endpoint(blk[1]);
      float row[8];
      if (lut) {
        memcpy(row, lut + ((size_t)(e1 + 127) * 255 + (e0 + 127)) * 8, sizeof row);
      } else {
        palette_row(e0, e1, row);
      }
      uint64_t bits = 0;
      for (int i = 0; i < 6; ++i) bits |= (uint64_t)blk[2 + i] << (8 * i);
      uint16_t *dst = out + (size_t)m * bpr * 16 + (size_t)b * 16;
      for (int p = 0; p < 16; ++p) {
        int s = (int)((bits >> (3 * p)) & 7u);
        float prod = row[s] * scale; /* one fp32 rounding */
        dst[p] = bf16_rne(prod);
      }
    }
  }
}

/* y[m] = sum_k w[m][k] * x[k] in double. */
void oracle_matvec_f64(const uint16_t *w, const uint16_t *x, int64_t M, int64_t K, double *y) {
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    const uint16_t *row = w + (size_t)m * K;
    double acc = 0.0;
    for (int64_t k = 0; k < K; ++k) acc += (double)bf16_to_f32(row[k]) * (double)bf16_to_f32(x[k]);
    y[m] = acc;
  }
}

/* Y[t][m] = sum_k x[t][k] * w[m][k] in double (each product of two bf16 values is exact in double).
 * x is converted to double once; each weight row once per thread; four tokens share each pass over
 * the row (four independent accumulators), so a whole prefill shape finishes in seconds. */
void oracle_gemm_f64(const uint16_t *x, const uint16_t *w, int64_t T, int64_t M, int64_t K, double *y) {
  double *xd = (double *)malloc((size_t)T * (size_t)K * sizeof(double));
  if (!xd) return;
  for (int64_t i = 0; i < T * K; ++i) xd[i] = (double)bf16_to_f32(x[i]);
#pragma omp parallel
  {
    double *wd = (double *)malloc((size_t)K * sizeof(double));
#pragma omp for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
      if (!wd) continue;
      const uint16_t *row = w + (size_t)m * K;
      for (int64_t k = 0; k < K; ++k) wd[k] = (double)bf16_to_f32(row[k]);
      int64_t t = 0;
      for (; t + 4 <= T; t += 4) {
        const double *x0 = xd + (size_t)t * K, *x1 = x0 + K, *x2 = x1 + K, *x3 = x2 + K;
        double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
        for (int64_t k = 0; k < K; ++k) {
          const double v = wd[k];
          a0 += v * x0[k];
          a1 += v * x1[k];
          a2 += v * x2[k];
          a3 += v * x3[k];
        }
        y[(size_t)t * M + m] = a0;
        y[(size_t)(t + 1) * M + m] = a1;
        y[(size_t)(t + 2) * M + m] = a2;
        y[(size_t)(t + 3) * M + m] = a3;
      }
      for (; t < T; ++t) {
        const double *xr = xd + (size_t)t * K;
        double acc = 0.0;
        for (int64_t k = 0; k < K; ++k) acc += wd[k] * xr[k];
        y[(size_t)t * M + m] = acc;
      }
    }
    free(wd);
  }
  free(xd);
}

/* CPU baseline: fused decode + fp32 matvec (the CPU analogue of the GEMV), y in float.
 * Uses the built-in palette; eight fp32 accumulators per row. */
void oracle_decode_matvec_f32(const uint8_t *blocks, const float *scales, const uint16_t *x,
                              int64_t M, int64_t bpr, float *y) {
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    float scale = scales[m];
    float acc[16];
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
    for (int64_t b = 0; b < bpr; ++b) {
      const uint8_t *blk = blocks + ((size_t)m * bpr + b) * 8;
      float row[8], w[8];
      palette_row(clamp_endpoint(blk[0]), clamp_endpoint(blk[1]), row);
      for (int s = 0; s < 8; ++s) w[s] = bf16_to_f32(bf16_rne(row[s] * scale));
      uint64_t bits = 0;
      for (int i = 0; i < 6; ++i) bits |= (uint64_t)blk[2 + i] << (8 * i);
      const uint16_t *xb = x + b * 16;
      for (int p = 0; p < 16; ++p) acc[p] += w[(bits >> (3 * p)) & 7u] * bf16_to_f32(xb[p]);
    }
    float total = 0.0f;
    for (int i = 0; i < 16; ++i) total += acc[i];
    y[m] = total;
  }
}

int oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void oracle_set_threads(int n) {
#ifdef _OPENMP
  omp_set_num_threads(n);
#else
  (void)n;
#endif
}
