/*
 * CPU restatement of the packed 4-bit affine quantized matmul — TEST INFRASTRUCTURE.
 *
 * Used only as the test reference in tests/ and as the timed CPU baseline ("port") in bench.py; the
 * product path never links it. Same arithmetic as oracle/qmm4_oracle.py:
 *   q[n, 8c+i] = (w[n, c] >> 4i) & 0xF                     src/mlx_tree_spec/qmm_packed.py:115, 200-201
 *   w_deq     = bf16_rne(fp32(s) * q + fp32(b)), g = k/64  qmm_packed.py:635-636, 630
 *   y[m, n]   = bf16_rne(sum_k fp32(x[m,k]) * w_deq[n,k])  tests/test_units.py:108 (fp32 accumulation)
 * Accumulation: 16 fp32 partial sums over k (k mod 16), summed pairwise at the end; the order
 * differs from the GPU kernels, the tolerance absorbs it.
 * Parallel over output columns with OpenMP; each thread dequantizes one weight row at a time
 * into an fp32 buffer and reuses it for every activation row.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bf16_to_f32(uint16_t u) {
  union { uint32_t i; float f; } v;
  v.i = (uint32_t)u << 16;
  return v.f;
}

static inline uint16_t f32_to_bf16(float f) {
  union { uint32_t i; float f; } v;
  v.f = f;
  if (isnan(f)) return (uint16_t)(((v.i >> 16) & 0x8000u) | 0x7FC0u);
  return (uint16_t)((v.i + 0x7FFFu + ((v.i >> 16) & 1u)) >> 16);
}

static void dequant_row(const uint32_t* w, const uint16_t* s, const uint16_t* b, int64_t K,
                        float* out) {
  for (int64_t c = 0; c < K / 8; ++c) {
    const float sf = bf16_to_f32(s[(c * 8) / 64]);
    const float bf = bf16_to_f32(b[(c * 8) / 64]);
    const uint32_t word = w[c];
    for (int i = 0; i < 8; ++i) {
      const float q = (float)((word >> (4 * i)) & 0xFu);
      out[c * 8 + i] = bf16_to_f32(f32_to_bf16(fmaf(q, sf, bf)));
    }
  }
}

int qmm4_oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* out: bf16 bits [N, K]. Returns 0, or -22 on bad arguments. */
int qmm4_oracle_dequant(const uint32_t* w, const uint16_t* s, const uint16_t* b, uint16_t* out,
                        int64_t N, int64_t K, int n_threads) {
  if (K % 64 != 0 || N < 0) return -22;
#ifdef _OPENMP
  if (n_threads > 0) omp_set_num_threads(n_threads);
#else
  (void)n_threads;
#endif
#pragma omp parallel
  {
    float* row = (float*)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
      dequant_row(w + n * (K / 8), s + n * (K / 64), b + n * (K / 64), K, row);
      for (int64_t k = 0; k < K; ++k) {
        union { uint32_t i; float f; } v;
        v.f = row[k];
        out[n * K + k] = (uint16_t)(v.i >> 16);
      }
    }
    free(row);
  }
  return 0;
}

/* Shared body: fp32 y[M, N] (yf != NULL) or bf16 bits (yb != NULL). */
static int qmm_impl(const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                    uint16_t* yb, float* yf, int64_t M, int64_t N, int64_t K, int n_threads) {
  if (K % 64 != 0 || M < 0 || N < 0) return -22;
#ifdef _OPENMP
  if (n_threads > 0) omp_set_num_threads(n_threads);
#else
  (void)n_threads;
#endif
  float* xf = (float*)malloc(sizeof(float) * (size_t)(M * K + 1));
  if (!xf) return -12;
  for (int64_t i = 0; i < M * K; ++i) xf[i] = bf16_to_f32(x[i]);
#pragma omp parallel
  {
    float* row = (float*)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
      dequant_row(w + n * (K / 8), s + n * (K / 64), b + n * (K / 64), K, row);
      for (int64_t m = 0; m < M; ++m) {
        const float* xr = xf + m * K;
        float acc[16];
        for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
        int64_t k = 0;
        for (; k + 16 <= K; k += 16)
          for (int j = 0; j < 16; ++j) acc[j] += xr[k + j] * row[k + j];
        for (; k < K; ++k) acc[k & 15] += xr[k] * row[k];
        for (int h = 8; h > 0; h >>= 1)
          for (int j = 0; j < h; ++j) acc[j] += acc[j + h];
        if (yf) yf[m * N + n] = acc[0];
        if (yb) yb[m * N + n] = f32_to_bf16(acc[0]);
      }
    }
    free(row);
  }
  free(xf);
  return 0;
}

/* y: bf16 bits [M, N]. Returns 0, or -22 on bad arguments. */
int qmm4_oracle_qmm(const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                    uint16_t* y, int64_t M, int64_t N, int64_t K, int n_threads) {
  return qmm_impl(x, w, s, b, y, NULL, M, N, K, n_threads);
}

/* y: fp32 [M, N], not rounded to bf16 (the fp32-accumulated reference). */
int qmm4_oracle_qmm_f32(const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                        float* y, int64_t M, int64_t N, int64_t K, int n_threads) {
  return qmm_impl(x, w, s, b, NULL, y, M, N, K, n_threads);
}
