/* Compiled CPU restatement of the reference's Q4_K dequantization, for the CPU
 * baseline of the dequant-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  Like oracle/gguf_ref.py this is part of the
 * oracle: only tests/ and the cpu_baseline leg of bench.py load it (through
 * ctypes), to pin it against the numpy oracle and to time the host.  The
 * product path (the HIP library and its Python host code) never calls it.
 *
 * Built by oracle/build_oracle.py:
 *   gcc -O3 -march=x86-64-v3 -fopenmp -shared -fPIC gguf_ref_c.c -o liboracle.so
 *
 * Arithmetic.  Each weight is d*sc*q - dmin*m computed in f32, as
 * webgpu/src/model/gguf-dequant.ts:255-281 computes it in f64 and stores to a
 * Float32Array: every product is exact in f32 (d*sc*q needs at most 21
 * significant bits, dmin*m at most 17) and the one rounding left, the
 * subtraction, rounds the same in f32 as f64-then-f32.  So the dequantized
 * values are bit-identical to the reference's (tests/test_oracle_c.py checks
 * them against the numpy oracle and the reference's golden samples).  The
 * matmul accumulates each output in f32 over K in a fixed order (8 partial
 * sums, element k into sum k mod 8, added in order at the end), independent
 * of the thread count.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define Q4K_BYTES 144
#define QK 256

/* IEEE half bits -> f32 (gguf-dequant.ts:64-71: sign, 5-bit exponent, 10-bit
 * mantissa; subnormals, Inf and NaN included). */
static float f16_to_f32(uint16_t h) {
  const uint32_t s = (uint32_t)(h >> 15), e = (h >> 10) & 31u, f = h & 1023u;
  float v;
  if (e == 0)
    v = ldexpf((float)f, -24);
  else if (e == 31)
    v = f ? NAN : INFINITY;
  else
    v = ldexpf((float)(f | 1024u), (int)e - 25);
  return s ? -v : v;
}

/* The 6-bit (scale, min) pair j of a superblock (gguf-dequant.ts:169-176). */
static void scale_min_k4(int j, const uint8_t *q, int *sc, int *m) {
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4);
    *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

/* One superblock to 256 f32 values (gguf-dequant.ts:255-281): four 64-element
 * chunks; chunk c's 32 bytes give sub-block 2c from the low nibbles and
 * sub-block 2c + 1 from the high nibbles. */
static void dequant_block_q4_k(const uint8_t *b, float *out) {
  uint16_t hd, hm;
  memcpy(&hd, b, 2);
  memcpy(&hm, b + 2, 2);
  const float d = f16_to_f32(hd), dmin = f16_to_f32(hm);
  const uint8_t *scales = b + 4, *qs = b + 16;
  for (int c = 0; c < 4; ++c) {
    int sc1, m1, sc2, m2;
    scale_min_k4(2 * c, scales, &sc1, &m1);
    scale_min_k4(2 * c + 1, scales, &sc2, &m2);
    const float d1 = d * (float)sc1, min1 = dmin * (float)m1;
    const float d2 = d * (float)sc2, min2 = dmin * (float)m2;
    for (int l = 0; l < 32; ++l) out[64 * c + l] = d1 * (float)(qs[32 * c + l] & 0x0F) - min1;
    for (int l = 0; l < 32; ++l) out[64 * c + 32 + l] = d2 * (float)(qs[32 * c + l] >> 4) - min2;
  }
}

static int set_threads(int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
  return omp_get_max_threads();
#else
  (void)threads;
  return 1;
#endif
}

/* out[n_rows][k] = the dequantized rows of raw GGUF Q4_K data (row-major,
 * k / 256 superblocks per row), rows split over the threads.  Returns the
 * thread count used, or -1 for a K that is not a multiple of 256. */
int oracle_dequant_rows_q4_k(const uint8_t *raw, int64_t n_rows, int64_t k, float *out, int threads) {
  if (k % QK != 0 || n_rows < 0) return -1;
  const int used = set_threads(threads);
  const int64_t nb = k / QK;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < n_rows; ++r)
    for (int64_t b = 0; b < nb; ++b)
      dequant_block_q4_k(raw + (r * nb + b) * Q4K_BYTES, out + r * k + b * QK);
  return used;
}

/* y[m][n] = sum_k x[m][k] * W[n][k] for W the n_rows x k Q4_K matrix in raw
 * (row-major GGUF layout) and x an m x k f32 matrix (m <= 64): each thread
 * takes whole weight rows, dequantizes one superblock at a time into a local
 * buffer and accumulates every activation row against it, element k into
 * partial sum k mod 8; the 8 partial sums are added in order at the end.
 * Returns the thread count used, or -1 for a bad shape. */
int oracle_matmul_q4_k(const uint8_t *raw, int64_t n_rows, int64_t k, const float *x, int64_t m,
                       float *y, int threads) {
  if (k % QK != 0 || n_rows < 0 || m < 0 || m > 64) return -1;
  const int used = set_threads(threads);
  const int64_t nb = k / QK;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < n_rows; ++r) {
    float w[QK];
    float acc[64][8];
    memset(acc, 0, sizeof(float) * (size_t)m * 8);
    for (int64_t b = 0; b < nb; ++b) {
      dequant_block_q4_k(raw + (r * nb + b) * Q4K_BYTES, w);
      for (int64_t i = 0; i < m; ++i) {
        const float *xr = x + i * k + b * QK;
        for (int l = 0; l < QK; l += 8)
          for (int v = 0; v < 8; ++v) acc[i][v] += xr[l + v] * w[l + v];
      }
    }
    for (int64_t i = 0; i < m; ++i) {
      float t = 0.f;
      for (int v = 0; v < 8; ++v) t += acc[i][v];
      y[i * n_rows + r] = t;
    }
  }
  return used;
}
