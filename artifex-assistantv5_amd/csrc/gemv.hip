// VALU GEMV: y[m, n] = sum_k x[m, k] * dequant(W)[n, k], one pass over the
// weights per activation row (grid.y = M), f32 accumulation.
//
// Replaces the reference's decode kernels matmul_gguf_q8_0 /
// matmul_gguf_q4_k_tiled_v4 / matmul_gguf_q6_k_tiled
// (webgpu/src/shaders/matmul_gguf.wgsl:2102-2133, :3191-3245, :2406-2464),
// which re-read the activation slice per row from workgroup memory and
// tree-reduce in LDS.  Here:
//   * a wave owns R consecutive weight rows; each lane owns a fixed 64-element
//     slice of K (one "lane unit"), so its slice of x is loaded into VGPRs
//     once per 4096-wide K segment and reused by all R rows;
//   * the weight stream is read with 16-byte nontemporal loads;
//   * quantized values are masked into f16 subnormal halves (q * 2^-24) and
//     multiplied with v_fma_mix_f32 (convert + FMA in one op); the 2^24 and
//     integer offsets (Q8_0 +128, Q6_K +32, Q4_K mins) are applied once per
//     block with per-slice sums of x;
//   * the R per-lane partial sums are reduced across the 64 lanes with a
//     transpose-butterfly (log2 R halving exchanges, then full reduction).
#include "common.hpp"

namespace gguf {

constexpr float kTwo24 = 16777216.0f;   // 2^24
constexpr float kTwo20 = 1048576.0f;    // 2^20

// x slice: 16 consecutive activations starting at p, converted to f32.
template <typename XT>
__device__ __forceinline__ void load_x16(const XT *p, float *v);
template <>
__device__ __forceinline__ void load_x16<float>(const float *p, float *v) {
  const float4 *q = (const float4 *)p;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 t = q[i];
    v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
  }
}
template <>
__device__ __forceinline__ void load_x16<half_t>(const half_t *p, float *v) {
  const uint4 *q = (const uint4 *)p;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint4 t = q[i];
    const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const half2_t h = as_h2(w[j]);
      v[8 * i + 2 * j] = (float)h.x;
      v[8 * i + 2 * j + 1] = (float)h.y;
    }
  }
}

__device__ __forceinline__ float sum16(const float *v) {
  float a = 0.f, b = 0.f;
#pragma unroll
  for (int i = 0; i < 16; i += 2) { a += v[i]; b += v[i + 1]; }
  return a + b;
}

// Transpose-reduce R per-lane partials across the wave.  After the call the
// lanes with (lane & (64/R - 1)) == 0 hold the full sum of row lane / (64/R)
// in acc[0].
template <int R>
__device__ __forceinline__ void wave_reduce_rows(float (&acc)[R], int lane) {
  static_assert(R >= 1 && R <= 64 && (R & (R - 1)) == 0, "R must be a power of two");
#pragma unroll
  for (int cnt = R, mask = 32; cnt > 1; cnt >>= 1, mask >>= 1) {
    const bool upper = (lane & mask) != 0;
#pragma unroll
    for (int i = 0; i < cnt / 2; ++i) {
      const float keep = upper ? acc[i + cnt / 2] : acc[i];
      const float send = upper ? acc[i] : acc[i + cnt / 2];
      acc[i] = keep + __shfl_xor(send, mask);
    }
  }
#pragma unroll
  for (int mask = 32 / R; mask >= 1; mask >>= 1) acc[0] += __shfl_xor(acc[0], mask);
}

template <int R>
__device__ __forceinline__ void store_rows(float (&acc)[R], int lane, int n0, int n_rows,
                                           float *yrow) {
  wave_reduce_rows<R>(acc, lane);
  constexpr int span = 64 / R;
  if ((lane & (span - 1)) == 0) {
    const int n = n0 + lane / span;
    if (n < n_rows) yrow[n] = acc[0];
  }
}

// ---------------------------------------------------------------------------
// Q4_K.  Lane unit = chunk c = lane & 3 of superblock sb = seg + lane / 4:
// 32 qs bytes holding sub-blocks 2c (low nibbles) and 2c + 1 (high nibbles).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float q4k_unit_dot(const uint4 hd, const uint4 qa, const uint4 qb,
                                              int c, const float *xv, float xs_lo, float xs_hi) {
  const uint32_t w[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
  float lo0 = 0.f, lo1 = 0.f, hi0 = 0.f, hi1 = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const half2_t l02 = as_h2(w[j] & 0x000F000Fu);          // bytes 0, 2: low nibbles
    const half2_t l13 = as_h2((w[j] >> 8) & 0x000F000Fu);   // bytes 1, 3
    const half2_t h02 = as_h2(w[j] & 0x00F000F0u);          // high nibbles * 16
    const half2_t h13 = as_h2((w[j] >> 8) & 0x00F000F0u);
    lo0 = fmix(l02.x, xv[4 * j + 0], lo0);
    lo1 = fmix(l13.x, xv[4 * j + 1], lo1);
    lo0 = fmix(l02.y, xv[4 * j + 2], lo0);
    lo1 = fmix(l13.y, xv[4 * j + 3], lo1);
    hi0 = fmix(h02.x, xv[32 + 4 * j + 0], hi0);
    hi1 = fmix(h13.x, xv[32 + 4 * j + 1], hi1);
    hi0 = fmix(h02.y, xv[32 + 4 * j + 2], hi0);
    hi1 = fmix(h13.y, xv[32 + 4 * j + 3], hi1);
  }
  const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
  uint32_t sc0, m0, sc1, m1;
  q4k_scale_min(2 * c, hd.y, hd.z, hd.w, sc0, m0);
  q4k_scale_min(2 * c + 1, hd.y, hd.z, hd.w, sc1, m1);
  const float s_lo = d * (float)sc0 * kTwo24;
  const float s_hi = d * (float)sc1 * kTwo20;
  return s_lo * (lo0 + lo1) + s_hi * (hi0 + hi1) - dmin * ((float)m0 * xs_lo + (float)m1 * xs_hi);
}

template <typename XT, int R>
__global__ __launch_bounds__(256) void gemv_q4k_kernel(const XT *__restrict__ x, int64_t ldx,
                                                       const uint8_t *__restrict__ W, int64_t trb,
                                                       int N, int K, float *__restrict__ y,
                                                       int64_t ldy) {
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
  if (n0 >= N) return;
  const int m = blockIdx.y;
  const XT *xr = x + (int64_t)m * ldx;
  const int nsb = K >> 8;
  const int c = lane & 3;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  for (int seg = 0; seg < nsb; seg += 16) {
    const int sb = seg + (lane >> 2);
    if (sb < nsb) {
      float xv[64];
      const XT *xp = xr + 256 * sb + 64 * c;
#pragma unroll
      for (int i = 0; i < 4; ++i) load_x16<XT>(xp + 16 * i, xv + 16 * i);
      const float xs_lo = sum16(xv) + sum16(xv + 16);
      const float xs_hi = sum16(xv + 32) + sum16(xv + 48);
      const uint8_t *wp = W + (int64_t)n0 * trb + 144 * sb;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (n0 + r < N) {
          const uint8_t *blk = wp + (int64_t)r * trb;
          const uint4 hd = ldg16_stream(blk);
          const uint4 qa = ldg16_stream(blk + 16 + 32 * c);
          const uint4 qb = ldg16_stream(blk + 32 + 32 * c);
          acc[r] += q4k_unit_dot(hd, qa, qb, c, xv, xs_lo, xs_hi);
        }
      }
    }
  }
  store_rows<R>(acc, lane, n0, N, y + (int64_t)m * ldy);
}

// ---------------------------------------------------------------------------
// Q8_0.  Lane unit = blocks 2*lane, 2*lane + 1 of the segment (64 elements).
// Bytes are biased to q + 128 (xor 0x80) so they mask into unsigned halves.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float q8_block_dot(const uint4 a, const uint4 b, const float *xv) {
  const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t u = w[j] ^ 0x80808080u;
    const half2_t e02 = as_h2(u & 0x00FF00FFu);
    const half2_t e13 = as_h2((u >> 8) & 0x00FF00FFu);
    s0 = fmix(e02.x, xv[4 * j + 0], s0);
    s1 = fmix(e13.x, xv[4 * j + 1], s1);
    s0 = fmix(e02.y, xv[4 * j + 2], s0);
    s1 = fmix(e13.y, xv[4 * j + 3], s1);
  }
  return s0 + s1;
}

template <typename XT, int R>
__global__ __launch_bounds__(256) void gemv_q8_0_kernel(const XT *__restrict__ x, int64_t ldx,
                                                        const uint8_t *__restrict__ W, int64_t trb,
                                                        int N, int K, float *__restrict__ y,
                                                        int64_t ldy) {
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
  if (n0 >= N) return;
  const int m = blockIdx.y;
  const XT *xr = x + (int64_t)m * ldx;
  const int nb = K >> 5;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  for (int seg = 0; seg < nb; seg += 128) {
    const int b0 = seg + 2 * lane;
    if (b0 < nb) {
      const bool two = b0 + 1 < nb;
      float xv[64];
      const XT *xp = xr + 32 * b0;
      load_x16<XT>(xp, xv);
      load_x16<XT>(xp + 16, xv + 16);
      if (two) {
        load_x16<XT>(xp + 32, xv + 32);
        load_x16<XT>(xp + 48, xv + 48);
      } else {
#pragma unroll
        for (int i = 32; i < 64; ++i) xv[i] = 0.f;
      }
      const float xs0 = 128.f * (sum16(xv) + sum16(xv + 16));
      const float xs1 = 128.f * (sum16(xv + 32) + sum16(xv + 48));
      const uint8_t *wp = W + (int64_t)n0 * trb;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (n0 + r < N) {
          const uint8_t *row = wp + (int64_t)r * trb;
          const uint4 q0 = ldg16_stream(row + 32 * b0);
          const uint4 q1 = ldg16_stream(row + 32 * b0 + 16);
          const uint32_t dd = *(const uint32_t *)(row + K + 2 * b0);  // d[b0] | d[b0+1] << 16
          float v = h2f(dd) * (kTwo24 * q8_block_dot(q0, q1, xv) - xs0);
          if (two) {
            const uint4 q2 = ldg16_stream(row + 32 * b0 + 32);
            const uint4 q3 = ldg16_stream(row + 32 * b0 + 48);
            v += h2f(dd >> 16) * (kTwo24 * q8_block_dot(q2, q3, xv + 32) - xs1);
          }
          acc[r] += v;
        }
      }
    }
  }
  store_rows<R>(acc, lane, n0, N, y + (int64_t)m * ldy);
}

// ---------------------------------------------------------------------------
// Q6_K.  Lane unit = (superblock sb = seg + lane / 4, half h = (lane >> 1) & 1,
// group g = lane & 1): 64 elements y[128h + 32t + 16g + i], t = 0..3, with
// scales sc[8h + g + 2t].  Values are biased (q + 32, 6-bit unsigned).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float q6k_unit_dot(const uint4 qa4, const uint4 qb4, const uint4 qh4,
                                              const float *xv, float (&dt)[4]) {
  const uint32_t qa[4] = {qa4.x, qa4.y, qa4.z, qa4.w};
  const uint32_t qb[4] = {qb4.x, qb4.y, qb4.z, qb4.w};
  const uint32_t qh[4] = {qh4.x, qh4.y, qh4.z, qh4.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) dt[t] = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t v[4] = {
        (qa[j] & 0x0F0F0F0Fu) | ((qh[j] << 4) & 0x30303030u),
        (qb[j] & 0x0F0F0F0Fu) | ((qh[j] << 2) & 0x30303030u),
        ((qa[j] >> 4) & 0x0F0F0F0Fu) | (qh[j] & 0x30303030u),
        ((qb[j] >> 4) & 0x0F0F0F0Fu) | ((qh[j] >> 2) & 0x30303030u)};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const half2_t e02 = as_h2(v[t] & 0x00FF00FFu);
      const half2_t e13 = as_h2((v[t] >> 8) & 0x00FF00FFu);
      const float *xt = xv + 16 * t + 4 * j;
      float s = fmix(e02.x, xt[0], dt[t]);
      s = fmix(e13.x, xt[1], s);
      s = fmix(e02.y, xt[2], s);
      dt[t] = fmix(e13.y, xt[3], s);
    }
  }
  return 0.f;
}

template <typename XT, int R>
__global__ __launch_bounds__(256) void gemv_q6_k_kernel(const XT *__restrict__ x, int64_t ldx,
                                                        const uint8_t *__restrict__ W, int64_t trb,
                                                        int N, int K, float *__restrict__ y,
                                                        int64_t ldy) {
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
  if (n0 >= N) return;
  const int m = blockIdx.y;
  const XT *xr = x + (int64_t)m * ldx;
  const int nsb = K >> 8;
  const int h = (lane >> 1) & 1, g = lane & 1;
  const int off_qh = K / 2, off_sc = K / 2 + K / 4, off_d = K / 2 + K / 4 + K / 16;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  for (int seg = 0; seg < nsb; seg += 16) {
    const int sb = seg + (lane >> 2);
    if (sb < nsb) {
      float xv[64];
      const XT *xp = xr + 256 * sb + 128 * h + 16 * g;
#pragma unroll
      for (int t = 0; t < 4; ++t) load_x16<XT>(xp + 32 * t, xv + 16 * t);
      float xs[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) xs[t] = 32.f * sum16(xv + 16 * t);
      const uint8_t *wp = W + (int64_t)n0 * trb;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (n0 + r < N) {
          const uint8_t *row = wp + (int64_t)r * trb;
          const uint4 qa = ldg16_stream(row + 128 * sb + 64 * h + 16 * g);
          const uint4 qb = ldg16_stream(row + 128 * sb + 64 * h + 32 + 16 * g);
          const uint4 qh = ldg16_stream(row + off_qh + 64 * sb + 32 * h + 16 * g);
          const uint2 scw = *(const uint2 *)(row + off_sc + 16 * sb + 8 * h);
          const float d = h2f(*(const uint16_t *)(row + off_d + 2 * sb));
          float dt[4];
          q6k_unit_dot(qa, qb, qh, xv, dt);
          // sc[8h + g + 2t]: bytes g, g+2 of word 0 and g, g+2 of word 1
          const int s0 = (int)(int8_t)(scw.x >> (8 * g));
          const int s1 = (int)(int8_t)(scw.x >> (8 * (g + 2)));
          const int s2 = (int)(int8_t)(scw.y >> (8 * g));
          const int s3 = (int)(int8_t)(scw.y >> (8 * (g + 2)));
          const float v = (float)s0 * (kTwo24 * dt[0] - xs[0]) + (float)s1 * (kTwo24 * dt[1] - xs[1]) +
                          (float)s2 * (kTwo24 * dt[2] - xs[2]) + (float)s3 * (kTwo24 * dt[3] - xs[3]);
          acc[r] += d * v;
        }
      }
    }
  }
  store_rows<R>(acc, lane, n0, N, y + (int64_t)m * ldy);
}

// ---------------------------------------------------------------------------

template <typename XT>
static hipError_t launch_gemv_t(const XT *x, int64_t ldx, const uint8_t *W, int type, int64_t n,
                                int64_t k, int64_t trb, float *y, int64_t ldy, int64_t m,
                                hipStream_t s) {
  constexpr int R = 8;
  const int64_t waves = (n + R - 1) / R;
  const dim3 grid((unsigned)((waves + 3) / 4), (unsigned)m);
  if (type == 12)
    hipLaunchKernelGGL((gemv_q4k_kernel<XT, R>), grid, dim3(256), 0, s, x, ldx, W, trb, (int)n,
                       (int)k, y, ldy);
  else if (type == 8)
    hipLaunchKernelGGL((gemv_q8_0_kernel<XT, R>), grid, dim3(256), 0, s, x, ldx, W, trb, (int)n,
                       (int)k, y, ldy);
  else
    hipLaunchKernelGGL((gemv_q6_k_kernel<XT, R>), grid, dim3(256), 0, s, x, ldx, W, trb, (int)n,
                       (int)k, y, ldy);
  return hipGetLastError();
}

hipError_t launch_gemv(const void *x, int x_type, int64_t ldx, const uint8_t *tiles, int type,
                       int64_t n, int64_t k, int64_t trb, float *y, int64_t ldy, int64_t m,
                       hipStream_t s) {
  if (x_type == 0)
    return launch_gemv_t<float>((const float *)x, ldx, tiles, type, n, k, trb, y, ldy, m, s);
  return launch_gemv_t<half_t>((const half_t *)x, ldx, tiles, type, n, k, trb, y, ldy, m, s);
}

}  // namespace gguf
