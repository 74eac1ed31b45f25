// Repack (raw GGUF bytes -> HBM row layout) and dequantization to f32.
//
// Dequantization is bit-exact to the reference CPU dequant
// (webgpu/src/model/gguf-dequant.ts:152-166 Q8_0, :255-281 Q4_K,
// :369-399 Q6_K): every product in these formats is exact in f32, so the
// only rounding is the final Q4_K subtraction, which f32 arithmetic (fused
// or not) rounds exactly once, as the reference's f64-then-Float32Array does.
#include "common.hpp"

namespace gguf {

// ---------------------------------------------------------------------------
// Per-unit decoders shared by the tile and raw kernels.
// ---------------------------------------------------------------------------

// Q4_K: 16 qs bytes (chunk c, half h) of a superblock -> 16 values of
// sub-block 2c (out_lo) and 16 of sub-block 2c + 1 (out_hi).
__device__ __forceinline__ void q4k_decode16(uint32_t hdr0, uint32_t s0, uint32_t s1, uint32_t s2,
                                             int c, const uint32_t q[4], float *out_lo,
                                             float *out_hi) {
  const float d = h2f(hdr0), dmin = h2f(hdr0 >> 16);
  uint32_t sc0, m0, sc1, m1;
  q4k_scale_min(2 * c, s0, s1, s2, sc0, m0);
  q4k_scale_min(2 * c + 1, s0, s1, s2, sc1, m1);
  const float d1 = d * (float)sc0, min1 = dmin * (float)m0;
  const float d2 = d * (float)sc1, min2 = dmin * (float)m1;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t b = (q[i >> 2] >> (8 * (i & 3))) & 0xFFu;
    out_lo[i] = d1 * (float)(b & 0x0Fu) - min1;
    out_hi[i] = d2 * (float)(b >> 4) - min2;
  }
}

// Q6_K: one (half h, lane-group g) unit = 64 values: for t = 0..3 the 16
// values y[128h + 32t + 16g + i], scaled by sc[8h + g + 2t].
// qa = ql[64h + 16g ..], qb = ql[64h + 32 + 16g ..], qh = qh[32h + 16g ..].
__device__ __forceinline__ void q6k_decode64(float d, const int sc[4], const uint32_t qa[4],
                                             const uint32_t qb[4], const uint32_t qh[4],
                                             float out[4][16]) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int w = i >> 2, sh = 8 * (i & 3);
    const uint32_t a = (qa[w] >> sh) & 0xFFu, b = (qb[w] >> sh) & 0xFFu, h = (qh[w] >> sh) & 0xFFu;
    const int q0 = (int)((a & 0x0Fu) | ((h & 3u) << 4)) - 32;
    const int q1 = (int)((b & 0x0Fu) | (((h >> 2) & 3u) << 4)) - 32;
    const int q2 = (int)((a >> 4) | (((h >> 4) & 3u) << 4)) - 32;
    const int q3 = (int)((b >> 4) | (((h >> 6) & 3u) << 4)) - 32;
    out[0][i] = d * (float)sc[0] * (float)q0;
    out[1][i] = d * (float)sc[1] * (float)q1;
    out[2][i] = d * (float)sc[2] * (float)q2;
    out[3][i] = d * (float)sc[3] * (float)q3;
  }
}

__device__ __forceinline__ uint32_t ld_u32_bytes(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
__device__ __forceinline__ uint32_t ld_u16_bytes(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8);
}

// ---------------------------------------------------------------------------
// Repack kernels (one thread per GGUF block)
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void repack_q8_0_kernel(const uint8_t *__restrict__ raw,
                                                          int64_t n_rows, int nb,
                                                          uint8_t *__restrict__ tiles,
                                                          int64_t trb) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= n_rows * nb) return;
  const int64_t n = g / nb;
  const int b = (int)(g - n * nb);
  const uint8_t *src = raw + g * 34;
  uint8_t *row = tiles + n * trb;
  uint32_t w[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) w[i] = ld_u32_bytes(src + 2 + 4 * i);
  uint4 *qdst = (uint4 *)(row + 32 * b);
  qdst[0] = make_uint4(w[0], w[1], w[2], w[3]);
  qdst[1] = make_uint4(w[4], w[5], w[6], w[7]);
  const int k = nb * 32;
  row[k + 2 * b] = src[0];
  row[k + 2 * b + 1] = src[1];
  if (b == nb - 1)
    for (int64_t p = (int64_t)k + 2 * nb; p < trb; ++p) row[p] = 0;
}

__global__ __launch_bounds__(256) void repack_q6_k_kernel(const uint8_t *__restrict__ raw,
                                                          int64_t n_rows, int nsb,
                                                          uint8_t *__restrict__ tiles,
                                                          int64_t trb) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= n_rows * nsb) return;
  const int64_t n = g / nsb;
  const int b = (int)(g - n * nsb);
  const int k = nsb * 256;
  const uint8_t *src = raw + g * 210;
  uint8_t *row = tiles + n * trb;
  uint4 *ql = (uint4 *)(row + 128 * b);
  uint4 *qh = (uint4 *)(row + k / 2 + 64 * b);
  uint4 *sc = (uint4 *)(row + k / 2 + k / 4 + 16 * b);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint8_t *s = src + 16 * i;
    ql[i] = make_uint4(ld_u32_bytes(s), ld_u32_bytes(s + 4), ld_u32_bytes(s + 8), ld_u32_bytes(s + 12));
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint8_t *s = src + 128 + 16 * i;
    qh[i] = make_uint4(ld_u32_bytes(s), ld_u32_bytes(s + 4), ld_u32_bytes(s + 8), ld_u32_bytes(s + 12));
  }
  {
    const uint8_t *s = src + 192;
    sc[0] = make_uint4(ld_u32_bytes(s), ld_u32_bytes(s + 4), ld_u32_bytes(s + 8), ld_u32_bytes(s + 12));
  }
  uint8_t *dd = row + k / 2 + k / 4 + k / 16 + 2 * b;
  dd[0] = src[208];
  dd[1] = src[209];
  if (b == nsb - 1)
    for (int64_t p = (int64_t)210 * nsb; p < trb; ++p) row[p] = 0;
}

hipError_t launch_repack(const uint8_t *raw, int type, int64_t n_rows, int64_t k, uint8_t *tiles,
                         int64_t trb, hipStream_t s) {
  if (type == 12) {  // Q4_K rows are the raw superblocks
    return hipMemcpyAsync(tiles, raw, (size_t)(n_rows * trb), hipMemcpyDeviceToDevice, s);
  }
  if (type == 8) {
    const int nb = (int)(k / 32);
    const int64_t total = n_rows * nb;
    hipLaunchKernelGGL(repack_q8_0_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                       raw, n_rows, nb, tiles, trb);
    return hipGetLastError();
  }
  const int nsb = (int)(k / 256);
  const int64_t total = n_rows * nsb;
  hipLaunchKernelGGL(repack_q6_k_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                     raw, n_rows, nsb, tiles, trb);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Dequantization of the HBM row layout
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void dequant_q8_0_kernel(const uint8_t *__restrict__ tiles,
                                                           int64_t n_rows, int nb, int64_t trb,
                                                           float *__restrict__ out, int64_t ldo) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= n_rows * nb) return;
  const int64_t n = g / nb;
  const int b = (int)(g - n * nb);
  const uint8_t *row = tiles + n * trb;
  const uint4 q0 = ldg16(row + 32 * b), q1 = ldg16(row + 32 * b + 16);
  const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
  const float d = h2f(*(const uint16_t *)(row + 32 * nb + 2 * b));
  float *o = out + n * ldo + 32 * b;
#pragma unroll
  for (int i = 0; i < 32; ++i) o[i] = d * (float)(int8_t)((q[i >> 2] >> (8 * (i & 3))) & 0xFFu);
}

__global__ __launch_bounds__(256) void dequant_q4_k_kernel(const uint8_t *__restrict__ tiles,
                                                           int64_t n_rows, int nsb, int64_t trb,
                                                           float *__restrict__ out, int64_t ldo) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= n_rows * nsb * 8) return;
  const int part = (int)(g & 7);
  const int64_t sbg = g >> 3;
  const int64_t n = sbg / nsb;
  const int b = (int)(sbg - n * nsb);
  const uint8_t *blk = tiles + n * trb + 144 * b;
  const int c = part >> 1, h = part & 1;
  const uint4 hd = ldg16(blk);
  const uint4 qv = ldg16(blk + 16 + 32 * c + 16 * h);
  const uint32_t q[4] = {qv.x, qv.y, qv.z, qv.w};
  float lo[16], hi[16];
  q4k_decode16(hd.x, hd.y, hd.z, hd.w, c, q, lo, hi);
  float *o = out + n * ldo + 256 * b + 64 * c + 16 * h;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    o[i] = lo[i];
    o[32 + i] = hi[i];
  }
}

__global__ __launch_bounds__(256) void dequant_q6_k_kernel(const uint8_t *__restrict__ tiles,
                                                           int64_t n_rows, int nsb, int64_t trb,
                                                           float *__restrict__ out, int64_t ldo) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= n_rows * nsb * 4) return;
  const int part = (int)(g & 3);
  const int64_t sbg = g >> 2;
  const int64_t n = sbg / nsb;
  const int b = (int)(sbg - n * nsb);
  const int k = nsb * 256;
  const int h = part >> 1, gg = part & 1;
  const uint8_t *row = tiles + n * trb;
  const uint4 a = ldg16(row + 128 * b + 64 * h + 16 * gg);
  const uint4 bq = ldg16(row + 128 * b + 64 * h + 32 + 16 * gg);
  const uint4 hq = ldg16(row + k / 2 + 64 * b + 32 * h + 16 * gg);
  const int8_t *scp = (const int8_t *)(row + k / 2 + k / 4 + 16 * b + 8 * h + gg);
  const int sc[4] = {scp[0], scp[2], scp[4], scp[6]};
  const float d = h2f(*(const uint16_t *)(row + k / 2 + k / 4 + k / 16 + 2 * b));
  const uint32_t qa[4] = {a.x, a.y, a.z, a.w}, qb[4] = {bq.x, bq.y, bq.z, bq.w};
  const uint32_t qh[4] = {hq.x, hq.y, hq.z, hq.w};
  float v[4][16];
  q6k_decode64(d, sc, qa, qb, qh, v);
  float *o = out + n * ldo + 256 * b + 128 * h + 16 * gg;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[32 * t + i] = v[t][i];
}

hipError_t launch_dequant(const uint8_t *tiles, int type, int64_t n_rows, int64_t k, int64_t trb,
                          float *out, int64_t ldo, hipStream_t s) {
  if (type == 8) {
    const int nb = (int)(k / 32);
    const int64_t total = n_rows * nb;
    hipLaunchKernelGGL(dequant_q8_0_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                       tiles, n_rows, nb, trb, out, ldo);
  } else if (type == 12) {
    const int nsb = (int)(k / 256);
    const int64_t total = n_rows * nsb * 8;
    hipLaunchKernelGGL(dequant_q4_k_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                       tiles, n_rows, nsb, trb, out, ldo);
  } else {
    const int nsb = (int)(k / 256);
    const int64_t total = n_rows * nsb * 4;
    hipLaunchKernelGGL(dequant_q6_k_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                       tiles, n_rows, nsb, trb, out, ldo);
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Dequantization of raw GGUF bytes (any alignment: byte loads)
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void dequant_raw_q8_0_kernel(const uint8_t *__restrict__ raw,
                                                               int64_t nb,
                                                               float *__restrict__ out) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nb) return;
  const uint8_t *src = raw + b * 34;
  const float d = h2f(ld_u16_bytes(src));
  float *o = out + 32 * b;
#pragma unroll
  for (int i = 0; i < 32; ++i) o[i] = d * (float)(int8_t)src[2 + i];
}

__global__ __launch_bounds__(256) void dequant_raw_q4_k_kernel(const uint8_t *__restrict__ raw,
                                                               int64_t nsb,
                                                               float *__restrict__ out) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= nsb * 8) return;
  const int part = (int)(g & 7);
  const int64_t b = g >> 3;
  const uint8_t *blk = raw + b * 144;
  const int c = part >> 1, h = part & 1;
  uint32_t q[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) q[i] = ld_u32_bytes(blk + 16 + 32 * c + 16 * h + 4 * i);
  float lo[16], hi[16];
  q4k_decode16(ld_u32_bytes(blk), ld_u32_bytes(blk + 4), ld_u32_bytes(blk + 8),
               ld_u32_bytes(blk + 12), c, q, lo, hi);
  float *o = out + 256 * b + 64 * c + 16 * h;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    o[i] = lo[i];
    o[32 + i] = hi[i];
  }
}

__global__ __launch_bounds__(256) void dequant_raw_q6_k_kernel(const uint8_t *__restrict__ raw,
                                                               int64_t nsb,
                                                               float *__restrict__ out) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= nsb * 4) return;
  const int part = (int)(g & 3);
  const int64_t b = g >> 2;
  const int h = part >> 1, gg = part & 1;
  const uint8_t *blk = raw + b * 210;
  uint32_t qa[4], qb[4], qh[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    qa[i] = ld_u32_bytes(blk + 64 * h + 16 * gg + 4 * i);
    qb[i] = ld_u32_bytes(blk + 64 * h + 32 + 16 * gg + 4 * i);
    qh[i] = ld_u32_bytes(blk + 128 + 32 * h + 16 * gg + 4 * i);
  }
  const int8_t *scp = (const int8_t *)(blk + 192 + 8 * h + gg);
  const int sc[4] = {scp[0], scp[2], scp[4], scp[6]};
  const float d = h2f(ld_u16_bytes(blk + 208));
  float v[4][16];
  q6k_decode64(d, sc, qa, qb, qh, v);
  float *o = out + 256 * b + 128 * h + 16 * gg;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[32 * t + i] = v[t][i];
}

hipError_t launch_dequant_raw(const uint8_t *raw, int type, int64_t n_elems, float *out,
                              hipStream_t s) {
  if (type == 8) {
    const int64_t nb = n_elems / 32;
    hipLaunchKernelGGL(dequant_raw_q8_0_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0,
                       s, raw, nb, out);
  } else if (type == 12) {
    const int64_t nsb = n_elems / 256;
    hipLaunchKernelGGL(dequant_raw_q4_k_kernel, dim3((unsigned)((nsb * 8 + 255) / 256)), dim3(256),
                       0, s, raw, nsb, out);
  } else {
    const int64_t nsb = n_elems / 256;
    hipLaunchKernelGGL(dequant_raw_q6_k_kernel, dim3((unsigned)((nsb * 4 + 255) / 256)), dim3(256),
                       0, s, raw, nsb, out);
  }
  return hipGetLastError();
}

}  // namespace gguf
