// Repack (raw GGUF bytes -> HBM row-tile layout) and dequantization to f32.
//
// Dequantization is bit-exact to the reference CPU dequant
// (webgpu/src/model/gguf-dequant.ts:110-127 Q4_0, :130-149 Q5_0, :152-166 Q8_0,
// :181-206 Q2_K, :217-252 Q3_K, :255-281 Q4_K, :283-314 Q5_K, :321-341 IQ4_NL, :344-366 IQ4_XS, :369-399 Q6_K): every
// product in these formats is exact in f32, so the
// only rounding is the final Q4_K subtraction, which f32 arithmetic (fused
// or not) rounds exactly once, as the reference's f64-then-Float32Array does.
// The row-tile layout itself is described in common.hpp.
#include "common.hpp"
#include "iq.hpp"

namespace gguf {

__device__ __forceinline__ uint32_t ld_u32_bytes(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
__device__ __forceinline__ uint32_t ld_u16_bytes(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8);
}
__device__ __forceinline__ uint2 ld_u64_bytes(const uint8_t *p) {
  return make_uint2(ld_u32_bytes(p), ld_u32_bytes(p + 4));
}

// 4-bit code of element k (0..31) of a 32-element GGUF block: the low nibble
// of qs[k] for k < 16, the high nibble of qs[k - 16] above
// (gguf-dequant.ts:110-127, :130-149, :321-341).
__device__ __forceinline__ uint32_t b32_code_of(const uint8_t *qs, int k) {
  return k < 16 ? (qs[k] & 0x0Fu) : (qs[k - 16] >> 4);
}

// IQ4_NL codebook (kvalues_iq4nl, gguf-dequant.ts:29).
__constant__ int8_t kIq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                  1,    13,   25,  38,  53,  69,  89,  113};

// Value of element k of a Q4_0 / Q5_0 / IQ4_NL block with scale d, code q (4 bits) and
// fifth bit h (Q5_0).  d * an integer of at most 8 bits: exact in f32.
template <int TYPE>
__device__ __forceinline__ float b32_value(float d, uint32_t q, uint32_t h) {
  if constexpr (TYPE == 2) return d * (float)((int)q - 8);
  if constexpr (TYPE == 6) return d * (float)((int)(q | (h << 4)) - 16);
  return d * (float)kIq4nl[q];
}

// ---------------------------------------------------------------------------
// Repack: one thread per (row n < 16 * tiles, unit u).  Rows past N write zeros.
// ---------------------------------------------------------------------------
template <int TYPE>
__global__ __launch_bounds__(256) void repack_kernel(const uint8_t *__restrict__ raw, int64_t n_rows,
                                                     int nu, int64_t n_pad,
                                                     uint8_t *__restrict__ tiles) {
  constexpr int UB = Fmt<TYPE>::UB, TU = Fmt<TYPE>::TU;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n_pad * nu) return;
  const int64_t n = gid / nu;
  const int u = (int)(gid - n * nu);
  const int r = (int)(n & 15);
  uint8_t *tu = tiles + ((n >> 4) * nu + u) * (int64_t)TU;
  if (n >= n_rows) {  // padding row of the last tile: every byte of its slots is zero
    const uint4 z = make_uint4(0, 0, 0, 0);
    if (TYPE == 12 || TYPE == 13) {
      *(uint4 *)(tu + 16 * r) = z;
#pragma unroll
      for (int p = 0; p < 8; ++p) *(uint4 *)(tu + 256 + (p * 16 + r) * 16) = z;
      if (TYPE == 13)
#pragma unroll
        for (int g = 0; g < 4; ++g) *(uint2 *)(tu + 2304 + (16 * g + r) * 8) = make_uint2(0, 0);
    } else if (TYPE == 14) {
#pragma unroll
      for (int p = 0; p < 12; ++p) *(uint4 *)(tu + (p * 16 + r) * 16) = z;
      *(uint4 *)(tu + 3072 + 16 * r) = z;
      *(uint16_t *)(tu + 3328 + 2 * r) = 0;
    } else if (TYPE == 11) {
      *(uint32_t *)(tu + 12 * r) = 0u;
      *(uint32_t *)(tu + 12 * r + 4) = 0u;
      *(uint32_t *)(tu + 12 * r + 8) = 0u;
      *(uint16_t *)(tu + 192 + 2 * r) = 0;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        *(uint2 *)(tu + 224 + (16 * g + r) * 8) = make_uint2(0, 0);
        *(uint4 *)(tu + 736 + (16 * g + r) * 16) = z;
      }
    } else if (TYPE == 10) {
      *(uint4 *)(tu + 16 * r) = z;
      *(uint32_t *)(tu + 256 + 4 * r) = 0u;
#pragma unroll
      for (int g = 0; g < 4; ++g) *(uint4 *)(tu + 320 + (16 * g + r) * 16) = z;
    } else if (TYPE == 23) {
      *(uint2 *)(tu + 8 * r) = make_uint2(0, 0);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        *(uint4 *)(tu + 128 + (16 * g + r) * 32) = z;
        *(uint4 *)(tu + 128 + (16 * g + r) * 32 + 16) = z;
      }
    } else if (is_b32(TYPE)) {
      *(uint16_t *)(tu + 2 * r) = 0;
      if (TYPE == 6) *(uint32_t *)(tu + 32 + 4 * r) = 0u;
#pragma unroll
      for (int g = 0; g < 4; ++g) *(uint32_t *)(tu + b32_code_off<TYPE>() + (16 * g + r) * 4) = 0u;
    } else {
      *(uint16_t *)(tu + 2 * r) = 0;
#pragma unroll
      for (int g = 0; g < 4; ++g) *(uint2 *)(tu + 32 + (16 * g + r) * 8) = make_uint2(0, 0);
    }
    return;
  }
  const uint8_t *src = raw + (n * nu + u) * UB;
  if (TYPE == 12 || TYPE == 13) {
    *(uint4 *)(tu + 16 * r) = make_uint4(ld_u32_bytes(src), ld_u32_bytes(src + 4),
                                         ld_u32_bytes(src + 8), ld_u32_bytes(src + 12));
    const uint8_t *qs = src + (TYPE == 13 ? 48 : 16);
    if (TYPE == 13)
#pragma unroll
      for (int g = 0; g < 4; ++g) *(uint2 *)(tu + 2304 + (16 * g + r) * 8) = ld_u64_bytes(src + 16 + 8 * g);
#pragma unroll
    for (int cp = 0; cp < 2; ++cp)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint2 a = ld_u64_bytes(qs + 64 * cp + 8 * g);
        const uint2 b = ld_u64_bytes(qs + 64 * cp + 32 + 8 * g);
        *(uint4 *)(tu + 256 + ((4 * cp + g) * 16 + r) * 16) = make_uint4(a.x, a.y, b.x, b.y);
      }
  } else if (TYPE == 14) {
    const uint8_t *ql = src, *qh = src + 128;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint32_t dw[12];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int hf = i >> 1, lh = i & 1;
        dw[3 * i] = ld_u32_bytes(ql + 64 * hf + 16 * lh + 4 * g);
        dw[3 * i + 1] = ld_u32_bytes(ql + 64 * hf + 32 + 16 * lh + 4 * g);
        dw[3 * i + 2] = ld_u32_bytes(qh + 32 * hf + 16 * lh + 4 * g);
      }
#pragma unroll
      for (int v = 0; v < 3; ++v)
        *(uint4 *)(tu + ((4 * v + g) * 16 + r) * 16) =
            make_uint4(dw[4 * v], dw[4 * v + 1], dw[4 * v + 2], dw[4 * v + 3]);
    }
    const uint8_t *sc = src + 192;
    *(uint4 *)(tu + 3072 + 16 * r) = make_uint4(ld_u32_bytes(sc), ld_u32_bytes(sc + 4),
                                                ld_u32_bytes(sc + 8), ld_u32_bytes(sc + 12));
    *(uint16_t *)(tu + 3328 + 2 * r) = (uint16_t)ld_u16_bytes(src + 208);
  } else if (TYPE == 11) {  // Q3_K: scales, d, then the lane's hmask and qs pieces
    *(uint32_t *)(tu + 12 * r) = ld_u32_bytes(src + 96);
    *(uint32_t *)(tu + 12 * r + 4) = ld_u32_bytes(src + 100);
    *(uint32_t *)(tu + 12 * r + 8) = ld_u32_bytes(src + 104);
    *(uint16_t *)(tu + 192 + 2 * r) = (uint16_t)ld_u16_bytes(src + 108);
    const uint8_t *qs = src + 32;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      *(uint2 *)(tu + 224 + (16 * g + r) * 8) = ld_u64_bytes(src + 8 * g);
      *(uint4 *)(tu + 736 + (16 * g + r) * 16) =
          make_uint4(ld_u32_bytes(qs + 8 * g), ld_u32_bytes(qs + 8 * g + 4),
                     ld_u32_bytes(qs + 32 + 8 * g), ld_u32_bytes(qs + 32 + 8 * g + 4));
    }
  } else if (TYPE == 10) {  // Q2_K: scales, d | dmin, then the lane's two 8-byte qs pieces
    *(uint4 *)(tu + 16 * r) = make_uint4(ld_u32_bytes(src), ld_u32_bytes(src + 4),
                                         ld_u32_bytes(src + 8), ld_u32_bytes(src + 12));
    *(uint32_t *)(tu + 256 + 4 * r) = ld_u32_bytes(src + 80);
    const uint8_t *qs = src + 16;
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *(uint4 *)(tu + 320 + (16 * g + r) * 16) =
          make_uint4(ld_u32_bytes(qs + 8 * g), ld_u32_bytes(qs + 8 * g + 4),
                     ld_u32_bytes(qs + 32 + 8 * g), ld_u32_bytes(qs + 32 + 8 * g + 4));
  } else if (TYPE == 23) {  // IQ4_XS: header, then each sub-block's codes regrouped per lane
    *(uint2 *)(tu + 8 * r) = ld_u64_bytes(src);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint32_t w[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint8_t *qs = src + 8 + 16 * j;
        w[j] = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          w[j] |= (b32_code_of(qs, 8 * g + i) | (b32_code_of(qs, 8 * g + 4 + i) << 4)) << (8 * i);
      }
      uint8_t *p = tu + 128 + (16 * g + r) * 32;
      *(uint4 *)p = make_uint4(w[0], w[1], w[2], w[3]);
      *(uint4 *)(p + 16) = make_uint4(w[4], w[5], w[6], w[7]);
    }
  } else if (is_b32(TYPE)) {  // Q4_0 / Q5_0 / IQ4_NL: codes regrouped per lane
    *(uint16_t *)(tu + 2 * r) = (uint16_t)ld_u16_bytes(src);
    if (TYPE == 6) *(uint32_t *)(tu + 32 + 4 * r) = ld_u32_bytes(src + 2);
    const uint8_t *qs = src + (TYPE == 6 ? 6 : 2);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint32_t w = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w |= (b32_code_of(qs, 8 * g + i) | (b32_code_of(qs, 8 * g + 4 + i) << 4)) << (8 * i);
      *(uint32_t *)(tu + b32_code_off<TYPE>() + (16 * g + r) * 4) = w;
    }
  } else {  // Q8_0
    *(uint16_t *)(tu + 2 * r) = (uint16_t)ld_u16_bytes(src);
#pragma unroll
    for (int g = 0; g < 4; ++g) *(uint2 *)(tu + 32 + (16 * g + r) * 8) = ld_u64_bytes(src + 2 + 8 * g);
  }
}

// IQ grid types: one thread per (row, unit); d and the rest of the block to
// their places in the tile unit (iq.hpp), zeros for the padding rows.
template <int TYPE>
__global__ __launch_bounds__(256) void repack_iq_kernel(const uint8_t *__restrict__ raw, int64_t n_rows,
                                                        int nu, int64_t n_pad,
                                                        uint8_t *__restrict__ tiles) {
  constexpr int BS = IqFmt<TYPE>::BS, HASD = IqFmt<TYPE>::HASD;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n_pad * nu) return;
  const int64_t n = gid / nu;
  const int u = (int)(gid - n * nu);
  const int r = (int)(n & 15);
  uint8_t *tu = tiles + ((n >> 4) * nu + u) * (int64_t)Fmt<TYPE>::TU;
  const bool pad = n >= n_rows;
  const uint8_t *src = raw + (n * nu + u) * BS;
  if (HASD) *(uint16_t *)(tu + 2 * r) = pad ? 0 : (uint16_t)ld_u16_bytes(src);
  uint32_t *rec = (uint32_t *)(tu + iq_rec_off<TYPE>(r));
  for (int i = 0; i < iq_rd<TYPE>(); ++i) rec[i] = pad ? 0u : ld_u32_bytes(src + 2 * HASD + 4 * i);
}

hipError_t launch_repack(const uint8_t *raw, int type, int64_t n_rows, int64_t k, uint8_t *tiles,
                         hipStream_t s) {
  const int nu = (int)(k / unit_elems(type));
  const int64_t n_pad = (n_rows + 15) & ~(int64_t)15;
  const int64_t total = n_pad * nu;
  const dim3 grid((unsigned)((total + 255) / 256)), block(256);
  if (type == 16)
    hipLaunchKernelGGL(repack_iq_kernel<16>, grid, block, 0, s, raw, n_rows, nu, n_pad, tiles);
  else if (type == 17)
    hipLaunchKernelGGL(repack_iq_kernel<17>, grid, block, 0, s, raw, n_rows, nu, n_pad, tiles);
  else if (type == 18)
    hipLaunchKernelGGL(repack_iq_kernel<18>, grid, block, 0, s, raw, n_rows, nu, n_pad, tiles);
  else if (type == 21)
    hipLaunchKernelGGL(repack_iq_kernel<21>, grid, block, 0, s, raw, n_rows, nu, n_pad, tiles);
  else if (type == 22)
    hipLaunchKernelGGL(repack_iq_kernel<22>, grid, block, 0, s, raw, n_rows, nu, n_pad, tiles);
  else if (type == 29)
    hipLaunchKernelGGL(repack_iq_kernel<29>, grid, block, 0, s, raw, n_rows, nu, n_pad, tiles);
  else if (type == 12)
    hipLaunchKernelGGL(repack_kernel<12>, grid, block, 0, s, raw, n_rows, nu, n_pad, tiles);
  else if (type == 13)
    hipLaunchKernelGGL(repack_kernel<13>, grid, block, 0, s, raw, n_rows, nu, n_pad, tiles);
  else if (type == 14)
    hipLaunchKernelGGL(repack_kernel<14>, grid, block, 0, s, raw, n_rows, nu, n_pad, tiles);
  else if (type == 2)
    hipLaunchKernelGGL(repack_kernel<2>, grid, block, 0, s, raw, n_rows, nu, n_pad, tiles);
  else if (type == 6)
    hipLaunchKernelGGL(repack_kernel<6>, grid, block, 0, s, raw, n_rows, nu, n_pad, tiles);
  else if (type == 20)
    hipLaunchKernelGGL(repack_kernel<20>, grid, block, 0, s, raw, n_rows, nu, n_pad, tiles);
  else if (type == 23)
    hipLaunchKernelGGL(repack_kernel<23>, grid, block, 0, s, raw, n_rows, nu, n_pad, tiles);
  else if (type == 10)
    hipLaunchKernelGGL(repack_kernel<10>, grid, block, 0, s, raw, n_rows, nu, n_pad, tiles);
  else if (type == 11)
    hipLaunchKernelGGL(repack_kernel<11>, grid, block, 0, s, raw, n_rows, nu, n_pad, tiles);
  else
    hipLaunchKernelGGL(repack_kernel<8>, grid, block, 0, s, raw, n_rows, nu, n_pad, tiles);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Per-unit decoders shared by the tile and raw dequant kernels.
// ---------------------------------------------------------------------------

// Q4_K chunk c (32 qs bytes in q[0..7]) -> 32 values of sub-block 2c (lo) and
// 32 of sub-block 2c + 1 (hi).
__device__ __forceinline__ void q4k_decode_chunk(uint32_t hdr0, uint32_t s0, uint32_t s1,
                                                 uint32_t s2, int c, const uint32_t q[8],
                                                 float *lo, float *hi) {
  const float d = h2f(hdr0), dmin = h2f(hdr0 >> 16);
  uint32_t sc0, m0, sc1, m1;
  q4k_scale_min(2 * c, s0, s1, s2, sc0, m0);
  q4k_scale_min(2 * c + 1, s0, s1, s2, sc1, m1);
  const float d1 = d * (float)sc0, min1 = dmin * (float)m0;
  const float d2 = d * (float)sc1, min2 = dmin * (float)m1;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const uint32_t b = (q[i >> 2] >> (8 * (i & 3))) & 0xFFu;
    lo[i] = d1 * (float)(b & 0x0Fu) - min1;
    hi[i] = d2 * (float)(b >> 4) - min2;
  }
}

// Q5_K chunk c: as q4k_decode_chunk, with 16 x bit 2c (lo) / 2c + 1 (hi) of
// qh[l] (bytes of h[0..7]) added to the codes (gguf-dequant.ts:283-314).
__device__ __forceinline__ void q5k_decode_chunk(uint32_t hdr0, uint32_t s0, uint32_t s1,
                                                 uint32_t s2, int c, const uint32_t q[8],
                                                 const uint32_t h[8], float *lo, float *hi) {
  const float d = h2f(hdr0), dmin = h2f(hdr0 >> 16);
  uint32_t sc0, m0, sc1, m1;
  q4k_scale_min(2 * c, s0, s1, s2, sc0, m0);
  q4k_scale_min(2 * c + 1, s0, s1, s2, sc1, m1);
  const float d1 = d * (float)sc0, min1 = dmin * (float)m0;
  const float d2 = d * (float)sc1, min2 = dmin * (float)m1;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const uint32_t b = (q[i >> 2] >> (8 * (i & 3))) & 0xFFu;
    const uint32_t hb = (h[i >> 2] >> (8 * (i & 3))) & 0xFFu;
    lo[i] = d1 * (float)((b & 0x0Fu) | (((hb >> (2 * c)) & 1u) << 4)) - min1;
    hi[i] = d2 * (float)((b >> 4) | (((hb >> (2 * c + 1)) & 1u) << 4)) - min2;
  }
}

// Q6_K 6-bit value (unsigned, q + 32) of element (hf, t, l) from the ql byte
// ql[64 hf + 32 (t & 1) + l] and the qh byte qh[32 hf + l] (gguf-dequant.ts:369-399).
__device__ __forceinline__ int q6k_value(uint32_t qlb, uint32_t qhb, int t) {
  const uint32_t nib = (t >> 1) ? (qlb >> 4) : (qlb & 0x0Fu);
  return (int)(nib | (((qhb >> (2 * t)) & 3u) << 4)) - 32;
}

// ---------------------------------------------------------------------------
// Dequantization of the row-tile layout: out[n * ldo + k], rows n < N.
// ---------------------------------------------------------------------------

// Q4_K / Q5_K: one thread per (row, unit, chunk c).
template <int TYPE>
__global__ __launch_bounds__(256) void dequant_q4_k_kernel(const uint8_t *__restrict__ tiles,
                                                           int64_t n_rows, int nu,
                                                           float *__restrict__ out, int64_t ldo) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n_rows * nu * 4) return;
  const int c = (int)(gid & 3);
  const int64_t nuid = gid >> 2;
  const int64_t n = nuid / nu;
  const int u = (int)(nuid - n * nu);
  const int r = (int)(n & 15);
  const uint8_t *tu = tiles + ((n >> 4) * nu + u) * (int64_t)Fmt<TYPE>::TU;
  const uint4 hd = ldg16(tu + 16 * r);
  const int cp = c >> 1, h = c & 1;
  uint32_t q[8];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint4 p = ldg16(tu + 256 + ((4 * cp + g) * 16 + r) * 16);
    q[2 * g] = h ? p.z : p.x;
    q[2 * g + 1] = h ? p.w : p.y;
  }
  float lo[32], hi[32];
  if constexpr (TYPE == 13) {
    uint32_t h[8];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint2 p = *(const uint2 *)(tu + 2304 + (16 * g + r) * 8);
      h[2 * g] = p.x;
      h[2 * g + 1] = p.y;
    }
    q5k_decode_chunk(hd.x, hd.y, hd.z, hd.w, c, q, h, lo, hi);
  } else {
    q4k_decode_chunk(hd.x, hd.y, hd.z, hd.w, c, q, lo, hi);
  }
  float *o = out + n * ldo + 256 * (int64_t)u + 64 * c;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    o[i] = lo[i];
    o[32 + i] = hi[i];
  }
}

// Q6_K: one thread per (row, unit, half hf).
__global__ __launch_bounds__(256) void dequant_q6_k_kernel(const uint8_t *__restrict__ tiles,
                                                           int64_t n_rows, int nu,
                                                           float *__restrict__ out, int64_t ldo) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n_rows * nu * 2) return;
  const int hf = (int)(gid & 1);
  const int64_t nuid = gid >> 1;
  const int64_t n = nuid / nu;
  const int u = (int)(nuid - n * nu);
  const int r = (int)(n & 15);
  const uint8_t *tu = tiles + ((n >> 4) * nu + u) * (int64_t)Fmt<14>::TU;
  const float d = h2f(*(const uint16_t *)(tu + 3328 + 2 * r));
  const int8_t *sc = (const int8_t *)(tu + 3072 + 16 * r);
  float *o = out + n * ldo + 256 * (int64_t)u + 128 * hf;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    uint32_t dw[12];
#pragma unroll
    for (int v = 0; v < 3; ++v) {
      const uint4 p = ldg16(tu + ((4 * v + g) * 16 + r) * 16);
      dw[4 * v] = p.x; dw[4 * v + 1] = p.y; dw[4 * v + 2] = p.z; dw[4 * v + 3] = p.w;
    }
#pragma unroll
    for (int lh = 0; lh < 2; ++lh) {
      const int i = 2 * hf + lh;
      const uint32_t qa = dw[3 * i], qb = dw[3 * i + 1], qh = dw[3 * i + 2];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int l = 16 * lh + 4 * g + b;
        const uint32_t ab = (qa >> (8 * b)) & 0xFFu, bb = (qb >> (8 * b)) & 0xFFu;
        const uint32_t hb = (qh >> (8 * b)) & 0xFFu;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int q = q6k_value((t & 1) ? bb : ab, hb, t);
          o[32 * t + l] = d * (float)sc[8 * hf + 2 * t + lh] * (float)q;
        }
      }
    }
  }
}

// Q8_0: one thread per (row, block).
__global__ __launch_bounds__(256) void dequant_q8_0_kernel(const uint8_t *__restrict__ tiles,
                                                           int64_t n_rows, int nu,
                                                           float *__restrict__ out, int64_t ldo) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n_rows * nu) return;
  const int64_t n = gid / nu;
  const int u = (int)(gid - n * nu);
  const int r = (int)(n & 15);
  const uint8_t *tu = tiles + ((n >> 4) * nu + u) * (int64_t)Fmt<8>::TU;
  const float d = h2f(*(const uint16_t *)(tu + 2 * r));
  float *o = out + n * ldo + 32 * (int64_t)u;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint2 p = *(const uint2 *)(tu + 32 + (16 * g + r) * 8);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t w = i < 4 ? p.x : p.y;
      o[8 * g + i] = d * (float)(int8_t)((w >> (8 * (i & 3))) & 0xFFu);
    }
  }
}

// Q4_0 / Q5_0 / IQ4_NL: one thread per (row, block).
template <int TYPE>
__global__ __launch_bounds__(256) void dequant_b32_kernel(const uint8_t *__restrict__ tiles,
                                                          int64_t n_rows, int nu,
                                                          float *__restrict__ out, int64_t ldo) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n_rows * nu) return;
  const int64_t n = gid / nu;
  const int u = (int)(gid - n * nu);
  const int r = (int)(n & 15);
  const uint8_t *tu = tiles + ((n >> 4) * nu + u) * (int64_t)Fmt<TYPE>::TU;
  const float d = h2f(*(const uint16_t *)(tu + 2 * r));
  const uint32_t qh = TYPE == 6 ? *(const uint32_t *)(tu + 32 + 4 * r) : 0u;
  float *o = out + n * ldo + 32 * (int64_t)u;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint32_t w = *(const uint32_t *)(tu + b32_code_off<TYPE>() + (16 * g + r) * 4);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int k = 8 * g + i;
      const uint32_t q = (w >> (8 * (i & 3) + 4 * (i >> 2))) & 0x0Fu;
      o[k] = b32_value<TYPE>(d, q, (qh >> k) & 1u);
    }
  }
}

// Q2_K: one thread per (row, unit, half h).  Element 128 h + 32 j + 8 g + i
// has code (qs[32 h + 8 g + i] >> 2 j) & 3 and scale group 8 h + 2 j + (g >> 1);
// d * sc * q (at most 17 bits) and dmin * m are exact, the difference is
// rounded once.
__global__ __launch_bounds__(256) void dequant_q2_k_kernel(const uint8_t *__restrict__ tiles,
                                                           int64_t n_rows, int nu,
                                                           float *__restrict__ out, int64_t ldo) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n_rows * nu * 2) return;
  const int h = (int)(gid & 1);
  const int64_t nuid = gid >> 1;
  const int64_t n = nuid / nu;
  const int u = (int)(nuid - n * nu);
  const int r = (int)(n & 15);
  const uint8_t *tu = tiles + ((n >> 4) * nu + u) * (int64_t)Fmt<10>::TU;
  const uint8_t *sc = tu + 16 * r;
  const uint32_t dm = *(const uint32_t *)(tu + 256 + 4 * r);
  const float d = h2f(dm), dmin = h2f(dm >> 16);
  float *o = out + n * ldo + 256 * (int64_t)u + 128 * h;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint8_t *q = tu + 320 + (16 * g + r) * 16 + 8 * h;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t s = sc[8 * h + 2 * j + (g >> 1)];
      const float dl = d * (float)(s & 15u), ml = dmin * (float)(s >> 4);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[32 * j + 8 * g + i] = dl * (float)((q[i] >> (2 * j)) & 3u) - ml;
    }
  }
}

// Q3_K: one thread per (row, unit, half h).  Element 128 h + 32 j + 8 g + i
// has low bits (qs[32 h + 8 g + i] >> 2 j) & 3, high bit (hmask[8 g + i] >> (4 h
// + j)) & 1 and scale group 8 h + 2 j + (g >> 1); d * (sc - 32) * (q3 - 4) is
// exact in f32 (at most 20 significant bits).
__global__ __launch_bounds__(256) void dequant_q3_k_kernel(const uint8_t *__restrict__ tiles,
                                                           int64_t n_rows, int nu,
                                                           float *__restrict__ out, int64_t ldo) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n_rows * nu * 2) return;
  const int h = (int)(gid & 1);
  const int64_t nuid = gid >> 1;
  const int64_t n = nuid / nu;
  const int u = (int)(nuid - n * nu);
  const int r = (int)(n & 15);
  const uint8_t *tu = tiles + ((n >> 4) * nu + u) * (int64_t)Fmt<11>::TU;
  uint32_t S[4];
  q3k_scales(*(const uint32_t *)(tu + 12 * r), *(const uint32_t *)(tu + 12 * r + 4),
             *(const uint32_t *)(tu + 12 * r + 8), S);
  const float d = h2f(*(const uint16_t *)(tu + 192 + 2 * r));
  float *o = out + n * ldo + 256 * (int64_t)u + 128 * h;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint8_t *q = tu + 736 + (16 * g + r) * 16 + 8 * h;
    const uint8_t *hm = tu + 224 + (16 * g + r) * 8;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int grp = 8 * h + 2 * j + (g >> 1);
      const float dl = d * (float)((int)((S[grp >> 2] >> (8 * (grp & 3))) & 0xFFu) - 32);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int q3 = (int)(((q[i] >> (2 * j)) & 3u) | (((hm[i] >> (4 * h + j)) & 1u) << 2));
        o[32 * j + 8 * g + i] = dl * (float)(q3 - 4);
      }
    }
  }
}

// IQ4_XS: one thread per (row, unit, sub-block j).  d * (ls - 32) has at most
// 16 significant bits and times a codebook entry at most 23: exact in f32.
__global__ __launch_bounds__(256) void dequant_iq4_xs_kernel(const uint8_t *__restrict__ tiles,
                                                             int64_t n_rows, int nu,
                                                             float *__restrict__ out, int64_t ldo) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n_rows * nu * 8) return;
  const int j = (int)(gid & 7);
  const int64_t nuid = gid >> 3;
  const int64_t n = nuid / nu;
  const int u = (int)(nuid - n * nu);
  const int r = (int)(n & 15);
  const uint8_t *tu = tiles + ((n >> 4) * nu + u) * (int64_t)Fmt<23>::TU;
  const uint2 h = *(const uint2 *)(tu + 8 * r);
  const float dl = h2f(h.x) * (float)((int)iq4xs_ls(h.x >> 16, h.y, j) - 32);
  float *o = out + n * ldo + 256 * (int64_t)u + 32 * j;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint32_t w = *(const uint32_t *)(tu + 128 + (16 * g + r) * 32 + 4 * j);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      o[8 * g + i] = dl * (float)kIq4nl[(w >> (8 * (i & 3) + 4 * (i >> 2))) & 0x0Fu];
  }
}

// IQ grid types: one thread per (row, unit, sub-block ib).
template <int TYPE>
__global__ __launch_bounds__(256) void dequant_iq_kernel(const uint8_t *__restrict__ tiles,
                                                         int64_t n_rows, int nu,
                                                         float *__restrict__ out, int64_t ldo) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n_rows * nu * 8) return;
  const int ib = (int)(gid & 7);
  const int64_t nuid = gid >> 3;
  const int64_t n = nuid / nu;
  const int u = (int)(nuid - n * nu);
  const int r = (int)(n & 15);
  const uint8_t *tu = tiles + ((n >> 4) * nu + u) * (int64_t)Fmt<TYPE>::TU;
  iq_piece<TYPE>([&](int o) { return iq_tile_byte<TYPE>(tu, r, o); }, ib,
                 out + n * ldo + 256 * (int64_t)u + 32 * ib);
}

hipError_t launch_dequant(const uint8_t *tiles, int type, int64_t n_rows, int64_t k, float *out,
                          int64_t ldo, hipStream_t s) {
  const int nu = (int)(k / unit_elems(type));
  const int parts = (type == 12 || type == 13) ? 4
                    : (type == 14 || type == 10 || type == 11) ? 2
                    : (type == 23 || is_iq(type) ? 8 : 1);
  const int64_t total = n_rows * nu * parts;
  const dim3 grid((unsigned)((total + 255) / 256)), block(256);
  if (type == 16)
    hipLaunchKernelGGL(dequant_iq_kernel<16>, grid, block, 0, s, tiles, n_rows, nu, out, ldo);
  else if (type == 17)
    hipLaunchKernelGGL(dequant_iq_kernel<17>, grid, block, 0, s, tiles, n_rows, nu, out, ldo);
  else if (type == 18)
    hipLaunchKernelGGL(dequant_iq_kernel<18>, grid, block, 0, s, tiles, n_rows, nu, out, ldo);
  else if (type == 21)
    hipLaunchKernelGGL(dequant_iq_kernel<21>, grid, block, 0, s, tiles, n_rows, nu, out, ldo);
  else if (type == 22)
    hipLaunchKernelGGL(dequant_iq_kernel<22>, grid, block, 0, s, tiles, n_rows, nu, out, ldo);
  else if (type == 29)
    hipLaunchKernelGGL(dequant_iq_kernel<29>, grid, block, 0, s, tiles, n_rows, nu, out, ldo);
  else if (type == 12)
    hipLaunchKernelGGL(dequant_q4_k_kernel<12>, grid, block, 0, s, tiles, n_rows, nu, out, ldo);
  else if (type == 13)
    hipLaunchKernelGGL(dequant_q4_k_kernel<13>, grid, block, 0, s, tiles, n_rows, nu, out, ldo);
  else if (type == 14)
    hipLaunchKernelGGL(dequant_q6_k_kernel, grid, block, 0, s, tiles, n_rows, nu, out, ldo);
  else if (type == 2)
    hipLaunchKernelGGL(dequant_b32_kernel<2>, grid, block, 0, s, tiles, n_rows, nu, out, ldo);
  else if (type == 6)
    hipLaunchKernelGGL(dequant_b32_kernel<6>, grid, block, 0, s, tiles, n_rows, nu, out, ldo);
  else if (type == 20)
    hipLaunchKernelGGL(dequant_b32_kernel<20>, grid, block, 0, s, tiles, n_rows, nu, out, ldo);
  else if (type == 23)
    hipLaunchKernelGGL(dequant_iq4_xs_kernel, grid, block, 0, s, tiles, n_rows, nu, out, ldo);
  else if (type == 10)
    hipLaunchKernelGGL(dequant_q2_k_kernel, grid, block, 0, s, tiles, n_rows, nu, out, ldo);
  else if (type == 11)
    hipLaunchKernelGGL(dequant_q3_k_kernel, grid, block, 0, s, tiles, n_rows, nu, out, ldo);
  else
    hipLaunchKernelGGL(dequant_q8_0_kernel, grid, block, 0, s, tiles, n_rows, nu, out, ldo);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Dequantization of raw GGUF bytes (any alignment: byte loads)
// ---------------------------------------------------------------------------

// One piece of a raw GGUF row: a Q8_0 block (32 values), a 64-value chunk c
// of a Q4_K superblock, or a 128-value half hf of a Q6_K superblock.
__device__ __forceinline__ void raw_piece_q8_0(const uint8_t *blk, float *o) {
  const float d = h2f(ld_u16_bytes(blk));
#pragma unroll
  for (int i = 0; i < 32; ++i) o[i] = d * (float)(int8_t)blk[2 + i];
}

__device__ __forceinline__ void raw_piece_q4_k(const uint8_t *blk, int c, float *o) {
  uint32_t q[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) q[i] = ld_u32_bytes(blk + 16 + 32 * c + 4 * i);
  float lo[32], hi[32];
  q4k_decode_chunk(ld_u32_bytes(blk), ld_u32_bytes(blk + 4), ld_u32_bytes(blk + 8),
                   ld_u32_bytes(blk + 12), c, q, lo, hi);
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    o[i] = lo[i];
    o[32 + i] = hi[i];
  }
}

__device__ __forceinline__ void raw_piece_q5_k(const uint8_t *blk, int c, float *o) {
  uint32_t q[8], h[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    q[i] = ld_u32_bytes(blk + 48 + 32 * c + 4 * i);
    h[i] = ld_u32_bytes(blk + 16 + 4 * i);
  }
  float lo[32], hi[32];
  q5k_decode_chunk(ld_u32_bytes(blk), ld_u32_bytes(blk + 4), ld_u32_bytes(blk + 8),
                   ld_u32_bytes(blk + 12), c, q, h, lo, hi);
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    o[i] = lo[i];
    o[32 + i] = hi[i];
  }
}

__device__ __forceinline__ void raw_piece_q6_k(const uint8_t *blk, int hf, float *o) {
  const float d = h2f(ld_u16_bytes(blk + 208));
  const int8_t *sc = (const int8_t *)(blk + 192);
  for (int l = 0; l < 32; ++l) {
    const uint32_t ab = blk[64 * hf + l], bb = blk[64 * hf + 32 + l], hb = blk[128 + 32 * hf + l];
#pragma unroll
    for (int t = 0; t < 4; ++t)
      o[32 * t + l] = d * (float)sc[8 * hf + 2 * t + l / 16] * (float)q6k_value((t & 1) ? bb : ab, hb, t);
  }
}

// Q4_0 / Q5_0 / IQ4_NL block (32 values) from raw GGUF bytes.
template <int TYPE>
__device__ __forceinline__ void raw_piece_b32(const uint8_t *blk, float *o) {
  const float d = h2f(ld_u16_bytes(blk));
  const uint32_t qh = TYPE == 6 ? ld_u32_bytes(blk + 2) : 0u;
  const uint8_t *qs = blk + (TYPE == 6 ? 6 : 2);
#pragma unroll
  for (int k = 0; k < 32; ++k) o[k] = b32_value<TYPE>(d, b32_code_of(qs, k), (qh >> k) & 1u);
}

// Half h (128 values) of a Q2_K superblock from raw GGUF bytes (gguf-dequant.ts:191-203).
__device__ __forceinline__ void raw_piece_q2_k(const uint8_t *blk, int h, float *o) {
  const float d = h2f(ld_u16_bytes(blk + 80)), dmin = h2f(ld_u16_bytes(blk + 82));
  const uint8_t *q = blk + 16 + 32 * h;
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const uint32_t s = blk[8 * h + 2 * j + sub];
      const float dl = d * (float)(s & 15u), ml = dmin * (float)(s >> 4);
#pragma unroll
      for (int l = 0; l < 16; ++l)
        o[32 * j + 16 * sub + l] = dl * (float)((q[16 * sub + l] >> (2 * j)) & 3u) - ml;
    }
}

// Half h (128 values) of a Q3_K superblock from raw GGUF bytes (gguf-dequant.ts:232-249).
__device__ __forceinline__ void raw_piece_q3_k(const uint8_t *blk, int h, float *o) {
  uint32_t S[4];
  q3k_scales(ld_u32_bytes(blk + 96), ld_u32_bytes(blk + 100), ld_u32_bytes(blk + 104), S);
  const float d = h2f(ld_u16_bytes(blk + 108));
  const uint8_t *q = blk + 32 + 32 * h;
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int grp = 8 * h + 2 * j + sub;
      const float dl = d * (float)((int)((S[grp >> 2] >> (8 * (grp & 3))) & 0xFFu) - 32);
#pragma unroll
      for (int l = 0; l < 16; ++l) {
        const int q3 = (int)(((q[16 * sub + l] >> (2 * j)) & 3u) |
                             (((blk[16 * sub + l] >> (4 * h + j)) & 1u) << 2));
        o[32 * j + 16 * sub + l] = dl * (float)(q3 - 4);
      }
    }
}

// Sub-block j (32 values) of an IQ4_XS superblock from raw GGUF bytes.
__device__ __forceinline__ void raw_piece_iq4_xs(const uint8_t *blk, int j, float *o) {
  const float dl = h2f(ld_u16_bytes(blk)) *
                   (float)((int)iq4xs_ls(ld_u16_bytes(blk + 2), ld_u32_bytes(blk + 4), j) - 32);
  const uint8_t *qs = blk + 8 + 16 * j;
#pragma unroll
  for (int k = 0; k < 32; ++k) o[k] = dl * (float)kIq4nl[b32_code_of(qs, k)];
}

// Pieces per 256-element superblock (per 32-element block for Q8_0) and values per piece.
template <int TYPE>
struct RawPiece;
template <>
struct RawPiece<2> {
  static constexpr int PER_UNIT = 1, VALUES = 32;
  __device__ static void run(const uint8_t *unit, int, float *o) { raw_piece_b32<2>(unit, o); }
};
template <>
struct RawPiece<6> {
  static constexpr int PER_UNIT = 1, VALUES = 32;
  __device__ static void run(const uint8_t *unit, int, float *o) { raw_piece_b32<6>(unit, o); }
};
template <>
struct RawPiece<20> {
  static constexpr int PER_UNIT = 1, VALUES = 32;
  __device__ static void run(const uint8_t *unit, int, float *o) { raw_piece_b32<20>(unit, o); }
};
template <>
struct RawPiece<10> {
  static constexpr int PER_UNIT = 2, VALUES = 128;
  __device__ static void run(const uint8_t *unit, int p, float *o) { raw_piece_q2_k(unit, p, o); }
};
template <>
struct RawPiece<11> {
  static constexpr int PER_UNIT = 2, VALUES = 128;
  __device__ static void run(const uint8_t *unit, int p, float *o) { raw_piece_q3_k(unit, p, o); }
};
template <>
struct RawPiece<23> {
  static constexpr int PER_UNIT = 8, VALUES = 32;
  __device__ static void run(const uint8_t *unit, int p, float *o) { raw_piece_iq4_xs(unit, p, o); }
};
template <>
struct RawPiece<8> {
  static constexpr int PER_UNIT = 1, VALUES = 32;
  __device__ static void run(const uint8_t *unit, int, float *o) { raw_piece_q8_0(unit, o); }
};
template <>
struct RawPiece<12> {
  static constexpr int PER_UNIT = 4, VALUES = 64;
  __device__ static void run(const uint8_t *unit, int p, float *o) { raw_piece_q4_k(unit, p, o); }
};
template <>
struct RawPiece<13> {
  static constexpr int PER_UNIT = 4, VALUES = 64;
  __device__ static void run(const uint8_t *unit, int p, float *o) { raw_piece_q5_k(unit, p, o); }
};
template <>
struct RawPiece<14> {
  static constexpr int PER_UNIT = 2, VALUES = 128;
  __device__ static void run(const uint8_t *unit, int p, float *o) { raw_piece_q6_k(unit, p, o); }
};

template <int TYPE>
struct RawPieceIq {
  static constexpr int PER_UNIT = 8, VALUES = 32;
  __device__ static void run(const uint8_t *unit, int p, float *o) {
    iq_piece<TYPE>([&](int off) { return (uint32_t)unit[off]; }, p, o);
  }
};
template <>
struct RawPiece<16> : RawPieceIq<16> {};
template <>
struct RawPiece<17> : RawPieceIq<17> {};
template <>
struct RawPiece<18> : RawPieceIq<18> {};
template <>
struct RawPiece<21> : RawPieceIq<21> {};
template <>
struct RawPiece<22> : RawPieceIq<22> {};
template <>
struct RawPiece<29> : RawPieceIq<29> {};

// Contiguous raw bytes: one thread per piece of the whole buffer.
template <int TYPE>
__global__ __launch_bounds__(256) void dequant_raw_kernel(const uint8_t *__restrict__ raw,
                                                          int64_t n_pieces,
                                                          float *__restrict__ out) {
  using P = RawPiece<TYPE>;
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= n_pieces) return;
  const int64_t u = g / P::PER_UNIT;
  P::run(raw + u * Fmt<TYPE>::UB, (int)(g % P::PER_UNIT), out + g * P::VALUES);
}

// Row gather: out[i * ldo + j] = dequant(raw row ids[i])[j].  One thread per
// (output row, piece).  An id outside [0, n_rows) reads nothing and writes a
// row of NaN, so a bad token id is visible in the output instead of faulting.
template <int TYPE>
__global__ __launch_bounds__(256) void get_rows_kernel(const uint8_t *__restrict__ raw,
                                                       int64_t n_rows, int64_t units_per_row,
                                                       const int64_t *__restrict__ ids,
                                                       int64_t n_ids, float *__restrict__ out,
                                                       int64_t ldo) {
  using P = RawPiece<TYPE>;
  const int64_t per_row = units_per_row * P::PER_UNIT;
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= n_ids * per_row) return;
  const int64_t i = g / per_row, p = g % per_row;
  const int64_t id = ids[i];
  float *o = out + i * ldo + p * P::VALUES;
  if (id < 0 || id >= n_rows) {
    for (int j = 0; j < P::VALUES; ++j) o[j] = __builtin_nanf("");
    return;
  }
  const uint8_t *unit = raw + (id * units_per_row + p / P::PER_UNIT) * Fmt<TYPE>::UB;
  P::run(unit, (int)(p % P::PER_UNIT), o);
}

template <int TYPE>
static void dequant_raw_type(const uint8_t *raw, int64_t n_elems, float *out, hipStream_t s) {
  const int64_t pieces = n_elems / RawPiece<TYPE>::VALUES;
  hipLaunchKernelGGL(dequant_raw_kernel<TYPE>, dim3((unsigned)((pieces + 255) / 256)), dim3(256),
                     0, s, raw, pieces, out);
}

hipError_t launch_dequant_raw(const uint8_t *raw, int type, int64_t n_elems, float *out,
                              hipStream_t s) {
  if (type == 16)
    dequant_raw_type<16>(raw, n_elems, out, s);
  else if (type == 17)
    dequant_raw_type<17>(raw, n_elems, out, s);
  else if (type == 18)
    dequant_raw_type<18>(raw, n_elems, out, s);
  else if (type == 21)
    dequant_raw_type<21>(raw, n_elems, out, s);
  else if (type == 22)
    dequant_raw_type<22>(raw, n_elems, out, s);
  else if (type == 29)
    dequant_raw_type<29>(raw, n_elems, out, s);
  else if (type == 8)
    dequant_raw_type<8>(raw, n_elems, out, s);
  else if (type == 2)
    dequant_raw_type<2>(raw, n_elems, out, s);
  else if (type == 6)
    dequant_raw_type<6>(raw, n_elems, out, s);
  else if (type == 20)
    dequant_raw_type<20>(raw, n_elems, out, s);
  else if (type == 23)
    dequant_raw_type<23>(raw, n_elems, out, s);
  else if (type == 10)
    dequant_raw_type<10>(raw, n_elems, out, s);
  else if (type == 11)
    dequant_raw_type<11>(raw, n_elems, out, s);
  else if (type == 12)
    dequant_raw_type<12>(raw, n_elems, out, s);
  else if (type == 13)
    dequant_raw_type<13>(raw, n_elems, out, s);
  else
    dequant_raw_type<14>(raw, n_elems, out, s);
  return hipGetLastError();
}

template <int TYPE>
static void get_rows_type(const uint8_t *raw, int64_t n_rows, int64_t k, const int64_t *ids,
                          int64_t n_ids, float *out, int64_t ldo, hipStream_t s) {
  const int64_t upr = k / Fmt<TYPE>::UE;
  const int64_t threads = n_ids * upr * RawPiece<TYPE>::PER_UNIT;
  hipLaunchKernelGGL(get_rows_kernel<TYPE>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     s, raw, n_rows, upr, ids, n_ids, out, ldo);
}

hipError_t launch_get_rows(const uint8_t *raw, int type, int64_t n_rows, int64_t k,
                           const int64_t *ids, int64_t n_ids, float *out, int64_t ldo,
                           hipStream_t s) {
  if (type == 16)
    get_rows_type<16>(raw, n_rows, k, ids, n_ids, out, ldo, s);
  else if (type == 17)
    get_rows_type<17>(raw, n_rows, k, ids, n_ids, out, ldo, s);
  else if (type == 18)
    get_rows_type<18>(raw, n_rows, k, ids, n_ids, out, ldo, s);
  else if (type == 21)
    get_rows_type<21>(raw, n_rows, k, ids, n_ids, out, ldo, s);
  else if (type == 22)
    get_rows_type<22>(raw, n_rows, k, ids, n_ids, out, ldo, s);
  else if (type == 29)
    get_rows_type<29>(raw, n_rows, k, ids, n_ids, out, ldo, s);
  else if (type == 8)
    get_rows_type<8>(raw, n_rows, k, ids, n_ids, out, ldo, s);
  else if (type == 2)
    get_rows_type<2>(raw, n_rows, k, ids, n_ids, out, ldo, s);
  else if (type == 6)
    get_rows_type<6>(raw, n_rows, k, ids, n_ids, out, ldo, s);
  else if (type == 20)
    get_rows_type<20>(raw, n_rows, k, ids, n_ids, out, ldo, s);
  else if (type == 23)
    get_rows_type<23>(raw, n_rows, k, ids, n_ids, out, ldo, s);
  else if (type == 10)
    get_rows_type<10>(raw, n_rows, k, ids, n_ids, out, ldo, s);
  else if (type == 11)
    get_rows_type<11>(raw, n_rows, k, ids, n_ids, out, ldo, s);
  else if (type == 12)
    get_rows_type<12>(raw, n_rows, k, ids, n_ids, out, ldo, s);
  else if (type == 13)
    get_rows_type<13>(raw, n_rows, k, ids, n_ids, out, ldo, s);
  else
    get_rows_type<14>(raw, n_rows, k, ids, n_ids, out, ldo, s);
  return hipGetLastError();
}

}  // namespace gguf
