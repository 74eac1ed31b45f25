// Shared device helpers and the internal launcher interface of libgguf_hip.
// gfx950 (CDNA4) only: wave64, MFMA, 160 KB LDS per CU.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gguf {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// IEEE half bits -> f32 with the hardware converter (subnormals, Inf and NaN
// preserved), the same mapping as f16ToF32 in gguf-dequant.ts:64-71.
__device__ __forceinline__ float h2f(uint32_t bits16) {
  return (float)__builtin_bit_cast(half_t, (uint16_t)(bits16 & 0xFFFFu));
}

// The two halves of a 32-bit word as f16 values.  Used with masks that leave a
// small unsigned integer q in each half: the half then holds q * 2^-24 (an f16
// subnormal) exactly, and `(float)h.x * a` compiles to v_fma_mix_f32, which
// converts the half and multiplies in one instruction.  The 2^24 factor is
// folded into the per-block scale afterwards (an exact power of two).
__device__ __forceinline__ half2_t as_h2(uint32_t w) { return __builtin_bit_cast(half2_t, w); }

__device__ __forceinline__ float fmix(half_t q, float a, float acc) {
  return __builtin_fmaf((float)q, a, acc);
}

// 6-bit (scale, min) pair j of a Q4_K superblock from its 12 scale bytes held
// in three little-endian words s0 = bytes 0-3, s1 = 4-7, s2 = 8-11
// (get_scale_min_k4, gguf-dequant.ts:169-176).
__device__ __forceinline__ void q4k_scale_min(int j, uint32_t s0, uint32_t s1, uint32_t s2,
                                              uint32_t &sc, uint32_t &m) {
  const int sh = 8 * (j & 3);
  const uint32_t b0 = (s0 >> sh) & 0xFFu;  // byte j (j < 4) or j - 4
  const uint32_t b1 = (s1 >> sh) & 0xFFu;  // byte j + 4 (j < 4) or j
  const uint32_t b2 = (s2 >> sh) & 0xFFu;  // byte j + 4 (j >= 4)
  if (j < 4) {
    sc = b0 & 63u;
    m = b1 & 63u;
  } else {
    sc = (b2 & 0x0Fu) | ((b0 >> 6) << 4);
    m = (b2 >> 4) | ((b1 >> 6) << 4);
  }
}

__device__ __forceinline__ uint4 ldg16(const void *p) { return *(const uint4 *)p; }

// Streaming (read-once) 16-byte load of weight data: nontemporal so the
// weight stream does not evict activations from L1/L2.
__device__ __forceinline__ uint4 ldg16_stream(const void *p) {
  const uint4 *q = (const uint4 *)p;
  uint4 r;
  r.x = __builtin_nontemporal_load(&q->x);
  r.y = __builtin_nontemporal_load(&q->y);
  r.z = __builtin_nontemporal_load(&q->z);
  r.w = __builtin_nontemporal_load(&q->w);
  return r;
}

}  // namespace gguf

// ---------------------------------------------------------------------------
// Internal launchers (host side).  Arguments are already validated by the API
// layer; each returns a hipError_t from the launch.
// ---------------------------------------------------------------------------
namespace gguf {

hipError_t launch_repack(const uint8_t *raw, int type, int64_t n_rows, int64_t k, uint8_t *tiles,
                         int64_t tile_row_bytes, hipStream_t s);
hipError_t launch_dequant(const uint8_t *tiles, int type, int64_t n_rows, int64_t k,
                          int64_t tile_row_bytes, float *out, int64_t ldo, hipStream_t s);
hipError_t launch_dequant_raw(const uint8_t *raw, int type, int64_t n_elems, float *out,
                              hipStream_t s);
hipError_t launch_gemv(const void *x, int x_type, int64_t ldx, const uint8_t *tiles, int type,
                       int64_t n, int64_t k, int64_t tile_row_bytes, float *y, int64_t ldy,
                       int64_t m, hipStream_t s);
hipError_t launch_mfma(const void *x, int x_type, int64_t ldx, const uint8_t *tiles, int type,
                       int64_t n, int64_t k, int64_t tile_row_bytes, float *y, int64_t ldy,
                       int64_t m, bool skinny, hipStream_t s);

}  // namespace gguf
