// Shared device helpers, the HBM row-tile layout and the internal launcher
// interface of libgguf_hip.  gfx950 (CDNA4) only: wave64, MFMA, 160 KB LDS/CU.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gguf {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// Shared-memory addressing by 32-bit LDS address.  A pointer into shared
// memory becomes its LDS address once (an address-space cast), and loads
// through such addresses fold constant offsets into the instruction, where
// offsets from the dynamic array's symbol each cost an add.
__device__ __forceinline__ uint32_t lds_addr32(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) unsigned char *)p;
}
template <typename T>
__device__ __forceinline__ T lds_ld(uint32_t a) {
  typedef uint32_t words_t __attribute__((ext_vector_type(sizeof(T) / 4)));
  return __builtin_bit_cast(T, *(const __attribute__((address_space(3))) words_t *)a);
}

// ---------------------------------------------------------------------------
// HBM row-tile layout.
//
// A weight of N rows x K columns is stored as ceil(N/16) row tiles of 16
// consecutive rows (rows past N are zero).  A tile holds, for each "unit" of
// the row (a 256-element superblock for Q4_K / Q5_K / Q6_K, a 32-element block for
// Q8_0) in K order, one tile-unit of 16 * (GGUF block bytes): the 16 rows'
// blocks interleaved at 16-byte (Q8_0 quant bytes: 8-byte) granularity so
// that one wave-wide load reads contiguous memory and lane (r = lane & 15,
// g = lane >> 4) receives exactly the bytes its MFMA operand needs:
//
//   Q4_K (2304 B)  [   0,  256) header of row r at 16 r: d, dmin, scales[12]
//                  [ 256, 2304) piece (cp, g, r) at 256 + ((4 cp + g) * 16 + r) * 16:
//                               qs[64 cp + 8 g, +8) | qs[64 cp + 32 + 8 g, +8)
//   Q5_K (2816 B)  [   0, 2304) as Q4_K (headers, then the qs pieces)
//                  [2304, 2816) piece (g, r) at 2304 + (16 g + r) * 8: qh[8 g, +8)
//   Q6_K (3360 B)  [   0, 3072) piece (v, g, r) at ((4 v + g) * 16 + r) * 16 holds
//                               dwords 4v..4v+3 of the lane's 12 quant dwords;
//                               for i = 2 hf + lh:  dword 3i   = ql[64 hf + 16 lh + 4 g, +4)
//                                                   dword 3i+1 = ql[64 hf + 32 + 16 lh + 4 g, +4)
//                                                   dword 3i+2 = qh[32 hf + 16 lh + 4 g, +4)
//                  [3072, 3328) scales sc[16] of row r at 3072 + 16 r
//                  [3328, 3360) d of row r at 3328 + 2 r
//   Q8_0 ( 544 B)  [   0,   32) d of row r at 2 r
//                  [  32,  544) piece (g, r) at 32 + (16 g + r) * 8: qs[8 g, +8)
//   Q4_0, IQ4_NL (288 B)  [0, 32) d of row r at 2 r
//                  [  32,  288) word (g, r) at 32 + (16 g + r) * 4: byte i holds the
//                               4-bit codes of elements 8 g + i (low nibble) and
//                               8 g + 4 + i (high nibble) of the block
//   Q5_0 ( 352 B)  [   0,   32) d of row r at 2 r
//                  [  32,   96) qh of row r at 32 + 4 r (bit k: fifth bit of element k)
//                  [  96,  352) word (g, r) at 96 + (16 g + r) * 4, as Q4_0
//   Q2_K (1344 B)  [   0,  256) scales[16] of row r at 16 r
//                  [ 256,  320) d | dmin << 16 of row r at 256 + 4 r
//                  [ 320, 1344) piece (g, r) at 320 + (16 g + r) * 16:
//                               qs[8 g, +8) | qs[32 + 8 g, +8)
//   Q3_K (1760 B)  [   0,  192) scales[12] of row r at 12 r
//                  [ 192,  224) d of row r at 192 + 2 r
//                  [ 224,  736) piece (g, r) at 224 + (16 g + r) * 8: hmask[8 g, +8)
//                  [ 736, 1760) piece (g, r) at 736 + (16 g + r) * 16:
//                               qs[8 g, +8) | qs[32 + 8 g, +8)
//   IQ4_XS (2176 B) [   0,  128) header of row r at 8 r: d, scales_h, scales_l[4]
//                  [ 128, 2176) piece (g, r) at 128 + (16 g + r) * 32: word j (j = 0..7)
//                               holds sub-block j's codes 8 g .. 8 g + 7, as Q4_0
//
// The 32-element block types (Q4_0, Q5_0, IQ4_NL; element k of a GGUF block
// is the low nibble of qs[k] for k < 16, the high nibble of qs[k - 16] above)
// and IQ4_XS (whose 32-element sub-blocks store their codes the same way) are
// the only ones whose bytes are reordered inside a row's block: each lane's
// eight codes of a (sub-)block sit in one word, in the order b32_codes unpacks.
//
// Byte offset of (tile t, unit u) = (t * units_per_row + u) * tile_unit_bytes.
// No bytes are added: a tile is exactly 16 rows of GGUF blocks.
// ---------------------------------------------------------------------------
constexpr int kTileRows = 16;

template <int TYPE>
struct Fmt;
template <>
struct Fmt<12> {  // Q4_K
  static constexpr int UE = 256, UB = 144, TU = 16 * 144;
};
template <>
struct Fmt<13> {  // Q5_K
  static constexpr int UE = 256, UB = 176, TU = 16 * 176;
};
template <>
struct Fmt<14> {  // Q6_K
  static constexpr int UE = 256, UB = 210, TU = 16 * 210;
};
template <>
struct Fmt<8> {  // Q8_0
  static constexpr int UE = 32, UB = 34, TU = 16 * 34;
};
template <>
struct Fmt<2> {  // Q4_0
  static constexpr int UE = 32, UB = 18, TU = 16 * 18;
};
template <>
struct Fmt<6> {  // Q5_0
  static constexpr int UE = 32, UB = 22, TU = 16 * 22;
};
template <>
struct Fmt<20> {  // IQ4_NL
  static constexpr int UE = 32, UB = 18, TU = 16 * 18;
};
template <>
struct Fmt<10> {  // Q2_K
  static constexpr int UE = 256, UB = 84, TU = 16 * 84;
};
template <>
struct Fmt<11> {  // Q3_K
  static constexpr int UE = 256, UB = 110, TU = 16 * 110;
};
template <>
struct Fmt<23> {  // IQ4_XS
  static constexpr int UE = 256, UB = 136, TU = 16 * 136;
};
// the grid-codebook IQ types (layout in iq.hpp)
template <>
struct Fmt<16> {  // IQ2_XXS
  static constexpr int UE = 256, UB = 66, TU = 16 * 66;
};
template <>
struct Fmt<17> {  // IQ2_XS
  static constexpr int UE = 256, UB = 74, TU = 16 * 74;
};
template <>
struct Fmt<18> {  // IQ3_XXS
  static constexpr int UE = 256, UB = 98, TU = 16 * 98;
};
template <>
struct Fmt<21> {  // IQ3_S
  static constexpr int UE = 256, UB = 110, TU = 16 * 110;
};
template <>
struct Fmt<22> {  // IQ2_S
  static constexpr int UE = 256, UB = 82, TU = 16 * 82;
};
template <>
struct Fmt<29> {  // IQ1_M
  static constexpr int UE = 256, UB = 56, TU = 16 * 56;
};

// Q3_K: the 16 6-bit scales (stored + 32) from the 12 scale bytes (words a0,
// a1, a2), one per byte of S[0..3]: low nibbles from a0 / a1 (scales 0-7) and
// their high nibbles (8-15), bits 4-5 from the 2-bit fields of a2
// (gguf-dequant.ts:227-231).
__host__ __device__ __forceinline__ void q3k_scales(uint32_t a0, uint32_t a1, uint32_t a2,
                                                    uint32_t (&S)[4]) {
  S[0] = (a0 & 0x0F0F0F0Fu) | ((a2 & 0x03030303u) << 4);
  S[1] = (a1 & 0x0F0F0F0Fu) | (((a2 >> 2) & 0x03030303u) << 4);
  S[2] = ((a0 >> 4) & 0x0F0F0F0Fu) | (((a2 >> 4) & 0x03030303u) << 4);
  S[3] = ((a1 >> 4) & 0x0F0F0F0Fu) | (((a2 >> 6) & 0x03030303u) << 4);
}

// IQ4_XS: the 6-bit scale of sub-block j, from nibble j of scales_l (bits
// 4j..4j+3 of the little-endian word sl) and bits 2j, 2j + 1 of scales_h
// (gguf-dequant.ts:354-356); the sub-block's values are d * (ls - 32) * kvalues[q].
__host__ __device__ __forceinline__ uint32_t iq4xs_ls(uint32_t sh, uint32_t sl, int j) {
  return ((sl >> (4 * j)) & 0xFu) | (((sh >> (2 * j)) & 3u) << 4);
}

// 32-element block types whose codes are nibbles (b32_codes below).
__host__ __device__ constexpr bool is_b32(int type) { return type == 2 || type == 6 || type == 20; }

__host__ __device__ inline int unit_elems(int type) {
  return (type == 8 || is_b32(type)) ? 32 : 256;
}
__host__ __device__ inline int unit_bytes(int type) {
  return type == 8    ? 34
         : type == 2  ? 18
         : type == 6  ? 22
         : type == 20 ? 18
         : type == 23 ? 136
         : type == 10 ? 84
         : type == 11 ? 110
         : type == 16 ? 66
         : type == 17 ? 74
         : type == 18 ? 98
         : type == 21 ? 110
         : type == 22 ? 82
         : type == 29 ? 56
         : (type == 12 ? 144 : (type == 13 ? 176 : 210));
}

// Byte offset of the code words in a 32-element-block tile-unit.
template <int TYPE>
constexpr int b32_code_off() {
  return TYPE == 6 ? 96 : 32;
}
// The unsigned code a block stores for value d * (code - offset): Q4_0
// d * (q - 8), Q5_0 d * (q5 - 16), IQ4_NL d * kvalues[q] coded as
// kvalues[q] + 128 (a table lookup in b32_codes), Q8_0 d * q coded as q + 128.
template <int TYPE>
constexpr float code_offset() {
  return TYPE == 2 ? 8.f : (TYPE == 6 ? 16.f : 128.f);
}

// IQ4_NL's 16-entry codebook (kvalues_iq4nl, gguf-dequant.ts:29) plus 128,
// four entries per little-endian word: entries 0-3, 4-7, 8-11, 12-15.
constexpr uint32_t kIq4Tab0 = 0x3F2D1801u;  //   1,  24,  45,  63
constexpr uint32_t kIq4Tab1 = 0x766A5D4Fu;  //  79,  93, 106, 118
constexpr uint32_t kIq4Tab2 = 0xA6998D81u;  // 129, 141, 153, 166
constexpr uint32_t kIq4Tab3 = 0xF1D9C5B5u;  // 181, 197, 217, 241

// Four 4-bit indices (one per byte of s) -> their codebook codes (one per byte).
// A third byte permute picks each byte from the upper half's lookup (selector
// 4 + j) where the index is >= 8, else from the lower half's (selector j).
__device__ __forceinline__ uint32_t iq4nl_lookup(uint32_t s) {
  const uint32_t lo3 = s & 0x07070707u;
  const uint32_t ra = __builtin_amdgcn_perm(kIq4Tab1, kIq4Tab0, lo3);  // entries 0-7
  const uint32_t rb = __builtin_amdgcn_perm(kIq4Tab3, kIq4Tab2, lo3);  // entries 8-15
  const uint32_t sel = ((s >> 1) & 0x04040404u) | 0x03020100u;        // bit 3 -> +4
  return __builtin_amdgcn_perm(rb, ra, sel);
}

// The eight codes of a lane in a 32-element-block unit, from its code word q
// (and, for Q5_0, its qh byte: bit i = fifth bit of the lane's element i), as
// four words of 16-bit halves: w[0] = (e0, e2), w[1] = (e1, e3),
// w[2] = (e4, e6), w[3] = (e5, e7) for the lane's elements e0..e7.
template <int TYPE>
__device__ __forceinline__ void b32_codes(uint32_t q, uint32_t qhb, uint32_t (&w)[4]) {
  if constexpr (TYPE == 20) {
    const uint32_t lo = iq4nl_lookup(q & 0x0F0F0F0Fu), hi = iq4nl_lookup((q >> 4) & 0x0F0F0F0Fu);
    w[0] = lo & 0x00FF00FFu;
    w[1] = (lo >> 8) & 0x00FF00FFu;
    w[2] = hi & 0x00FF00FFu;
    w[3] = (hi >> 8) & 0x00FF00FFu;
  } else {
    w[0] = q & 0x000F000Fu;
    w[1] = (q >> 8) & 0x000F000Fu;
    w[2] = (q >> 4) & 0x000F000Fu;
    w[3] = (q >> 12) & 0x000F000Fu;
    if constexpr (TYPE == 6) {
      // bit i of qhb to bit 4 of the half holding element i: e0 / e2 sit at
      // bits 4 / 20 of t, and the other words read t shifted by 1, 4 and 5
      const uint32_t t = qhb * 0x00040010u;
      w[0] |= t & 0x00100010u;
      w[1] |= (t >> 1) & 0x00100010u;
      w[2] |= (t >> 4) & 0x00100010u;
      w[3] |= (t >> 5) & 0x00100010u;
    }
  }
}

// IEEE half bits -> f32 with the hardware converter (subnormals, Inf and NaN
// preserved), the same mapping as f16ToF32 in gguf-dequant.ts:64-71.
__device__ __forceinline__ float h2f(uint32_t bits16) {
  return (float)__builtin_bit_cast(half_t, (uint16_t)(bits16 & 0xFFFFu));
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

// The fifth bits of a Q5_K code word.  w holds four code bytes (k = b0..b0+3
// of a lane's 8), h the qh bytes of the same k; sub-block j's fifth bit is
// bit j of the qh byte.  Returns the words of 16-bit halves that add
// 16 * bit to the codes the decoders extract with the masks 0x000F000F
// (even bytes) and (w >> 8) & 0x000F000F (odd bytes) for the low-nibble
// sub-block j = 2c, and 256 * bit (16 x the high nibble's 16) for the
// high-nibble sub-block j = 2c + 1 (masks 0x00F000F0).
__device__ __forceinline__ uint32_t q5k_lo_even(uint32_t h, int c) {
  return ((h >> (2 * c)) & 0x00010001u) << 4;
}
__device__ __forceinline__ uint32_t q5k_lo_odd(uint32_t h, int c) {
  return ((h >> (8 + 2 * c)) & 0x00010001u) << 4;
}
__device__ __forceinline__ uint32_t q5k_hi_even(uint32_t h, int c) {
  return ((h >> (2 * c + 1)) & 0x00010001u) << 8;
}
__device__ __forceinline__ uint32_t q5k_hi_odd(uint32_t h, int c) {
  return ((h >> (9 + 2 * c)) & 0x00010001u) << 8;
}

// All eight 6-bit scales and mins of a Q4_K superblock, one per byte:
// sc_lo = scales 0-3, sc_hi = scales 4-7, m_lo / m_hi likewise.
__device__ __forceinline__ void q4k_scales_packed(uint32_t s0, uint32_t s1, uint32_t s2,
                                                  uint32_t &sc_lo, uint32_t &sc_hi,
                                                  uint32_t &m_lo, uint32_t &m_hi) {
  sc_lo = s0 & 0x3F3F3F3Fu;
  m_lo = s1 & 0x3F3F3F3Fu;
  sc_hi = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
  m_hi = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
}

__device__ __forceinline__ float ubyte(uint32_t w, int i) {
  return (float)((w >> (8 * i)) & 0xFFu);
}

// Range of f32 activations on the f16 matrix-core paths.  A block of
// activations whose largest magnitude is mx is multiplied by 2^e with
// e = stage_exp(mx), which puts mx in [2^14, 2^15): no f16 overflow (65504),
// and the hi / lo split keeps 22 significant bits of the block's large
// values whatever the f32 range of the input.  Products with 2^e are exact;
// the inverse 2^-e is applied to the block's dot products in f32.  e is
// clamped to [-126, 126] so that both 2^e and 2^-e are normal floats (a zero
// or subnormal block gets 2^126; an Inf / NaN block stays non-finite).
__device__ __forceinline__ int stage_exp(float mx) {
  // biased exponent E of mx: mx in [2^(E-127), 2^(E-126)) for normal mx
  const int E = (int)((__float_as_uint(mx) >> 23) & 0xFFu);
  const int e = 141 - E;  // 15 - (E - 126)
  return e < -126 ? -126 : (e > 126 ? 126 : e);
}
__device__ __forceinline__ float pow2f(int e) {  // 2^e for e in [-126, 127]
  return __uint_as_float((uint32_t)(e + 127) << 23);
}

// Cross-lane reductions on the VALU (DPP and gfx950 permlane swaps) rather than
// through the LDS crossbar (ds_bpermute, tens of cycles each).  Every lane of
// the wave must be active.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;         // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within each 8
constexpr int kDppMirror = 0x140;      // lane i <-> 15 - i within each 16
__device__ __forceinline__ float max_lanes2(float v) { return fmaxf(v, dpp<kDppXor1>(v)); }
// max over each aligned group of 16 lanes, in every lane of the group
__device__ __forceinline__ float max_lanes16(float v) {
  v = fmaxf(v, dpp<kDppXor1>(v));
  v = fmaxf(v, dpp<kDppXor2>(v));
  v = fmaxf(v, dpp<kDppHalfMirror>(v));
  return fmaxf(v, dpp<kDppMirror>(v));
}
// max(v, v of lane ^ 16 / lane ^ 32)
__device__ __forceinline__ float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// v + v of lane ^ 16 / lane ^ 32
__device__ __forceinline__ float sum_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// (a & m) | c.  Plain code on purpose: an inline-asm v_and_or_b32 whose input
// was a buffer-load destination read the register before the load had landed
// in a deeply pipelined kernel (results varied run to run); the compiler's
// wait-count insertion is only trusted for instructions it selects itself.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) {
  return (a & m) | c;
}

__device__ __forceinline__ uint4 ldg16(const void *p) { return *(const uint4 *)p; }

// Streaming (read-once) 16-byte load of weight data: nontemporal, so the
// weight stream does not evict the activations from the caches.
__device__ __forceinline__ uint4 ldg16_stream(const void *p) {
  const uint4 *q = (const uint4 *)p;
  uint4 r;
  r.x = __builtin_nontemporal_load(&q->x);
  r.y = __builtin_nontemporal_load(&q->y);
  r.z = __builtin_nontemporal_load(&q->z);
  r.w = __builtin_nontemporal_load(&q->w);
  return r;
}

__device__ __forceinline__ uint2 ldg8_stream(const void *p) {
  const uint2 *q = (const uint2 *)p;
  uint2 r;
  r.x = __builtin_nontemporal_load(&q->x);
  r.y = __builtin_nontemporal_load(&q->y);
  return r;
}

}  // namespace gguf

// ---------------------------------------------------------------------------
// Internal launchers (host side).  Arguments are already validated by the API
// layer; each returns a hipError_t from the launch.
// ---------------------------------------------------------------------------
namespace gguf {

// Decode attention splits the causal range 0..p into workgroups of
// kAttnSplit cache slots.  Each writes one partial-softmax record per query
// head: o[hd] (the unnormalized sum_t e_t v_t), then m (the largest score) and
// l (sum_t e_t, e_t = exp(score_t - m)), at a stride of hd + 4 floats, so
// every record starts 16-byte aligned.  The record of KV head g, split s and
// query head j of the group sits at ((g * S + s) * grp + j) * (hd + 4),
// S = ceil(max_seq / kAttnSplit).  Records are merged in split order:
//   M = max_s m_s,  w_s = exp(m_s - M),  L = sum_s w_s l_s,
//   out = (sum_s w_s o_s) * (1 / L).
constexpr int kAttnSplit = 64;
constexpr int attn_record_stride(int hd) { return hd + 4; }
struct AttnRecords {
  const float *work;     // the records
  const int64_t *pos;    // device position p; the range holds slots 0..p
  int nh, nkv, hd;       // query heads, KV heads, head dim
  int max_seq;
};

hipError_t launch_repack(const uint8_t *raw, int type, int64_t n_rows, int64_t k, uint8_t *tiles,
                         hipStream_t s);
hipError_t launch_dequant(const uint8_t *tiles, int type, int64_t n_rows, int64_t k, float *out,
                          int64_t ldo, hipStream_t s);
hipError_t launch_dequant_raw(const uint8_t *raw, int type, int64_t n_elems, float *out,
                              hipStream_t s);
hipError_t launch_get_rows(const uint8_t *raw, int type, int64_t n_rows, int64_t k,
                           const int64_t *ids, int64_t n_ids, float *out, int64_t ldo,
                           hipStream_t s);
// A matmul workspace starts with kWsPrefix bytes of counters (zero before the
// workspace's first use; every call leaves them zero); the kernels' data
// follows.  Only the batched decode's range reduction uses the counters, so
// a workspace can be shared by calls of any shape and path.
constexpr int64_t kWsPrefix = 65536;
hipError_t launch_decode(const void *x, int x_type, int64_t ldx, const uint8_t *tiles, int type,
                         int64_t n, int64_t k, float *y, int64_t ldy, int64_t m, float *work,
                         int64_t work_floats, hipStream_t s);
// Workspace floats launch_decode uses for these shapes (0: it needs none).
int64_t launch_decode_work(int type, int x_type, int64_t n, int64_t k, int64_t m);
// The GEMM (gemm.hip); with a workspace of launch_gemm_work floats, small grids
// split K over the chip and add the partial sums in a second launch, and f32
// activations on large grids are staged once as an fp16 image for the wide tile.
hipError_t launch_gemm(const void *x, int x_type, int64_t ldx, const uint8_t *tiles, int type,
                       int64_t n, int64_t k, float *y, int64_t ldy, int64_t m, float *work,
                       int64_t work_floats, hipStream_t s);
int64_t launch_gemm_work(int type, int x_type, int64_t n, int64_t k, int64_t m);
hipError_t launch_decode_fused(const float *x, const uint8_t *tiles, int type, int64_t n,
                               int64_t k, float *y, int prologue, const float *pw, float eps,
                               int epilogue, hipStream_t s);
hipError_t launch_decode_attn_merge(const AttnRecords &ar, const uint8_t *tiles, int type,
                                   int64_t n, float *y, int epilogue, hipStream_t s);
hipError_t launch_rmsnorm(float *x, const float *r, const float *w, float eps, float *y,
                          int64_t rows, int64_t n, hipStream_t s);
hipError_t launch_swiglu(const float *gu, float *out, int64_t rows, int64_t ffn, hipStream_t s);
int64_t attention_work_bytes(int nh, int nkv, int hd, int64_t max_seq);
hipError_t launch_attention_decode(const float *qkv, const int64_t *pos, const float *cs,
                                   const float *sn, float *kc, float *vc, float *out, float *work,
                                   int nh, int nkv, int hd, int64_t max_seq, hipStream_t s);
hipError_t launch_attention_prefill(const float *qkv, int64_t ldq, const int64_t *pos, int64_t m,
                                    const float *cs, const float *sn, float *kc, float *vc,
                                    float *out, int64_t ldo, int nh, int nkv, int hd,
                                    int64_t max_seq, hipStream_t s);
// The attention of gguf_hip_attention_decode_noalloc keeps its workspace
// (records and counters) in a device array of this many bytes.
constexpr int64_t kNoAllocAttentionBytes = (int64_t)8 << 20;
hipError_t launch_attention_decode_noalloc(const float *qkv, const int64_t *pos, const float *cs,
                                           const float *sn, float *kc, float *vc, float *out,
                                           int nh, int nkv, int hd, int64_t max_seq,
                                           hipStream_t s);
int64_t argmax_work_bytes();
hipError_t launch_argmax(const float *x, int64_t n, int64_t *out, void *work, hipStream_t s);

}  // namespace gguf
