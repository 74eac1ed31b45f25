// MFMA decode kernel: y[m, n] = sum_k x[m, k] * dequant(W)[n, k] for up to
// 32 activation rows, one pass over the weights, f32 result.
//
// Replaces the reference's decode GEMVs matmul_gguf_q8_0 /
// matmul_gguf_q4_k_tiled_v4 / matmul_gguf_q6_k_tiled
// (webgpu/src/shaders/matmul_gguf.wgsl:2102-2133, :3191-3245, :2406-2464),
// and its batched decode, which re-reads the weights once per activation row
// (grid.y = M, webgpu/src/engine/forward-pass.ts:1536-1539).
//
// Arithmetic.  The reference computes sum_k a_k * (d1 * q_k - min1) per unit
// in f32.  Here the quantized codes are fed to the matrix cores *exactly*, as
// normal f16 integers (f16_codes): the signed code q - offset for the types
// whose values are d * (q - offset) (Q8_0 q, Q4_0 q - 8, Q5_0 q - 16, IQ4_NL /
// IQ4_XS the codebook value, Q6_K q - 32, Q3_K 128 (q - 4)), the unsigned code
// for the types with mins (Q4_K / Q5_K q and, for the high-nibble sub-blocks,
// 16 q; Q2_K 256 q).
// Each unit of each activation row (256 or 32 elements) is scaled by a power
// of two 2^e that puts its largest magnitude in [2^14, 2^15) (stage_exp), then
// split into f16 hi + lo parts (x 2^e = hi + lo to 22 significant bits), so
// any f32 activation is in range.  One v_mfma_f32_16x16x32_f16 (Q6_K:
// 16x16x16, one 16-element scale group) then yields the exact-product,
// f32-accumulated dot of one scale group of 16 weight rows with up to 16
// activation rows, and the unit's 2^-e, the group's scale and min are applied
// in f32 afterwards:
//     acc += 2^-e ((d * sc) * D  -  (dmin * m) * sum(hi + lo of group))
// (the min term only for Q4_K / Q5_K / Q2_K).  Nothing is rounded to f16 on
// the weight side, unlike an fp16 dequant-GEMM.
//
// Work split.  A workgroup is four waves; each wave owns one 16-row tile of
// the weight (lane (r, g) = (lane & 15, lane >> 4) holds row r's operand
// bytes, loaded from the row-tile layout as 1 KB-contiguous wave loads) and
// every KS-th unit of K.  TS = 4 / KS tiles share a workgroup.  Activations
// are staged per chunk of units into LDS (hi, lo, per-group sums), shared by
// all waves.  Unit loads are double-buffered across chunks so the next
// chunk's weight bytes are in flight while the current one is computed.  The
// KS partial sums of a row are added in a fixed order (deterministic).
#pragma once

#include "common.hpp"
#include "decode_types.hpp"
#include "iq.hpp"
#include "iq_ops.hpp"

namespace gguf {

namespace {

constexpr int kXPad = 8;               // halves of padding per staged activation row

template <int TYPE>
struct Unit;
template <>
struct Unit<12> {  // header, qs pieces cp = 0, 1
  uint4 h, a, b;
};
template <>
struct Unit<13> {  // as Q4_K, plus the lane's qh bytes 8g..8g+7
  uint4 h, a, b;
  uint2 qh;
};
template <>
struct Unit<14> {  // quant pieces v = 0..2, scales, d
  uint4 p0, p1, p2, sc;
  uint32_t d;
};
template <>
struct Unit<8> {  // qs bytes 8g..8g+7, d
  uint2 q;
  uint32_t d;
};
// Q4_0 / Q5_0 / IQ4_NL: the lane's code word, d, and (Q5_0) the row's qh
template <>
struct Unit<2> {
  uint32_t q, d;
};
template <>
struct Unit<6> {
  uint32_t q, d, qh;
};
template <>
struct Unit<20> {
  uint32_t q, d;
};
template <>
struct Unit<10> {  // Q2_K: the lane's qs pieces, the row's 16 scale bytes, d | dmin << 16
  uint4 q, sc;
  uint32_t dm;
};
template <>
struct Unit<11> {  // Q3_K: the lane's qs and hmask pieces, the row's scale words and d
  uint4 q;
  uint2 hm;
  uint32_t s0, s1, s2, d;
};
template <>
struct Unit<23> {  // IQ4_XS: the row's header; the lane's code words of sub-blocks 0-3, 4-7
  uint2 h;
  uint4 a, b;
};

// Scale group size (elements sharing one scale), units in flight per wave
// (P; deepest for a single activation row, whose staged chunk is small),
// whether the kernels need the group sums of the activations (mins dmin * m,
// or a code offset taken off through the sums), and whether the codes enter
// in natural k order (the FP8-converted codes of at most 4 bits) rather than
// the (0, 2, 1, 3) quad order of the masked 16-bit halves.
#ifndef GGUF_DECODE_P_Q4K
#define GGUF_DECODE_P_Q4K 4
#endif
#ifndef GGUF_DECODE_P_Q6K
#define GGUF_DECODE_P_Q6K 2
#endif
#ifndef GGUF_DECODE_P_Q8
#define GGUF_DECODE_P_Q8 8
#endif
template <int TYPE>
struct Dec;
template <>
struct Dec<12> {
  static constexpr int GS = 32, P1 = GGUF_DECODE_P_Q4K;
  static constexpr bool SUMS = true, NAT = true;
};
template <>
struct Dec<13> {
  static constexpr int GS = 32, P1 = GGUF_DECODE_P_Q4K;
  static constexpr bool SUMS = true, NAT = false;
};
template <>
struct Dec<14> {
  static constexpr int GS = 16, P1 = GGUF_DECODE_P_Q6K;
  static constexpr bool SUMS = false, NAT = false;
};
template <>
struct Dec<8> {
  static constexpr int GS = 32, P1 = GGUF_DECODE_P_Q8;
  static constexpr bool SUMS = false, NAT = false;
};
template <>
struct Dec<2> {
  static constexpr int GS = 32, P1 = GGUF_DECODE_P_Q8;
  static constexpr bool SUMS = true, NAT = true;
};
template <>
struct Dec<6> {
  static constexpr int GS = 32, P1 = GGUF_DECODE_P_Q8;
  static constexpr bool SUMS = false, NAT = false;
};
template <>
struct Dec<20> {
  static constexpr int GS = 32, P1 = GGUF_DECODE_P_Q8;
  static constexpr bool SUMS = false, NAT = false;
};
template <>
struct Dec<10> {
  static constexpr int GS = 16, P1 = GGUF_DECODE_P_Q4K;
  static constexpr bool SUMS = true, NAT = true;
};
template <>
struct Dec<11> {
  static constexpr int GS = 16, P1 = GGUF_DECODE_P_Q4K;
  static constexpr bool SUMS = true, NAT = true;
};
template <>
struct Dec<23> {
  static constexpr int GS = 32, P1 = GGUF_DECODE_P_Q4K;
  static constexpr bool SUMS = false, NAT = false;
};
template <int TYPE, int MT, int MR>
constexpr int decode_p() {
  return MR == 1 ? Dec<TYPE>::P1
                 : (MT == 1 ? (Dec<TYPE>::P1 + 1) / 2 : ((TYPE == 8 || is_b32(TYPE)) ? 4 : 1));
}

// Weight loads go through a buffer resource spanning the wave's row tile
// (base = tile start, num_records = its byte count): the per-unit offset is a
// scalar (soffset), the lane's offset a loop-invariant VGPR, and a load of a
// tile that does not exist (num_records = 0) returns zeros instead of
// touching memory.  Loads are nontemporal (aux bit 1).
constexpr int kNT = 2;
constexpr int kRsrcWord3 = 0x00020000;

__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t rs, int voff, int soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, kNT);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint2 bload8(__amdgpu_buffer_rsrc_t rs, int voff, int soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, voff, soff, kNT);
  return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint32_t bload2(__amdgpu_buffer_rsrc_t rs, int voff, int soff) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, voff, soff, kNT);
}

// soff = unit * tile_unit_bytes; r = lane & 15, g = lane >> 4.
__device__ __forceinline__ void load_unit(__amdgpu_buffer_rsrc_t rs, int soff, int r, int g,
                                          Unit<12> &u) {
  const int qa = 256 + (16 * g + r) * 16;
  u.h = bload16(rs, 16 * r, soff);
  u.a = bload16(rs, qa, soff);
  u.b = bload16(rs, qa + 1024, soff);
}
__device__ __forceinline__ void load_unit(__amdgpu_buffer_rsrc_t rs, int soff, int r, int g,
                                          Unit<13> &u) {
  const int qa = 256 + (16 * g + r) * 16;
  u.h = bload16(rs, 16 * r, soff);
  u.a = bload16(rs, qa, soff);
  u.b = bload16(rs, qa + 1024, soff);
  u.qh = bload8(rs, 2304 + (16 * g + r) * 8, soff);
}
__device__ __forceinline__ void load_unit(__amdgpu_buffer_rsrc_t rs, int soff, int r, int g,
                                          Unit<14> &u) {
  const int p0 = (16 * g + r) * 16;
  u.p0 = bload16(rs, p0, soff);
  u.p1 = bload16(rs, p0 + 1024, soff);
  u.p2 = bload16(rs, p0 + 2048, soff);
  u.sc = bload16(rs, 3072 + 16 * r, soff);
  u.d = bload2(rs, 3328 + 2 * r, soff);
}
__device__ __forceinline__ void load_unit(__amdgpu_buffer_rsrc_t rs, int soff, int r, int g,
                                          Unit<8> &u) {
  u.q = bload8(rs, 32 + (16 * g + r) * 8, soff);
  u.d = bload2(rs, 2 * r, soff);
}
__device__ __forceinline__ uint32_t bload4(__amdgpu_buffer_rsrc_t rs, int voff, int soff) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs, voff, soff, kNT);
}
__device__ __forceinline__ void load_unit(__amdgpu_buffer_rsrc_t rs, int soff, int r, int g,
                                          Unit<2> &u) {
  u.q = bload4(rs, 32 + (16 * g + r) * 4, soff);
  u.d = bload2(rs, 2 * r, soff);
}
__device__ __forceinline__ void load_unit(__amdgpu_buffer_rsrc_t rs, int soff, int r, int g,
                                          Unit<6> &u) {
  u.q = bload4(rs, 96 + (16 * g + r) * 4, soff);
  u.d = bload2(rs, 2 * r, soff);
  u.qh = bload4(rs, 32 + 4 * r, soff);
}
__device__ __forceinline__ void load_unit(__amdgpu_buffer_rsrc_t rs, int soff, int r, int g,
                                          Unit<20> &u) {
  u.q = bload4(rs, 32 + (16 * g + r) * 4, soff);
  u.d = bload2(rs, 2 * r, soff);
}
__device__ __forceinline__ void load_unit(__amdgpu_buffer_rsrc_t rs, int soff, int r, int g,
                                          Unit<10> &u) {
  u.q = bload16(rs, 320 + (16 * g + r) * 16, soff);
  u.sc = bload16(rs, 16 * r, soff);
  u.dm = bload4(rs, 256 + 4 * r, soff);
}
__device__ __forceinline__ void load_unit(__amdgpu_buffer_rsrc_t rs, int soff, int r, int g,
                                          Unit<11> &u) {
  u.q = bload16(rs, 736 + (16 * g + r) * 16, soff);
  u.hm = bload8(rs, 224 + (16 * g + r) * 8, soff);
  u.s0 = bload4(rs, 12 * r, soff);
  u.s1 = bload4(rs, 12 * r + 4, soff);
  u.s2 = bload4(rs, 12 * r + 8, soff);
  u.d = bload2(rs, 192 + 2 * r, soff);
}
__device__ __forceinline__ void load_unit(__amdgpu_buffer_rsrc_t rs, int soff, int r, int g,
                                          Unit<23> &u) {
  const int qa = 128 + (16 * g + r) * 32;
  u.h = bload8(rs, 8 * r, soff);
  u.a = bload16(rs, qa, soff);
  u.b = bload16(rs, qa + 16, soff);
}

__device__ __forceinline__ half8_t as_h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  return __builtin_bit_cast(half8_t, make_uint4(a, b, c, d));
}
__device__ __forceinline__ half4_t as_h4(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(half4_t, make_uint2(a, b));
}

// Quant codes as exact normal f16 integers.  A code c < 1024 OR-ed into the
// mantissa of 1024.0 (0x6400) is 1024 + c; one packed f16 subtraction of
// 1024 + off then leaves c - off exactly.  The codes masked into the low bits
// of an f16 would be exact subnormals c * 2^-24, but the matrix cores keep
// only about 18 significant bits of a dot product whose B operand is a deep
// subnormal (measured on gfx950: 2^-18.6 of sum |a b| with 4-bit codes, and
// 2^-12 when the activations of one dot span 2^16), against 2^-24 (2^-21
// with such a span) for normal operands.
constexpr uint32_t kF16Base = 0x64006400u;  // 1024.0 in both halves
constexpr uint32_t neg_base(uint32_t off) { return (0xE400u + off) * 0x00010001u; }  // -(1024 + off) x 2
// kF16Base in a vector register.  With the mask and the base both literals
// the compiler splits every (w & m) | base into a v_and and a v_or (a VOP3
// v_and_or_b32 takes at most one constant from the scalar side); with the base
// in a register it is one v_and_or_b32.  The asm has no inputs and no side
// effects, so identical copies fold into one per kernel.
__device__ __forceinline__ uint32_t f16_base() {
  uint32_t v;
  asm("v_mov_b32 %0, %1" : "=v"(v) : "i"(kF16Base));
  return v;
}
// the two codes (w & m) (each < 1024, one per half) minus off, as f16
__device__ __forceinline__ uint32_t f16_codes(uint32_t w, uint32_t m, uint32_t nb) {
  const half2_t v = __builtin_bit_cast(half2_t, and_or(w, m, f16_base())) + __builtin_bit_cast(half2_t, nb);
  return __builtin_bit_cast(uint32_t, v);
}
// the same for codes already masked into the low bits of their halves
__device__ __forceinline__ uint32_t f16_codes(uint32_t two, uint32_t nb) {
  const half2_t v = __builtin_bit_cast(half2_t, two | kF16Base) + __builtin_bit_cast(half2_t, nb);
  return __builtin_bit_cast(uint32_t, v);
}

// Four codes of at most 4 bits, one per byte of w, as exact f16 integers in
// byte order (two words of two halves).  A byte c < 16 read as FP8 E4M3 is
// c * 2^-9 (the subnormals and the first binade are evenly spaced), and the
// converter scales it by 2^9: measured exact on gfx950 for every byte value.
__device__ __forceinline__ uint32_t fp8_codes_lo(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 512.0f, false));
}
__device__ __forceinline__ uint32_t fp8_codes_hi(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 512.0f, true));
}
// eight such codes: bytes 0-3 of a, then bytes 0-3 of b
__device__ __forceinline__ half8_t fp8_operand(uint32_t a, uint32_t b) {
  return as_h8(fp8_codes_lo(a), fp8_codes_hi(a), fp8_codes_lo(b), fp8_codes_hi(b));
}

// The eight codes of a lane in a 32-element-block unit (as b32_codes: w[0] =
// (e0, e2), w[1] = (e1, e3), w[2] = (e4, e6), w[3] = (e5, e7)) minus the
// type's code offset, as f16.
template <int TYPE>
__device__ __forceinline__ void b32_f16(uint32_t q, uint32_t qhb, uint32_t (&w)[4]) {
  constexpr uint32_t nb = neg_base((uint32_t)code_offset<TYPE>());
  if constexpr (TYPE == 20) {
    const uint32_t lo = iq4nl_lookup(q & 0x0F0F0F0Fu), hi = iq4nl_lookup((q >> 4) & 0x0F0F0F0Fu);
    w[0] = f16_codes(lo, 0x00FF00FFu, nb);
    w[1] = f16_codes(lo >> 8, 0x00FF00FFu, nb);
    w[2] = f16_codes(hi, 0x00FF00FFu, nb);
    w[3] = f16_codes(hi >> 8, 0x00FF00FFu, nb);
  } else if constexpr (TYPE == 6) {
    uint32_t c[4];
    b32_codes<6>(q, qhb, c);
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = f16_codes(c[i], nb);
  } else {
    w[0] = f16_codes(q, 0x000F000Fu, nb);
    w[1] = f16_codes(q >> 8, 0x000F000Fu, nb);
    w[2] = f16_codes(q >> 4, 0x000F000Fu, nb);
    w[3] = f16_codes(q >> 12, 0x000F000Fu, nb);
  }
}

// The B operand of a 32-element-block unit for lane group g: Q4_0 the codes
// (natural order), Q5_0 / IQ4_NL the signed codes q - offset (halves in the
// staged (0, 2, 1, 3) quad order).
template <int TYPE>
__device__ __forceinline__ half8_t b32_operand(const Unit<TYPE> &u, int g) {
  if constexpr (TYPE == 2)  // codes 0..15 in natural order; the offset 8 goes through the sums
    return fp8_operand(u.q & 0x0F0F0F0Fu, (u.q >> 4) & 0x0F0F0F0Fu);
  uint32_t qhb = 0;
  if constexpr (TYPE == 6) qhb = (u.qh >> (8 * g)) & 0xFFu;
  uint32_t w[4];
  b32_f16<TYPE>(u.q, qhb, w);
  return as_h8(w[0], w[1], w[2], w[3]);
}

// The B operand of one Q8_0 block for lane group g: the signed int8 codes.
__device__ __forceinline__ half8_t q8_operand(const Unit<8> &u) {
  const uint32_t u0 = u.q.x ^ 0x80808080u, u1 = u.q.y ^ 0x80808080u;  // q + 128
  constexpr uint32_t nb = neg_base(128);
  return as_h8(f16_codes(u0, 0x00FF00FFu, nb), f16_codes(u0 >> 8, 0x00FF00FFu, nb),
               f16_codes(u1, 0x00FF00FFu, nb), f16_codes(u1 >> 8, 0x00FF00FFu, nb));
}

// Q6_K: the B operand (q - 32) of the four 6-bit codes held in the bytes of v.
__device__ __forceinline__ half4_t q6_operand(uint32_t v) {
  constexpr uint32_t nb = neg_base(32);
  return as_h4(f16_codes(v, 0x00FF00FFu, nb), f16_codes(v >> 8, 0x00FF00FFu, nb));
}

// Dynamic LDS of the decode kernel.  Stage records offsets into it (not
// pointers), so every access below is an explicit ds_read / ds_write.
extern __shared__ __align__(16) unsigned char g_lds[];

struct Stage {
  int xh, xl;  // half offsets of [M][ce + kXPad] hi and lo parts of the scaled activations,
               // quads in (0, 2, 1, 3) order
  int xs;      // float offset of [ce / GS][MS] per-group sums of hi + lo, rows M..MS-1 zero
  int xf;      // float offset of [ce / UE][MS] per-unit inverse scales 2^-e
  int zero;    // half offset of kZeroHalves zeros: the A operand of lanes that contribute nothing
  int ld;      // ce + kXPad
  int ms;      // 16 * MT
  int tbl;     // byte offset of the IQ decode tables (grid-codebook types)
};

__device__ __forceinline__ half8_t lds_h8b(int byte_off) {
  return *(const half8_t *)(g_lds + byte_off);
}
__device__ __forceinline__ half4_t lds_h4b(int byte_off) {
  return *(const half4_t *)(g_lds + byte_off);
}
__device__ __forceinline__ half8_t lds_h8(int half_off) {
  return *(const half8_t *)((const half_t *)g_lds + half_off);
}
__device__ __forceinline__ half4_t lds_h4(int half_off) {
  return *(const half4_t *)((const half_t *)g_lds + half_off);
}
__device__ __forceinline__ float lds_f(int float_off) { return ((const float *)g_lds)[float_off]; }
__device__ __forceinline__ float4 lds_f4(int float_off) {
  return *(const float4 *)((const float *)g_lds + float_off);
}

// The eight selector-row A fragments of an IQ unit (M = 1): fragment j holds
// the lane's activations (LDS address own + 64 j) where its row belongs to
// sub-block j (jo == j), and zeros elsewhere.  The lane reads its one
// fragment and selects the other seven to zero, where the K-quant units read
// all eight (seven from the zero block): the IQ units' table lookups keep the
// LDS busy (IQ2_XXS M = 1 10.5 -> 10.0 us), while Q4_K, whose VALU sets the
// pace, measured slower with the selects (7.9-8.2 -> 8.5-8.8 us).
__device__ __forceinline__ void iq_frags(uint32_t own, uint32_t zero, bool live, int jo,
                                         half8_t (&a)[8]) {
  const half8_t mine = lds_ld<half8_t>(live ? own + 64 * jo : zero), z = {};
#pragma unroll
  for (int j = 0; j < 8; ++j) a[j] = jo == j ? mine : z;
}

#include "iq_decode.hpp"

// D = (hi + lo parts of A) x B; lanes with on == false read the zero operand.
template <int PARTS>
__device__ __forceinline__ float4_t mfma32(int ah, int al, int zero, half8_t b, bool on) {
  float4_t d = {0.f, 0.f, 0.f, 0.f};
  d = __builtin_amdgcn_mfma_f32_16x16x32_f16(lds_h8(on ? ah : zero), b, d, 0, 0, 0);
  if (PARTS == 2) d = __builtin_amdgcn_mfma_f32_16x16x32_f16(lds_h8(on ? al : zero), b, d, 0, 0, 0);
  return d;
}

template <int PARTS>
__device__ __forceinline__ float4_t mfma16(int ah, int al, int zero, half4_t b, bool on) {
  float4_t d = {0.f, 0.f, 0.f, 0.f};
  d = __builtin_amdgcn_mfma_f32_16x16x16f16(lds_h4(on ? ah : zero), b, d, 0, 0, 0);
  if (PARTS == 2) d = __builtin_amdgcn_mfma_f32_16x16x16f16(lds_h4(on ? al : zero), b, d, 0, 0, 0);
  return d;
}

// acc[i] += f[i] (s D[i] - o xs[i]) for the MR activation rows a lane holds
// (f: the rows' inverse unit scales 2^-e).
// The batched kernels keep two row tiles per wave (two inlined copies of the
// unit arithmetic): every accumulation is an explicit fmaf with contraction
// off, so that a row's rounding never depends on which copy computed it (the
// compiler may otherwise fuse the products of a * b + c * d differently in
// the two copies, and rows would differ in the last bit by tile position).
template <int MR>
__device__ __forceinline__ void apply(float (&acc)[4], const float4_t &D, float s, float o, int xs,
                                      const float (&f)[4]) {
#pragma clang fp contract(off)
  if (MR == 1) {
    acc[0] = fmaf(f[0], fmaf(s, D[0], -(o * lds_f(xs))), acc[0]);
  } else {
    const float4 v = lds_f4(xs);
    acc[0] = fmaf(f[0], fmaf(s, D[0], -(o * v.x)), acc[0]);
    acc[1] = fmaf(f[1], fmaf(s, D[1], -(o * v.y)), acc[1]);
    acc[2] = fmaf(f[2], fmaf(s, D[2], -(o * v.z)), acc[2]);
    acc[3] = fmaf(f[3], fmaf(s, D[3], -(o * v.w)), acc[3]);
  }
}

// acc[i] += f[i] (s D[i]) (types without mins).
template <int MR>
__device__ __forceinline__ void apply_s(float (&acc)[4], const float4_t &D, float s,
                                        const float (&f)[4]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int i = 0; i < MR; ++i) acc[i] = fmaf(f[i], s * D[i], acc[i]);
}

// The inverse unit scales of unit ul for the MR rows of each activation tile a lane holds.
template <int MT, int MR>
__device__ __forceinline__ void unit_scales(const Stage &st, int ul, int g, float (&f)[MT][4]) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int o = st.xf + ul * st.ms + 16 * mt + 4 * g;
    if (MR == 1) {
      f[mt][0] = lds_f(o);
    } else {
      const float4 v = lds_f4(o);
      f[mt][0] = v.x;
      f[mt][1] = v.y;
      f[mt][2] = v.z;
      f[mt][3] = v.w;
    }
  }
}

// Shared-memory view of one staged chunk of activations.
constexpr int kZeroHalves = 256;  // covers every immediate offset added to a selected address
constexpr size_t kMaxLds = 160 * 1024;  // LDS a gfx950 workgroup may use

// ---------------------------------------------------------------------------
// Single activation row (M = 1).  The 16 A rows of the MFMA are then free to
// act as selectors: row 2j + p carries part p (hi / lo) of the activations of
// scale group j and is zero in every MFMA that does not belong to group j, so
// one accumulator chain over a unit's groups leaves group j's dot in rows
// 2j, 2j + 1.  Lane (n, g) ends up holding the groups of "its" quarter and
// applies their scales; a 4-lane sum per row finishes the unit.
// ---------------------------------------------------------------------------

// B operands of chunk c of a Q4_K / Q5_K unit: the lane's 8 codes of
// sub-block 2c (low nibbles) and 2c + 1 (high nibbles) as f16 integers.  Q4_K:
// both as q, natural order (FP8 conversion).  Q5_K (with the fifth bits): q
// and 16 q, halves in (0, 2, 1, 3) order per quad.
template <int TYPE>
__device__ __forceinline__ void k_codes(const Unit<TYPE> &u, int c, half8_t &blo, half8_t &bhi) {
  const uint32_t w[8] = {u.a.x, u.a.y, u.a.z, u.a.w, u.b.x, u.b.y, u.b.z, u.b.w};
  const uint32_t wa = w[2 * c], wb = w[2 * c + 1];
  const uint32_t wa8 = wa >> 8, wb8 = wb >> 8;
  constexpr uint32_t nb = neg_base(0), ML = 0x000F000Fu, MH = 0x00F000F0u;
  if constexpr (TYPE == 12) {  // FP8-converted nibbles, natural order; both sub-blocks as q
    blo = fp8_operand(wa & 0x0F0F0F0Fu, wb & 0x0F0F0F0Fu);
    bhi = fp8_operand((wa >> 4) & 0x0F0F0F0Fu, (wb >> 4) & 0x0F0F0F0Fu);
  } else {
    const uint32_t qa = u.qh.x, qb = u.qh.y;
    blo = as_h8(f16_codes((wa & ML) | q5k_lo_even(qa, c), nb), f16_codes((wa8 & ML) | q5k_lo_odd(qa, c), nb),
                f16_codes((wb & ML) | q5k_lo_even(qb, c), nb), f16_codes((wb8 & ML) | q5k_lo_odd(qb, c), nb));
    bhi = as_h8(f16_codes((wa & MH) | q5k_hi_even(qa, c), nb), f16_codes((wa8 & MH) | q5k_hi_odd(qa, c), nb),
                f16_codes((wb & MH) | q5k_hi_even(qb, c), nb), f16_codes((wb8 & MH) | q5k_hi_odd(qb, c), nb));
  }
}
// Scale of the high-nibble sub-blocks' codes: Q4_K enters them as q, Q5_K as 16 q.
template <int TYPE>
constexpr float k_hi_scale() {
  return TYPE == 13 ? 0.0625f : 1.0f;
}

// Q4_K / Q5_K: 8 sub-blocks, one chain; lane (n, g) keeps sub-blocks 2g (lo
// nibbles of chunk g) and 2g + 1 (hi nibbles).
template <int PARTS, int TYPE>
__device__ __forceinline__ void unit_m1_k(const Unit<TYPE> &u, const Stage &st, int ul, int lane,
                                          float &acc) {
  const int r = lane & 15, g = lane >> 4;
  const int jo = r >> 1;
  const bool live = PARTS == 2 || (r & 1) == 0;
  // byte addresses: the lane's own activation row and the zero operand
  const int own = 2 * (st.xh + (r & 1) * (st.xl - st.xh) + 256 * ul + 8 * g);
  const int zero = 2 * st.zero;
  // all eight A fragments first, so their LDS latency overlaps the decode below
  half8_t a[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) a[j] = lds_h8b(((live && jo == j) ? own : zero) + 64 * j);
  uint32_t sc_lo, sc_hi, m_lo, m_hi;
  q4k_scales_packed(u.h.y, u.h.z, u.h.w, sc_lo, sc_hi, m_lo, m_hi);
  const uint32_t scw = g < 2 ? sc_lo : sc_hi, mw = g < 2 ? m_lo : m_hi;
  const int sh = 16 * (g & 1);
  const float sc0 = (float)((scw >> sh) & 0xFFu), sc1 = (float)((scw >> (sh + 8)) & 0xFFu);
  const float m0 = (float)((mw >> sh) & 0xFFu), m1 = (float)((mw >> (sh + 8)) & 0xFFu);
  const int xs = st.xs + (ul * 8 + 2 * g) * st.ms;
  const float mx = m0 * lds_f(xs) + m1 * lds_f(xs + st.ms);
  const float d = h2f(u.h.x), dmin = h2f(u.h.x >> 16), fu = lds_f(st.xf + ul * st.ms);
  float4_t D = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < 4; ++c) {  // codes of chunk c decoded just before its two MFMAs
    half8_t blo, bhi;
    k_codes(u, c, blo, bhi);
    D = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[2 * c], blo, D, 0, 0, 0);
    D = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[2 * c + 1], bhi, D, 0, 0, 0);
  }
  // rows 4g + i: sub-block 2g (i = 0, 1) and 2g + 1 (i = 2, 3), part i & 1
  acc += fu * (d * (sc0 * (D[0] + D[1])) + (d * k_hi_scale<TYPE>()) * (sc1 * (D[2] + D[3])) -
               dmin * mx);
}
template <int PARTS>
__device__ __forceinline__ void unit_m1(const Unit<12> &u, const Stage &st, int ul, int lane,
                                        float &acc) {
  unit_m1_k<PARTS, 12>(u, st, ul, lane, acc);
}
template <int PARTS>
__device__ __forceinline__ void unit_m1(const Unit<13> &u, const Stage &st, int ul, int lane,
                                        float &acc) {
  unit_m1_k<PARTS, 13>(u, st, ul, lane, acc);
}

// IQ grid types: the B operand of sub-block j is the lane's grid entries with
// signs and odd factor (exact f16 integers, iq_b); one chain over the 8
// sub-blocks leaves sub-block j in rows 2j, 2j + 1, and every row takes the
// same unit scale.  Types with one factor per sub-block leave it out of the
// operand and apply it to the two rows of the sub-block (four packed
// multiplies per sub-block fewer).
template <int PARTS, int TYPE>
__device__ __forceinline__ void unit_m1_iq(const Unit<TYPE> &u, const Stage &st, int ul, int lane,
                                           float &acc) {
  const int r = lane & 15, g = lane >> 4;
  const int jo = r >> 1;
  const bool live = PARTS == 2 || (r & 1) == 0;
  const uint32_t own = lds_addr32(g_lds) + 2 * (st.xh + (r & 1) * (st.xl - st.xh) + 256 * ul + 8 * g);
  const uint32_t zero = lds_addr32(g_lds) + 2 * st.zero;
  half8_t a[8];
  iq_frags(own, zero, live, jo, a);
  constexpr bool BF = iq_block_factor<TYPE>();
  float4_t D = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 8; ++j)
    D = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[j], iq_b<TYPE, !BF>(u, j, g, g_lds + st.tbl), D, 0, 0, 0);
  const float fu = lds_f(st.xf + ul * st.ms);
  // rows 4g + i: sub-block 2g (i = 0, 1) and 2g + 1 (i = 2, 3)
  float f0 = 1.f, f1 = 1.f;
  if constexpr (BF) iq_factors<TYPE>(u, g, f0, f1);
  const float s = f0 * (D[0] + D[1]) + f1 * (D[2] + D[3]);
  acc += fu * (iq_unit_scale<TYPE>(u) * s);
}
#define GGUF_IQ_M1(T)                                                                        \
  template <int PARTS>                                                                       \
  __device__ __forceinline__ void unit_m1(const Unit<T> &u, const Stage &st, int ul, int lane, \
                                          float &acc) {                                      \
    unit_m1_iq<PARTS, T>(u, st, ul, lane, acc);                                              \
  }
GGUF_IQ_M1(16)
GGUF_IQ_M1(17)
GGUF_IQ_M1(18)
GGUF_IQ_M1(21)
GGUF_IQ_M1(22)
GGUF_IQ_M1(29)
#undef GGUF_IQ_M1

// Q6_K: 16 groups of 16 elements, two chains of 8 (halves hf = 0, 1); lane
// (n, g) keeps groups 8 hf + 2 g + lh, lh = 0, 1.
template <int PARTS>
__device__ __forceinline__ void unit_m1(const Unit<14> &u, const Stage &st, int ul, int lane,
                                        float &acc) {
  const int r = lane & 15, g = lane >> 4;
  const int so = r >> 1;
  const bool live = PARTS == 2 || (r & 1) == 0;
  const int own = 2 * (st.xh + (r & 1) * (st.xl - st.xh) + 256 * ul + 4 * g);
  const int zero = 2 * st.zero;
  const uint32_t dw[12] = {u.p0.x, u.p0.y, u.p0.z, u.p0.w, u.p1.x, u.p1.y,
                           u.p1.z, u.p1.w, u.p2.x, u.p2.y, u.p2.z, u.p2.w};
  const uint32_t scw[4] = {u.sc.x, u.sc.y, u.sc.z, u.sc.w};
  const float d = h2f(u.d);
  float sd = 0.f;
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    // the chain's eight A fragments first (LDS latency overlaps the decode)
    half4_t a[8];
#pragma unroll
    for (int sl = 0; sl < 8; ++sl) {
      const int t = sl >> 1, lh = sl & 1;
      a[sl] = lds_h4b(((live && so == sl) ? own : zero) + 2 * (128 * hf + 32 * t + 16 * lh));
    }
    half4_t b[8];
#pragma unroll
    for (int lh = 0; lh < 2; ++lh) {
      const int i = 2 * hf + lh;
      const uint32_t qa = dw[3 * i], qb = dw[3 * i + 1], qh = dw[3 * i + 2];
      const uint32_t v[4] = {(qa & 0x0F0F0F0Fu) | ((qh << 4) & 0x30303030u),
                             (qb & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u),
                             ((qa >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u),
                             ((qb >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u)};
#pragma unroll
      for (int t = 0; t < 4; ++t) b[2 * t + lh] = q6_operand(v[t]);
    }
    // rows 4g + i: group 8 hf + 2 g + (i >> 1), part i & 1
    const uint32_t sw = scw[2 * hf + (g >> 1)];
    const int sh = 16 * (g & 1);
    const float s0 = (float)(int8_t)((sw >> sh) & 0xFFu), s1 = (float)(int8_t)((sw >> (sh + 8)) & 0xFFu);
    float4_t D = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sl = 0; sl < 8; ++sl) D = __builtin_amdgcn_mfma_f32_16x16x16f16(a[sl], b[sl], D, 0, 0, 0);
    sd += s0 * (D[0] + D[1]) + s1 * (D[2] + D[3]);
  }
  acc += lds_f(st.xf + ul * st.ms) * (d * sd);
}

// Q8_0: one block; rows 0 (hi) and 1 (lo) carry the activations, lanes g = 0
// hold the result.
template <int PARTS>
__device__ __forceinline__ void unit_m1(const Unit<8> &u, const Stage &st, int ul, int lane,
                                        float &acc) {
  const int r = lane & 15, g = lane >> 4;
  const bool live = r == 0 || (PARTS == 2 && r == 1);
  const int pa = live ? st.xh + r * (st.xl - st.xh) + 32 * ul + 8 * g : st.zero;
  float4_t D = {0.f, 0.f, 0.f, 0.f};
  D = __builtin_amdgcn_mfma_f32_16x16x32_f16(lds_h8(pa), q8_operand(u), D, 0, 0, 0);
  // D is zero outside rows 0 and 1 (lanes g = 0), so every lane adds its own value
  acc += lds_f(st.xf + ul * st.ms) * (h2f(u.d) * (D[0] + D[1]));
}

// Q4_0 / Q5_0 / IQ4_NL: as Q8_0, with the codes from the lane's word.
template <int PARTS, int TYPE>
__device__ __forceinline__ void unit_m1_b32(const Unit<TYPE> &u, const Stage &st, int ul, int lane,
                                            float &acc) {
  const int r = lane & 15, g = lane >> 4;
  const bool live = r == 0 || (PARTS == 2 && r == 1);
  const int pa = live ? st.xh + r * (st.xl - st.xh) + 32 * ul + 8 * g : st.zero;
  const half8_t b = b32_operand<TYPE>(u, g);
  float4_t D = {0.f, 0.f, 0.f, 0.f};
  D = __builtin_amdgcn_mfma_f32_16x16x32_f16(lds_h8(pa), b, D, 0, 0, 0);
  const float d = h2f(u.d);
  float v = d * (D[0] + D[1]);  // zero outside rows 0 and 1 (lanes g = 0)
  if constexpr (TYPE == 2) v -= (g == 0 ? 8.f * d : 0.f) * lds_f(st.xs + ul * st.ms);
  acc += lds_f(st.xf + ul * st.ms) * v;
}
template <int PARTS>
__device__ __forceinline__ void unit_m1(const Unit<2> &u, const Stage &st, int ul, int lane,
                                        float &acc) {
  unit_m1_b32<PARTS, 2>(u, st, ul, lane, acc);
}
template <int PARTS>
__device__ __forceinline__ void unit_m1(const Unit<6> &u, const Stage &st, int ul, int lane,
                                        float &acc) {
  unit_m1_b32<PARTS, 6>(u, st, ul, lane, acc);
}
template <int PARTS>
__device__ __forceinline__ void unit_m1(const Unit<20> &u, const Stage &st, int ul, int lane,
                                        float &acc) {
  unit_m1_b32<PARTS, 20>(u, st, ul, lane, acc);
}

// Q2_K: the B operand of 32-element window w = 4 h + j: the lane's 8 codes
// (k = 8 g .. 8 g + 7 of the window), bits 2 j of its qs bytes 32 h + 8 g + i,
// natural order.
__device__ __forceinline__ half8_t q2k_codes(const Unit<10> &u, int w) {
  const uint32_t qw[4] = {u.q.x, u.q.y, u.q.z, u.q.w};
  const int h = w >> 2, sh = 2 * (w & 3);
  return fp8_operand((qw[2 * h] >> sh) & 0x03030303u, (qw[2 * h + 1] >> sh) & 0x03030303u);
}

// Q2_K: 16 scale groups of 16.  Two chains (h = 0, 1) of four MFMAs, one per
// window j; selector row 2 i + p of chain h carries group 8 h + i, whose k-half
// (i & 1) of window i >> 1 only the lanes g >> 1 == (i & 1) supply.  Lane
// (n, g) keeps groups 8 h + 2 g and 8 h + 2 g + 1 of each chain.
template <int PARTS>
__device__ __forceinline__ void unit_m1(const Unit<10> &u, const Stage &st, int ul, int lane,
                                        float &acc) {
  const int r = lane & 15, g = lane >> 4;
  const int gi = r >> 1;
  const bool on = (PARTS == 2 || (r & 1) == 0) && (gi & 1) == (g >> 1);
  const int own = 2 * (st.xh + (r & 1) * (st.xl - st.xh) + 256 * ul + 8 * g);
  const int zero = 2 * st.zero;
  half8_t a[8];
#pragma unroll
  for (int w = 0; w < 8; ++w) a[w] = lds_h8b((on && (gi >> 1) == (w & 3)) ? own + 64 * w : zero);
  float4_t D0 = {0.f, 0.f, 0.f, 0.f}, D1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    D0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[j], q2k_codes(u, j), D0, 0, 0, 0);
    D1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[4 + j], q2k_codes(u, 4 + j), D1, 0, 0, 0);
  }
  const int sh = 16 * (g & 1);
  const uint32_t w0 = (g >> 1) ? u.sc.y : u.sc.x, w1 = (g >> 1) ? u.sc.w : u.sc.z;  // groups 2g.., 8+2g..
  const uint32_t a0 = (w0 >> sh) & 0xFFu, a1 = (w0 >> (sh + 8)) & 0xFFu;
  const uint32_t b0 = (w1 >> sh) & 0xFFu, b1 = (w1 >> (sh + 8)) & 0xFFu;
  const float s = (float)(a0 & 15u) * (D0[0] + D0[1]) + (float)(a1 & 15u) * (D0[2] + D0[3]) +
                  (float)(b0 & 15u) * (D1[0] + D1[1]) + (float)(b1 & 15u) * (D1[2] + D1[3]);
  const int xs = st.xs + (ul * 16 + 2 * g) * st.ms;
  const float m = (float)(a0 >> 4) * lds_f(xs) + (float)(a1 >> 4) * lds_f(xs + st.ms) +
                  (float)(b0 >> 4) * lds_f(xs + 8 * st.ms) + (float)(b1 >> 4) * lds_f(xs + 9 * st.ms);
  acc += lds_f(st.xf + ul * st.ms) * (h2f(u.dm) * s - h2f(u.dm >> 16) * m);
}

// Q3_K: the B operand of window w = 4 h + j: the codes q3 = low bits | high
// bit << 2 <= 7 (natural order; the offset 4 goes through the group sums), the
// lane's codes as in Q2_K plus bit 4 h + j of its hmask bytes 8 g + i.
__device__ __forceinline__ half8_t q3k_codes(const Unit<11> &u, int w) {
  const uint32_t qw[4] = {u.q.x, u.q.y, u.q.z, u.q.w};
  const int h = w >> 2, j = w & 3;
  const uint32_t t0 = ((qw[2 * h] >> (2 * j)) & 0x03030303u) |
                      (((u.hm.x >> (4 * h + j)) & 0x01010101u) << 2);
  const uint32_t t1 = ((qw[2 * h + 1] >> (2 * j)) & 0x03030303u) |
                      (((u.hm.y >> (4 * h + j)) & 0x01010101u) << 2);
  return fp8_operand(t0, t1);
}
__device__ __forceinline__ float q3k_scale(const uint32_t (&S)[4], int grp) {
  return (float)((int)((S[grp >> 2] >> (8 * (grp & 3))) & 0xFFu) - 32);
}

// Q3_K: the Q2_K scheme (two chains, two groups per MFMA) with signed 6-bit
// scales and the code offset 4 taken off through the group sums.
template <int PARTS>
__device__ __forceinline__ void unit_m1(const Unit<11> &u, const Stage &st, int ul, int lane,
                                        float &acc) {
  const int r = lane & 15, g = lane >> 4;
  const int gi = r >> 1;
  const bool on = (PARTS == 2 || (r & 1) == 0) && (gi & 1) == (g >> 1);
  const int own = 2 * (st.xh + (r & 1) * (st.xl - st.xh) + 256 * ul + 8 * g);
  const int zero = 2 * st.zero;
  half8_t a[8];
#pragma unroll
  for (int w = 0; w < 8; ++w) a[w] = lds_h8b((on && (gi >> 1) == (w & 3)) ? own + 64 * w : zero);
  float4_t D0 = {0.f, 0.f, 0.f, 0.f}, D1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    D0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[j], q3k_codes(u, j), D0, 0, 0, 0);
    D1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[4 + j], q3k_codes(u, 4 + j), D1, 0, 0, 0);
  }
  uint32_t S[4];
  q3k_scales(u.s0, u.s1, u.s2, S);
  const float a0 = q3k_scale(S, 2 * g), a1 = q3k_scale(S, 2 * g + 1);
  const float b0 = q3k_scale(S, 8 + 2 * g), b1 = q3k_scale(S, 9 + 2 * g);
  const float s = a0 * (D0[0] + D0[1]) + a1 * (D0[2] + D0[3]) + b0 * (D1[0] + D1[1]) +
                  b1 * (D1[2] + D1[3]);
  const int xs = st.xs + (ul * 16 + 2 * g) * st.ms;
  const float m = a0 * lds_f(xs) + a1 * lds_f(xs + st.ms) + b0 * lds_f(xs + 8 * st.ms) +
                  b1 * lds_f(xs + 9 * st.ms);
  const float d = h2f(u.d);
  acc += lds_f(st.xf + ul * st.ms) * (d * s - (4.f * d) * m);
}

// IQ4_XS: the B operand of sub-block j (the codebook values).
__device__ __forceinline__ half8_t xs_codes(const Unit<23> &u, int j) {
  const uint32_t w[8] = {u.a.x, u.a.y, u.a.z, u.a.w, u.b.x, u.b.y, u.b.z, u.b.w};
  uint32_t c[4];
  b32_f16<20>(w[j], 0u, c);
  return as_h8(c[0], c[1], c[2], c[3]);
}

// IQ4_XS: 8 sub-blocks, one chain as Q4_K; lane (n, g) keeps sub-blocks 2g
// and 2g + 1, whose scales are d * (ls - 32).
template <int PARTS>
__device__ __forceinline__ void unit_m1(const Unit<23> &u, const Stage &st, int ul, int lane,
                                        float &acc) {
  const int r = lane & 15, g = lane >> 4;
  const int jo = r >> 1;
  const bool live = PARTS == 2 || (r & 1) == 0;
  const int own = 2 * (st.xh + (r & 1) * (st.xl - st.xh) + 256 * ul + 8 * g);
  const int zero = 2 * st.zero;
  half8_t a[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) a[j] = lds_h8b(((live && jo == j) ? own : zero) + 64 * j);
  float4_t D = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 8; ++j) D = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[j], xs_codes(u, j), D, 0, 0, 0);
  const float d = h2f(u.h.x);
  const float l0 = (float)((int)iq4xs_ls(u.h.x >> 16, u.h.y, 2 * g) - 32);
  const float l1 = (float)((int)iq4xs_ls(u.h.x >> 16, u.h.y, 2 * g + 1) - 32);
  acc += lds_f(st.xf + ul * st.ms) * (d * (l0 * (D[0] + D[1]) + l1 * (D[2] + D[3])));
}

// One unit of Q4_K / Q5_K: 8 sub-blocks x MT activation tiles.  Per
// activation row the sub-block dots are folded as
//   acc += d 2^24 sum_even sc_j D_j + d 2^20 sum_odd sc_j D_j - dmin sum_j m_j xs_j
// (odd sub-blocks hold high nibbles, coded as 16 q).
template <int PARTS, int MT, int MR, int TYPE>
__device__ __forceinline__ void unit_compute_k(const Unit<TYPE> &u, const Stage &st, int ul,
                                               int lane, int M, float (&acc)[MT][4]) {
#pragma clang fp contract(off)
  const int r = lane & 15, g = lane >> 4;
  uint32_t sc_lo, sc_hi, m_lo, m_hi;
  q4k_scales_packed(u.h.y, u.h.z, u.h.w, sc_lo, sc_hi, m_lo, m_hi);
  float se[MT][4], so[MT][4], sm[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) se[mt][i] = so[mt][i] = sm[mt][i] = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    half8_t blo, bhi;
    k_codes(u, c, blo, bhi);
    const uint32_t scw = c < 2 ? sc_lo : sc_hi, mw = c < 2 ? m_lo : m_hi;
    const int b0 = (2 * c) & 3, b1 = (2 * c + 1) & 3;
    const float sc0 = ubyte(scw, b0), m0 = ubyte(mw, b0);
    const float sc1 = ubyte(scw, b1), m1 = ubyte(mw, b1);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = 16 * mt + r;
      const bool on = m < M;
      const int off = m * st.ld + 256 * ul + 64 * c + 8 * g;
      const float4_t D0 = mfma32<PARTS>(st.xh + off, st.xl + off, st.zero, blo, on);
      const float4_t D1 = mfma32<PARTS>(st.xh + off + 32, st.xl + off + 32, st.zero, bhi, on);
      const int xs = st.xs + (ul * 8 + 2 * c) * st.ms + 16 * mt + 4 * g;
      if (MR == 1) {
        se[mt][0] = fmaf(sc0, D0[0], se[mt][0]);
        so[mt][0] = fmaf(sc1, D1[0], so[mt][0]);
        sm[mt][0] = fmaf(m0, lds_f(xs), fmaf(m1, lds_f(xs + st.ms), sm[mt][0]));
      } else {
        const float4 x0 = lds_f4(xs), x1 = lds_f4(xs + st.ms);
        const float xv0[4] = {x0.x, x0.y, x0.z, x0.w}, xv1[4] = {x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          se[mt][i] = fmaf(sc0, D0[i], se[mt][i]);
          so[mt][i] = fmaf(sc1, D1[i], so[mt][i]);
          sm[mt][i] = fmaf(m0, xv0[i], fmaf(m1, xv1[i], sm[mt][i]));
        }
      }
    }
  }
  const float d = h2f(u.h.x), dmin = h2f(u.h.x >> 16);
  const float d24 = d, d20 = d * k_hi_scale<TYPE>();
  float f[MT][4];
  unit_scales<MT, MR>(st, ul, g, f);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < MR; ++i)
      acc[mt][i] = fmaf(f[mt][i], fmaf(d24, se[mt][i], fmaf(d20, so[mt][i], -(dmin * sm[mt][i]))),
                        acc[mt][i]);
}
template <int PARTS, int MT, int MR>
__device__ __forceinline__ void unit_compute(const Unit<12> &u, const Stage &st, int ul, int lane,
                                             int M, float (&acc)[MT][4]) {
  unit_compute_k<PARTS, MT, MR, 12>(u, st, ul, lane, M, acc);
}
template <int PARTS, int MT, int MR>
__device__ __forceinline__ void unit_compute(const Unit<13> &u, const Stage &st, int ul, int lane,
                                             int M, float (&acc)[MT][4]) {
  unit_compute_k<PARTS, MT, MR, 13>(u, st, ul, lane, M, acc);
}

// One unit of Q6_K: 16 scale groups of 16 elements.
template <int PARTS, int MT, int MR>
__device__ __forceinline__ void unit_compute(const Unit<14> &u, const Stage &st, int ul, int lane,
                                             int M, float (&acc)[MT][4]) {
  const int r = lane & 15, g = lane >> 4;
  const float d = h2f(u.d);
  const uint32_t dw[12] = {u.p0.x, u.p0.y, u.p0.z, u.p0.w, u.p1.x, u.p1.y,
                           u.p1.z, u.p1.w, u.p2.x, u.p2.y, u.p2.z, u.p2.w};
  const uint32_t scw[4] = {u.sc.x, u.sc.y, u.sc.z, u.sc.w};
  float f[MT][4];
  unit_scales<MT, MR>(st, ul, g, f);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int hf = i >> 1, lh = i & 1;
    const uint32_t qa = dw[3 * i], qb = dw[3 * i + 1], qh = dw[3 * i + 2];
    const uint32_t v[4] = {(qa & 0x0F0F0F0Fu) | ((qh << 4) & 0x30303030u),
                           (qb & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u),
                           ((qa >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u),
                           ((qb >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u)};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const half4_t b = q6_operand(v[t]);
      const int s = 8 * hf + 2 * t + lh;
      const float sd = d * (float)(int8_t)((scw[s >> 2] >> (8 * (s & 3))) & 0xFFu);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = 16 * mt + r;
        const int off = m * st.ld + 256 * ul + 128 * hf + 32 * t + 16 * lh + 4 * g;
        const float4_t D = mfma16<PARTS>(st.xh + off, st.xl + off, st.zero, b, m < M);
        apply_s<MR>(acc[mt], D, sd, f[mt]);
      }
    }
  }
}

// One Q8_0 block.
template <int PARTS, int MT, int MR>
__device__ __forceinline__ void unit_compute(const Unit<8> &u, const Stage &st, int ul, int lane,
                                             int M, float (&acc)[MT][4]) {
  const int r = lane & 15, g = lane >> 4;
  const half8_t b = q8_operand(u);
  const float sd = h2f(u.d);
  float f[MT][4];
  unit_scales<MT, MR>(st, ul, g, f);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + r;
    const int off = m * st.ld + 32 * ul + 8 * g;
    const float4_t D = mfma32<PARTS>(st.xh + off, st.xl + off, st.zero, b, m < M);
    apply_s<MR>(acc[mt], D, sd, f[mt]);
  }
}

// One Q4_0 / Q5_0 / IQ4_NL block.
template <int PARTS, int MT, int MR, int TYPE>
__device__ __forceinline__ void unit_compute_b32(const Unit<TYPE> &u, const Stage &st, int ul,
                                                 int lane, int M, float (&acc)[MT][4]) {
  const int r = lane & 15, g = lane >> 4;
  const half8_t b = b32_operand<TYPE>(u, g);
  const float sd = h2f(u.d);
  float f[MT][4];
  unit_scales<MT, MR>(st, ul, g, f);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + r;
    const int off = m * st.ld + 32 * ul + 8 * g;
    const float4_t D = mfma32<PARTS>(st.xh + off, st.xl + off, st.zero, b, m < M);
    if constexpr (TYPE == 2)
      apply<MR>(acc[mt], D, sd, 8.f * sd, st.xs + ul * st.ms + 16 * mt + 4 * g, f[mt]);
    else
      apply_s<MR>(acc[mt], D, sd, f[mt]);
  }
}
template <int PARTS, int MT, int MR>
__device__ __forceinline__ void unit_compute(const Unit<2> &u, const Stage &st, int ul, int lane,
                                             int M, float (&acc)[MT][4]) {
  unit_compute_b32<PARTS, MT, MR, 2>(u, st, ul, lane, M, acc);
}
template <int PARTS, int MT, int MR>
__device__ __forceinline__ void unit_compute(const Unit<6> &u, const Stage &st, int ul, int lane,
                                             int M, float (&acc)[MT][4]) {
  unit_compute_b32<PARTS, MT, MR, 6>(u, st, ul, lane, M, acc);
}
template <int PARTS, int MT, int MR>
__device__ __forceinline__ void unit_compute(const Unit<20> &u, const Stage &st, int ul, int lane,
                                             int M, float (&acc)[MT][4]) {
  unit_compute_b32<PARTS, MT, MR, 20>(u, st, ul, lane, M, acc);
}
// Q2_K: each window twice, once per 16-element group (the other k-half reads
// the zero operand), with that group's d * sc and dmin * m.
template <int PARTS, int MT, int MR>
__device__ __forceinline__ void unit_compute(const Unit<10> &u, const Stage &st, int ul, int lane,
                                             int M, float (&acc)[MT][4]) {
  const int r = lane & 15, g = lane >> 4;
  const float d = h2f(u.dm), dmin = h2f(u.dm >> 16);
  const uint32_t scw[4] = {u.sc.x, u.sc.y, u.sc.z, u.sc.w};
  float f[MT][4];
  unit_scales<MT, MR>(st, ul, g, f);
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    const half8_t b = q2k_codes(u, w);
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int grp = 2 * w + sub;
      const uint32_t sb = (scw[grp >> 2] >> (8 * (grp & 3))) & 0xFFu;
      const float sd = d * (float)(sb & 15u), so = dmin * (float)(sb >> 4);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = 16 * mt + r;
        const int off = m * st.ld + 256 * ul + 32 * w + 8 * g;
        const float4_t Dv = mfma32<PARTS>(st.xh + off, st.xl + off, st.zero, b,
                                          m < M && (g >> 1) == sub);
        apply<MR>(acc[mt], Dv, sd, so, st.xs + (ul * 16 + grp) * st.ms + 16 * mt + 4 * g, f[mt]);
      }
    }
  }
}
// Q3_K: as Q2_K, with the group's d * (sc - 32) and the code offset 4.
template <int PARTS, int MT, int MR>
__device__ __forceinline__ void unit_compute(const Unit<11> &u, const Stage &st, int ul, int lane,
                                             int M, float (&acc)[MT][4]) {
  const int r = lane & 15, g = lane >> 4;
  const float d = h2f(u.d);
  uint32_t S[4];
  q3k_scales(u.s0, u.s1, u.s2, S);
  float f[MT][4];
  unit_scales<MT, MR>(st, ul, g, f);
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    const half8_t b = q3k_codes(u, w);
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int grp = 2 * w + sub;
      const float sd = d * q3k_scale(S, grp), so = 4.f * sd;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = 16 * mt + r;
        const int off = m * st.ld + 256 * ul + 32 * w + 8 * g;
        const float4_t Dv = mfma32<PARTS>(st.xh + off, st.xl + off, st.zero, b,
                                          m < M && (g >> 1) == sub);
        apply<MR>(acc[mt], Dv, sd, so, st.xs + (ul * 16 + grp) * st.ms + 16 * mt + 4 * g, f[mt]);
      }
    }
  }
}
// IQ4_XS: sub-block j as an IQ4_NL block with scale d * (ls_j - 32).
template <int PARTS, int MT, int MR>
__device__ __forceinline__ void unit_compute(const Unit<23> &u, const Stage &st, int ul, int lane,
                                             int M, float (&acc)[MT][4]) {
  const int r = lane & 15, g = lane >> 4;
  const float d = h2f(u.h.x);
  float f[MT][4];
  unit_scales<MT, MR>(st, ul, g, f);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const half8_t b = xs_codes(u, j);
    const float sd = d * (float)((int)iq4xs_ls(u.h.x >> 16, u.h.y, j) - 32);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = 16 * mt + r;
      const int off = m * st.ld + 256 * ul + 32 * j + 8 * g;
      const float4_t D = mfma32<PARTS>(st.xh + off, st.xl + off, st.zero, b, m < M);
      apply_s<MR>(acc[mt], D, sd, f[mt]);
    }
  }
}

// Activation staging.  Activations are converted in items of 16 consecutive
// elements of one row, one item per thread and step.
constexpr int kItem = 16;
constexpr int kMergeChunk = 8;  // attention records per item held in registers (merge prologue)

template <typename XT>
__device__ __forceinline__ void load_item(const XT *__restrict__ x, int64_t ldx, int K, int k0,
                                          int per_row, int total, int q, float (&v)[kItem]) {
#pragma unroll
  for (int i = 0; i < kItem; ++i) v[i] = 0.f;
  if (q < total) {
    const int m = q / per_row, e = kItem * (q - m * per_row), k = k0 + e;
    if (k < K) {  // K is a multiple of 32, so an item is either all in or all out
      if constexpr (sizeof(XT) == 4) {
        const float4 *src = (const float4 *)(x + (int64_t)m * ldx + k);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 t = src[i];
          v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
        }
      } else {
        const half8_t *src = (const half8_t *)(x + (int64_t)m * ldx + k);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const half8_t t = src[i];
#pragma unroll
          for (int j = 0; j < 8; ++j) v[8 * i + j] = (float)t[j];
        }
      }
    }
  }
}

// hi / lo parts of the scaled item (natural order, or each quad in (0, 2, 1, 3) order),
// group sums of hi + lo and the unit's inverse scale.  A group
// (16 or 32 elements) spans one or two consecutive threads of a wave, a unit
// (UE = 32 or 256 elements) UE / 16 of them; every lane of the wave takes part
// (items past the end hold zeros).
template <int PARTS, int GS, int UE, bool SUMS, bool NAT>
__device__ __forceinline__ void store_item(int per_row, int total, int q, const float (&v)[kItem],
                                           const Stage &st) {
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < kItem; ++i) mx = fmaxf(mx, fabsf(v[i]));
  mx = UE / kItem == 16 ? max_lanes16(mx) : max_lanes2(mx);  // a unit is one or two DPP rows
  const int ex = stage_exp(mx);
  const float sc = pow2f(ex);
  half8_t hi[2], lo[2];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kItem; ++i) {
    const int pos = NAT ? i : (i & ~3) | ((i & 1) << 1) | ((i >> 1) & 1);  // swap 1 <-> 2 per quad
    // Split the f32 value itself: when the compiler folds the multiply that
    // produced it into the f16 conversions (v_fma_mix), the RMSNorm prologue
    // measured ~15x the error of the plain kernel on the same products.
    float vi = v[i];
    asm volatile("" : "+v"(vi));
    const float t = vi * sc;  // exact: a power of two
    const half_t h = (half_t)t;
    const half_t l = (half_t)(t - (float)h);
    hi[pos >> 3][pos & 7] = h;
    lo[pos >> 3][pos & 7] = l;
    if (SUMS) s += (float)h + (PARTS == 2 ? (float)l : 0.f);
  }
  if (SUMS && GS == 2 * kItem) s += dpp<kDppXor1>(s);
  if (q < total) {
    const int m = q / per_row, e = kItem * (q - m * per_row);
    half_t *lh = (half_t *)g_lds;
    *(half8_t *)(lh + st.xh + m * st.ld + e) = hi[0];
    *(half8_t *)(lh + st.xh + m * st.ld + e + 8) = hi[1];
    if (PARTS == 2) {
      *(half8_t *)(lh + st.xl + m * st.ld + e) = lo[0];
      *(half8_t *)(lh + st.xl + m * st.ld + e + 8) = lo[1];
    }
    if (SUMS && (e & (GS - 1)) == 0) ((float *)g_lds)[st.xs + (e / GS) * st.ms + m] = s;
    if ((e & (UE - 1)) == 0) ((float *)g_lds)[st.xf + (e / UE) * st.ms + m] = pow2f(-ex);
  }
}

// ---------------------------------------------------------------------------
// Batched decode: 2 <= M <= 32 activation rows in one pass over the weights
// (and M = 1 beyond the one-shot kernel's K).
//
// The reference re-reads the weights once per activation row
// (forward-pass.ts:1536-1539).  Here a workgroup of 8 waves owns 4 row tiles
// (two pairs) and one or more K slices of `us` units.  A slice's activations
// (M rows: scaled hi / lo parts, group sums, unit scales) are staged in LDS at
// once; wave (pair p, lane kl) takes tile pair p and every 4th unit of the
// slice, so every A fragment read from LDS feeds the MFMAs of two row tiles.
// The 4 waves of a pair add their partial sums in a fixed order.
//
// Split K.  With a workspace the slices are spread over the grid (grid.y =
// number of slices): a workgroup stages one slice and writes its partial sums
// to the workspace, and mb_reduce_kernel adds the slices in a fixed order.
// For a small N (the FFN down projection: 256 row tiles for 256 CUs) this is
// what keeps the per-CU activation staging small: without it every CU would
// convert and stage all M x K activations for its one tile.  Without a
// workspace each workgroup walks all slices (spw of them) itself.  Either way
// the sums are deterministic.
// ---------------------------------------------------------------------------
#ifndef GGUF_MB_MIN_WGS
#define GGUF_MB_MIN_WGS 512  // split K further while the grid has fewer workgroups
#endif
#ifndef GGUF_MB_DEPTH_K
#define GGUF_MB_DEPTH_K 2    // units in flight per tile per wave, 256-element units
#endif
#ifndef GGUF_MB_DEPTH_K2
#define GGUF_MB_DEPTH_K2 2   // the same, two 16-row activation tiles
#endif
#ifndef GGUF_MB_DEPTH_B
#define GGUF_MB_DEPTH_B 4    // the same, 32-element blocks
#endif
constexpr int kMbThreads = 512;
constexpr int kMbTiles = 4;  // row tiles per workgroup
template <int TYPE, int MT>
constexpr int mb_depth() {  // units in flight per tile per wave
  return (TYPE == 8 || is_b32(TYPE)) ? GGUF_MB_DEPTH_B : (MT == 2 ? GGUF_MB_DEPTH_K2 : GGUF_MB_DEPTH_K);
}

template <int TYPE, typename XT, int MT>
__global__ __launch_bounds__(kMbThreads) void mb_kernel(const XT *__restrict__ x, int64_t ldx,
                                                        const uint8_t *__restrict__ W, int N,
                                                        int K, int M, int us, int spw,
                                                        float *__restrict__ out, int64_t ldo) {
  constexpr int PARTS = sizeof(XT) == 4 ? 2 : 1;
  constexpr int UE = Fmt<TYPE>::UE, TU = Fmt<TYPE>::TU, GS = Dec<TYPE>::GS;
  constexpr int P = mb_depth<TYPE, MT>();
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int pr = wave & 1, kl = wave >> 1;
  const int ntiles = (N + 15) >> 4, nu = K / UE;
  const int nsl = (nu + us - 1) / us;
  const int tt = kMbTiles * blockIdx.x + 2 * pr;  // the wave's first tile
  const int ce = us * UE;

  Stage st;
  st.ld = ce + kXPad;
  st.ms = 16 * MT;
  st.xh = 0;
  st.xl = M * st.ld;
  st.xs = (st.xl + (PARTS == 2 ? M * st.ld : 0)) / 2;
  st.xf = st.xs + (ce / GS) * st.ms;
  st.zero = 2 * (st.xf + (ce / UE) * st.ms);
  // rows M..ms-1 of the group sums / unit scales and the zero operand stay zero
  // throughout (only those rows: the staging below writes rows < M without a
  // barrier in between)
  for (int i = threadIdx.x; i < (ce / GS + ce / UE) * st.ms; i += kMbThreads)
    if (i % st.ms >= M) ((float *)g_lds)[st.xs + i] = 0.f;
  if (threadIdx.x < kZeroHalves / 2) ((uint32_t *)((half_t *)g_lds + st.zero))[threadIdx.x] = 0u;

  // one buffer resource per tile; a tile past the weight's end has no records (loads read 0)
  const int tb = nu * TU;
  const __amdgpu_buffer_rsrc_t rs0 = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(W + (int64_t)min(tt, ntiles - 1) * tb), 0, tt < ntiles ? tb : 0, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs1 = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(W + (int64_t)min(tt + 1, ntiles - 1) * tb), 0, tt + 1 < ntiles ? tb : 0,
      kRsrcWord3);
  float acc[2][MT][4];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[t][mt][i] = 0.f;

  const int sl0 = blockIdx.y * spw, sl1 = min(sl0 + spw, nsl);
  for (int sl = sl0; sl < sl1; ++sl) {  // uniform over the workgroup
    const int u0 = sl * us, nus = min(us, nu - u0);
    const int cnt = (nus - kl + 3) >> 2;  // the wave's units: u0 + kl + 4 j, j < cnt
    // weights first (the staging below overlaps their latency)
    Unit<TYPE> b0[P], b1[P];
#pragma unroll
    for (int j = 0; j < P; ++j)
      if (j < cnt) {
        const int soff = (u0 + kl + 4 * j) * TU;
        load_unit(rs0, soff, r, g, b0[j]);
        load_unit(rs1, soff, r, g, b1[j]);
      }
    if (sl > sl0) __syncthreads();  // the previous slice is consumed
    const int per_row = ce / kItem, total = M * per_row;
    for (int q0 = 0; q0 < total; q0 += kMbThreads) {
      float v[kItem];
      load_item<XT>(x, ldx, K, u0 * UE, per_row, total, q0 + (int)threadIdx.x, v);
      store_item<PARTS, GS, UE, Dec<TYPE>::SUMS, Dec<TYPE>::NAT>(per_row, total,
                                                                 q0 + (int)threadIdx.x, v, st);
    }
    __syncthreads();
    for (int j0 = 0; j0 < cnt; j0 += P) {
#pragma unroll
      for (int jj = 0; jj < P; ++jj) {
        const int j = j0 + jj;
        if (j < cnt) {
          const int ul = kl + 4 * j;  // unit within the slice
          unit_compute<PARTS, MT, 4>(b0[jj], st, ul, lane, M, acc[0]);
          unit_compute<PARTS, MT, 4>(b1[jj], st, ul, lane, M, acc[1]);
          if (j + P < cnt) {
            const int soff = (u0 + kl + 4 * (j + P)) * TU;
            load_unit(rs0, soff, r, g, b0[jj]);
            load_unit(rs1, soff, r, g, b1[jj]);
          }
        }
      }
    }
  }

  // fixed-order sum of the 4 waves of each pair (kl = 0, 1, 2, 3), through LDS
  __syncthreads();  // the staged activations are consumed
  float *red = (float *)g_lds;  // [8 waves][2][MT][4][64]
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[(((wave * 2 + t) * MT + mt) * 4 + i) * 64 + lane] = acc[t][mt][i];
  __syncthreads();
  if (kl != 0) return;
  float *o = out + (int64_t)blockIdx.y * (gridDim.y > 1 ? (int64_t)M * N : 0);
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int n = 16 * (tt + t) + r;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = acc[t][mt][i];
#pragma unroll
        for (int w2 = 1; w2 < 4; ++w2) v += red[((((pr + 2 * w2) * 2 + t) * MT + mt) * 4 + i) * 64 + lane];
        const int m = 16 * mt + 4 * g + i;
        if (m < M && n < N) o[(int64_t)m * ldo + n] = v;
      }
  }
}

// y[m, n] = sum over the S slices of part[s][m][n], in slice order.
__global__ __launch_bounds__(256) void mb_reduce_kernel(const float *__restrict__ part, int S, int M,
                                                        int N, float *__restrict__ y, int64_t ldy) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x, mn = (int64_t)M * N;
  if (i >= mn) return;
  float v = part[i];
  for (int s = 1; s < S; ++s) v += part[(int64_t)s * mn + i];
  y[(i / N) * ldy + i % N] = v;
}

// Staged slice width: the units whose staged activations (hi / lo parts of M
// rows, group sums and unit scales of the MT * 16 padded rows) fit in
// kMbStageBytes of LDS next to the row padding and the zero operand.
constexpr size_t kMbStageBytes = 150 * 1024;
template <int TYPE, typename XT>
int mb_units_per_slice(int M, int K) {
  constexpr int UE = Fmt<TYPE>::UE, GS = Dec<TYPE>::GS, PARTS = sizeof(XT) == 4 ? 2 : 1;
  const int MT = M <= 16 ? 1 : 2;
  const size_t per_unit = (size_t)M * UE * 2 * PARTS + (size_t)(UE / GS + 1) * 16 * MT * 4;
  const size_t fixed = (size_t)M * kXPad * 2 * PARTS + kZeroHalves * 2;
  int us = (int)((kMbStageBytes - fixed) / per_unit);
  us = us < 1 ? 1 : us;
  const int nu = K / UE;
  return us < nu ? us : nu;
}
// Slices and workspace: at least ~2 workgroups per CU, split K further while
// the grid is smaller; the workspace holds the slices' partial sums.
template <int TYPE, typename XT>
void mb_plan(int M, int N, int K, int *us, int *nsl) {
  constexpr int UE = Fmt<TYPE>::UE;
  const int nu = K / UE, groups = ((N + 15) / 16 + kMbTiles - 1) / kMbTiles;
  int u = mb_units_per_slice<TYPE, XT>(M, K);
  while (u > 1 && (int64_t)groups * ((nu + u - 1) / u) < GGUF_MB_MIN_WGS) u = (u + 1) / 2;
  *us = u;
  *nsl = (nu + u - 1) / u;
}

template <int TYPE, typename XT, int MT>
hipError_t launch_mb(const XT *x, int64_t ldx, const uint8_t *W, int N, int K, float *y,
                     int64_t ldy, int M, float *work, int64_t work_floats, hipStream_t s) {
  constexpr int PARTS = sizeof(XT) == 4 ? 2 : 1;
  constexpr int UE = Fmt<TYPE>::UE, GS = Dec<TYPE>::GS;
  int us, nsl;
  mb_plan<TYPE, XT>(M, N, K, &us, &nsl);
  // the partial sums follow the workspace's counter prefix
  const bool split = nsl > 1 && work && work_floats >= kWsPrefix / 4 + (int64_t)nsl * M * N;
  float *part = split ? work + kWsPrefix / 4 : nullptr;
  if (!split) {  // every workgroup walks all of K, in the widest slices that fit
    us = mb_units_per_slice<TYPE, XT>(M, K);
    nsl = (K / UE + us - 1) / us;
  }
  const int ce = us * UE;
  size_t lds = (size_t)M * (ce + kXPad) * 2 * PARTS + (size_t)(ce / GS + ce / UE) * 16 * MT * 4 +
               kZeroHalves * 2;
  const size_t red = (size_t)8 * 2 * MT * 4 * 64 * 4;
  lds = lds > red ? lds : red;
  auto kern = mb_kernel<TYPE, XT, MT>;
  if (lds > 65536) {
    const hipError_t ea =
        hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (ea != hipSuccess) return ea;
  }
  const unsigned groups = (unsigned)(((N + 15) / 16 + kMbTiles - 1) / kMbTiles);
  const dim3 grid(groups, split ? (unsigned)nsl : 1u), block(kMbThreads);
  hipLaunchKernelGGL(kern, grid, block, lds, s, x, ldx, W, N, K, M, us, split ? 1 : nsl,
                     split ? part : y, split ? (int64_t)N : ldy);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !split) return e;
  const int64_t mn = (int64_t)M * N;
  hipLaunchKernelGGL(mb_reduce_kernel, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, s, part,
                     nsl, M, N, y, ldy);
  return hipGetLastError();
}

#include "decode_mk.hpp"

// Workspace floats the split-K batched decode uses for M rows (0: none).
template <int TYPE, typename XT>
int64_t mb_work_floats(int M, int N, int K) {
  if (M < 2) return 0;
  if constexpr (TYPE == 12 || TYPE == 14 || TYPE == 8)
    if (K % 256 == 0) return (int64_t)((mk_work_bytes<TYPE, XT>(M, N, K) + 3) / 4);
  int us, nsl;
  mb_plan<TYPE, XT>(M, N, K, &us, &nsl);
  return nsl > 1 ? kWsPrefix / 4 + (int64_t)nsl * M * N : 0;
}

// ---------------------------------------------------------------------------
// M = 1: a wave's whole share of the weights sits in registers.
//
// A workgroup of NW waves (8 when K > 4096, ks_n = 8 or the grid has at least
// 1536 waves, else 4) covers NW / ks_n
// row tiles;
// the ks_n waves of a tile split its units (wave ks takes units ks, ks + ks_n,
// ...), at most U per wave.  The activation vector is requested before the
// weights (the memory counter retires in issue order, so staging never waits
// on weight bytes) and staged once for all of K.  DP units of each wave are in
// flight at a time (DP = 0: all U at once), and each is consumed as it
// arrives.  The depth matters when the grid is one round of waves: with every
// unit of every wave requested at once (48 MB for a 4096 x 14336 Q6_K weight)
// the memory system returns them in no useful order, a wave's first unit lands
// as late as its last, and the decode runs after the transfer instead of
// under it.  A few units per wave (about 12 MB over the chip) keep the
// transfer at full rate and the arrivals in order.
//
// Fused variants for a decoder step (PRO, f32 activations only):
//   PRO = 1  the input norm of the projection, rmsnorm(x) * w
//            (rmsnorm.wgsl:58-67).  The scale r = 1 / rms(x) is common to the
//            whole row, so W (x * w * r) = r (W (x * w)): x * w is staged at
//            once, every thread publishes its partial sum of x^2 with the
//            staging barrier that exists anyway, and the sum is reduced and
//            applied only to the final sums.  No extra launch, buffer or
//            barrier, and nothing ahead of the staging writes;
//   PRO = 2  x is a row [gate (K) | up (K)] and is replaced by up * silu(gate)
//            (elementwise.wgsl:96-102);
//   PRO = 3  x is the attention output, merged here from the partial-softmax
//            records that the decode attention wrote (no merge pass of its
//            own): each thread's item is a 16-element slice of one query
//            head, and the records of the first kMergeChunk splits are
//            requested with the activations, ahead of the weights;
// and the epilogue `epi`:
//   0  y = result;
//   1  y += result (the residual add after the output and down projections);
//   2  SwiGLU over tile pairs: the weight holds gate and up row tiles
//      interleaved (tile 2m = gate rows 16m..16m+15, tile 2m + 1 = the same up
//      rows), and y[16 m + r] = up * silu(gate) (N / 2 outputs), so the FFN
//      activation never takes a separate pass.
// ---------------------------------------------------------------------------
#ifndef GGUF_M1_PRIO
#define GGUF_M1_PRIO 1  // wave priority from the units still to do
#endif
template <int TYPE, typename XT, int U, int XI, int PRO, int DP>
__global__ __launch_bounds__(512) void decode_m1_kernel(const XT *__restrict__ x,
                                                        const uint8_t *__restrict__ W, int N,
                                                        int K, float *__restrict__ y, int ks_n,
                                                        const float *__restrict__ pw, float eps,
                                                        int epi, AttnRecords ar, int rows_wg) {
  constexpr int PARTS = sizeof(XT) == 4 ? 2 : 1;
  constexpr int UE = Fmt<TYPE>::UE, TU = Fmt<TYPE>::TU, GS = Dec<TYPE>::GS;
  const int nthr = blockDim.x;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int ts_n = (nthr >> 6) / ks_n;
  const int ts = wave / ks_n, ks = wave - ts * ks_n;
  const int ntiles = (N + 15) >> 4;
  // rows_wg > 0: the workgroup owns rows [rows_wg b, rows_wg b + rows_wg) (a
  // multiple of 8, so that every CU gets the same share of a weight whose tiles
  // do not divide evenly over the grid); tile slot ts is the ts-th tile they
  // touch, and lanes of rows outside the range load nothing (their offsets are
  // past the buffer's end, which reads as zero) and store nothing
  int tile, lo, hi;
  if (rows_wg > 0) {
    const int row0 = blockIdx.x * rows_wg;
    tile = (row0 >> 4) + ts;
    lo = max(row0, 16 * tile);
    hi = min(min(row0 + rows_wg, N), 16 * tile + 16);
  } else {
    tile = blockIdx.x * ts_n + ts;
    lo = 16 * tile;
    hi = min(N, 16 * tile + 16);
  }
  const bool active = tile < ntiles && lo < hi;
  const int rl = (16 * tile + r >= lo && 16 * tile + r < hi) ? r : r + (1 << 20);  // row of the loads
  const int nu = K / UE;
  const int iters = (nu + ks_n - 1) / ks_n;  // <= U

  Stage st;
  st.ld = K + kXPad;
  st.ms = 1;
  st.xh = 0;
  st.xl = st.ld;
  st.xs = (st.xl + (PARTS == 2 ? st.ld : 0)) / 2;
  st.xf = st.xs + K / GS;
  const int red_off = st.xf + K / UE;  // floats: [waves][64]
  st.zero = 2 * (red_off + (nthr >> 6) * 64);
  float *red = (float *)g_lds + red_off;
  float *ssq = (float *)g_lds + st.zero / 2 + kZeroHalves / 2;  // [threads] partial sums of x^2
  if (threadIdx.x < kZeroHalves / 2) ((uint32_t *)((half_t *)g_lds + st.zero))[threadIdx.x] = 0u;
  // IQ types: the decode tables behind the rest, requested first, written with the staging
  st.tbl = (4 * (st.zero / 2 + kZeroHalves / 2 + nthr) + 15) & ~15;
  IqTabRegs<TYPE, 256> tab;
  if constexpr (is_iq(TYPE)) iq_get_tables<TYPE, 256>(tab);

  // activations first: item q = threadIdx.x + nthr * i of the K / 16 items
  const int per_row = K / kItem;
  float xv[XI][kItem];
  float pv[PRO == 1 || PRO == 2 ? XI : 1][kItem];  // norm weights (PRO 1) or up values (PRO 2)
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int q = (int)threadIdx.x + nthr * i;
    if constexpr (PRO != 3) load_item<XT>(x, 0, K, 0, per_row, per_row, q, xv[i]);
    if constexpr (PRO == 1) load_item<float>(pw, 0, K, 0, per_row, per_row, q, pv[i]);
    if constexpr (PRO == 2) load_item<float>((const float *)x + K, 0, K, 0, per_row, per_row, q, pv[i]);
  }
  // PRO 3: the item's 16-element slice of the first RC attention records of
  // its query head (the slots past the range are not loaded and get weight
  // zero), and where the rest would be
  constexpr int RC = PRO == 3 ? kMergeChunk : 1;
  float4 ro[PRO == 3 ? XI : 1][RC][4];
  float2 rml[PRO == 3 ? XI : 1][RC];
  const float *ro_base[PRO == 3 ? XI : 1], *rml_base[PRO == 3 ? XI : 1];
  int mn = 0;              // records to merge: ceil((p + 1) / kAttnSplit), 0 for a bad p
  int64_t rstride = 0;     // floats from one split's record to the next
  if constexpr (PRO == 3) {
    const int64_t p = ar.pos[0];
    mn = (p >= 0 && p < ar.max_seq) ? (int)(p / kAttnSplit) + 1 : 0;
    const int grp = ar.nh / ar.nkv, S = (ar.max_seq + kAttnSplit - 1) / kAttnSplit;
    const int rs = attn_record_stride(ar.hd);
    rstride = (int64_t)grp * rs;
    const int last = mn > 0 ? mn - 1 : 0;
#pragma unroll
    for (int i = 0; i < XI; ++i) {
      const int q = min((int)threadIdx.x + nthr * i, per_row - 1);
      const int k0 = kItem * q, h = k0 / ar.hd, i0 = k0 - h * ar.hd;
      const int gk = h / grp, jh = h - gk * grp;
      const float *rec = ar.work + ((int64_t)gk * S * grp + jh) * rs;
      ro_base[i] = rec + i0;
      rml_base[i] = rec + ar.hd;
#pragma unroll
      for (int c = 0; c < RC; ++c) {
        if (c > last) break;  // uniform: the loads of splits past the range are not issued
        const int64_t off = (int64_t)c * rstride;
        const float4 *o4 = (const float4 *)(ro_base[i] + off);
#pragma unroll
        for (int v = 0; v < 4; ++v) ro[i][c][v] = o4[v];
        rml[i][c] = *(const float2 *)(rml_base[i] + off);
      }
    }
  }

  // Branch-free over the U slots, so that the compiler can interleave the
  // units: a slot past the wave's share loads a valid unit of the tile (the
  // last one) and contributes zero; a wave past the last tile reads the last
  // tile and stores nothing.
  const int tile_c = active ? tile : ntiles - 1;
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(W + (int64_t)tile_c * nu * TU), 0, nu * TU, kRsrcWord3);
  // D units in flight: slot j + D is requested once unit j is consumed.  The
  // issue order is pinned (sched_barrier) because the memory counter retires
  // in order.
  constexpr int D = (DP == 0 || DP >= U) ? U : DP;
  // Half the window (at least one unit) is requested before the activations
  // are staged and the rest after the staging barrier, so that the activation
  // loads queue behind less weight traffic (256-element units; graph replays,
  // medians of four to six: 4096 x 4096 4.68 -> 4.20 us, 6144 x 4096 5.55 ->
  // 5.42, Q6_K 4096 x 14336 13.09 -> 12.53, Q5_K 14336 x 4096 11.32 -> 10.99,
  // the headline level).  Q8_0 (32-element units) lost 5-8% and Q3_K 3%:
  // they request the whole window first.
  constexpr int D0 = UE == 256 && TYPE != 11 ? (D / 2 > 1 ? D / 2 : 1) : D;
  Unit<TYPE> buf[D];
#pragma unroll
  for (int j = 0; j < D0; ++j) {
    const int u = ks + ks_n * j;
    const int uc = u < nu ? u : nu - 1;
    load_unit(wrs, uc * TU, rl, g, buf[j]);
  }

  if constexpr (PRO == 1) {  // stage x * w; the row's sum of x^2 rides on the staging barrier
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < XI; ++i)
#pragma unroll
      for (int e = 0; e < kItem; ++e) {
        ss += xv[i][e] * xv[i][e];
        xv[i][e] *= pv[i][e];
      }
    ssq[threadIdx.x] = ss;
  }
  if constexpr (PRO == 2) {
#pragma unroll
    for (int i = 0; i < XI; ++i)
#pragma unroll
      for (int e = 0; e < kItem; ++e) {
        const float gt = xv[i][e];
        xv[i][e] = pv[i][e] * (gt / (1.0f + expf(-gt)));
      }
  }
  if constexpr (PRO == 3) {  // merge in split order (attention_kernel's merge, same arithmetic)
#pragma unroll
    for (int i = 0; i < XI; ++i) {
      float M = -INFINITY;
#pragma unroll
      for (int c = 0; c < RC; ++c)
        if (c < mn) M = fmaxf(M, rml[i][c].x);
      for (int s2 = RC; s2 < mn; ++s2) M = fmaxf(M, rml_base[i][s2 * rstride]);
      float L = 0.f, a[kItem];
#pragma unroll
      for (int e = 0; e < kItem; ++e) a[e] = 0.f;
#pragma unroll
      for (int c = 0; c < RC; ++c) {
        if (c >= mn) break;  // uniform; the slots past the range were never loaded
        const float w = expf(rml[i][c].x - M);
        L = fmaf(w, rml[i][c].y, L);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          a[4 * v] = fmaf(w, ro[i][c][v].x, a[4 * v]);
          a[4 * v + 1] = fmaf(w, ro[i][c][v].y, a[4 * v + 1]);
          a[4 * v + 2] = fmaf(w, ro[i][c][v].z, a[4 * v + 2]);
          a[4 * v + 3] = fmaf(w, ro[i][c][v].w, a[4 * v + 3]);
        }
      }
      for (int s2 = RC; s2 < mn; ++s2) {  // ranges beyond RC splits: one record at a time
        const float *rp = ro_base[i] + s2 * rstride, *ml = rml_base[i] + s2 * rstride;
        const float w = expf(ml[0] - M);
        L = fmaf(w, ml[1], L);
#pragma unroll
        for (int e = 0; e < kItem; ++e) a[e] = fmaf(w, rp[e], a[e]);
      }
      const float inv = 1.0f / L;  // no records (bad position): 0 * inf = NaN
#pragma unroll
      for (int e = 0; e < kItem; ++e) xv[i][e] = a[e] * inv;
    }
  }
#pragma unroll
  for (int i = 0; i < XI; ++i)
    store_item<PARTS, GS, UE, Dec<TYPE>::SUMS, Dec<TYPE>::NAT>(per_row, per_row,
                                                               (int)threadIdx.x + nthr * i, xv[i], st);
  if constexpr (is_iq(TYPE)) iq_put_tables<TYPE, 256>(tab, g_lds + st.tbl);
  __syncthreads();
#pragma unroll
  for (int j = D0; j < D; ++j) {
    const int u = ks + ks_n * j;
    const int uc = u < nu ? u : nu - 1;
    load_unit(wrs, uc * TU, rl, g, buf[j]);
  }
  float ssp = 0.f;  // this lane's share of the row's sum of x^2 (reduced after the units)
  if constexpr (PRO == 1)
    for (int t = lane; t < nthr; t += 64) ssp += ssq[t];

  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < U; ++j) {
    // Wave priority from the units still to do (3 while at least 6 remain,
    // down to 0 for the last): the two waves of a SIMD otherwise issue oldest
    // first, and the younger one finished its units ~1 us after the older one
    // at the headline shape (per-wave timestamps), which set the kernel's
    // length.  The wave that is behind now issues first.
    if (GGUF_M1_PRIO) {
      const int rem = U - j;
      if (rem >= 6) __builtin_amdgcn_s_setprio(3);
      else if (rem >= 4) __builtin_amdgcn_s_setprio(2);
      else if (rem >= 2) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
    }
    const int u = ks + ks_n * j;
    const bool valid = u < nu;  // implies j < iters
    float t = 0.f;
    unit_m1<PARTS>(buf[j % D], st, valid ? u : nu - 1, lane, t);
    acc += valid ? t : 0.f;
    if (j + D < U) {
      const int un = ks + ks_n * (j + D);
      const int ucn = un < nu ? un : nu - 1;
      __builtin_amdgcn_sched_barrier(0);
      load_unit(wrs, ucn * TU, rl, g, buf[j % D]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (GGUF_M1_PRIO) __builtin_amdgcn_s_setprio(0);
  acc = sum_xor32(sum_xor16(acc));  // the four lane groups of each row
  float scale = 1.0f;
  if constexpr (PRO == 1) {
    ssp = sum_xor32(sum_xor16(ssp));
    ssp += dpp<kDppMirror>(ssp);
    ssp += dpp<kDppHalfMirror>(ssp);
    ssp += dpp<kDppXor2>(ssp);
    ssp += dpp<kDppXor1>(ssp);
    scale = 1.0f / sqrtf(ssp / (float)K + eps);
  }

  const int n = 16 * tile + r;
  if (ks_n > 1) {  // fixed-order sum of the ks_n partial sums of each tile
    red[wave * 64 + lane] = acc;
    __syncthreads();
    if (ks == 0)
      for (int j = 1; j < ks_n; ++j) acc += red[(wave + j) * 64 + lane];
  }
  acc *= scale;
  if (epi == 2) {  // every wave reaches both barriers
    __syncthreads();  // the partial sums above are read
    if (ks == 0 && (ts & 1) && g == 0) red[(ts >> 1) * 16 + r] = acc;  // up rows
    __syncthreads();
    if (ks == 0 && !(ts & 1) && g == 0 && active && n < N) {
      const float up = red[(ts >> 1) * 16 + r];
      y[16 * (tile >> 1) + r] = up * (acc / (1.0f + expf(-acc)));
    }
    return;
  }
  if (ks == 0 && active && n >= lo && n < hi && g == 0) y[n] = epi == 1 ? y[n] + acc : acc;
}

// Units per wave a kernel may own (K-quant units stay in registers whole; a
// fused prologue or long K leaves less room for them).
#ifndef GGUF_M1_PRO_TIGHT
#define GGUF_M1_PRO_TIGHT 1  // a fused prologue takes the tight unit budget
#endif
#ifndef GGUF_M1_NW_MIN
#define GGUF_M1_NW_MIN 4     // waves per workgroup, at least
#endif
#ifndef GGUF_M1_MIN_WAVES
#define GGUF_M1_MIN_WAVES 1024  // K split until the grid has this many waves
#endif
#ifndef GGUF_M1_FILL
#define GGUF_M1_FILL 1  // K-quants too: split K while the doubled grid fits one round of waves
                        // and keeps 4 units per wave (16384 x 4096: 11.7 -> 9.1 us)
#endif
#ifndef GGUF_M1_ROWS
#define GGUF_M1_ROWS 1  // spread rows evenly over the CUs when the tiles do not divide
#endif
constexpr int kM1Cus = 256;  // compute units of the MI355X
#ifndef GGUF_M1_ROUND_WAVES
#define GGUF_M1_ROUND_WAVES 2048  // waves resident at once (256 CUs x 8)
#endif
template <int TYPE>
constexpr int m1_umax(bool tight) {
  // 32-element blocks: up to 64 per wave (K = 16384 over 8 waves); past 32 at
  // most GGUF_M1_DEEP are in flight (m1_depth), so the register cost stays small
  return (TYPE == 8 || is_b32(TYPE)) ? 64 : (TYPE == 14 || TYPE == 13 || is_iq(TYPE) || tight ? 8 : 16);
}

#ifndef GGUF_M1_DEEP
#define GGUF_M1_DEEP 8  // units in flight of a wave holding more than 32 small blocks
#endif
// Units in flight per wave for a grid of `waves` waves holding `per` units
// of `unit_bytes` each: about 12 MB over the chip when the grid is one round
// (at most 2048 resident waves), one unit when later rounds stream in behind
// the first anyway.  0 = all of them (the transfer is small enough to issue
// at once).
#ifndef GGUF_M1_FLIGHT_MB
#define GGUF_M1_FLIGHT_MB 12.0
#endif
constexpr double kM1Flight = GGUF_M1_FLIGHT_MB * 1024 * 1024;
inline int m1_depth(int waves, int per, int unit_bytes) {
  if (waves > 2 * 2048) return 1;
  const int resident = waves < 2048 ? waves : 2048;
  const int d = (int)(kM1Flight / ((double)resident * unit_bytes) + 0.5);
  if (d < 1) return 1;
  if (per > 32)  // 32-element blocks only: never all in registers, a deep window instead
    return d > 3 ? GGUF_M1_DEEP : d;
  if (d > 3 || d >= per) return 0;
  return d;
}

// Returns hipErrorNotSupported (nothing launched) when K is beyond the
// one-shot staging (16384) or the units per wave exceed the register budget.
template <int TYPE, typename XT, int PRO>
hipError_t launch_m1(const XT *x, const uint8_t *W, int N, int K, float *y, const float *pw,
                     float eps, int epi, const AttnRecords &ar, hipStream_t s) {
  constexpr int UE = Fmt<TYPE>::UE, GS = Dec<TYPE>::GS;
  constexpr int PARTS = sizeof(XT) == 4 ? 2 : 1;
  const int ntiles = (N + 15) / 16, nu = K / UE;
  if (K > 16384) return hipErrorNotSupported;
  const bool long_k = K > 4096;
  const int umax = m1_umax<TYPE>(long_k || (PRO != 0 && GGUF_M1_PRO_TIGHT));
  // K split: units per wave within the budget, and at least ~1024 waves when
  // possible (at most 4 with the SwiGLU epilogue, which needs two tiles per workgroup);
  // 32-element blocks (one MFMA per unit, latency-bound) split further while the
  // grid stays one round of resident waves (Q8_0 4096 x 4096: 7.5 -> 6.4 us), and
  // so do the K-quants while each wave keeps at least 4 units
  int ks = 1;
  const int ks_max = epi == 2 ? 4 : 8;
  while (ks < ks_max && ks < nu &&
         ((nu + ks - 1) / ks > umax || ntiles * ks < GGUF_M1_MIN_WAVES ||
          (UE == 32 && 2 * ntiles * ks <= GGUF_M1_ROUND_WAVES) ||
          (GGUF_M1_FILL && 2 * ntiles * ks <= GGUF_M1_ROUND_WAVES && nu >= 8 * ks)))
    ks <<= 1;
  // 2- and 3-bit K-quants: the most VALU per byte, and a wave's units decode
  // one after another on its own dependency chain, so one more K split while
  // the grid stays under 4096 waves and every wave keeps 4 units (14336 x
  // 4096: Q2_K 2193 -> 2384 GB/s, Q3_K 2432 -> 2646; IQ4_XS lost 4% with it,
  // and 2 units per wave lost a third)
  if (TYPE == 10 || TYPE == 11)
    while (ks < ks_max && ks < nu && ntiles * ks < 4096 && nu >= 8 * ks) ks <<= 1;
  const int per = (nu + ks - 1) / ks;
  if (per > umax) return hipErrorNotSupported;
  // 8 waves per workgroup (half as many workgroups staging the activations)
  // once the grid keeps at least 192 of them; smaller grids keep 4 so that
  // every CU gets a workgroup
  int nw = (long_k || ks > 4 || GGUF_M1_NW_MIN > 4 || ntiles * ks >= 1536) ? 8 : 4;
  if (epi == 2 && nw / ks < 2) nw = 8;  // the SwiGLU epilogue pairs tiles 2m, 2m + 1
  const int nthr = 64 * nw, ts = nw / ks;
  if (epi == 2 && (ts < 2 || (ntiles & 1))) return hipErrorNotSupported;
  const int xi = (K / kItem + nthr - 1) / nthr;  // 1 or 2
  size_t lds = (size_t)(K + kXPad) * 2 * PARTS + (size_t)(K / GS + K / UE) * 4 +
               (size_t)nw * 64 * 4 + kZeroHalves * 2 + (size_t)nthr * 4;
  if constexpr (is_iq(TYPE)) lds = ((lds + 15) & ~(size_t)15) + iq_tbl_bytes<TYPE>();
  if (lds > kMaxLds) return hipErrorNotSupported;
  // Rows per workgroup instead of whole tiles when the tiles leave more than a
  // fifth of the CUs without a workgroup (6144 or 12288 rows: 192 workgroups
  // on 256 CUs): a multiple of 8 rows each, so that the bytes per CU are even
  // (6144 x 4096: 6.02 -> 5.55 us, 12288 x 4096: 9.60 -> 7.97 us).  At 224 of
  // 256 (14336 rows) it measured no faster, and the tile layout stays.
  unsigned groups = (unsigned)((ntiles + ts - 1) / ts);
  int rows_wg = 0;
  if (GGUF_M1_ROWS && epi != 2 && 5 * groups < 4u * kM1Cus) {
    const int R = 8 * ((N + 8 * kM1Cus - 1) / (8 * kM1Cus));
    if ((R + 15) / 16 <= ts) {
      rows_wg = R;
      groups = (unsigned)((N + R - 1) / R);
    }
  }
  const dim3 grid(groups), block(nthr);
  int dp = m1_depth(grid.x * nw, per, Fmt<TYPE>::TU);
  if (is_iq(TYPE) && (dp == 0 || dp > 3)) dp = 3;  // the IQ records are large: 3 in flight at most
  // template U is clamped to the compile-time budget (runtime per <= umax already);
  // above 64 KB of dynamic LDS the kernel's limit is raised first (gfx950: 160 KB)
#define GGUF_M1_K(UU, XX, DD)                                                                    \
  do {                                                                                           \
    auto kern = decode_m1_kernel<TYPE, XT,                                                       \
                                 ((UU) < m1_umax<TYPE>((XX) > 1 || (PRO != 0 && GGUF_M1_PRO_TIGHT)) \
                                      ? (UU)                                                     \
                                      : m1_umax<TYPE>((XX) > 1 || (PRO != 0 && GGUF_M1_PRO_TIGHT))), \
                                 XX, PRO, DD>;                                                   \
    if (lds > 65536) {                                                                           \
      const hipError_t ea = hipFuncSetAttribute((const void *)kern,                              \
                                                hipFuncAttributeMaxDynamicSharedMemorySize,      \
                                                (int)lds);                                       \
      if (ea != hipSuccess) return ea;                                                           \
    }                                                                                            \
    hipLaunchKernelGGL(kern, grid, block, lds, s, x, W, N, K, y, ks, pw, eps, epi, ar, rows_wg); \
  } while (0)
#define GGUF_M1(UU, XX)                                                                          \
  do {                                                                                           \
    if (dp == 1) GGUF_M1_K(UU, XX, 1);                                                           \
    else if (dp == 2) GGUF_M1_K(UU, XX, 2);                                                      \
    else if (dp == 3) GGUF_M1_K(UU, XX, 3);                                                      \
    else if (dp == GGUF_M1_DEEP)                                                                 \
      GGUF_M1_K(UU, XX, ((UU) == 64 && Fmt<TYPE>::UE == 32 ? GGUF_M1_DEEP : is_iq(TYPE) ? 3 : 0)); \
    else GGUF_M1_K(UU, XX, (is_iq(TYPE) ? 3 : 0));  /* IQ: never all units at once */          \
  } while (0)
  if (xi <= 1) {
    if (per <= 4) GGUF_M1(4, 1);
    else if (per <= 8) GGUF_M1(8, 1);
    else if (per <= 16) GGUF_M1(16, 1);
    else if (per <= 32) GGUF_M1(32, 1);
    else GGUF_M1(64, 1);
  } else if constexpr (PRO != 3) {
    if (per <= 4) GGUF_M1(4, 2);
    else if (per <= 8) GGUF_M1(8, 2);
    else if (per <= 16) GGUF_M1(16, 2);
    else if (per <= 32) GGUF_M1(32, 2);
    else GGUF_M1(64, 2);
  } else {
    return hipErrorNotSupported;  // the merge prologue holds one item per thread
  }
#undef GGUF_M1
#undef GGUF_M1_K
  return hipGetLastError();
}

template <int TYPE, typename XT>
hipError_t launch_m(const XT *x, int64_t ldx, const uint8_t *W, int N, int K, float *y,
                    int64_t ldy, int M, float *work, int64_t work_floats, hipStream_t s) {
  if (M == 1) {
    const hipError_t e = launch_m1<TYPE, XT, 0>(x, W, N, K, y, nullptr, 0.f, 0, AttnRecords{}, s);
    if (e != hipErrorNotSupported) return e;
  }
  if constexpr (TYPE == 12 || TYPE == 14 || TYPE == 8) {  // the batched kernel (decode_mk.hpp)
    const hipError_t e = launch_mk<TYPE, XT>(x, ldx, W, N, K, y, ldy, M, work, work_floats, s);
    if (e != hipErrorNotSupported) return e;
  }
  if (M <= 16) return launch_mb<TYPE, XT, 1>(x, ldx, W, N, K, y, ldy, M, work, work_floats, s);
  return launch_mb<TYPE, XT, 2>(x, ldx, W, N, K, y, ldy, M, work, work_floats, s);
}

}  // namespace

// Per-type entry points of the decode kernels; each ggml type is compiled in
// a translation unit of its own (decode_<type>.hip) that expands this macro.
#define GGUF_DECODE_DEFINE(T, NAME)                                                              \
  hipError_t decode_##NAME(const void *x, int x_type, int64_t ldx, const uint8_t *tiles, int n,  \
                           int k, float *y, int64_t ldy, int m, float *work, int64_t work_floats, \
                           hipStream_t s) {                                                      \
    return x_type == 0 ? launch_m<T, float>((const float *)x, ldx, tiles, n, k, y, ldy, m, work, \
                                            work_floats, s)                                      \
                       : launch_m<T, half_t>((const half_t *)x, ldx, tiles, n, k, y, ldy, m,     \
                                             work, work_floats, s);                              \
  }                                                                                              \
  int64_t decode_work_##NAME(int x_type, int n, int k, int m) {                                  \
    return x_type == 0 ? mb_work_floats<T, float>(m, n, k) : mb_work_floats<T, half_t>(m, n, k); \
  }                                                                                              \
  hipError_t decode_fused_##NAME(const float *x, const uint8_t *tiles, int n, int k, float *y,   \
                                 int prologue, const float *pw, float eps, int epi,              \
                                 hipStream_t s) {                                                \
    return prologue == 1   ? launch_m1<T, float, 1>(x, tiles, n, k, y, pw, eps, epi,             \
                                                    AttnRecords{}, s)                            \
           : prologue == 2 ? launch_m1<T, float, 2>(x, tiles, n, k, y, pw, eps, epi,             \
                                                    AttnRecords{}, s)                            \
                           : launch_m1<T, float, 0>(x, tiles, n, k, y, pw, eps, epi,             \
                                                    AttnRecords{}, s);                           \
  }                                                                                              \
  hipError_t decode_merge_##NAME(const AttnRecords &ar, const uint8_t *tiles, int n, float *y,   \
                                 int epi, hipStream_t s) {                                       \
    return launch_m1<T, float, 3>(nullptr, tiles, n, ar.nh * ar.hd, y, nullptr, 0.f, epi, ar, s); \
  }

// The grid-codebook IQ types: the one-shot kernel for M = 1 (K <= 16384), the
// batched kernel (decode_mk.hpp) for M >= 2 when the caller's workspace holds
// its image and partial sums; without one (K <= 16384) the one-shot kernel
// runs once per activation row, which needs no workspace.  K > 16384 always
// takes the batched kernel (hipErrorNotSupported without a workspace, before
// anything is launched).  The fused prologue / epilogue and merge kernels are
// the one-shot kernel's, as for the other types.
template <int TYPE, typename XT>
hipError_t launch_iq(const XT *x, int64_t ldx, const uint8_t *W, int N, int K, float *y,
                     int64_t ldy, int M, float *work, int64_t work_floats, hipStream_t s) {
  if (M == 1) {
    const hipError_t e = launch_m1<TYPE, XT, 0>(x, W, N, K, y, nullptr, 0.f, 0, AttnRecords{}, s);
    if (e != hipErrorNotSupported) return e;
  }
  hipError_t e = launch_mk<TYPE, XT>(x, ldx, W, N, K, y, ldy, M, work, work_floats, s);
  if (e != hipErrorNotSupported) return e;
  for (int m = 0; m < M; ++m) {  // row 0 answers NotSupported before anything is launched
    e = launch_m1<TYPE, XT, 0>(x + (int64_t)m * ldx, W, N, K, y + (int64_t)m * ldy, nullptr, 0.f, 0,
                               AttnRecords{}, s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}
#define GGUF_DECODE_DEFINE_IQ(T, NAME)                                                           \
  hipError_t decode_##NAME(const void *x, int x_type, int64_t ldx, const uint8_t *tiles, int n,  \
                           int k, float *y, int64_t ldy, int m, float *work, int64_t work_floats, \
                           hipStream_t s) {                                                      \
    return x_type == 0 ? launch_iq<T, float>((const float *)x, ldx, tiles, n, k, y, ldy, m, work, \
                                             work_floats, s)                                     \
                       : launch_iq<T, half_t>((const half_t *)x, ldx, tiles, n, k, y, ldy, m,    \
                                              work, work_floats, s);                             \
  }                                                                                              \
  int64_t decode_work_##NAME(int x_type, int n, int k, int m) {                                  \
    const size_t b = x_type == 0 ? mk_work_bytes<T, float>(m, n, k) : mk_work_bytes<T, half_t>(m, n, k); \
    return (int64_t)((b + 3) / 4);                                                               \
  }                                                                                              \
  hipError_t decode_fused_##NAME(const float *x, const uint8_t *tiles, int n, int k, float *y,   \
                                 int prologue, const float *pw, float eps, int epi,              \
                                 hipStream_t s) {                                                \
    return prologue == 1   ? launch_m1<T, float, 1>(x, tiles, n, k, y, pw, eps, epi,             \
                                                    AttnRecords{}, s)                            \
           : prologue == 2 ? launch_m1<T, float, 2>(x, tiles, n, k, y, pw, eps, epi,             \
                                                    AttnRecords{}, s)                            \
                           : launch_m1<T, float, 0>(x, tiles, n, k, y, pw, eps, epi,             \
                                                    AttnRecords{}, s);                           \
  }                                                                                              \
  hipError_t decode_merge_##NAME(const AttnRecords &ar, const uint8_t *tiles, int n, float *y,   \
                                 int epi, hipStream_t s) {                                       \
    return launch_m1<T, float, 3>(nullptr, tiles, n, ar.nh * ar.hd, y, nullptr, 0.f, epi, ar, s); \
  }

}  // namespace gguf
