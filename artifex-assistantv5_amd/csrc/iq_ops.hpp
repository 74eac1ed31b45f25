// Arithmetic of the grid-codebook IQ types on the matrix cores, shared by the
// decode kernels and the GEMM: the shared-memory tables (the grid as f16 and
// the sign masks), the exact f16 B operand of one sub-block and group, and the
// unit scales.  The caller passes the tables' shared-memory address.
#pragma once

#include "common.hpp"
#include "iq.hpp"

namespace gguf {

template <int TYPE>
struct IqTab {
  static constexpr int NG = TYPE == 16 ? 256 : TYPE == 17 ? 512 : TYPE == 22 ? 1024
                          : TYPE == 18 ? 256 : TYPE == 21 ? 512 : 2048;
  static constexpr int W = (TYPE == 18 || TYPE == 21) ? 4 : 8;
  static constexpr int NS = TYPE == 29 ? 0 : (TYPE == 22 || TYPE == 21) ? 256 : 128;
  static constexpr bool KS = TYPE == 16 || TYPE == 17 || TYPE == 18;
  static constexpr int GB = NG * W * 2;  // grid bytes (the masks follow)
};
template <int TYPE>
constexpr int iq_tbl_bytes() {
  if constexpr (is_iq(TYPE)) return IqTab<TYPE>::GB + IqTab<TYPE>::NS * 16;
  return 0;
}

// ---------------------------------------------------------------------------
// The B operand of sub-block ib for lane group g
// (elements 8 g .. 8 g + 7, group l = g of the format) is the grid entry's
// magnitudes with the signs applied (an XOR of f16 sign bits) times the
// group's odd sub-block factor f (2 ls + 1, 2 s + 1): exact f16 integers
// (at most 43 x 31, 62 x 31, 15 x 31, 9 x 15).  The unit scale (d / 8, d / 4
// or d) is applied to the f32 result.
// ---------------------------------------------------------------------------
template <int TYPE>
struct IqUnit {
  uint32_t w[iq_rd<TYPE>()];  // the row's record (the block without its d)
  uint32_t d;                 // the f16 d (types that have one)
};
template <int TYPE>
__device__ __forceinline__ const void *iq_grid() {
  if constexpr (TYPE == 16) return kIq2xxsGrid;
  if constexpr (TYPE == 17) return kIq2xsGrid;
  if constexpr (TYPE == 22) return kIq2sGrid;
  if constexpr (TYPE == 18) return kIq3xxsGrid;
  if constexpr (TYPE == 21) return kIq3sGrid;
  return kIq1sGrid;
}
// Table loads (16 grid bytes per chunk, at most CH chunks per thread), requested
// with the other loads; written to shared memory by iq_put_tables.
template <int TYPE, int NT>
struct IqTabRegs {
  static constexpr int CHUNKS = is_iq(TYPE) ? IqTab<TYPE>::NG * IqTab<TYPE>::W / 16 : 0;
  static constexpr int CH = (CHUNKS + NT - 1) / NT;
  uint4 v[CH > 0 ? CH : 1];
};
template <int TYPE, int NT>
__device__ __forceinline__ void iq_get_tables(IqTabRegs<TYPE, NT> &t) {
  using R = IqTabRegs<TYPE, NT>;
  const uint4 *src = (const uint4 *)iq_grid<TYPE>();
#pragma unroll
  for (int c = 0; c < R::CH; ++c) t.v[c] = src[min((int)threadIdx.x + NT * c, R::CHUNKS - 1)];
}
template <int TYPE, int NT>
__device__ __forceinline__ void iq_put_tables(const IqTabRegs<TYPE, NT> &t, unsigned char *tb) {
  using R = IqTabRegs<TYPE, NT>;
  using Q = IqTab<TYPE>;
#pragma unroll
  for (int c = 0; c < R::CH; ++c) {
    const int q = (int)threadIdx.x + NT * c;
    if (q < R::CHUNKS) {
      const uint32_t b[4] = {t.v[c].x, t.v[c].y, t.v[c].z, t.v[c].w};
      half8_t h[2];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const uint32_t byte = (b[i >> 2] >> (8 * (i & 3))) & 0xFFu;
        h[i >> 3][i & 7] = TYPE == 29 ? (half_t)(8.f * (float)(int8_t)byte) : (half_t)(float)byte;
      }
      *(half8_t *)(tb + 32 * q) = h[0];
      *(half8_t *)(tb + 32 * q + 16) = h[1];
    }
  }
  // sign masks: entry e, bit j of its sign byte (ksigns[e] = e with bit 7 making
  // the popcount even, or e itself) -> 0x8000 in half j
  for (int q = threadIdx.x; q < Q::NS; q += NT) {
    const uint32_t sb = Q::KS ? (uint32_t)q | ((__builtin_popcount(q) & 1u) << 7) : (uint32_t)q;
    uint32_t m[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) m[i] = (((sb >> (2 * i)) & 1u) << 15) | (((sb >> (2 * i + 1)) & 1u) << 31);
    *(uint4 *)(tb + Q::GB + 16 * q) = make_uint4(m[0], m[1], m[2], m[3]);
  }
}

__device__ __forceinline__ uint32_t iq_byte(uint32_t w, int i) { return __builtin_amdgcn_ubfe(w, 8 * i, 8); }
// a0 for lane groups 0, 1 and a1 for 2, 3, selected as values (a select of the
// two array elements' addresses keeps the record out of registers)
__device__ __forceinline__ uint32_t pick2(uint32_t a0, uint32_t a1, int g) { return (g & 2) ? a1 : a0; }

// The B operand of sub-block ib for lane group g, and (scale) the f32 factor
// of the unit.
// Types whose odd factor is one per sub-block (not per pair of groups).
template <int TYPE>
constexpr bool iq_block_factor() {
  return TYPE == 16 || TYPE == 18 || TYPE == 21;
}
// Those factors of sub-blocks 2g and 2g + 1 (the rows lane group g holds), as
// f32 integers; the words are picked with selects (no indexing by g).
__device__ __forceinline__ uint32_t sel4(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3, int g) {
  return (g & 2) ? ((g & 1) ? a3 : a2) : ((g & 1) ? a1 : a0);
}
template <int TYPE>
__device__ __forceinline__ void iq_factors(const IqUnit<TYPE> &u, int g, float &f0, float &f1) {
  uint32_t l0, l1;
  if constexpr (TYPE == 16) {  // ls in the top nibble of word 2 ib + 1
    l0 = sel4(u.w[1], u.w[5], u.w[9], u.w[13], g) >> 28;
    l1 = sel4(u.w[3], u.w[7], u.w[11], u.w[15], g) >> 28;
  } else if constexpr (TYPE == 18) {  // ls in the top nibble of word 16 + ib
    l0 = sel4(u.w[16], u.w[18], u.w[20], u.w[22], g) >> 28;
    l1 = sel4(u.w[17], u.w[19], u.w[21], u.w[23], g) >> 28;
  } else {  // IQ3_S: scale byte g, low nibble for the even sub-block
    const uint32_t sc = iq_byte(u.w[26], g);
    l0 = sc & 15u;
    l1 = sc >> 4;
  }
  f0 = (float)(2u * l0 + 1u);
  f1 = (float)(2u * l1 + 1u);
}

// FACTOR false (iq_block_factor types only): the operand without the odd
// factor, which the caller applies to the sub-block's f32 result.
template <int TYPE, bool FACTOR = true>
__device__ __forceinline__ half8_t iq_b(const IqUnit<TYPE> &u, int ib, int g, const unsigned char *tb) {
  using Q = IqTab<TYPE>;
  uint32_t idx0, idx1 = 0, sidx = 0, f;
  half2_t delta = {(half_t)0.f, (half_t)0.f};
  if constexpr (TYPE == 16) {  // IQ2_XXS: (4 index bytes, u32 7-bit sign indices | ls << 28)
    const uint32_t aux1 = u.w[2 * ib + 1];
    idx0 = iq_byte(u.w[2 * ib], g);
    sidx = __builtin_amdgcn_ubfe(aux1, 7 * g, 7);
    f = 2u * (aux1 >> 28) + 1u;
  } else if constexpr (TYPE == 17) {  // IQ2_XS: u16 (9-bit index | 7-bit sign index); scales
    const uint32_t q = (pick2(u.w[2 * ib], u.w[2 * ib + 1], g) >> (16 * (g & 1))) & 0xFFFFu;
    const uint32_t sc = iq_byte(u.w[16 + (ib >> 2)], ib & 3);
    idx0 = q & 511u;
    sidx = q >> 9;
    f = 2u * (g < 2 ? sc & 15u : sc >> 4) + 1u;
  } else if constexpr (TYPE == 22) {  // IQ2_S: qs[32] | signs[32] | qh[8] | scales[8]
    const uint32_t qh = iq_byte(u.w[16 + (ib >> 2)], ib & 3), sc = iq_byte(u.w[18 + (ib >> 2)], ib & 3);
    idx0 = iq_byte(u.w[ib], g) | ((qh << (8 - 2 * g)) & 0x300u);
    sidx = iq_byte(u.w[8 + ib], g);
    f = 2u * (g < 2 ? sc & 15u : sc >> 4) + 1u;
  } else if constexpr (TYPE == 18) {  // IQ3_XXS: qs[64] | u32 (7-bit sign indices | ls << 28)
    const uint32_t q = pick2(u.w[2 * ib], u.w[2 * ib + 1], g) >> (16 * (g & 1)), aux = u.w[16 + ib];
    idx0 = q & 0xFFu;
    idx1 = (q >> 8) & 0xFFu;
    sidx = __builtin_amdgcn_ubfe(aux, 7 * g, 7);
    f = 2u * (aux >> 28) + 1u;
  } else if constexpr (TYPE == 21) {  // IQ3_S: qs[64] | qh[8] | signs[32] | scales[4]
    const uint32_t q = pick2(u.w[2 * ib], u.w[2 * ib + 1], g) >> (16 * (g & 1));
    const uint32_t qh = iq_byte(u.w[16 + (ib >> 2)], ib & 3), sc = iq_byte(u.w[26], ib >> 1);
    idx0 = (q & 0xFFu) | ((qh << (8 - 2 * g)) & 256u);
    idx1 = ((q >> 8) & 0xFFu) | ((qh << (7 - 2 * g)) & 256u);
    sidx = iq_byte(u.w[18 + ib], g);
    f = 2u * ((ib & 1) ? sc >> 4 : sc & 15u) + 1u;
  } else {  // IQ1_M: qs[32] | qh[16] | scales[4] u16
    const uint32_t qh = iq_byte(u.w[8 + (ib >> 1)], 2 * (ib & 1) + (g >> 1));
    const uint32_t wk = (u.w[12 + (ib >> 2)] >> (16 * ((ib >> 1) & 1))) & 0xFFFFu;
    const int sh = 6 * (ib & 1) + (g < 2 ? 0 : 3);
    idx0 = iq_byte(u.w[ib], g) | ((qh << ((g & 1) ? 4 : 8)) & 0x700u);
    f = 2u * ((wk >> sh) & 7u) + 1u;
    const half_t dl = (qh & ((g & 1) ? 0x80u : 0x08u)) ? (half_t)-1.f : (half_t)1.f;  // 8 x (+-1/8)
    delta = {dl, dl};
  }
  const half_t fh = (half_t)(float)f;
  const half2_t fp = {fh, fh};
  uint32_t v[4];
  const uint32_t ta = lds_addr32(tb);  // entry i at ta + entry bytes * i: one shift-add each
  if constexpr (Q::W == 8) {
    const uint4 gr = lds_ld<uint4>(ta + 16 * idx0);
    v[0] = gr.x; v[1] = gr.y; v[2] = gr.z; v[3] = gr.w;
  } else {
    const uint2 g1 = lds_ld<uint2>(ta + 8 * idx0), g2 = lds_ld<uint2>(ta + 8 * idx1);
    v[0] = g1.x; v[1] = g1.y; v[2] = g2.x; v[3] = g2.y;
  }
  if constexpr (Q::NS > 0) {
    const uint4 m = lds_ld<uint4>(ta + Q::GB + 16 * sidx);
    v[0] ^= m.x; v[1] ^= m.y; v[2] ^= m.z; v[3] ^= m.w;
  }
  half8_t b;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const half2_t h = __builtin_bit_cast(half2_t, v[i]);
    const half2_t r = TYPE == 29 ? __builtin_elementwise_fma(h, fp, delta * fp) : FACTOR ? h * fp : h;
    b[2 * i] = r[0];
    b[2 * i + 1] = r[1];
  }
  return b;
}
template <int TYPE>
__device__ __forceinline__ float iq_unit_scale(const IqUnit<TYPE> &u) {
  if constexpr (TYPE == 29) {
    const uint32_t s01 = u.w[12], s23 = u.w[13];
    const uint32_t bits = ((s01 >> 12) & 0x000Fu) | ((s01 >> 24) & 0x00F0u) | ((s23 >> 4) & 0x0F00u) |
                          ((s23 >> 16) & 0xF000u);
    return h2f(bits) * 0.125f;
  }
  return h2f(u.d) * (TYPE == 18 ? 0.25f : TYPE == 21 ? 1.f : 0.125f);
}

}  // namespace gguf
