// The grid-codebook IQ types: IQ2_XXS (16), IQ2_XS (17), IQ3_XXS (18),
// IQ3_S (21), IQ2_S (22), IQ1_M (29).  256-element superblocks whose values
// are d * (sub-block factor) * grid[index][j] * sign (IQ1_M: d * (2 s + 1) *
// (grid[index][j] +- 1/8)), decoded as the reference's CPU dequant does
// (webgpu/src/model/gguf-dequant.ts:406-672).
//
// Row-tile layout (tile unit of 16 rows, 16 * block bytes, nothing added):
//   types with an f16 d in bytes 0-1 of the block:
//     [0, 32)                     d of row r at 2 r
//     [32, 32 + 16 (BS - 2))      the rest of row r's block (bytes 2 .. BS - 1)
//                                 at 32 + r (BS - 2), as stored (4-byte aligned)
//   IQ1_M (no d field):           row r's block at 56 r
// A lane that decodes row r loads the row's whole rest as words (IqFmt::RD).
#pragma once

#include "common.hpp"
#include "iq_tables.hpp"

namespace gguf {

__host__ __device__ constexpr bool is_iq(int t) {
  return t == 16 || t == 17 || t == 18 || t == 21 || t == 22 || t == 29;
}

template <int TYPE>
struct IqFmt;
template <>
struct IqFmt<16> {  // IQ2_XXS: qs[8 groups x (4 index bytes, u32 signs/scale)]
  static constexpr int BS = 66, HASD = 1;
};
template <>
struct IqFmt<17> {  // IQ2_XS: qs[32] u16 (9-bit index | 7-bit sign index), scales[8]
  static constexpr int BS = 74, HASD = 1;
};
template <>
struct IqFmt<22> {  // IQ2_S: qs[32], signs[32], qh[8], scales[8]
  static constexpr int BS = 82, HASD = 1;
};
template <>
struct IqFmt<18> {  // IQ3_XXS: qs[64], scales_and_signs[8] u32
  static constexpr int BS = 98, HASD = 1;
};
template <>
struct IqFmt<21> {  // IQ3_S: qs[64], qh[8], signs[32], scales[4]
  static constexpr int BS = 110, HASD = 1;
};
template <>
struct IqFmt<29> {  // IQ1_M: qs[32], qh[16], scales[4] u16 (the f16 d in their top nibbles)
  static constexpr int BS = 56, HASD = 0;
};
// words of a row's record (the block without its d) and its offset in the tile unit
template <int TYPE>
constexpr int iq_rd() {
  return (IqFmt<TYPE>::BS - 2 * IqFmt<TYPE>::HASD) / 4;
}
template <int TYPE>
__host__ __device__ constexpr int iq_rec_off(int r) {
  return IqFmt<TYPE>::HASD ? 32 + r * (IqFmt<TYPE>::BS - 2) : r * IqFmt<TYPE>::BS;
}

// Byte o of row r's raw block, read from a tile unit.
template <int TYPE>
__device__ __forceinline__ uint32_t iq_tile_byte(const uint8_t *tu, int r, int o) {
  if constexpr (IqFmt<TYPE>::HASD) return o < 2 ? tu[2 * r + o] : tu[iq_rec_off<TYPE>(r) + o - 2];
  return tu[iq_rec_off<TYPE>(r) + o];
}

// Values 32 ib .. 32 ib + 31 of a superblock whose raw byte o is byte(o).
// Every value is exact in f32 (a d of 11 significant bits times a factor of
// at most 5 and a grid magnitude of at most 6), so the order of the products
// does not matter: bit-exact to the reference.
template <int TYPE, typename Byte>
__device__ __forceinline__ void iq_piece(const Byte &byte, int ib, float *o) {
  auto u16 = [&](int off) { return byte(off) | (byte(off + 1) << 8); };
  auto u32 = [&](int off) { return u16(off) | (u16(off + 2) << 16); };
  if constexpr (TYPE == 16) {  // gguf-dequant.ts:406-431
    const float d = h2f(u16(0));
    const int g = 2 + 8 * ib;
    const uint32_t aux1 = u32(g + 4);
    const float db = d * (0.5f + (float)(aux1 >> 28)) * 0.25f;
    for (int l = 0; l < 4; ++l) {
      const uint32_t idx = byte(g + l), sg = kKsigns[(aux1 >> (7 * l)) & 127u];
      for (int j = 0; j < 8; ++j)
        o[8 * l + j] = db * (float)kIq2xxsGrid[8 * idx + j] * (((sg >> j) & 1u) ? -1.f : 1.f);
    }
  } else if constexpr (TYPE == 17) {  // :440-470
    const float d = h2f(u16(0));
    const uint32_t sc = byte(66 + ib);
    const float db0 = d * (0.5f + (float)(sc & 15u)) * 0.25f, db1 = d * (0.5f + (float)(sc >> 4)) * 0.25f;
    for (int l = 0; l < 4; ++l) {
      const uint32_t q = u16(2 + 2 * (4 * ib + l)), idx = q & 511u, sg = kKsigns[q >> 9];
      for (int j = 0; j < 8; ++j)
        o[8 * l + j] = (l < 2 ? db0 : db1) * (float)kIq2xsGrid[8 * idx + j] * (((sg >> j) & 1u) ? -1.f : 1.f);
    }
  } else if constexpr (TYPE == 22) {  // :621-648
    const float d = h2f(u16(0));
    const uint32_t sc = byte(74 + ib), qh = byte(66 + ib);
    const float db0 = d * (0.5f + (float)(sc & 15u)) * 0.25f, db1 = d * (0.5f + (float)(sc >> 4)) * 0.25f;
    for (int l = 0; l < 4; ++l) {
      const uint32_t idx = byte(2 + 4 * ib + l) | ((qh << (8 - 2 * l)) & 0x300u), sg = byte(34 + 4 * ib + l);
      for (int j = 0; j < 8; ++j)
        o[8 * l + j] = (l < 2 ? db0 : db1) * (float)kIq2sGrid[8 * idx + j] * (((sg >> j) & 1u) ? -1.f : 1.f);
    }
  } else if constexpr (TYPE == 18) {  // :532-561
    const float d = h2f(u16(0));
    const uint32_t aux = u32(66 + 4 * ib);
    const float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
    for (int l = 0; l < 4; ++l) {
      const uint32_t sg = kKsigns[(aux >> (7 * l)) & 127u];
      const uint32_t g1 = byte(2 + 8 * ib + 2 * l), g2 = byte(2 + 8 * ib + 2 * l + 1);
      for (int j = 0; j < 4; ++j) {
        o[8 * l + j] = db * (float)kIq3xxsGrid[4 * g1 + j] * (((sg >> j) & 1u) ? -1.f : 1.f);
        o[8 * l + 4 + j] = db * (float)kIq3xxsGrid[4 * g2 + j] * (((sg >> (j + 4)) & 1u) ? -1.f : 1.f);
      }
    }
  } else if constexpr (TYPE == 21) {  // :569-613 (sub-block ib = 2 p + half)
    const float d = h2f(u16(0));
    const uint32_t sc = byte(106 + (ib >> 1)), qh = byte(66 + ib);
    const float db = d * (float)(1u + 2u * ((ib & 1) ? (sc >> 4) : (sc & 15u)));
    for (int l = 0; l < 4; ++l) {
      const uint32_t g1 = byte(2 + 8 * ib + 2 * l) | ((qh << (8 - 2 * l)) & 256u);
      const uint32_t g2 = byte(2 + 8 * ib + 2 * l + 1) | ((qh << (7 - 2 * l)) & 256u);
      const uint32_t sg = byte(74 + 4 * ib + l);
      for (int j = 0; j < 4; ++j) {
        o[8 * l + j] = db * (float)kIq3sGrid[4 * g1 + j] * (((sg >> j) & 1u) ? -1.f : 1.f);
        o[8 * l + 4 + j] = db * (float)kIq3sGrid[4 * g2 + j] * (((sg >> (j + 4)) & 1u) ? -1.f : 1.f);
      }
    }
  } else {  // 29, IQ1_M, :478-524
    const uint32_t s0 = u16(48), s1 = u16(50), s2 = u16(52), s3 = u16(54);
    const float d = h2f(((s0 >> 12) | ((s1 >> 8) & 0x00F0u) | ((s2 >> 4) & 0x0F00u) | (s3 & 0xF000u)) & 0xFFFFu);
    const uint32_t w = (ib >> 1) == 0 ? s0 : (ib >> 1) == 1 ? s1 : (ib >> 1) == 2 ? s2 : s3;
    const int sh = 6 * (ib & 1);
    const float dl1 = d * (float)(2u * ((w >> sh) & 7u) + 1u), dl2 = d * (float)(2u * ((w >> (sh + 3)) & 7u) + 1u);
    const uint32_t qh0 = byte(32 + 2 * ib), qh1 = byte(33 + 2 * ib);
    for (int l = 0; l < 4; ++l) {
      const uint32_t qh = l < 2 ? qh0 : qh1;
      const uint32_t idx = byte(4 * ib + l) | ((qh << ((l & 1) ? 4 : 8)) & 0x700u);
      const float delta = (qh & ((l & 1) ? 0x80u : 0x08u)) ? -0.125f : 0.125f;
      for (int j = 0; j < 8; ++j) o[8 * l + j] = (l < 2 ? dl1 : dl2) * ((float)kIq1sGrid[8 * idx + j] + delta);
    }
  }
}

}  // namespace gguf
