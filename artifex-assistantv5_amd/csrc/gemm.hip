// MFMA dequant-GEMM for prefill: y[m, n] = sum_k x[m, k] * dequant(W)[n, k].
//
// The reference has no GEMM for these types: prefill re-runs its GEMV once
// per activation row (webgpu/src/engine/forward-pass.ts:1536-1539).
//
// A workgroup of eight waves owns a 128 x 256 output tile; wave w owns all 128
// rows and the 32 columns [32 w, 32 w + 32) (two row tiles of the weight), so
// no two waves need the same weight bytes and one staged activation tile
// feeds 256 columns.  K is walked in 64-wide steps:
//
//   weights      the row-tile layout (common.hpp) hands lane (r, g) exactly
//                the 8 consecutive k of row r that form its operand of
//                v_mfma_f32_16x16x32_f16, so each wave dequantizes its weight
//                bytes straight into MFMA B registers.  A quant code enters
//                as an f16 subnormal (code x 2^-24, exact) and one
//                v_fma_mix computes fp16(d*sc*q - dmin*m) with f32 internals:
//                the exact f32 dequant value rounded once to fp16.
//   activations  staged through LDS as fp16, two buffers, rows of 128 B whose
//                16-byte chunks are rotated by the row index so that fragment
//                reads and row writes are free of bank conflicts.  f32 input
//                is scaled per row by the power of two 2^e that puts the row's
//                largest magnitude in [2^14, 2^15) (a pass over the block's
//                rows before the K loop), rounded to fp16, and the row's
//                outputs take 2^-e: any f32 range, 11 significant bits.  Q6_K's lanes hold k in the order
//                16 lh + 4 g + b; its activation columns are permuted the same
//                way when staged, so both MFMA operands agree.
//
// Pipeline, one barrier per step: issue the global loads of step s+1, run
// step s's 32 MFMAs per wave, dequantize step s+1's weights into registers,
// store its activations into the other LDS buffer, barrier.  All loads are
// buffer loads; their scalar offsets only ever address bytes inside the
// weight / activation block, and rows past M or N fall outside the buffer
// resource by their vector offset and read as zero.  Tiles are assigned XCD
// by XCD (workgroup b runs on XCD b % 8): each XCD gets a contiguous range of
// tiles in bands of 4 tile columns, n fastest within a band, so the
// workgroups resident on an XCD at once cover a block of a few row tiles by 4
// column tiles and share both operands in its L2 (M=2048, N=14336: 872 -> 896
// TFLOP/s against m fastest over whole columns).
#include "common.hpp"
#include "iq_ops.hpp"

namespace gguf {

namespace {

#ifndef GGUF_GEMM_WAVES
#define GGUF_GEMM_WAVES 8
#endif
#ifndef GGUF_GEMM_TN
#define GGUF_GEMM_TN 2
#endif
constexpr int kWaves = GGUF_GEMM_WAVES;
constexpr int kTN = GGUF_GEMM_TN;  // 16-column MFMA tiles (row tiles of W) per wave
constexpr int kBM = 128, kBN = 16 * kTN * kWaves, kBK = 64;
constexpr int kThreads = 64 * kWaves;
constexpr int kTM = kBM / 16;  // 16-row MFMA tiles per wave
constexpr int kAI = kBM * 8 / kThreads;  // activation chunks staged per thread
constexpr int kARows = kThreads / 8;     // row distance between a thread's chunks
constexpr int kRowB = 2 * kBK;             // LDS bytes per activation row
constexpr int kStageB = kBM * kRowB;       // LDS bytes per pipeline stage
#ifndef GGUF_GEMM_WIDE_MIN
#define GGUF_GEMM_WIDE_MIN 192  // Q4_K fp16: the wide tile once it gives this many workgroups
#endif
#ifndef GGUF_GEMM_GN
#define GGUF_GEMM_GN 4  // tile order: column bands of this many tiles (0: row tiles fastest)
#endif
constexpr float kTwo24 = 16777216.0f, kTwo20 = 1048576.0f;

typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)base, 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bl16(rsrc_t rs, int voff, int soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint2 bl8(rsrc_t rs, int voff, int soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, voff, soff, 0);
  return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint32_t bl4(rsrc_t rs, int voff, int soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(rs, voff, soff, 0);
}
__device__ __forceinline__ uint32_t bl2(rsrc_t rs, int voff, int soff) {
  return __builtin_amdgcn_raw_buffer_load_b16(rs, voff, soff, 0);
}

// Two f16 results packed in a word: fp16(s * x + c) for the f16 x taken from
// the low halves (mix_lo) or the high halves (mix_hi) of a and b, computed in
// f32 and rounded once (v_fma_mixlo_f16 / v_fma_mixhi_f16).  Plain code
// (fmaf of the widened halves, then a conversion) compiles to cvt + fma +
// cvt_pk and rounds twice, hence the asm.  Every operand passed here is the
// result of ordinary arithmetic (masks, shifts, products), never a load's
// destination register, so the compiler's memory-counter waits precede the
// instructions that produce them; the compiled assembly has no v_fma_mix
// whose source register was last written by a load.
__device__ __forceinline__ uint32_t mix_lo(uint32_t a, uint32_t b, float s, float c) {
  uint32_t r;
  asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[1,0,0]\n\t"
      "v_fma_mixhi_f16 %0, %4, %2, %3 op_sel_hi:[1,0,0]"
      : "=&v"(r)
      : "v"(a), "v"(s), "v"(c), "v"(b));
  return r;
}
__device__ __forceinline__ uint32_t mix_hi(uint32_t a, uint32_t b, float s, float c) {
  uint32_t r;
  asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
      "v_fma_mixhi_f16 %0, %4, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
      : "=&v"(r)
      : "v"(a), "v"(s), "v"(c), "v"(b));
  return r;
}
__device__ __forceinline__ half8_t h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  return __builtin_bit_cast(half8_t, make_uint4(a, b, c, d));
}

// ---------------------------------------------------------------------------
// Weight operands.  Item j in {0, 1} is the wave's row tile 2 w + j; bf[j][h]
// is its B operand for k in [k0 + 32 h, k0 + 32 h + 32).
// ---------------------------------------------------------------------------
template <int TYPE>
struct BRaw;
template <>
struct BRaw<12> {
  uint2 q[kTN];  // the lane's 8 code bytes of the 64-wide window
};
template <>
struct BRaw<13> {
  uint2 q[kTN];  // the lane's 8 code bytes of the 64-wide window
};
template <>
struct BRaw<14> {
  uint4 pa[kTN], pb[kTN];  // the two pieces holding the window's quant dwords
};
template <>
struct BRaw<8> {
  uint2 q[kTN][2];  // block b of the step: 8 int8 codes
  uint32_t d[kTN][2];
};
template <>
struct BRaw<2> {
  uint32_t q[kTN][2];  // block b of the step: the lane's code word
  uint32_t d[kTN][2];
};
template <>
struct BRaw<20> {
  uint32_t q[kTN][2];
  uint32_t d[kTN][2];
};
template <>
struct BRaw<6> {
  uint32_t q[kTN][2];
  uint32_t d[kTN][2];
  uint32_t qh[kTN][2];  // the row's fifth bits of block b
};

template <>
struct BRaw<10> {
  uint2 q[kTN];  // the lane's 8 qs bytes of half c >> 1 (windows 2c, 2c + 1 share them)
};
template <>
struct BRaw<11> {
  uint2 q[kTN];  // as Q2_K
};
template <>
struct BRaw<23> {
  uint2 q[kTN];  // the lane's code words of sub-blocks 2c, 2c + 1 (window c)
};

// Per-superblock fields of row r, loaded with the superblock's first window.
template <int TYPE>
struct BHdr {};
template <>
struct BHdr<12> {
  uint4 hd[kTN];  // d, dmin, 12 scale bytes
};
template <>
struct BHdr<13> {
  uint4 hd[kTN];  // d, dmin, 12 scale bytes
  uint2 qh[kTN];  // qh bytes 8g .. 8g + 7: the fifth bits of every window
};
template <>
struct BHdr<14> {
  uint4 sc[kTN];  // 16 int8 scales
  uint32_t d[kTN];
};

template <>
struct BHdr<10> {
  uint4 sc[kTN];  // the row's 16 scale bytes
  uint32_t dm[kTN];  // d | dmin << 16
};
template <>
struct BHdr<11> {
  uint32_t s[kTN][3];  // the row's 12 scale bytes
  uint32_t d[kTN];
  uint2 hm[kTN];       // the lane's hmask bytes 8 g .. 8 g + 7
};
template <>
struct BHdr<23> {
  uint2 hd[kTN];  // d | scales_h << 16, scales_l[4]
};

// The same fields in the form the dequantization uses, derived once per superblock.
template <int TYPE>
struct BCur {
  __device__ __forceinline__ void set(const BHdr<TYPE> &) {}
};
template <>
struct BCur<12> {
  uint32_t sc[kTN][2], mn[kTN][2];  // 6-bit scales / mins 0-3 and 4-7, one per byte
  float d24[kTN], d20[kTN], dmin[kTN];
  template <class H>
  __device__ __forceinline__ void set(const H &h) {
#pragma unroll
    for (int j = 0; j < kTN; ++j) {
      q4k_scales_packed(h.hd[j].y, h.hd[j].z, h.hd[j].w, sc[j][0], sc[j][1], mn[j][0], mn[j][1]);
      const float d = h2f(h.hd[j].x);
      d24[j] = d * kTwo24;
      d20[j] = d * kTwo20;
      dmin[j] = h2f(h.hd[j].x >> 16);
    }
  }
};
template <>
struct BCur<13> : BCur<12> {
  uint2 qh[kTN];
  __device__ __forceinline__ void set(const BHdr<13> &h) {
    BCur<12>::set(h);
#pragma unroll
    for (int j = 0; j < kTN; ++j) qh[j] = h.qh[j];
  }
};
template <>
struct BCur<14> {
  uint4 sc[kTN];
  float d[kTN];
  __device__ __forceinline__ void set(const BHdr<14> &h) {
#pragma unroll
    for (int j = 0; j < kTN; ++j) {
      sc[j] = h.sc[j];
      d[j] = h2f(h.d[j]);
    }
  }
};

template <>
struct BCur<10> {
  uint4 sc[kTN];
  float d24[kTN], dmin[kTN];
  __device__ __forceinline__ void set(const BHdr<10> &h) {
#pragma unroll
    for (int j = 0; j < kTN; ++j) {
      sc[j] = h.sc[j];
      d24[j] = h2f(h.dm[j]) * kTwo24;
      dmin[j] = h2f(h.dm[j] >> 16);
    }
  }
};
template <>
struct BCur<11> {
  uint32_t S[kTN][4];  // the 16 scales (+ 32), one per byte
  float d[kTN];
  uint2 hm[kTN];
  __device__ __forceinline__ void set(const BHdr<11> &h) {
#pragma unroll
    for (int j = 0; j < kTN; ++j) {
      q3k_scales(h.s[j][0], h.s[j][1], h.s[j][2], S[j]);
      d[j] = h2f(h.d[j]);
      hm[j] = h.hm[j];
    }
  }
};
template <>
struct BCur<23> {
  uint2 hd[kTN];
  float d[kTN];
  __device__ __forceinline__ void set(const BHdr<23> &h) {
#pragma unroll
    for (int j = 0; j < kTN; ++j) {
      hd[j] = h.hd[j];
      d[j] = h2f(h.hd[j].x);
    }
  }
};

struct BOff {       // per-lane vector offsets, fixed for the whole K loop
  int v0, v1, v2, v3;
};

template <int TYPE>
__device__ __forceinline__ BOff b_offsets(int r, int g);
template <>
__device__ __forceinline__ BOff b_offsets<12>(int r, int g) {
  return BOff{16 * r, 256 + (16 * g + r) * 16, 0, 0};
}
template <>
__device__ __forceinline__ BOff b_offsets<13>(int r, int g) {
  return BOff{16 * r, 256 + (16 * g + r) * 16, 2304 + (16 * g + r) * 8, 0};
}
template <>
__device__ __forceinline__ BOff b_offsets<14>(int r, int g) {
  return BOff{(16 * g + r) * 16, 3328 + 2 * r, 3072 + 16 * r, 0};
}
template <>
__device__ __forceinline__ BOff b_offsets<8>(int r, int g) {
  return BOff{32 + (16 * g + r) * 8, 2 * r, 0, 0};
}
template <>
__device__ __forceinline__ BOff b_offsets<2>(int r, int g) {
  return BOff{32 + (16 * g + r) * 4, 2 * r, 0, 0};
}
template <>
__device__ __forceinline__ BOff b_offsets<20>(int r, int g) {
  return BOff{32 + (16 * g + r) * 4, 2 * r, 0, 0};
}
template <>
__device__ __forceinline__ BOff b_offsets<10>(int r, int g) {
  return BOff{320 + (16 * g + r) * 16, 16 * r, 256 + 4 * r, 0};
}
template <>
__device__ __forceinline__ BOff b_offsets<11>(int r, int g) {
  return BOff{736 + (16 * g + r) * 16, 12 * r, 192 + 2 * r, 224 + (16 * g + r) * 8};
}
template <>
__device__ __forceinline__ BOff b_offsets<23>(int r, int g) {
  return BOff{8 * r, 128 + (16 * g + r) * 32, 0, 0};
}
template <>
__device__ __forceinline__ BOff b_offsets<6>(int r, int g) {
  return BOff{96 + (16 * g + r) * 4, 2 * r, 32 + 4 * r, 0};
}

// Loads for the 64-wide window c (0..3) of unit u (K-quants) or for blocks
// 2u, 2u + 1 (Q8_0; c unused).  ts = bytes of one row tile.
template <int C>
__device__ __forceinline__ void load_b(rsrc_t rs, const BOff &o, int ts, int u, int nu,
                                       BRaw<12> &b, BHdr<12> &h) {
  constexpr int TU = Fmt<12>::TU;
  const int su = u * TU;
#pragma unroll
  for (int j = 0; j < kTN; ++j) {
    if (C == 0) h.hd[j] = bl16(rs, o.v0 + j * ts, su);
    b.q[j] = bl8(rs, o.v1 + j * ts, su + (C >> 1) * 1024 + 8 * (C & 1));
  }
}
template <int C>
__device__ __forceinline__ void load_b(rsrc_t rs, const BOff &o, int ts, int u, int nu,
                                       BRaw<13> &b, BHdr<13> &h) {
  constexpr int TU = Fmt<13>::TU;
  const int su = u * TU;
#pragma unroll
  for (int j = 0; j < kTN; ++j) {
    if (C == 0) {
      h.hd[j] = bl16(rs, o.v0 + j * ts, su);
      h.qh[j] = bl8(rs, o.v2 + j * ts, su);
    }
    b.q[j] = bl8(rs, o.v1 + j * ts, su + (C >> 1) * 1024 + 8 * (C & 1));
  }
}
template <int C>
__device__ __forceinline__ void load_b(rsrc_t rs, const BOff &o, int ts, int u, int nu,
                                       BRaw<14> &b, BHdr<14> &h) {
  constexpr int TU = Fmt<14>::TU, HF = C >> 1;
  const int su = u * TU;
#pragma unroll
  for (int j = 0; j < kTN; ++j) {
    b.pa[j] = bl16(rs, o.v0 + j * ts, su + HF * 1024);
    b.pb[j] = bl16(rs, o.v0 + j * ts, su + HF * 1024 + 1024);
    if (C == 0) {
      h.d[j] = bl2(rs, o.v1 + j * ts, su);
      h.sc[j] = bl16(rs, o.v2 + j * ts, su);
    }
  }
}
template <int C>
__device__ __forceinline__ void load_b(rsrc_t rs, const BOff &o, int ts, int u, int nu,
                                       BRaw<8> &b, BHdr<8> &) {
  constexpr int TU = Fmt<8>::TU;
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    const int ub = 2 * u + blk;
    if (ub < nu) {  // uniform: K may end after the first block of the step
#pragma unroll
      for (int j = 0; j < kTN; ++j) {
        b.q[j][blk] = bl8(rs, o.v0 + j * ts, ub * TU);
        b.d[j][blk] = bl2(rs, o.v1 + j * ts, ub * TU);
      }
    } else {
#pragma unroll
      for (int j = 0; j < kTN; ++j) {
        b.q[j][blk] = make_uint2(0, 0);
        b.d[j][blk] = 0;
      }
    }
  }
}

// Q4_0 / Q5_0 / IQ4_NL: blocks 2u, 2u + 1 (as Q8_0).
template <int C, int TYPE>
__device__ __forceinline__ void load_b_b32(rsrc_t rs, const BOff &o, int ts, int u, int nu,
                                           BRaw<TYPE> &b) {
  constexpr int TU = Fmt<TYPE>::TU;
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    const int ub = 2 * u + blk;
    if (ub < nu) {  // uniform: K may end after the first block of the step
#pragma unroll
      for (int j = 0; j < kTN; ++j) {
        b.q[j][blk] = bl4(rs, o.v0 + j * ts, ub * TU);
        b.d[j][blk] = bl2(rs, o.v1 + j * ts, ub * TU);
        if constexpr (TYPE == 6) b.qh[j][blk] = bl4(rs, o.v2 + j * ts, ub * TU);
      }
    } else {
#pragma unroll
      for (int j = 0; j < kTN; ++j) {
        b.q[j][blk] = 0;
        b.d[j][blk] = 0;
        if constexpr (TYPE == 6) b.qh[j][blk] = 0;
      }
    }
  }
}
template <int C>
__device__ __forceinline__ void load_b(rsrc_t rs, const BOff &o, int ts, int u, int nu,
                                       BRaw<2> &b, BHdr<2> &) {
  load_b_b32<C, 2>(rs, o, ts, u, nu, b);
}
template <int C>
__device__ __forceinline__ void load_b(rsrc_t rs, const BOff &o, int ts, int u, int nu,
                                       BRaw<6> &b, BHdr<6> &) {
  load_b_b32<C, 6>(rs, o, ts, u, nu, b);
}
template <int C>
__device__ __forceinline__ void load_b(rsrc_t rs, const BOff &o, int ts, int u, int nu,
                                       BRaw<20> &b, BHdr<20> &) {
  load_b_b32<C, 20>(rs, o, ts, u, nu, b);
}

template <int C>
__device__ __forceinline__ void load_b(rsrc_t rs, const BOff &o, int ts, int u, int nu,
                                       BRaw<10> &b, BHdr<10> &h) {
  constexpr int TU = Fmt<10>::TU;
  const int su = u * TU;
#pragma unroll
  for (int j = 0; j < kTN; ++j) {
    if (C == 0) {
      h.sc[j] = bl16(rs, o.v1 + j * ts, su);
      h.dm[j] = bl4(rs, o.v2 + j * ts, su);
    }
    b.q[j] = bl8(rs, o.v0 + j * ts, su + 8 * (C >> 1));
  }
}
template <int C>
__device__ __forceinline__ void load_b(rsrc_t rs, const BOff &o, int ts, int u, int nu,
                                       BRaw<11> &b, BHdr<11> &h) {
  constexpr int TU = Fmt<11>::TU;
  const int su = u * TU;
#pragma unroll
  for (int j = 0; j < kTN; ++j) {
    if (C == 0) {
      h.s[j][0] = bl4(rs, o.v1 + j * ts, su);
      h.s[j][1] = bl4(rs, o.v1 + 4 + j * ts, su);
      h.s[j][2] = bl4(rs, o.v1 + 8 + j * ts, su);
      h.d[j] = bl2(rs, o.v2 + j * ts, su);
      h.hm[j] = bl8(rs, o.v3 + j * ts, su);
    }
    b.q[j] = bl8(rs, o.v0 + j * ts, su + 8 * (C >> 1));
  }
}
template <int C>
__device__ __forceinline__ void load_b(rsrc_t rs, const BOff &o, int ts, int u, int nu,
                                       BRaw<23> &b, BHdr<23> &h) {
  constexpr int TU = Fmt<23>::TU;
  const int su = u * TU;
#pragma unroll
  for (int j = 0; j < kTN; ++j) {
    if (C == 0) h.hd[j] = bl8(rs, o.v0 + j * ts, su);
    b.q[j] = bl8(rs, o.v1 + j * ts, su + 8 * C);
  }
}

// Q4_K / Q5_K: lane (r, g), window c = chunk c of the superblock: low
// nibbles are sub-block 2c (k = 8 g .. 8 g + 7 of the first 32), high nibbles
// sub-block 2c + 1.  Q5_K ORs the fifth bits into the codes first.
template <int C, int TYPE>
__device__ __forceinline__ void dequant_b_k(const BRaw<TYPE> &b, const BCur<TYPE> &h,
                                            half8_t (&bf)[kTN][2]) {
  constexpr int W = C >> 1, B0 = (2 * C) & 3;  // scale word, byte of sub-block 2C
#pragma unroll
  for (int j = 0; j < kTN; ++j) {
    const float s0 = h.d24[j] * ubyte(h.sc[j][W], B0), c0 = -(h.dmin[j] * ubyte(h.mn[j][W], B0));
    const float s1 = h.d20[j] * ubyte(h.sc[j][W], B0 + 1),
                c1 = -(h.dmin[j] * ubyte(h.mn[j][W], B0 + 1));
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const uint32_t q = w ? b.q[j].y : b.q[j].x, q8 = q >> 8;
      uint32_t el = q & 0x000F000Fu, ol = q8 & 0x000F000Fu;  // bytes 0, 2 / 1, 3: low nibble
      uint32_t eh = q & 0x00F000F0u, oh = q8 & 0x00F000F0u;  // high nibble (x 16)
      if constexpr (TYPE == 13) {
        const uint32_t hb = w ? h.qh[j].y : h.qh[j].x;
        el |= q5k_lo_even(hb, C);
        ol |= q5k_lo_odd(hb, C);
        eh |= q5k_hi_even(hb, C);
        oh |= q5k_hi_odd(hb, C);
      }
      lo[2 * w] = mix_lo(el, ol, s0, c0);
      lo[2 * w + 1] = mix_hi(el, ol, s0, c0);
      hi[2 * w] = mix_lo(eh, oh, s1, c1);
      hi[2 * w + 1] = mix_hi(eh, oh, s1, c1);
    }
    bf[j][0] = h8(lo[0], lo[1], lo[2], lo[3]);
    bf[j][1] = h8(hi[0], hi[1], hi[2], hi[3]);
  }
}

template <int C>
__device__ __forceinline__ void dequant_b(const BRaw<12> &b, const BCur<12> &h,
                                          half8_t (&bf)[kTN][2], int) {
  dequant_b_k<C, 12>(b, h, bf);
}
template <int C>
__device__ __forceinline__ void dequant_b(const BRaw<13> &b, const BCur<13> &h,
                                          half8_t (&bf)[kTN][2], int) {
  dequant_b_k<C, 13>(b, h, bf);
}

// Q6_K: window c = quarters 2 (c & 1), 2 (c & 1) + 1 of half c >> 1.  The
// lane's operand for k-block t2 (32 wide) holds the window columns
// 32 t2 + 16 lh + 4 g + e at position 4 lh + e.
template <int C>
__device__ __forceinline__ void dequant_b(const BRaw<14> &b, const BCur<14> &h,
                                          half8_t (&bf)[kTN][2], int) {
  constexpr int HF = C >> 1, TP = C & 1;
#pragma unroll
  for (int j = 0; j < kTN; ++j) {
    const uint4 pa = b.pa[j], pb = b.pb[j];
    // quant dwords 3i .. 3i + 2 of i = 2 HF + lh, taken from pieces HF and HF + 1
    const uint32_t dq[2][3] = {{HF ? pa.z : pa.x, HF ? pa.w : pa.y, HF ? pb.x : pa.z},
                               {HF ? pb.y : pa.w, HF ? pb.z : pb.x, HF ? pb.w : pb.y}};
    const float d = h.d[j];
    // scale bytes 8 HF + 4 TP .. + 3 of the window
    const uint32_t scw = (2 * HF + TP) == 0 ? h.sc[j].x
                         : (2 * HF + TP) == 1 ? h.sc[j].y
                         : (2 * HF + TP) == 2 ? h.sc[j].z
                                              : h.sc[j].w;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      uint32_t v[4];
#pragma unroll
      for (int lh = 0; lh < 2; ++lh) {
        const int t = 2 * TP + t2;
        const uint32_t ql = dq[lh][t & 1], qh = dq[lh][2];
        const uint32_t n4 = (t >> 1) ? ((ql >> 4) & 0x0F0F0F0Fu) : (ql & 0x0F0F0F0Fu);
        const uint32_t q6 = n4 | (((qh >> (2 * t)) & 0x03030303u) << 4);
        const uint32_t ev = q6 & 0x00FF00FFu, od = (q6 >> 8) & 0x00FF00FFu;
        const float sv = d * (float)(int8_t)((scw >> (8 * (2 * t2 + lh))) & 0xFFu);
        const float s = sv * kTwo24, c = -32.0f * sv;
        v[2 * lh] = mix_lo(ev, od, s, c);
        v[2 * lh + 1] = mix_hi(ev, od, s, c);
      }
      bf[j][t2] = h8(v[0], v[1], v[2], v[3]);
    }
  }
}

// Q8_0: block b of the step is k-block b; code + 128 enters as a subnormal.
template <int C>
__device__ __forceinline__ void dequant_b(const BRaw<8> &b, const BCur<8> &,
                                          half8_t (&bf)[kTN][2], int) {
#pragma unroll
  for (int j = 0; j < kTN; ++j)
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      const float d = h2f(b.d[j][blk]);
      const float s = d * kTwo24, c = -128.0f * d;
      uint32_t v[4];
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        const uint32_t q = (w ? b.q[j][blk].y : b.q[j][blk].x) ^ 0x80808080u;
        const uint32_t ev = q & 0x00FF00FFu, od = (q >> 8) & 0x00FF00FFu;
        v[2 * w] = mix_lo(ev, od, s, c);
        v[2 * w + 1] = mix_hi(ev, od, s, c);
      }
      bf[j][blk] = h8(v[0], v[1], v[2], v[3]);
    }
}

// Q4_0 / Q5_0 / IQ4_NL: block b of the step is k-block b; the code (minus the
// type's offset, times d) is dequantized in f32 and rounded once to fp16.
template <int TYPE>
__device__ __forceinline__ void dequant_b_b32(const BRaw<TYPE> &b, half8_t (&bf)[kTN][2], int g) {
#pragma unroll
  for (int j = 0; j < kTN; ++j)
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      const float d = h2f(b.d[j][blk]);
      const float s = d * kTwo24, c = -code_offset<TYPE>() * d;
      uint32_t qhb = 0;
      if constexpr (TYPE == 6) qhb = (b.qh[j][blk] >> (8 * g)) & 0xFFu;
      uint32_t w[4];
      b32_codes<TYPE>(b.q[j][blk], qhb, w);
      bf[j][blk] = h8(mix_lo(w[0], w[1], s, c), mix_hi(w[0], w[1], s, c), mix_lo(w[2], w[3], s, c),
                      mix_hi(w[2], w[3], s, c));
    }
}
template <int C>
__device__ __forceinline__ void dequant_b(const BRaw<2> &b, const BCur<2> &, half8_t (&bf)[kTN][2],
                                          int g) {
  dequant_b_b32<2>(b, bf, g);
}
template <int C>
__device__ __forceinline__ void dequant_b(const BRaw<6> &b, const BCur<6> &, half8_t (&bf)[kTN][2],
                                          int g) {
  dequant_b_b32<6>(b, bf, g);
}
template <int C>
__device__ __forceinline__ void dequant_b(const BRaw<20> &b, const BCur<20> &,
                                          half8_t (&bf)[kTN][2], int g) {
  dequant_b_b32<20>(b, bf, g);
}

// Q2_K: the 64-wide step c holds 32-element windows w = 2c, 2c + 1 (bits 2 (w & 3)
// of the lane's qs bytes of half c >> 1); the lane's 8 k of a window lie in scale
// group 2 w + (g >> 1), dequantized as fp16(d sc q - dmin m).
template <int C>
__device__ __forceinline__ void dequant_b(const BRaw<10> &b, const BCur<10> &h,
                                          half8_t (&bf)[kTN][2], int g) {
#pragma unroll
  for (int j = 0; j < kTN; ++j)
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      const int w = 2 * C + hb, sh = 2 * (w & 3);
      const uint32_t scw = (w >> 1) == 0 ? h.sc[j].x
                           : (w >> 1) == 1 ? h.sc[j].y
                           : (w >> 1) == 2 ? h.sc[j].z
                                           : h.sc[j].w;
      const uint32_t sb = (scw >> (8 * (2 * (w & 1) + (g >> 1)))) & 0xFFu;
      const float s = h.d24[j] * (float)(sb & 15u), c = -(h.dmin[j] * (float)(sb >> 4));
      const uint32_t t0 = (b.q[j].x >> sh) & 0x03030303u, t1 = (b.q[j].y >> sh) & 0x03030303u;
      const uint32_t e0 = t0 & 0x00FF00FFu, o0 = (t0 >> 8) & 0x00FF00FFu;
      const uint32_t e1 = t1 & 0x00FF00FFu, o1 = (t1 >> 8) & 0x00FF00FFu;
      bf[j][hb] = h8(mix_lo(e0, o0, s, c), mix_hi(e0, o0, s, c), mix_lo(e1, o1, s, c),
                     mix_hi(e1, o1, s, c));
    }
}

// Q3_K: as Q2_K, codes q3 = low bits | hmask bit 4 (c >> 1) + (w & 3) << 2,
// dequantized as fp16(d (sc - 32) (q3 - 4)) (exact in f32, rounded once).
template <int C>
__device__ __forceinline__ void dequant_b(const BRaw<11> &b, const BCur<11> &h,
                                          half8_t (&bf)[kTN][2], int g) {
#pragma unroll
  for (int j = 0; j < kTN; ++j)
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      const int w = 2 * C + hb, jj = w & 3, hh = w >> 2;
      const uint32_t sb = (h.S[j][w >> 1] >> (8 * (2 * (w & 1) + (g >> 1)))) & 0xFFu;
      const float dl = h.d[j] * (float)((int)sb - 32);
      const float s = dl * kTwo24, c = -4.0f * dl;
      const uint32_t t0 = ((b.q[j].x >> (2 * jj)) & 0x03030303u) |
                          (((h.hm[j].x >> (4 * hh + jj)) & 0x01010101u) << 2);
      const uint32_t t1 = ((b.q[j].y >> (2 * jj)) & 0x03030303u) |
                          (((h.hm[j].y >> (4 * hh + jj)) & 0x01010101u) << 2);
      const uint32_t e0 = t0 & 0x00FF00FFu, o0 = (t0 >> 8) & 0x00FF00FFu;
      const uint32_t e1 = t1 & 0x00FF00FFu, o1 = (t1 >> 8) & 0x00FF00FFu;
      bf[j][hb] = h8(mix_lo(e0, o0, s, c), mix_hi(e0, o0, s, c), mix_lo(e1, o1, s, c),
                     mix_hi(e1, o1, s, c));
    }
}

// IQ4_XS: window c = sub-blocks 2c, 2c + 1, each an IQ4_NL block with scale
// d * (ls - 32) (exact in f32), rounded once to fp16.
template <int C>
__device__ __forceinline__ void dequant_b(const BRaw<23> &b, const BCur<23> &h,
                                          half8_t (&bf)[kTN][2], int) {
#pragma unroll
  for (int j = 0; j < kTN; ++j)
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      const float dl = h.d[j] * (float)((int)iq4xs_ls(h.hd[j].x >> 16, h.hd[j].y, 2 * C + hb) - 32);
      const float s = dl * kTwo24, c = -128.0f * dl;
      uint32_t w[4];
      b32_codes<20>(hb ? b.q[j].y : b.q[j].x, 0u, w);
      bf[j][hb] = h8(mix_lo(w[0], w[1], s, c), mix_hi(w[0], w[1], s, c), mix_lo(w[2], w[3], s, c),
                     mix_hi(w[2], w[3], s, c));
    }
}

// ---------------------------------------------------------------------------
// Grid-codebook IQ types (iq_ops.hpp).  Window c is sub-blocks 2c, 2c + 1; the
// lane (r, g) loads the words of its row's record those two sub-blocks use
// (indices as in the record: the block without its d, 4-byte words) into a
// sparse IqUnit, builds the exact f16 operand of grid entry, signs and odd
// factor (iq_b, tables in shared memory) and rounds unit scale x operand to
// fp16 once (v_fma_mix).
// ---------------------------------------------------------------------------
#define GGUF_GEMM_IQ(T)                                                                          \
  template <>                                                                                    \
  struct BRaw<T> {                                                                               \
    IqUnit<T> u[kTN];                                                                            \
  };                                                                                             \
  template <>                                                                                    \
  struct BHdr<T> {                                                                               \
    uint32_t d[kTN];                                                                             \
  };                                                                                             \
  template <>                                                                                    \
  struct BCur<T> {                                                                               \
    float us[kTN];                                                                               \
    const unsigned char *tb;                                                                     \
    __device__ __forceinline__ void set(const BHdr<T> &h) {                                      \
      _Pragma("unroll") for (int j = 0; j < kTN; ++j) us[j] = h2f(h.d[j]) * iq_d_factor<T>();    \
    }                                                                                            \
  };                                                                                             \
  template <>                                                                                    \
  __device__ __forceinline__ BOff b_offsets<T>(int r, int) {                                     \
    return BOff{iq_rec_off<T>(r), 2 * r, 0, 0};                                                  \
  }                                                                                              \
  template <int C>                                                                               \
  __device__ __forceinline__ void load_b(rsrc_t rs, const BOff &o, int ts, int u, int,           \
                                         BRaw<T> &b, BHdr<T> &h) {                               \
    load_b_iq<C, T>(rs, o, ts, u, b, h);                                                         \
  }                                                                                              \
  template <int C>                                                                               \
  __device__ __forceinline__ void dequant_b(const BRaw<T> &b, const BCur<T> &h,                  \
                                            half8_t (&bf)[kTN][2], int g) {                      \
    dequant_b_iq<C, T>(b, h, bf, g);                                                             \
  }

// the unit scale over the f16 d (IQ1_M: d assembled from its scale words)
template <int T>
constexpr float iq_d_factor() {
  return T == 18 ? 0.25f : T == 21 ? 1.f : 0.125f;
}
template <int T>
struct BRaw;
template <int T>
struct BHdr;
template <int T>
struct BCur;

// fp16(s * x) of both f16 halves of w, computed in f32 and rounded once
__device__ __forceinline__ uint32_t mix_w(uint32_t w, float s) {
  uint32_t r;
  asm("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel_hi:[1,0,0]\n\t"
      "v_fma_mixhi_f16 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
      : "=&v"(r)
      : "v"(w), "v"(s));
  return r;
}

// The record words of window C (sub-blocks 2C, 2C + 1) of the lane's row: v =
// the record's offset in the resource, su = the unit's.
template <int C, int T>
__device__ __forceinline__ void iq_load_window(rsrc_t rs, int v, int su, uint32_t *w) {
    if constexpr (T == 16 || T == 17 || T == 18 || T == 21) {  // index words 4C .. 4C + 3
      const uint4 q = bl16(rs, v + 16 * C, su);
      w[4 * C] = q.x; w[4 * C + 1] = q.y; w[4 * C + 2] = q.z; w[4 * C + 3] = q.w;
    }
    if constexpr (T == 17) w[16 + (C >> 1)] = bl4(rs, v + 4 * (16 + (C >> 1)), su);
    if constexpr (T == 18) {
      const uint2 a = bl8(rs, v + 4 * (16 + 2 * C), su);
      w[16 + 2 * C] = a.x; w[17 + 2 * C] = a.y;
    }
    if constexpr (T == 21) {
      w[16 + (C >> 1)] = bl4(rs, v + 4 * (16 + (C >> 1)), su);
      const uint2 sg = bl8(rs, v + 4 * (18 + 2 * C), su);
      w[18 + 2 * C] = sg.x; w[19 + 2 * C] = sg.y;
      w[26] = bl4(rs, v + 4 * 26, su);
    }
    if constexpr (T == 22) {
      const uint2 q = bl8(rs, v + 8 * C, su), sg = bl8(rs, v + 4 * (8 + 2 * C), su);
      w[2 * C] = q.x; w[2 * C + 1] = q.y; w[8 + 2 * C] = sg.x; w[9 + 2 * C] = sg.y;
      w[16 + (C >> 1)] = bl4(rs, v + 4 * (16 + (C >> 1)), su);
      w[18 + (C >> 1)] = bl4(rs, v + 4 * (18 + (C >> 1)), su);
    }
    if constexpr (T == 29) {
      const uint2 q = bl8(rs, v + 8 * C, su), sw = bl8(rs, v + 48, su);
      w[2 * C] = q.x; w[2 * C + 1] = q.y; w[12] = sw.x; w[13] = sw.y;
      w[8 + C] = bl4(rs, v + 4 * (8 + C), su);
    }
}

template <int C, int T>
__device__ __forceinline__ void load_b_iq(rsrc_t rs, const BOff &o, int ts, int u, BRaw<T> &b,
                                          BHdr<T> &h) {
  const int su = u * Fmt<T>::TU;
#pragma unroll
  for (int j = 0; j < kTN; ++j) {
    iq_load_window<C, T>(rs, o.v0 + j * ts, su, b.u[j].w);  // the record of the lane's row in tile j
    if constexpr (T != 29)
      if (C == 0) h.d[j] = bl2(rs, o.v1 + j * ts, su);
  }
}

template <int C, int T>
__device__ __forceinline__ void dequant_b_iq(const BRaw<T> &b, const BCur<T> &h,
                                             half8_t (&bf)[kTN][2], int g) {
#pragma unroll
  for (int j = 0; j < kTN; ++j) {
    const float us = T == 29 ? iq_unit_scale<T>(b.u[j]) : h.us[j];
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      const uint4 v = __builtin_bit_cast(uint4, iq_b<T>(b.u[j], 2 * C + hb, g, h.tb));
      bf[j][hb] = h8(mix_w(v.x, us), mix_w(v.y, us), mix_w(v.z, us), mix_w(v.w, us));
    }
  }
}

GGUF_GEMM_IQ(16)
GGUF_GEMM_IQ(17)
GGUF_GEMM_IQ(18)
GGUF_GEMM_IQ(21)
GGUF_GEMM_IQ(22)
GGUF_GEMM_IQ(29)
#undef GGUF_GEMM_IQ

// ---------------------------------------------------------------------------
// Activations.  Thread t stages rows (t >> 3) + kARows i, i < kAI, 16-byte
// column chunk t & 7 of the 64-wide step.
// ---------------------------------------------------------------------------
template <typename XT>
struct ARaw {
  static constexpr int W = sizeof(XT) / 2;  // 16-byte loads per item
  uint4 v[kAI][W];
};

template <int TYPE, typename XT>
__device__ __forceinline__ void load_a(rsrc_t rs, int voff, int64_t ldxb, int k0, int K, int cc,
                                       ARaw<XT> &a) {
  constexpr int W = ARaw<XT>::W;
  const int soff = k0 * (int)sizeof(XT);
  // only 32-element-block weights can end K halfway through a step; chunks past K read as zero
  const bool ok = (TYPE != 8 && !is_b32(TYPE)) || k0 + 8 * cc < K;
#pragma unroll
  for (int i = 0; i < kAI; ++i)
#pragma unroll
    for (int w = 0; w < W; ++w)
      a.v[i][w] =
          ok ? bl16(rs, voff + (int)(kARows * i * ldxb) + 16 * w, soff) : make_uint4(0, 0, 0, 0);
}

__device__ __forceinline__ uint4 to_f16x8(const uint4 (&v)[1], float) { return v[0]; }
// eight f32 values times the row's power-of-two scale (exact), rounded to fp16
__device__ __forceinline__ uint4 to_f16x8(const uint4 (&v)[2], float sc) {
  half8_t h;
  const uint4 a = v[0], b = v[1];
  h[0] = (half_t)(__uint_as_float(a.x) * sc);
  h[1] = (half_t)(__uint_as_float(a.y) * sc);
  h[2] = (half_t)(__uint_as_float(a.z) * sc);
  h[3] = (half_t)(__uint_as_float(a.w) * sc);
  h[4] = (half_t)(__uint_as_float(b.x) * sc);
  h[5] = (half_t)(__uint_as_float(b.y) * sc);
  h[6] = (half_t)(__uint_as_float(b.z) * sc);
  h[7] = (half_t)(__uint_as_float(b.w) * sc);
  return __builtin_bit_cast(uint4, h);
}

// Largest magnitude of the f32 values of a raw activation item.
__device__ __forceinline__ float absmax(const uint4 (&v)[2], float m) {
  const uint4 a = v[0], b = v[1];
  m = fmaxf(m, fmaxf(fabsf(__uint_as_float(a.x)), fabsf(__uint_as_float(a.y))));
  m = fmaxf(m, fmaxf(fabsf(__uint_as_float(a.z)), fabsf(__uint_as_float(a.w))));
  m = fmaxf(m, fmaxf(fabsf(__uint_as_float(b.x)), fabsf(__uint_as_float(b.y))));
  return fmaxf(m, fmaxf(fabsf(__uint_as_float(b.z)), fabsf(__uint_as_float(b.w))));
}

// LDS byte address of (row, 16-byte chunk): chunks rotate by the row index.
__device__ __forceinline__ int lds_at(int row, int chunk) {
  return row * kRowB + ((chunk + row) & 7) * 16;
}

template <int TYPE, typename XT>
__device__ __forceinline__ void store_a(unsigned char *lds, int stage, int row0, int cc,
                                        const ARaw<XT> &a, const float (&rsc)[kAI]) {
#pragma unroll
  for (int i = 0; i < kAI; ++i) {
    const uint4 h = to_f16x8(a.v[i], rsc[i]);
    const int row = row0 + kARows * i;
    unsigned char *base = lds + stage * kStageB;
    if constexpr (TYPE == 14) {
      // columns 8 q + e (q = cc & 3, e = 0..7) of k-block cc >> 2 go to
      // position 8 g + 4 lh + (e & 3) with g = 2 (q & 1) + (e >> 2), lh = q >> 1
      const int q = cc & 3, ch = 4 * (cc >> 2) + 2 * (q & 1), half = 8 * (q >> 1);
      *(uint2 *)(base + lds_at(row, ch) + half) = make_uint2(h.x, h.y);
      *(uint2 *)(base + lds_at(row, ch + 1) + half) = make_uint2(h.z, h.w);
    } else {
      *(uint4 *)(base + lds_at(row, cc)) = h;
    }
  }
}

// ---------------------------------------------------------------------------

template <int TYPE, typename XT>
struct Gemm {
  rsrc_t ars, brs;
  int avoff, row0, cc, lg;  // lg: the lane's group (lane >> 4)
  int64_t ldxb;
  int K, nu, ts;
  BOff bo;
  int afrag[2];  // LDS byte address of the lane's A fragment, k-block 0 / 1
  float rsc[kAI];     // power-of-two scales of the staged rows (f32 input)
  ARaw<XT> ar[2];     // raw loads of the next two steps, by step parity
  BRaw<TYPE> br[2];
  BHdr<TYPE> hn;       // superblock fields loaded ahead
  BCur<TYPE> hc;       // superblock fields in use
  half8_t bf[kTN][2];  // B operands of the current step
  float4_t acc[kTM][kTN];
  unsigned char *lds;

  template <int C, int P>
  __device__ __forceinline__ void load(int u, int k0) {
    load_a<TYPE, XT>(ars, avoff, ldxb, k0, K, cc, ar[P]);
    load_b<C>(brs, bo, ts, u, nu, br[P], hn);
  }

  template <int C, int P>
  __device__ __forceinline__ void prepare(int stage) {
    if (C == 0) hc.set(hn);
    dequant_b<C>(br[P], hc, bf, lg);
    store_a<TYPE, XT>(lds, stage, row0, cc, ar[P], rsc);
  }

  // Step s (parity P = s & 1) from LDS stage P.  Loads step s + 2 (window C2 of
  // unit u2, k = k2) into raw set P when `load2`; dequantizes / stages step
  // s + 1 (window C1) from raw set P ^ 1 when `next`.  The schedule is pinned:
  // global loads first, then all sixteen A fragment reads, then the 32 MFMAs
  // with the dequantization of the next step's weights interleaved.
  template <int P, int C1, int C2>
  __device__ __forceinline__ void step(bool next, bool load2, int u2, int k2) {
    if (load2) load<C2, P>(u2, k2);
    const unsigned char *base = lds + P * kStageB;
    half8_t a[2][kTM];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < kTM; ++i) a[h][i] = *(const half8_t *)(base + afrag[h] + i * 16 * kRowB);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < kTM; ++i)
#pragma unroll
        for (int j = 0; j < kTN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[h][i], bf[j][h], acc[i][j], 0, 0, 0);
    if (next) {
      prepare<C1, P ^ 1>(P ^ 1);
#pragma unroll
      for (int i = 0; i < 2 * kTM * kTN; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // four VALU
      }
    }
    __syncthreads();
  }
};

template <int TYPE, typename XT>
__global__ __launch_bounds__(kThreads) void gemm_kernel(const XT *__restrict__ x, int64_t ldx,
                                                           const uint8_t *__restrict__ W, int M,
                                                           int N, int K, float *__restrict__ y,
                                                           int64_t ldy, int tiles_m, int kunits,
                                                           const float *__restrict__ rowf_g) {
  constexpr int TU = Fmt<TYPE>::TU, UE = Fmt<TYPE>::UE;
  __shared__ __align__(16) unsigned char lds[2 * kStageB];
  __shared__ __align__(16) float rowf[kBM];  // f32 input: the rows' inverse scales 2^-e
  // IQ types: the decode tables, requested first and written before the first dequantization
  __shared__ __align__(16) unsigned char iqtbl[is_iq(TYPE) ? iq_tbl_bytes<TYPE>() : 16];
  IqTabRegs<TYPE, kThreads> tab;
  if constexpr (is_iq(TYPE)) iq_get_tables<TYPE, kThreads>(tab);

  int bid = blockIdx.x;
  if ((gridDim.x & 7) == 0) bid = (bid & 7) * (gridDim.x >> 3) + (bid >> 3);
  int m0, n0;
  if (GGUF_GEMM_GN > 0) {
    // bands of GGUF_GEMM_GN tile columns, n fastest within a band: the
    // workgroups resident on one XCD at a time cover a few row tiles by
    // several column tiles, and share both operands in its L2
    const int band = bid / (tiles_m * GGUF_GEMM_GN), in = bid - band * tiles_m * GGUF_GEMM_GN;
    const int tiles_n = (int)gridDim.x / tiles_m;
    const int gn = min(GGUF_GEMM_GN, tiles_n - band * GGUF_GEMM_GN);
    m0 = (in / gn) * kBM;
    n0 = (band * GGUF_GEMM_GN + in % gn) * kBN;
  } else {
    m0 = (bid % tiles_m) * kBM;
    n0 = (bid / tiles_m) * kBN;
  }

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;

  Gemm<TYPE, XT> s;
  s.lds = lds;
  s.K = K;
  s.nu = K / UE;
  s.ts = s.nu * TU;
  // the wave's kTN row tiles; tiles past the weight's end are outside the resource
  const int ntiles = (N + 15) >> 4, t0 = (n0 >> 4) + kTN * wave;
  const int nt = __builtin_amdgcn_readfirstlane(max(0, min(kTN, ntiles - t0)));
  s.brs = make_rsrc(W + (int64_t)t0 * s.ts, (uint32_t)__builtin_amdgcn_readfirstlane(nt * s.ts));
  s.bo = b_offsets<TYPE>(r, g);
  s.lg = g;
  // activation rows m0 .. m0 + rows - 1; rows past M are outside the resource
  const int rows = min(kBM, M - m0);
  s.ldxb = ldx * (int64_t)sizeof(XT);
  s.ars = make_rsrc(x + (int64_t)m0 * ldx,
                    (uint32_t)__builtin_amdgcn_readfirstlane(
                        (int)((int64_t)(rows - 1) * s.ldxb + (int64_t)K * sizeof(XT))));
  s.row0 = tid >> 3;
  s.cc = tid & 7;
  s.avoff = (int)(s.row0 * s.ldxb) + s.cc * 16 * (int)ARaw<XT>::W;
  s.afrag[0] = lds_at(r, g);
  s.afrag[1] = lds_at(r, 4 + g);
#pragma unroll
  for (int i = 0; i < kTM; ++i)
#pragma unroll
    for (int j = 0; j < kTN; ++j) s.acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kAI; ++i) s.rsc[i] = 1.0f;
  if constexpr (sizeof(XT) == 4) {
    // row scales: each thread reads its staged rows' column chunk of every
    // step; the 8 threads of a row are lanes 8 j .. 8 j + 7 of a wave
    float mx[kAI];
#pragma unroll
    for (int i = 0; i < kAI; ++i) mx[i] = 0.f;
#pragma unroll 4
    for (int k0 = 0; k0 < K; k0 += kBK) {
      ARaw<XT> a;
      load_a<TYPE, XT>(s.ars, s.avoff, s.ldxb, k0, K, s.cc, a);
#pragma unroll
      for (int i = 0; i < kAI; ++i) mx[i] = absmax(a.v[i], mx[i]);
    }
#pragma unroll
    for (int i = 0; i < kAI; ++i) {
#pragma unroll
      for (int o = 1; o < 8; o <<= 1) mx[i] = fmaxf(mx[i], __shfl_xor(mx[i], o));
      const int e = stage_exp(mx[i]);
      s.rsc[i] = pow2f(e);
      if (s.cc == 0) rowf[s.row0 + kARows * i] = pow2f(-e);
    }
  }

  if constexpr (UE == 256) {
    // step s = 4 u + c covers window c of superblock u; 4 nu >= 4 steps
    // split K (gridDim.y > 1): units blockIdx.y kunits .. + kunits - 1, partial
    // sums written to y + blockIdx.y M ldy
    const int ub = blockIdx.y * kunits, ue = min(s.nu, ub + kunits);
    s.template load<0, 0>(ub, ub * 256);
    s.template load<1, 1>(ub, ub * 256 + 64);
    if constexpr (is_iq(TYPE)) {
      iq_put_tables<TYPE, kThreads>(tab, iqtbl);
      s.hc.tb = iqtbl;
      __syncthreads();
    }
    s.template prepare<0, 0>(0);
    __syncthreads();
    for (int u = ub; u < ue; ++u) {
      const int k = u * 256;
      const bool more = u + 1 < ue;
      s.template step<0, 1, 2>(true, true, u, k + 128);
      s.template step<1, 2, 3>(true, true, u, k + 192);
      s.template step<0, 3, 0>(true, more, u + 1, k + 256);
      s.template step<1, 0, 1>(more, more, u + 1, k + 320);
    }
  } else {
    // step s covers blocks 2 s, 2 s + 1
    const int steps = (s.nu + 1) >> 1;
    s.template load<0, 0>(0, 0);
    if (steps > 1) s.template load<0, 1>(1, kBK);
    s.template prepare<0, 0>(0);
    __syncthreads();
    for (int st = 0; st < steps; st += 2) {
      s.template step<0, 0, 0>(st + 1 < steps, st + 2 < steps, st + 2, (st + 2) * kBK);
      if (st + 1 < steps)
        s.template step<1, 0, 0>(st + 2 < steps, st + 3 < steps, st + 3, (st + 3) * kBK);
    }
  }

  y += (int64_t)blockIdx.y * M * ldy;  // this split's partial sums
  // D layout of the 16x16 MFMA: lane holds rows 4 g + e of column r
#pragma unroll
  for (int i = 0; i < kTM; ++i) {
    float f[4] = {1.f, 1.f, 1.f, 1.f};
    // the rows' inverse scales: staged here (f32 input) or by stage_rows_kernel
    // (rowf_g, kBM of them per row tile; entries past M are read, not used)
    const float *rf = sizeof(XT) == 4 ? rowf + 16 * i + 4 * g
                                      : (rowf_g ? rowf_g + m0 + 16 * i + 4 * g : nullptr);
    if (rf) {
      const float4 v = *(const float4 *)rf;
      f[0] = v.x;
      f[1] = v.y;
      f[2] = v.z;
      f[3] = v.w;
    }
#pragma unroll
    for (int j = 0; j < kTN; ++j) {
      const int n = n0 + 16 * (kTN * wave + j) + r;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + 16 * i + 4 * g + e;
        if (m < M && n < N) y[(int64_t)m * ldy + n] = s.acc[i][j][e] * f[e];
      }
    }
  }
}

// y[m, n] = sum over the S splits of part[s][m][n] (M x N each), in split order.
__global__ __launch_bounds__(256) void gemm_reduce_kernel(const float *__restrict__ part, int S,
                                                          int M, int N, float *__restrict__ y,
                                                          int64_t ldy) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)M * N) return;
  const int64_t st = (int64_t)M * N;
  float a = part[i];
  for (int t = 1; t < S; ++t) a += part[i + t * st];
  y[(i / N) * ldy + i % N] = a;
}

// The same, four outputs per thread (N and ldy multiples of 4, y 16-byte
// aligned), the splits' partials requested four at a time; the same order of
// additions.
__global__ __launch_bounds__(256) void gemm_reduce4_kernel(const float4 *__restrict__ part, int S,
                                                           int M, int N4, float *__restrict__ y,
                                                           int64_t ldy) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)M * N4) return;
  const int64_t st = (int64_t)M * N4;
  float4 a = part[i];
  for (int t0 = 1; t0 < S; t0 += 4) {
    float4 v[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) v[t] = t0 + t < S ? part[i + (t0 + t) * st] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int t = 0; t < 4; ++t)
      if (t0 + t < S) {
        a.x += v[t].x;
        a.y += v[t].y;
        a.z += v[t].z;
        a.w += v[t].w;
      }
  }
  const int64_t m = i / N4;
  *(float4 *)(y + m * ldy + 4 * (i - m * N4)) = a;
}

// Splits of K for a grid of `tiles` workgroups: while the grid leaves most CUs
// idle (fewer than 192 tiles) and each split keeps at least 4 superblocks,
// double the splits up to 256 workgroups (M=512, N=4096: 64 tiles, 4 splits).
#ifndef GGUF_GEMM_SPLIT_WGS
#define GGUF_GEMM_SPLIT_WGS 256  // the split grid stays within this many workgroups
#endif
#ifndef GGUF_GEMM_SPLIT_MIN
#define GGUF_GEMM_SPLIT_MIN 4  // doubling the splits keeps at least half this many superblocks each
#endif
inline int gemm_splits(int type, int64_t tiles, int nu) {
  if (unit_elems(type) != 256) return 1;
  int sp = 1;
  while (tiles * sp < 192 && tiles * 2 * sp <= GGUF_GEMM_SPLIT_WGS && nu >= GGUF_GEMM_SPLIT_MIN * sp) sp <<= 1;
  return sp;
}

// ---------------------------------------------------------------------------
// Wide-tile GEMM for large grids (every type but IQ3_XXS, fp16 activations, K a
// multiple of 256).  A workgroup of 8 waves owns a
// 128 x 512 output tile (Q6_K, Q5_K, Q3_K 128 x 384); wave w owns all 128 rows
// and the 64 columns [64 w, 64 w + 64) (four row tiles of the weight; Q6_K,
// Q5_K, Q3_K three): 32 accumulator tiles, 255 VGPRs, two waves per SIMD.  Against gemm_kernel's 128 x 32 per
// wave, each activation fragment read from LDS feeds twice the MFMAs and a
// step holds twice the MFMA work per barrier; each dequantized B operand
// still feeds 8 MFMAs.
//   Per 64-wide step: the activations of the step after next go from
//   registers to their LDS stage (four stages) and the following step's are
//   requested; then k-half by k-half the 8 fragments of the half are read and
//   each tile's B operand is dequantized (fp16(d sc q - dmin m), one rounding,
//   as gemm_kernel) just before its 8 MFMAs; a tile's codes for two steps
//   ahead are requested once both its operands of this step are built; a
//   barrier after every second step.  The step is branch-free: past the end
//   of K the loads stay inside their buffer resources and their data is never
//   used.
// The MFMAs of an output element run in the same k order as gemm_kernel's,
// so the results are the same bit for bit.
// Measured (one box, fp16, K = 4096 unless noted), TFLOP/s against
// gemm_kernel: M = 2048, N = 14336 778 -> 864; M = 8192, N = 14336
// 968 -> 1053; M = 8192, N = 4096, K = 14336 970 -> 1092.  Four stages and a
// barrier every second step instead of two stages and one per step: another
// +3% (852 -> 877, 1048 -> 1071); eight stages and one barrier per
// superblock measured level with four (868 / 1056).
//   - One wave per SIMD with 128 x 128 per wave (256 accumulators) spills
//     (136-164 dwords: the allocator copies accumulators between AGPRs and
//     VGPRs).
//   - Pinning an MFMA / VALU interleave (sched_group_barrier, 2-3 VALU per
//     MFMA) forces 55-89 dwords of spill and runs at 410-626.
//   - Reading the A fragments a few ahead of their MFMAs instead of all at
//     the start of a half (gemm_kernel, 2-8 ahead): 734-770 against 786.
//   - The same wave tile on v_mfma_f32_32x32x16_f16 (each lane dequantizes
//     its own weight row per 32-column block, so the sub-block scales are
//     derived once per row; 217 VGPRs): bit-identical results, 868-875
//     against 865-869 at M = 2048, 1-2% slower at M = 8192.
//   - Q8_0 on it (bit-identical to gemm_kernel): 702 -> 820 TFLOP/s at
//     M = 2048, N = 14336; 803 -> 1025 at M = 8192, N = 4096, K = 14336.
//   - Q6_K runs 3 tiles per wave (128 x 384 per workgroup, 242 VGPRs, two code
//     sets three steps ahead): 676 -> 699 TFLOP/s at M = 2048, N = 14336;
//     809 -> 877 at M = 8192, N = 4096, K = 14336; 800 -> 882 at M = 8192,
//     N = 14336 (bit-identical to gemm_kernel).  At 4 tiles per wave its 6
//     quant dwords per tile and half superblock left room for one set only
//     (one step ahead) and still spilled 31 dwords: 678 -> 624, 811 -> 729.
//   - Q5_K at 3 tiles per wave (222 VGPRs; 4 spilled 30 dwords): 703 -> 737
//     at M = 2048, 844 -> 920 at M = 8192 (bit-identical to gemm_kernel).
//   - Q2_K (4 tiles, 256 VGPRs): 751 -> 848 at M = 2048, 897 -> 1032 at
//     M = 8192 (3 tiles: 785 / 973).  Q3_K (3 tiles, 226 VGPRs): 681 -> 715,
//     829 -> 896.  IQ4_XS (4 tiles, 254 VGPRs): 671 -> 742, 797 -> 896.  All
//     bit-identical to gemm_kernel.
//   - Q4_0 / Q5_0 / IQ4_NL (4 tiles): 736 -> 873, 642 -> 744, 641 -> 749 at
//     M = 2048; 915 -> 1061, 791 -> 928, 793 -> 914 at M = 8192.
//   - Grid-codebook IQ types (tables in shared memory beside the stages, up to
//     96 KB): IQ2_XXS, IQ2_XS (4 tiles) 723 -> 804, 668 -> 746; IQ3_S, IQ2_S,
//     IQ1_M (3 tiles) 530 -> 573, 553 -> 613, 648 -> 679.  IQ3_XXS (3 tiles)
//     measured 685 -> 671 and keeps gemm_kernel.
// ---------------------------------------------------------------------------
constexpr int kWW = 8, kWTM = 8;
// weight row tiles per wave: 4 (a 128 x 512 workgroup tile); Q6_K, Q5_K, Q3_K, IQ3_S,
// IQ2_S and IQ1_M 3 (128 x 384), whose quant and header words need the registers of a
// fourth tile's accumulators.  No configuration may spill inside the main loop: IQ1_M
// at 4 tiles reloaded one spilled dword there, into a register the allocator also used
// for an accumulator, and one accumulator tile per wave came out wrong.
constexpr int wide_tn(int type) {
  return type == 14 || type == 13 || type == 11 || type == 21 || type == 22 || type == 29 ? 3 : 4;
}
template <int TYPE>
constexpr int wide_tn() {
  return wide_tn(TYPE);
}
template <int TYPE>
constexpr int wide_bn() {
  return 16 * wide_tn<TYPE>() * kWW;
}
// the grid (in workgroups) from which the wide tile runs: Q6_K from two full
// rounds of the chip (M = 1024, N = 14336: 304 workgroups, 611 -> 551 TFLOP/s)
constexpr int wide_min(int type) { return wide_tn(type) == 3 ? 512 : GGUF_GEMM_WIDE_MIN; }
template <int TYPE>
constexpr int wide_min() {
  return wide_min(TYPE);
}
// every type but IQ3_XXS (685 -> 671 TFLOP/s on the wide tile at M = 2048)
constexpr bool has_wide(int type) {
  return type == 12 || type == 8 || type == 14 || type == 13 || type == 10 || type == 11 ||
         type == 23 || type == 2 || type == 6 || type == 20 || type == 16 || type == 17 ||
         type == 21 || type == 22 || type == 29;
}
template <int TYPE>
constexpr bool has_wide() {
  return has_wide(TYPE);
}
constexpr int kWBM = 16 * kWTM;
constexpr int kWThr = 64 * kWW;
constexpr int kWAI = kWBM * 8 / kWThr;  // 16-byte activation chunks a thread stages per step
constexpr int kWAR = kWThr / 8;         // row distance between them
constexpr int kWStB = kWBM * kRowB;

// The B side of a wide wave tile: kWTN row tiles of 16 weight rows in the
// row-tile layout.  Per type: the code words of the steps ahead (two sets),
// the fields of the current superblock, and the operand build, with the
// arithmetic of gemm_kernel's dequant_b.  Each tile has its own buffer
// resource (none past the weight's end: its loads read zero), and every load
// addresses bytes inside its tile: a request for a unit past the end of K
// re-reads the last unit (its data is never used).
//   begin<C>(u)    at the start of step C of unit u
//   done<C>(j, u)  once both operands of tile j at step C are built
//   bop<C, H>(j)   the B operand of tile j, k-half H of step C
template <int TYPE, int TN>
struct WB;

// Q4_K: set P holds the 8 code bytes of the steps of parity P, requested two
// steps ahead; the header of unit u + 1 is requested at step 2 of unit u.
template <int TN>
struct WB<12, TN> {
  static constexpr int kWTN = TN;
  rsrc_t brs[kWTN];
  int ts, nu;
  BOff bo;
  uint2 cq[2][kWTN];
  uint4 hd[kWTN];
  uint32_t sc[kWTN][2], mn[kWTN][2];
  float d24[kWTN], dmin[kWTN];

  __device__ __forceinline__ void load_codes(int set, int j, int u, int c) {
    cq[set][j] = bl8(brs[j], bo.v1, u * Fmt<12>::TU + (c >> 1) * 1024 + 8 * (c & 1));
  }
  __device__ __forceinline__ void load_hdr(int u) {
#pragma unroll
    for (int j = 0; j < kWTN; ++j) hd[j] = bl16(brs[j], bo.v0, u * Fmt<12>::TU);
  }
  __device__ __forceinline__ void prologue() {
    load_hdr(0);
#pragma unroll
    for (int j = 0; j < kWTN; ++j) {
      load_codes(0, j, 0, 0);
      load_codes(1, j, 0, 1);
    }
  }
  template <int C>
  __device__ __forceinline__ void begin(int u) {
    if (C == 2) load_hdr(min(u + 1, nu - 1));
  }
  template <int C>
  __device__ __forceinline__ void done(int j, int u) {
    const int s2 = 4 * u + C + 2;
    load_codes(C & 1, j, min(s2 >> 2, nu - 1), (C + 2) & 3);
  }
  __device__ __forceinline__ void set_cur() {
#pragma unroll
    for (int j = 0; j < kWTN; ++j) {
      q4k_scales_packed(hd[j].y, hd[j].z, hd[j].w, sc[j][0], sc[j][1], mn[j][0], mn[j][1]);
      const float d = h2f(hd[j].x);
      d24[j] = d * kTwo24;
      dmin[j] = h2f(hd[j].x >> 16);
    }
  }
  // sub-block 2C + H: low (H = 0) or high nibbles of the step's codes
  template <int C, int H>
  __device__ __forceinline__ half8_t bop(int j) const {
    constexpr int Wd = C >> 1, B0 = ((2 * C) & 3) + H;
    // the high nibble enters as 16 q: its scale carries 1/16 (exact)
    const float s = (H ? d24[j] * 0.0625f : d24[j]) * ubyte(sc[j][Wd], B0),
                c = -(dmin[j] * ubyte(mn[j][Wd], B0));
    constexpr uint32_t m = H ? 0x00F000F0u : 0x000F000Fu;
    const uint2 q2 = cq[C & 1][j];
    uint32_t v[4];
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const uint32_t q = w ? q2.y : q2.x, q8 = q >> 8;
      const uint32_t e = q & m, o = q8 & m;
      v[2 * w] = mix_lo(e, o, s, c);
      v[2 * w + 1] = mix_hi(e, o, s, c);
    }
    return h8(v[0], v[1], v[2], v[3]);
  }
};

// Q5_K: Q4_K's codes and header, and the lane's 8 bytes of fifth bits (every
// window's) with the header; they are ORed into the nibbles as gemm_kernel does.
template <int TN>
struct WB<13, TN> {
  static constexpr int kWTN = TN;
  rsrc_t brs[kWTN];
  int ts, nu;
  BOff bo;
  uint2 cq[2][kWTN];
  uint4 hd[kWTN];
  uint2 hqh[kWTN], qh[kWTN];
  uint32_t sc[kWTN][2], mn[kWTN][2];
  float d24[kWTN], dmin[kWTN];

  __device__ __forceinline__ void load_codes(int set, int j, int u, int c) {
    cq[set][j] = bl8(brs[j], bo.v1, u * Fmt<13>::TU + (c >> 1) * 1024 + 8 * (c & 1));
  }
  __device__ __forceinline__ void load_hdr(int u) {
#pragma unroll
    for (int j = 0; j < kWTN; ++j) {
      hd[j] = bl16(brs[j], bo.v0, u * Fmt<13>::TU);
      hqh[j] = bl8(brs[j], bo.v2, u * Fmt<13>::TU);
    }
  }
  __device__ __forceinline__ void prologue() {
    load_hdr(0);
#pragma unroll
    for (int j = 0; j < kWTN; ++j) {
      load_codes(0, j, 0, 0);
      load_codes(1, j, 0, 1);
    }
  }
  template <int C>
  __device__ __forceinline__ void begin(int u) {
    if (C == 2) load_hdr(min(u + 1, nu - 1));
  }
  template <int C>
  __device__ __forceinline__ void done(int j, int u) {
    const int s2 = 4 * u + C + 2;
    load_codes(C & 1, j, min(s2 >> 2, nu - 1), (C + 2) & 3);
  }
  __device__ __forceinline__ void set_cur() {
#pragma unroll
    for (int j = 0; j < kWTN; ++j) {
      q4k_scales_packed(hd[j].y, hd[j].z, hd[j].w, sc[j][0], sc[j][1], mn[j][0], mn[j][1]);
      const float d = h2f(hd[j].x);
      d24[j] = d * kTwo24;
      dmin[j] = h2f(hd[j].x >> 16);
      qh[j] = hqh[j];
    }
  }
  template <int C, int H>
  __device__ __forceinline__ half8_t bop(int j) const {
    constexpr int Wd = C >> 1, B0 = ((2 * C) & 3) + H;
    const float s = (H ? d24[j] * 0.0625f : d24[j]) * ubyte(sc[j][Wd], B0),
                c = -(dmin[j] * ubyte(mn[j][Wd], B0));
    constexpr uint32_t m = H ? 0x00F000F0u : 0x000F000Fu;
    const uint2 q2 = cq[C & 1][j];
    uint32_t v[4];
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const uint32_t q = w ? q2.y : q2.x, q8 = q >> 8, hb = w ? qh[j].y : qh[j].x;
      const uint32_t e = (q & m) | (H ? q5k_hi_even(hb, C) : q5k_lo_even(hb, C));
      const uint32_t o = (q8 & m) | (H ? q5k_hi_odd(hb, C) : q5k_lo_odd(hb, C));
      v[2 * w] = mix_lo(e, o, s, c);
      v[2 * w + 1] = mix_hi(e, o, s, c);
    }
    return h8(v[0], v[1], v[2], v[3]);
  }
};

// Q2_K: the step's 8 qs bytes of half c >> 1 (windows 2c, 2c + 1 take bit
// pairs 2 (w & 3) of them); the header (16 scale bytes, d | dmin << 16).  The
// lane's 8 k of a window lie in scale group 2 w + (g >> 1).
template <int TN>
struct WB<10, TN> {
  static constexpr int kWTN = TN;
  rsrc_t brs[kWTN];
  int ts, nu, lg;
  BOff bo;
  uint2 cq[2][kWTN];
  uint4 hsc[kWTN], sc[kWTN];
  uint32_t hdm[kWTN];
  float d24[kWTN], dmin[kWTN];

  __device__ __forceinline__ void load_codes(int set, int j, int u, int c) {
    cq[set][j] = bl8(brs[j], bo.v0, u * Fmt<10>::TU + 8 * (c >> 1));
  }
  __device__ __forceinline__ void load_hdr(int u) {
#pragma unroll
    for (int j = 0; j < kWTN; ++j) {
      hsc[j] = bl16(brs[j], bo.v1, u * Fmt<10>::TU);
      hdm[j] = bl4(brs[j], bo.v2, u * Fmt<10>::TU);
    }
  }
  __device__ __forceinline__ void prologue() {
    load_hdr(0);
#pragma unroll
    for (int j = 0; j < kWTN; ++j) {
      load_codes(0, j, 0, 0);
      load_codes(1, j, 0, 1);
    }
  }
  template <int C>
  __device__ __forceinline__ void begin(int u) {
    if (C == 2) load_hdr(min(u + 1, nu - 1));
  }
  template <int C>
  __device__ __forceinline__ void done(int j, int u) {
    const int s2 = 4 * u + C + 2;
    load_codes(C & 1, j, min(s2 >> 2, nu - 1), (C + 2) & 3);
  }
  __device__ __forceinline__ void set_cur() {
#pragma unroll
    for (int j = 0; j < kWTN; ++j) {
      sc[j] = hsc[j];
      d24[j] = h2f(hdm[j]) * kTwo24;
      dmin[j] = h2f(hdm[j] >> 16);
    }
  }
  template <int C, int H>
  __device__ __forceinline__ half8_t bop(int j) const {
    constexpr int w = 2 * C + H, sh = 2 * (w & 3);
    const uint32_t scw = (w >> 1) == 0 ? sc[j].x : (w >> 1) == 1 ? sc[j].y : (w >> 1) == 2 ? sc[j].z : sc[j].w;
    const uint32_t sb = (scw >> (8 * (2 * (w & 1) + (lg >> 1)))) & 0xFFu;
    const float s = d24[j] * (float)(sb & 15u), c = -(dmin[j] * (float)(sb >> 4));
    const uint2 q2 = cq[C & 1][j];
    const uint32_t t0 = (q2.x >> sh) & 0x03030303u, t1 = (q2.y >> sh) & 0x03030303u;
    const uint32_t e0 = t0 & 0x00FF00FFu, o0 = (t0 >> 8) & 0x00FF00FFu;
    const uint32_t e1 = t1 & 0x00FF00FFu, o1 = (t1 >> 8) & 0x00FF00FFu;
    return h8(mix_lo(e0, o0, s, c), mix_hi(e0, o0, s, c), mix_lo(e1, o1, s, c), mix_hi(e1, o1, s, c));
  }
};

// Q3_K: as Q2_K, codes q3 = low bits | hmask bit 4 (c >> 1) + (w & 3) << 2,
// value d (sc - 32) (q3 - 4); the header (12 scale bytes, d, the lane's hmask
// bytes 8 g .. 8 g + 7).
template <int TN>
struct WB<11, TN> {
  static constexpr int kWTN = TN;
  rsrc_t brs[kWTN];
  int ts, nu, lg;
  BOff bo;
  uint2 cq[2][kWTN];
  uint32_t hs[kWTN][3], hd[kWTN];
  uint2 hhm[kWTN], hm[kWTN];
  uint32_t S[kWTN][4];
  float d[kWTN];

  __device__ __forceinline__ void load_codes(int set, int j, int u, int c) {
    cq[set][j] = bl8(brs[j], bo.v0, u * Fmt<11>::TU + 8 * (c >> 1));
  }
  __device__ __forceinline__ void load_hdr(int u) {
#pragma unroll
    for (int j = 0; j < kWTN; ++j) {
      const int su = u * Fmt<11>::TU;
      hs[j][0] = bl4(brs[j], bo.v1, su);
      hs[j][1] = bl4(brs[j], bo.v1 + 4, su);
      hs[j][2] = bl4(brs[j], bo.v1 + 8, su);
      hd[j] = bl2(brs[j], bo.v2, su);
      hhm[j] = bl8(brs[j], bo.v3, su);
    }
  }
  __device__ __forceinline__ void prologue() {
    load_hdr(0);
#pragma unroll
    for (int j = 0; j < kWTN; ++j) {
      load_codes(0, j, 0, 0);
      load_codes(1, j, 0, 1);
    }
  }
  template <int C>
  __device__ __forceinline__ void begin(int u) {
    if (C == 2) load_hdr(min(u + 1, nu - 1));
  }
  template <int C>
  __device__ __forceinline__ void done(int j, int u) {
    const int s2 = 4 * u + C + 2;
    load_codes(C & 1, j, min(s2 >> 2, nu - 1), (C + 2) & 3);
  }
  __device__ __forceinline__ void set_cur() {
#pragma unroll
    for (int j = 0; j < kWTN; ++j) {
      q3k_scales(hs[j][0], hs[j][1], hs[j][2], S[j]);
      d[j] = h2f(hd[j]);
      hm[j] = hhm[j];
    }
  }
  template <int C, int H>
  __device__ __forceinline__ half8_t bop(int j) const {
    constexpr int w = 2 * C + H, jj = w & 3, hh = w >> 2;
    const uint32_t sb = (S[j][w >> 1] >> (8 * (2 * (w & 1) + (lg >> 1)))) & 0xFFu;
    const float dl = d[j] * (float)((int)sb - 32);
    const float s = dl * kTwo24, c = -4.0f * dl;
    const uint2 q2 = cq[C & 1][j];
    const uint32_t t0 = ((q2.x >> (2 * jj)) & 0x03030303u) | (((hm[j].x >> (4 * hh + jj)) & 0x01010101u) << 2);
    const uint32_t t1 = ((q2.y >> (2 * jj)) & 0x03030303u) | (((hm[j].y >> (4 * hh + jj)) & 0x01010101u) << 2);
    const uint32_t e0 = t0 & 0x00FF00FFu, o0 = (t0 >> 8) & 0x00FF00FFu;
    const uint32_t e1 = t1 & 0x00FF00FFu, o1 = (t1 >> 8) & 0x00FF00FFu;
    return h8(mix_lo(e0, o0, s, c), mix_hi(e0, o0, s, c), mix_lo(e1, o1, s, c), mix_hi(e1, o1, s, c));
  }
};

// IQ4_XS: step c is sub-blocks 2c, 2c + 1 (the lane's code words, one each),
// each an IQ4_NL block with scale d (ls - 32); the header (d | scales_h << 16,
// scales_l[4]).
template <int TN>
struct WB<23, TN> {
  static constexpr int kWTN = TN;
  rsrc_t brs[kWTN];
  int ts, nu;
  BOff bo;
  uint2 cq[2][kWTN];
  uint2 hhd[kWTN], hd[kWTN];
  float d[kWTN];

  __device__ __forceinline__ void load_codes(int set, int j, int u, int c) {
    cq[set][j] = bl8(brs[j], bo.v1, u * Fmt<23>::TU + 8 * c);
  }
  __device__ __forceinline__ void load_hdr(int u) {
#pragma unroll
    for (int j = 0; j < kWTN; ++j) hhd[j] = bl8(brs[j], bo.v0, u * Fmt<23>::TU);
  }
  __device__ __forceinline__ void prologue() {
    load_hdr(0);
#pragma unroll
    for (int j = 0; j < kWTN; ++j) {
      load_codes(0, j, 0, 0);
      load_codes(1, j, 0, 1);
    }
  }
  template <int C>
  __device__ __forceinline__ void begin(int u) {
    if (C == 2) load_hdr(min(u + 1, nu - 1));
  }
  template <int C>
  __device__ __forceinline__ void done(int j, int u) {
    const int s2 = 4 * u + C + 2;
    load_codes(C & 1, j, min(s2 >> 2, nu - 1), (C + 2) & 3);
  }
  __device__ __forceinline__ void set_cur() {
#pragma unroll
    for (int j = 0; j < kWTN; ++j) {
      hd[j] = hhd[j];
      d[j] = h2f(hhd[j].x);
    }
  }
  template <int C, int H>
  __device__ __forceinline__ half8_t bop(int j) const {
    const float dl = d[j] * (float)((int)iq4xs_ls(hd[j].x >> 16, hd[j].y, 2 * C + H) - 32);
    const float s = dl * kTwo24, c = -128.0f * dl;
    const uint2 q2 = cq[C & 1][j];
    uint32_t w[4];
    b32_codes<20>(H ? q2.y : q2.x, 0u, w);
    return h8(mix_lo(w[0], w[1], s, c), mix_hi(w[0], w[1], s, c), mix_lo(w[2], w[3], s, c),
              mix_hi(w[2], w[3], s, c));
  }
};

// Q8_0: step c of unit u (256 elements) is blocks 8 u + 2 c + H; set P holds
// their codes and d for the steps of parity P, requested two steps ahead.
template <int TN>
struct WB<8, TN> {
  static constexpr int kWTN = TN;
  rsrc_t brs[kWTN];
  int ts, nu;
  BOff bo;
  uint2 cq[2][kWTN][2];
  uint32_t dq[2][kWTN][2];

  __device__ __forceinline__ void load_codes(int set, int j, int u, int c) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int so = (8 * u + 2 * c + h) * Fmt<8>::TU;
      cq[set][j][h] = bl8(brs[j], bo.v0, so);
      dq[set][j][h] = bl2(brs[j], bo.v1, so);
    }
  }
  __device__ __forceinline__ void prologue() {
#pragma unroll
    for (int j = 0; j < kWTN; ++j) {
      load_codes(0, j, 0, 0);
      load_codes(1, j, 0, 1);
    }
  }
  template <int C>
  __device__ __forceinline__ void begin(int) {}
  template <int C>
  __device__ __forceinline__ void done(int j, int u) {
    const int s2 = 4 * u + C + 2;
    load_codes(C & 1, j, min(s2 >> 2, nu - 1), (C + 2) & 3);
  }
  __device__ __forceinline__ void set_cur() {}
  // code + 128 enters as a subnormal: fp16(d q) rounded once
  template <int C, int H>
  __device__ __forceinline__ half8_t bop(int j) const {
    const float d = h2f(dq[C & 1][j][H]);
    const float s = d * kTwo24, c = -128.0f * d;
    const uint2 q2 = cq[C & 1][j][H];
    uint32_t v[4];
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const uint32_t q = (w ? q2.y : q2.x) ^ 0x80808080u;
      const uint32_t ev = q & 0x00FF00FFu, od = (q >> 8) & 0x00FF00FFu;
      v[2 * w] = mix_lo(ev, od, s, c);
      v[2 * w + 1] = mix_hi(ev, od, s, c);
    }
    return h8(v[0], v[1], v[2], v[3]);
  }
};

// Q6_K: steps 2 HF and 2 HF + 1 of a unit use the same 6 quant dwords of half
// HF (set HF), requested for unit u + 1 once step 2 HF + 1 of unit u has built
// the tile's operands (three steps ahead).  The step's scale dword (4 of the 16
// int8 scales) is requested two steps ahead with set P of the steps of parity
// P, the d of unit u + 1 at step 2 of unit u.  The lane's operand for k-half t2
// holds the window columns 32 t2 + 16 lh + 4 g + e at position 4 lh + e (the
// activations are staged in that order).
template <int TN>
struct WB<14, TN> {
  static constexpr int kWTN = TN;
  rsrc_t brs[kWTN];
  int ts, nu;
  BOff bo;
  uint32_t dq[2][kWTN][6];  // half HF: dwords 3 lh + i (i = 0, 1 low bits, 2 high bits)
  uint32_t scq[2][kWTN];    // scale dword of the steps of parity P
  uint32_t hd[kWTN];        // d of the next unit
  float d[kWTN];            // d of the current unit

  // half HF's dwords 6 HF .. 6 HF + 5 of the lane's 12, from pieces of 16 bytes
  __device__ __forceinline__ void load_half(int hf, int j, int u) {
    const int su = u * Fmt<14>::TU;
    if (hf == 0) {
      const uint4 a = bl16(brs[j], bo.v0, su);
      const uint2 b = bl8(brs[j], bo.v0, su + 1024);
      dq[0][j][0] = a.x; dq[0][j][1] = a.y; dq[0][j][2] = a.z;
      dq[0][j][3] = a.w; dq[0][j][4] = b.x; dq[0][j][5] = b.y;
    } else {
      const uint2 a = bl8(brs[j], bo.v0, su + 1024 + 8);
      const uint4 b = bl16(brs[j], bo.v0, su + 2048);
      dq[1][j][0] = a.x; dq[1][j][1] = a.y; dq[1][j][2] = b.x;
      dq[1][j][3] = b.y; dq[1][j][4] = b.z; dq[1][j][5] = b.w;
    }
  }
  __device__ __forceinline__ void load_scale(int set, int j, int u, int c) {
    scq[set][j] = bl4(brs[j], bo.v2, u * Fmt<14>::TU + 4 * c);
  }
  __device__ __forceinline__ void load_d(int u) {
#pragma unroll
    for (int j = 0; j < kWTN; ++j) hd[j] = bl2(brs[j], bo.v1, u * Fmt<14>::TU);
  }
  __device__ __forceinline__ void prologue() {
    load_d(0);
#pragma unroll
    for (int j = 0; j < kWTN; ++j) {
      load_half(0, j, 0);
      load_half(1, j, 0);
      load_scale(0, j, 0, 0);
      load_scale(1, j, 0, 1);
    }
  }
  template <int C>
  __device__ __forceinline__ void begin(int u) {
    if (C == 2) load_d(min(u + 1, nu - 1));
  }
  template <int C>
  __device__ __forceinline__ void done(int j, int u) {
    const int s2 = 4 * u + C + 2;
    load_scale(C & 1, j, min(s2 >> 2, nu - 1), (C + 2) & 3);
    if (C & 1) load_half(C >> 1, j, min(u + 1, nu - 1));
  }
  __device__ __forceinline__ void set_cur() {
#pragma unroll
    for (int j = 0; j < kWTN; ++j) d[j] = h2f(hd[j]);
  }
  template <int C, int H>
  __device__ __forceinline__ half8_t bop(int j) const {
    constexpr int HF = C >> 1, TP = C & 1, t = 2 * TP + H;
    const uint32_t scw = scq[C & 1][j];
    uint32_t v[4];
#pragma unroll
    for (int lh = 0; lh < 2; ++lh) {
      const uint32_t ql = dq[HF][j][3 * lh + (t & 1)], qh = dq[HF][j][3 * lh + 2];
      const uint32_t n4 = (t >> 1) ? ((ql >> 4) & 0x0F0F0F0Fu) : (ql & 0x0F0F0F0Fu);
      const uint32_t q6 = n4 | (((qh >> (2 * t)) & 0x03030303u) << 4);
      const uint32_t ev = q6 & 0x00FF00FFu, od = (q6 >> 8) & 0x00FF00FFu;
      const float sv = d[j] * (float)(int8_t)((scw >> (8 * (2 * H + lh))) & 0xFFu);
      const float s = sv * kTwo24, c = -32.0f * sv;
      v[2 * lh] = mix_lo(ev, od, s, c);
      v[2 * lh + 1] = mix_hi(ev, od, s, c);
    }
    return h8(v[0], v[1], v[2], v[3]);
  }
};

// Q4_0 / Q5_0 / IQ4_NL: as Q8_0, the step's blocks 8 u + 2 c + H; per block
// the lane's code word, the f16 d and (Q5_0) the row's fifth-bit word.
template <int T, int TN>
struct WB32 {
  static constexpr int kWTN = TN;
  rsrc_t brs[kWTN];
  int ts, nu, lg;
  BOff bo;
  uint32_t cq[2][kWTN][2], dq[2][kWTN][2], hq[2][kWTN][T == 6 ? 2 : 1];

  __device__ __forceinline__ void load_codes(int set, int j, int u, int c) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int so = (8 * u + 2 * c + h) * Fmt<T>::TU;
      cq[set][j][h] = bl4(brs[j], bo.v0, so);
      dq[set][j][h] = bl2(brs[j], bo.v1, so);
      if constexpr (T == 6) hq[set][j][h] = bl4(brs[j], bo.v2, so);
    }
  }
  __device__ __forceinline__ void prologue() {
#pragma unroll
    for (int j = 0; j < kWTN; ++j) {
      load_codes(0, j, 0, 0);
      load_codes(1, j, 0, 1);
    }
  }
  template <int C>
  __device__ __forceinline__ void begin(int) {}
  template <int C>
  __device__ __forceinline__ void done(int j, int u) {
    const int s2 = 4 * u + C + 2;
    load_codes(C & 1, j, min(s2 >> 2, nu - 1), (C + 2) & 3);
  }
  __device__ __forceinline__ void set_cur() {}
  // the code minus the type's offset, times d, rounded once to fp16
  template <int C, int H>
  __device__ __forceinline__ half8_t bop(int j) const {
    const float d = h2f(dq[C & 1][j][H]);
    const float s = d * kTwo24, c = -code_offset<T>() * d;
    uint32_t qhb = 0;
    if constexpr (T == 6) qhb = (hq[C & 1][j][H] >> (8 * lg)) & 0xFFu;
    uint32_t w[4];
    b32_codes<T>(cq[C & 1][j][H], qhb, w);
    return h8(mix_lo(w[0], w[1], s, c), mix_hi(w[0], w[1], s, c), mix_lo(w[2], w[3], s, c),
              mix_hi(w[2], w[3], s, c));
  }
};
// The grid-codebook IQ types: set P holds, per tile, the record words of the
// window of the steps of parity P (iq_load_window), requested two steps
// ahead; the operand is built from the workgroup's tables in shared memory
// (iq_b) and rounded once with the unit scale, as in gemm_kernel.
template <int T, int TN>
struct WBIq {
  static constexpr int kWTN = TN;
  rsrc_t brs[kWTN];
  int ts, nu, lg;
  BOff bo;
  const unsigned char *tb;
  IqUnit<T> cu[2][kWTN];
  uint32_t hd[kWTN];
  float us[kWTN];

  template <int C>
  __device__ __forceinline__ void load_win(int j, int u) {
    iq_load_window<C, T>(brs[j], bo.v0, u * Fmt<T>::TU, cu[C & 1][j].w);
  }
  __device__ __forceinline__ void load_hdr(int u) {
    if constexpr (T != 29)
#pragma unroll
      for (int j = 0; j < kWTN; ++j) hd[j] = bl2(brs[j], bo.v1, u * Fmt<T>::TU);
  }
  __device__ __forceinline__ void prologue() {
    load_hdr(0);
#pragma unroll
    for (int j = 0; j < kWTN; ++j) {
      load_win<0>(j, 0);
      load_win<1>(j, 0);
    }
  }
  template <int C>
  __device__ __forceinline__ void begin(int u) {
    if (C == 2) load_hdr(min(u + 1, nu - 1));
  }
  template <int C>
  __device__ __forceinline__ void done(int j, int u) {
    load_win<(C + 2) & 3>(j, min((4 * u + C + 2) >> 2, nu - 1));
  }
  __device__ __forceinline__ void set_cur() {
    if constexpr (T != 29)
#pragma unroll
      for (int j = 0; j < kWTN; ++j) us[j] = h2f(hd[j]) * iq_d_factor<T>();
  }
  template <int C, int H>
  __device__ __forceinline__ half8_t bop(int j) const {
    const float s = T == 29 ? iq_unit_scale<T>(cu[C & 1][j]) : us[j];
    const uint4 v = __builtin_bit_cast(uint4, iq_b<T>(cu[C & 1][j], 2 * C + H, lg, tb));
    return h8(mix_w(v.x, s), mix_w(v.y, s), mix_w(v.z, s), mix_w(v.w, s));
  }
};
template <int TN>
struct WB<16, TN> : WBIq<16, TN> {};
template <int TN>
struct WB<17, TN> : WBIq<17, TN> {};
template <int TN>
struct WB<18, TN> : WBIq<18, TN> {};
template <int TN>
struct WB<21, TN> : WBIq<21, TN> {};
template <int TN>
struct WB<22, TN> : WBIq<22, TN> {};
template <int TN>
struct WB<29, TN> : WBIq<29, TN> {};

template <int TN>
struct WB<2, TN> : WB32<2, TN> {};
template <int TN>
struct WB<6, TN> : WB32<6, TN> {};
template <int TN>
struct WB<20, TN> : WB32<20, TN> {};

template <int TYPE, int TN>
struct Wide : WB<TYPE, TN> {
  static constexpr int kWTN = TN;
  rsrc_t ars[kWAI];  // rows m0 + kWAR i + (0 .. kWAR - 1)
  int av, row0, cc, K, af0, af1;
  uint4 ar[kWAI];
  float4_t acc[kWTM][kWTN];
  unsigned char *lds;

  // the row within its resource is in the vector offset (rows past M read as
  // zero); the k offset stops at the last step (steps past K are never staged)
  __device__ __forceinline__ void load_a(int k0) {
    const int so = 2 * min(k0, K - 64);
#pragma unroll
    for (int i = 0; i < kWAI; ++i) ar[i] = bl16(ars[i], av, so);
  }
  __device__ __forceinline__ void store_a(int stage) {
    unsigned char *base = lds + stage * kWStB;
#pragma unroll
    for (int i = 0; i < kWAI; ++i) {
      const int row = row0 + kWAR * i;
      if constexpr (TYPE == 14) {
        // columns 8 q + e (q = cc & 3) of k-block cc >> 2 go to position
        // 8 g + 4 lh + (e & 3) with g = 2 (q & 1) + (e >> 2), lh = q >> 1
        const int q = cc & 3, ch = 4 * (cc >> 2) + 2 * (q & 1), half = 8 * (q >> 1);
        *(uint2 *)(base + lds_at(row, ch) + half) = make_uint2(ar[i].x, ar[i].y);
        *(uint2 *)(base + lds_at(row, ch + 1) + half) = make_uint2(ar[i].z, ar[i].w);
      } else {
        *(uint4 *)(base + lds_at(row, cc)) = ar[i];
      }
    }
  }

  // step s = 4 u + C: A from stage s & 3 (= C).  First the A of step s + 2
  // (loaded during step s - 1) goes to stage (s + 2) & 3 and step s + 3's A is
  // requested; then k-half by k-half the fragments of this step, each tile's B
  // operand built before its 8 MFMAs and the tile's codes ahead requested once
  // both halves are built.  A barrier after odd steps only: stage (s + 2) & 3
  // was last read at step s - 2 and is next read at step s + 2, and a barrier
  // at the end of an odd step lies between each pair.
  template <int C>
  __device__ __forceinline__ void step(int u) {
    const int s = 4 * u + C;
    store_a((C + 2) & 3);
    load_a(64 * (s + 3));
    this->template begin<C>(u);
    const unsigned char *base = lds + C * kWStB;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      half8_t a[kWTM];
#pragma unroll
      for (int i = 0; i < kWTM; ++i) a[i] = *(const half8_t *)(base + (h ? af1 : af0) + i * 16 * kRowB);
#pragma unroll
      for (int j = 0; j < kWTN; ++j) {
        const half8_t b = h ? this->template bop<C, 1>(j) : this->template bop<C, 0>(j);
        if (h == 1) this->template done<C>(j, u);
#pragma unroll
        for (int i = 0; i < kWTM; ++i) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b, acc[i][j], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);  // one half's fragments live at a time
    }
    if (C & 1) __syncthreads();
  }
};

// K a multiple of 256; TN weight row tiles per wave (a workgroup tile of
// 128 x 128 TN).
template <int TYPE, typename XT, int TN>
__global__ __launch_bounds__(kWThr) void gemm_wide(const XT *__restrict__ x, int64_t ldx,
                                                  const uint8_t *__restrict__ W, int M, int N,
                                                  int K, float *__restrict__ y, int64_t ldy,
                                                  int tiles_m, const float *__restrict__ rowf) {
  constexpr int kWTN = TN;
  __shared__ __align__(16) unsigned char lds[4 * kWStB];
  // IQ types: the decode tables, requested first and written before the first barrier
  __shared__ __align__(16) unsigned char iqtbl[is_iq(TYPE) ? iq_tbl_bytes<TYPE>() : 16];
  IqTabRegs<TYPE, kWThr> tab;
  if constexpr (is_iq(TYPE)) iq_get_tables<TYPE, kWThr>(tab);
  int bid = blockIdx.x;
  if ((gridDim.x & 7) == 0) bid = (bid & 7) * (gridDim.x >> 3) + (bid >> 3);
  int m0, n0;
  {
    const int band = bid / (tiles_m * GGUF_GEMM_GN), in = bid - band * tiles_m * GGUF_GEMM_GN;
    const int tiles_n = (int)gridDim.x / tiles_m;
    const int gn = min(GGUF_GEMM_GN, tiles_n - band * GGUF_GEMM_GN);
    m0 = (in / gn) * kWBM;
    n0 = (band * GGUF_GEMM_GN + in % gn) * (16 * TN * kWW);
  }
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  Wide<TYPE, TN> s;
  s.lds = lds;
  s.K = K;
  s.nu = K / 256;
  s.ts = (K / Fmt<TYPE>::UE) * Fmt<TYPE>::TU;
  const int ntiles = (N + 15) >> 4, t0 = __builtin_amdgcn_readfirstlane((n0 >> 4) + kWTN * wave);
#pragma unroll
  for (int j = 0; j < kWTN; ++j)  // tile t0 + j, or none past the weight's end
    s.brs[j] = make_rsrc(W + (int64_t)min(t0 + j, ntiles - 1) * s.ts, t0 + j < ntiles ? s.ts : 0);
  s.bo = b_offsets<TYPE>(r, g);
  if constexpr (TYPE == 10 || TYPE == 11 || TYPE == 6 || is_iq(TYPE)) s.lg = g;
  const int rows = min(kWBM, M - m0);
  const int64_t ldxb = ldx * (int64_t)sizeof(XT);
#pragma unroll
  for (int i = 0; i < kWAI; ++i) {  // rows m0 + kWAR i .. of which ri exist
    const int ri = rows - kWAR * i;
    s.ars[i] = make_rsrc(x + (int64_t)(m0 + min(kWAR * i, rows - 1)) * ldx,
                         ri > 0 ? (int)((int64_t)(ri - 1) * ldxb + (int64_t)K * sizeof(XT)) : 0);
  }
  s.row0 = tid >> 3;
  s.cc = tid & 7;
  s.av = (int)(s.row0 * ldxb) + s.cc * 16;
  s.af0 = lds_at(r, g);
  s.af1 = lds_at(r, 4 + g);
#pragma unroll
  for (int i = 0; i < kWTM; ++i)
#pragma unroll
    for (int j = 0; j < kWTN; ++j) s.acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};
  // prologue: header of unit 0 and the codes of its first steps, A of steps 0
  // and 1 into stages 0 and 1, A of step 2 requested
  s.prologue();
  s.load_a(0);
  s.store_a(0);
  s.load_a(64);
  s.store_a(1);
  s.load_a(128);
  if constexpr (is_iq(TYPE)) {
    iq_put_tables<TYPE, kWThr>(tab, iqtbl);
    s.tb = iqtbl;
  }
  __syncthreads();
  for (int u = 0; u < s.nu; ++u) {
    s.set_cur();
    s.template step<0>(u);
    s.template step<1>(u);
    s.template step<2>(u);
    s.template step<3>(u);
  }
  // rowf (staged f32 rows): the rows' inverse scales 2^-e, kWBM of them per
  // row tile (entries past M are read, not used)
#pragma unroll
  for (int i = 0; i < kWTM; ++i) {
    float4 f = make_float4(1.f, 1.f, 1.f, 1.f);
    if (rowf) f = *(const float4 *)(rowf + m0 + 16 * i + 4 * g);
    const float fe[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
    for (int j = 0; j < kWTN; ++j) {
      const int n = n0 + 16 * (kWTN * wave + j) + r;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + 16 * i + 4 * g + e;
        if (m < M && n < N) y[(int64_t)m * ldy + n] = s.acc[i][j][e] * fe[e];
      }
    }
  }
}

// f32 activation rows -> the fp16 image the GEMM kernels read: row m times
// 2^e, e = stage_exp of the row's largest magnitude, rounded to fp16, and
// rowf[m] = 2^-e.  The same values gemm_kernel stages in LDS for f32 input
// (the row maximum, exact, does not depend on the reduction order), so both
// paths give the same result bit for bit.  One workgroup of NT threads per
// row; with NC > 0 the row (K <= 4 NT NC) is loaded once into registers, all
// loads in flight together, otherwise it is read twice.  K % 8 == 0, x rows
// 16-byte aligned.
template <int NT, int NC>
__global__ __launch_bounds__(NT) void stage_rows_kernel(const float *__restrict__ x, int64_t ldx,
                                                        int K, half_t *__restrict__ img,
                                                        float *__restrict__ rowf) {
  __shared__ float wmx[NT / 64];
  const int m = blockIdx.x, tid = threadIdx.x, K4 = K / 4;
  const float4 *xr = (const float4 *)(x + (int64_t)m * ldx);
  uint2 *ir = (uint2 *)(img + (int64_t)m * K);  // four fp16 values per float4 of x
  float4 v[NC > 0 ? NC : 1];
  float mx = 0.f;
  if constexpr (NC > 0) {
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = tid + NT * i;
      v[i] = c < K4 ? xr[c] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int i = 0; i < NC; ++i)
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
  } else {
    for (int c = tid; c < K4; c += NT) {
      const float4 a = xr[c];
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
    }
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((tid & 63) == 0) wmx[tid >> 6] = mx;
  __syncthreads();
  mx = wmx[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) mx = fmaxf(mx, wmx[w]);
  const int e = stage_exp(mx);
  const float sc = pow2f(e);
  if (tid == 0) rowf[m] = pow2f(-e);
  auto put = [&](int c, const float4 &a) {
    half4_t h;
    h[0] = (half_t)(a.x * sc);
    h[1] = (half_t)(a.y * sc);
    h[2] = (half_t)(a.z * sc);
    h[3] = (half_t)(a.w * sc);
    ir[c] = __builtin_bit_cast(uint2, h);
  };
  if constexpr (NC > 0) {
#pragma unroll
    for (int i = 0; i < NC; ++i)
      if (tid + NT * i < K4) put(tid + NT * i, v[i]);
  } else {
    for (int c = tid; c < K4; c += NT) put(c, xr[c]);
  }
}

hipError_t launch_stage_rows(const float *x, int64_t ldx, int M, int K, half_t *img, float *rowf,
                             hipStream_t s) {
  const dim3 g((unsigned)M);
  if (K <= 2048)
    hipLaunchKernelGGL((stage_rows_kernel<256, 2>), g, dim3(256), 0, s, x, ldx, K, img, rowf);
  else if (K <= 4096)
    hipLaunchKernelGGL((stage_rows_kernel<256, 4>), g, dim3(256), 0, s, x, ldx, K, img, rowf);
  else if (K <= 8192)
    hipLaunchKernelGGL((stage_rows_kernel<256, 8>), g, dim3(256), 0, s, x, ldx, K, img, rowf);
  else if (K <= 16384)
    hipLaunchKernelGGL((stage_rows_kernel<1024, 4>), g, dim3(1024), 0, s, x, ldx, K, img, rowf);
  else if (K <= 32768)
    hipLaunchKernelGGL((stage_rows_kernel<1024, 8>), g, dim3(1024), 0, s, x, ldx, K, img, rowf);
  else
    hipLaunchKernelGGL((stage_rows_kernel<1024, 0>), g, dim3(1024), 0, s, x, ldx, K, img, rowf);
  return hipGetLastError();
}

// Workspace floats of the staged f32 rows: M inverse row scales, padded to
// whole 128-row tiles, then the M x K fp16 image.
static_assert(kWBM == kBM, "both GEMM kernels read kBM row scales per row tile");
int64_t stage_floats(int64_t m, int64_t k) { return (m + kBM - 1) / kBM * kBM + m * k / 2; }

// Compute units of the current device (256 on MI355X), read once per device.
int device_cus() {
  static int cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] <= 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
      v = 256;
    cus[dev] = v;
  }
  return cus[dev];
}

// The wide tile's launch plan over wn column tiles.  Its workgroups hold a
// CU each for about the same time, so a grid of wm x wn runs in
// ceil(wm wn / CUs) rounds.  When the last round is partly empty, the wide
// launch keeps the columns of its whole rounds and the rest goes to
// gemm_kernel (128 x 256 tiles, one K range) or, for Q4_K and Q8_0, to
// their three-tile wide tile, whichever the round estimate says ends sooner by a
// twentieth of a round.  A round of gemm_kernel takes 0.52 of a four-tile
// wide round and 0.81 of a three-tile one, a three-tile round 0.91 of a
// four-tile one (measured: Q4_K 134 against 69 us, Q6_K 121 against 98 us,
// Q4_K 145 against 132 us).  Q6_K at M = 2048, N = 14336: 608 workgroups (3
// rounds, the last 37.5% full) -> 512 + 128 of gemm_kernel, 656-663 ->
// 684-696 TFLOP/s; Q4_K M = 4096 896-906 -> 933-945, M = 1536 685 -> 761-785
// (gemm_kernel); Q4_K M = 2048 (448: 2 rounds) -> 256 + 256 three-tile
// workgroups, 826-831 -> 866 (with gemm_kernel for the rest: 802-808).
#ifndef GGUF_GEMM_WIDE_SPLIT
#define GGUF_GEMM_WIDE_SPLIT 1  // 0: the wide tile covers every column
#endif
#ifndef GGUF_GEMM_RHO3
#define GGUF_GEMM_RHO3 0.91  // a round of three-tile workgroups against one of four-tile ones
#endif
// Q4_K and Q8_0 also have a three-tile wide tile for the columns past the
// whole rounds (exact against gemm_kernel and repeatable at M = 2048, N =
// 14336).  The other four-tile types do not use theirs: the three-tile builds
// of IQ4_NL and IQ2_XS gave wrong values in a few percent of the elements,
// different from call to call (M = 2048, N = 14336, K = 4096), while those of
// Q4_0, Q5_0, Q2_K, IQ4_XS and IQ2_XXS matched.  The compiled loop of the
// IQ4_NL build shows no read of, or write to, a register with a load
// outstanding; the cause is not known.
template <int TYPE>
constexpr bool has_wide3() {
  return TYPE == 12 || TYPE == 8;
}
// Q6_K, Q5_K and Q3_K (three tiles per wave) have a two-tile wide tile for
// those columns.
template <int TYPE>
constexpr bool has_wide2() {
  return TYPE == 14 || TYPE == 13 || TYPE == 11;
}
#ifndef GGUF_GEMM_RHO2
#define GGUF_GEMM_RHO2 0.7  // a round of two-tile workgroups against one of three-tile ones
#endif
struct WidePlan {
  int wn1;   // column tiles of the wide launch
  int rest;  // the columns past them: 0 none, 1 gemm_kernel, 2 / 3 the three- / two-tile wide tile
};
WidePlan wide_plan(int wm, int wn, int M, int N, int tn, bool three, bool two) {
  WidePlan p{wn, 0};
  if (!GGUF_GEMM_WIDE_SPLIT) return p;
  const int64_t cus = device_cus(), g = (int64_t)wm * wn;
  const int64_t r = g / cus, rounds = (g + cus - 1) / cus;
  if (r < 1 || g % cus == 0) return p;
  const int w1 = (int)(r * cus / wm);
  if (w1 < 1 || w1 >= wn) return p;
  const int64_t left = N - (int64_t)w1 * 16 * tn * kWW;
  double best = (double)rounds - 0.05;
  const int64_t gk = (int64_t)((M + kBM - 1) / kBM) * ((left + kBN - 1) / kBN);
  const double ck = (double)r + (double)((gk + cus - 1) / cus) * (tn == 3 ? 0.81 : 0.52);
  if (ck < best) {
    best = ck - 0.05;
    p = WidePlan{w1, 1};
  }
  if (three) {
    const int64_t g3 = (int64_t)wm * ((left + 16 * 3 * kWW - 1) / (16 * 3 * kWW));
    const double c3 = (double)r + (double)((g3 + cus - 1) / cus) * GGUF_GEMM_RHO3;
    if (c3 < best) p = WidePlan{w1, 2};
  }
  if (two) {
    const int64_t g2 = (int64_t)wm * ((left + 16 * 2 * kWW - 1) / (16 * 2 * kWW));
    const double c2 = (double)r + (double)((g2 + cus - 1) / cus) * GGUF_GEMM_RHO2;
    if (c2 < best) p = WidePlan{w1, 3};
  }
  return p;
}

// rowf: the rows' inverse scales when x is the fp16 image of f32 rows.
template <int TYPE, typename XT>
hipError_t launch_type(const XT *x, int64_t ldx, const uint8_t *W, int M, int N, int K, float *y,
                       int64_t ldy, float *work, int64_t work_floats, hipStream_t s,
                       const float *rowf = nullptr) {
  if constexpr (sizeof(XT) == 4) {
    // f32 activations with room for their fp16 image: stage the rows once,
    // then the fp16 kernels run on the image (the K split's partial sums, if
    // any, follow it in the workspace)
    const int64_t sf = stage_floats(M, K);
    if (work && work_floats >= sf) {
      half_t *img = (half_t *)(work + (sf - (int64_t)M * K / 2));
      const hipError_t e = launch_stage_rows(x, ldx, M, K, img, work, s);
      if (e != hipSuccess) return e;
      return launch_type<TYPE, half_t>(img, (int64_t)K, W, M, N, K, y, ldy, work + sf,
                                       work_floats - sf, s, work);
    }
  }
  if constexpr (has_wide<TYPE>() && sizeof(XT) == 2) {
    // fp16 activations on a grid that fills the chip: the wide tile
    constexpr int bn = wide_bn<TYPE>();
    const int wm = (M + kWBM - 1) / kWBM, wn = (N + bn - 1) / bn;
    if ((int64_t)wm * wn >= wide_min<TYPE>() && K % 256 == 0) {
      const WidePlan pl =
          wide_plan(wm, wn, M, N, wide_tn<TYPE>(), has_wide3<TYPE>(), has_wide2<TYPE>());
      const int n1 = min(N, pl.wn1 * bn);
      hipLaunchKernelGGL((gemm_wide<TYPE, XT, wide_tn<TYPE>()>), dim3((unsigned)(wm * pl.wn1)),
                         dim3(kWThr), 0, s, x, ldx, W, M, n1, K, y, ldy, wm, rowf);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess || n1 == N) return e;
      // the columns past the wide tile's whole rounds: the three-tile wide tile
      // or gemm_kernel with one K range (the same bits per element either way)
      const int64_t ts = (int64_t)(K / Fmt<TYPE>::UE) * Fmt<TYPE>::TU;
      if constexpr (has_wide3<TYPE>()) {
        if (pl.rest == 2) {
          const int wn3 = (N - n1 + 16 * 3 * kWW - 1) / (16 * 3 * kWW);
          hipLaunchKernelGGL((gemm_wide<TYPE, XT, 3>), dim3((unsigned)(wm * wn3)), dim3(kWThr), 0,
                             s, x, ldx, W + (int64_t)(n1 / 16) * ts, M, N - n1, K, y + n1, ldy, wm,
                             rowf);
          return hipGetLastError();
        }
      }
      if constexpr (has_wide2<TYPE>()) {
        if (pl.rest == 3) {
          const int wn2 = (N - n1 + 16 * 2 * kWW - 1) / (16 * 2 * kWW);
          hipLaunchKernelGGL((gemm_wide<TYPE, XT, 2>), dim3((unsigned)(wm * wn2)), dim3(kWThr), 0,
                             s, x, ldx, W + (int64_t)(n1 / 16) * ts, M, N - n1, K, y + n1, ldy, wm,
                             rowf);
          return hipGetLastError();
        }
      }
      const int tm = (M + kBM - 1) / kBM, tn = (N - n1 + kBN - 1) / kBN;
      hipLaunchKernelGGL((gemm_kernel<TYPE, XT>), dim3((unsigned)(tm * tn), 1u), dim3(kThreads), 0,
                         s, x, ldx, W + (int64_t)(n1 / 16) * ts, M, N - n1, K, y + n1, ldy, tm,
                         K / Fmt<TYPE>::UE, rowf);
      return hipGetLastError();
    }
  }
  const int tiles_m = (M + kBM - 1) / kBM, tiles_n = (N + kBN - 1) / kBN, nu = K / Fmt<TYPE>::UE;
  // sp ranges of kunits superblocks each (the last one shorter); the
  // workspace is checked against the rounded count, the one
  // launch_gemm_work sizes it for
  int sp = gemm_splits(TYPE, (int64_t)tiles_m * tiles_n, nu);
  int kunits = (nu + sp - 1) / sp;
  sp = (nu + kunits - 1) / kunits;
  if (!work || work_floats < (int64_t)sp * M * N) {
    sp = 1;
    kunits = nu;
  }
  hipLaunchKernelGGL((gemm_kernel<TYPE, XT>), dim3((unsigned)(tiles_m * tiles_n), (unsigned)sp),
                     dim3(kThreads), 0, s, x, ldx, W, M, N, K, sp > 1 ? work : y,
                     sp > 1 ? (int64_t)N : ldy, tiles_m, kunits, rowf);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || sp == 1) return e;
  const int64_t mn = (int64_t)M * N;
  if (N % 4 == 0 && ldy % 4 == 0 && ((uintptr_t)y & 15) == 0 && ((uintptr_t)work & 15) == 0)
    hipLaunchKernelGGL(gemm_reduce4_kernel, dim3((unsigned)((mn / 4 + 255) / 256)), dim3(256), 0, s,
                       (const float4 *)work, sp, M, N / 4, y, ldy);
  else
    hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, s, work,
                       sp, M, N, y, ldy);
  return hipGetLastError();
}

template <typename XT>
hipError_t launch_x(const XT *x, int64_t ldx, const uint8_t *W, int type, int64_t n, int64_t k,
                    float *y, int64_t ldy, int64_t m, float *work, int64_t work_floats,
                    hipStream_t s) {
  hipError_t e;
  if (type == 12)
    e = launch_type<12, XT>(x, ldx, W, (int)m, (int)n, (int)k, y, ldy, work, work_floats, s);
  else if (type == 13)
    e = launch_type<13, XT>(x, ldx, W, (int)m, (int)n, (int)k, y, ldy, work, work_floats, s);
  else if (type == 8)
    e = launch_type<8, XT>(x, ldx, W, (int)m, (int)n, (int)k, y, ldy, work, work_floats, s);
  else if (type == 2)
    e = launch_type<2, XT>(x, ldx, W, (int)m, (int)n, (int)k, y, ldy, work, work_floats, s);
  else if (type == 6)
    e = launch_type<6, XT>(x, ldx, W, (int)m, (int)n, (int)k, y, ldy, work, work_floats, s);
  else if (type == 20)
    e = launch_type<20, XT>(x, ldx, W, (int)m, (int)n, (int)k, y, ldy, work, work_floats, s);
  else if (type == 23)
    e = launch_type<23, XT>(x, ldx, W, (int)m, (int)n, (int)k, y, ldy, work, work_floats, s);
  else if (type == 16)
    e = launch_type<16, XT>(x, ldx, W, (int)m, (int)n, (int)k, y, ldy, work, work_floats, s);
  else if (type == 17)
    e = launch_type<17, XT>(x, ldx, W, (int)m, (int)n, (int)k, y, ldy, work, work_floats, s);
  else if (type == 18)
    e = launch_type<18, XT>(x, ldx, W, (int)m, (int)n, (int)k, y, ldy, work, work_floats, s);
  else if (type == 21)
    e = launch_type<21, XT>(x, ldx, W, (int)m, (int)n, (int)k, y, ldy, work, work_floats, s);
  else if (type == 22)
    e = launch_type<22, XT>(x, ldx, W, (int)m, (int)n, (int)k, y, ldy, work, work_floats, s);
  else if (type == 29)
    e = launch_type<29, XT>(x, ldx, W, (int)m, (int)n, (int)k, y, ldy, work, work_floats, s);
  else if (type == 10)
    e = launch_type<10, XT>(x, ldx, W, (int)m, (int)n, (int)k, y, ldy, work, work_floats, s);
  else if (type == 11)
    e = launch_type<11, XT>(x, ldx, W, (int)m, (int)n, (int)k, y, ldy, work, work_floats, s);
  else
    e = launch_type<14, XT>(x, ldx, W, (int)m, (int)n, (int)k, y, ldy, work, work_floats, s);
  return e;
}

}  // namespace

// Workspace floats of the GEMM for these shapes (0: none): for f32
// activations their fp16 image (of the largest launch_gemm chunk of rows),
// then the K split's partial sums.
int64_t launch_gemm_work(int type, int x_type, int64_t n, int64_t k, int64_t m) {
  const int64_t chunk = ((int64_t)1 << 30) / ((n + kBN - 1) / kBN) * kBM;
  const int64_t img = x_type == 0 ? stage_floats(m < chunk ? m : chunk, k) : 0;
  const int64_t tiles = ((m + kBM - 1) / kBM) * ((n + kBN - 1) / kBN);
  const int nu = (int)(k / unit_elems(type));
  const int sp = m <= chunk ? gemm_splits(type, tiles, nu) : 1;
  if (sp == 1) return img;
  const int kunits = (nu + sp - 1) / sp;
  return img + (int64_t)((nu + kunits - 1) / kunits) * m * n;
}

hipError_t launch_gemm(const void *x, int x_type, int64_t ldx, const uint8_t *tiles, int type,
                       int64_t n, int64_t k, float *y, int64_t ldy, int64_t m, float *work,
                       int64_t work_floats, hipStream_t s) {
  const int esize = x_type == 0 ? 4 : 2;
  // one launch covers at most 2^30 output tiles; split M beyond that
  const int64_t tiles_n = (n + kBN - 1) / kBN;
  const int64_t chunk = ((int64_t)1 << 30) / tiles_n * kBM;
  hipError_t e = hipSuccess;
  for (int64_t m0 = 0; m0 < m && e == hipSuccess; m0 += chunk) {
    const int64_t mc = (m - m0) < chunk ? (m - m0) : chunk;
    const char *xb = (const char *)x + m0 * ldx * esize;
    e = x_type == 0 ? launch_x<float>((const float *)xb, ldx, tiles, type, n, k, y + m0 * ldy, ldy,
                                      mc, work, work_floats, s)
                    : launch_x<half_t>((const half_t *)xb, ldx, tiles, type, n, k, y + m0 * ldy,
                                       ldy, mc, work, work_floats, s);
  }
  return e;
}

}  // namespace gguf
