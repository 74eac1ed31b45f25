// Batched decode of Q4_K, Q6_K, Q8_0 and the grid-codebook IQ weights
// (2 <= M <= 32 activation rows, and M = 1 beyond the one-shot kernel's K).
//
// Replaces the reference's batched decode, which runs its Q4_K GEMV once per
// activation row (grid.y = M, webgpu/src/engine/forward-pass.ts:1536-1539;
// kernel webgpu/src/shaders/matmul_gguf.wgsl:3191-3245): here the weights are
// read once for all M rows.
//
// The activations are converted into an image laid out exactly as a
// workgroup's shared memory holds them, one block of mk_unit_bytes<MA>() per
// 256-element unit (MA activation tiles of 16 MFMA rows each).  Up to 24 rows
// of f32 (48 of f16, MA <= 3), and 32 when K >= 8192 or for Q6_K, each workgroup of
// mk_kernel converts its own K range; otherwise the batch is converted once
// per call into the workspace (mk_prep_kernel), and the workgroups copy their
// range.  K is split over
// workgroups (ranges); each range writes its partial sums and
// mk_reduce_kernel adds them in range order.
//   A [16 MA][kMkLd] f16  MFMA row 2m + p holds part p (hi, lo) of activation
//                         row m for f32 inputs (8 rows per tile); row m holds
//                         row m for 16-bit inputs (16 rows per tile).  The
//                         elements are x * 2^e(m, unit), with e putting the
//                         unit's largest magnitude in [2^14, 2^15) (stage_exp),
//                         each quad in (0, 2, 1, 3) order.
//   S [16 MA][16] f16     the unit's 8 group sums sum(hi + lo) / 32, as hi and
//                         lo f16 parts, on the row of part 0 (zeros on the row
//                         of part 1): the A operand of the mins MFMA.
//   F [16 MA] f32         2^-e(m, unit) on every row of m.
//
// Arithmetic per unit, weight row n, activation row m.  The B operand is the
// sub-block's codes times its 6-bit scale, exact f16 integers (q sc <= 945,
// one v_pk_fma_f16 per two codes, mk_scaled), so the 8 sub-block
// MFMAs of a unit chain into one f32 accumulator D[m, n] = sum_j sc_j sum_k q x;
// one 16x16x16 MFMA gives the mins' dot M[m, n] = sum_j m_j S_j[m]; then
//     acc[m, n] += F[m] (d D[m, n] - 32 dmin M[m, n])
// in f32, and the parts are added at the end.
#pragma once

constexpr int kMkLd = 256 + 8;  // halves per staged row: a 16-byte pad (bank spread)
// The image of one 256-element unit: A, then (Q4_K) the group sums S, then F,
// NF inverse scales per row (one per unit, or one per 32-element block for
// Q8_0, whose blocks carry independent scales).
template <int MA, bool S = true, int NF = 1>
constexpr int mk_unit_bytes() {
  return 16 * MA * (kMkLd * 2 + (S ? 32 : 0) + 4 * NF);
}
template <int MA>
constexpr int mk_s_off() {
  return 16 * MA * kMkLd * 2;
}
template <int MA, bool S = true>
constexpr int mk_f_off() {
  return 16 * MA * (kMkLd * 2 + (S ? 32 : 0));
}

// Per-type traits of the batched kernel.  A unit is 256 elements of K: one
// superblock, or eight Q8_0 blocks (a super-unit of eight tile-units).
//   ORDER  0: natural k order (the IQ grid types); 1: each quad in (0, 2, 1, 3)
//          order (codes masked into the halves of a word: Q4_K, Q8_0);
//          2: as 1, and within each 32-element window the quads of its two
//          16-element groups interleaved (Q6_K: lane group g's 8 k are quad g
//          of group 2t, then quad g of group 2t + 1)
//   NF     inverse scales per unit and row (Q8_0: one per block)
template <int TYPE>
struct MkFmt {
  static constexpr int ORDER = TYPE == 12 ? 1 : 0, NF = 1;
  static constexpr bool SUMS = TYPE == 12;
  static constexpr int TU = Fmt<TYPE>::TU;  // bytes of a row tile's unit
};
template <>
struct MkFmt<14> {
  static constexpr int ORDER = 2, NF = 1;
  static constexpr bool SUMS = false;
  static constexpr int TU = Fmt<14>::TU;
};
template <>
struct MkFmt<8> {
  static constexpr int ORDER = 1, NF = 8;
  static constexpr bool SUMS = false;
  static constexpr int TU = 8 * Fmt<8>::TU;
};
template <int TYPE, int MA>
constexpr int mk_ub() {
  return mk_unit_bytes<MA, MkFmt<TYPE>::SUMS, MkFmt<TYPE>::NF>();
}

// The weight unit a lane holds: Unit<TYPE>, or eight Q8_0 blocks.
struct Q8Super {
  Unit<8> b[8];
};
template <int TYPE>
struct MkUnitOf {
  using type = Unit<TYPE>;
};
template <>
struct MkUnitOf<8> {
  using type = Q8Super;
};
__device__ __forceinline__ void load_unit(__amdgpu_buffer_rsrc_t rs, int soff, int r, int g,
                                          Q8Super &u) {
#pragma unroll
  for (int b = 0; b < 8; ++b) load_unit(rs, soff + b * Fmt<8>::TU, r, g, u.b[b]);
}

#ifndef GGUF_MK_LDS
#define GGUF_MK_LDS (159 * 1024)  // shared memory a workgroup's staged range may take
#endif
#ifndef GGUF_MK_MIN_WGS
#define GGUF_MK_MIN_WGS 224  // split K further while the grid has fewer workgroups
#endif
#ifndef GGUF_MK_DEPTH
#define GGUF_MK_DEPTH 2  // units in flight per wave, 1 or 2 activation tiles
#endif
#ifndef GGUF_MK_DEPTH_WIDE
#define GGUF_MK_DEPTH_WIDE 2  // the same, 3 or 4 activation tiles
#endif
#ifndef GGUF_MK_FUSE
#define GGUF_MK_FUSE 1  // each workgroup converts its own range of x (no prep launch)
#endif
constexpr int kMkFuseKw = 4;  // units per K range when the workgroups convert their own range
constexpr int kMkBatch = 8;  // ranges whose partial sums are requested at a time by the reduction
#ifndef GGUF_MK_WIDE_T
#define GGUF_MK_WIDE_T 1  // row tiles per wave for 3 or 4 activation tiles (16 T tiles per workgroup)
#endif
template <int TYPE, int MA>
constexpr int mk_kw_max() {  // units a workgroup can stage
  return (GGUF_MK_LDS - 1024 - iq_tbl_bytes<TYPE>()) / mk_ub<TYPE, MA>();
}

// Convert one (unit, activation row) into the unit's image block at blk;
// lane l holds elements 4l .. 4l + 3 in v (zeros for a padding row).  Every
// lane of the wave takes part.  NF = 1: one power of two for the unit (its
// 64 lanes); NF = 8: one per 32-element block (8 lanes).
template <int PARTS, int MA, int ORDER, bool SUMS, int NF>
__device__ __forceinline__ void mk_stage(const float (&v)[4], int m, int l, uint8_t *blk) {
  float mx = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  if constexpr (NF == 8) {
    mx = fmaxf(mx, dpp<kDppXor1>(mx));
    mx = fmaxf(mx, dpp<kDppXor2>(mx));
    mx = fmaxf(mx, dpp<kDppHalfMirror>(mx));
  } else {
    mx = max_xor32(max_xor16(max_lanes16(mx)));
  }
  const int ex = stage_exp(mx);
  const float sc = pow2f(ex);
  half4_t h, lo;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int pos = ORDER ? ((i & 1) << 1 | (i >> 1)) : i;  // quad order (0, 2, 1, 3) or natural
    float vi = v[i];
    asm volatile("" : "+v"(vi));  // keep the product out of the f16 conversions (no v_fma_mix)
    const float t = vi * sc;      // exact: a power of two
    const half_t hh = (half_t)t;
    const half_t ll = (half_t)(t - (float)hh);
    h[pos] = hh;
    lo[pos] = ll;
    s += (float)hh + (PARTS == 2 ? (float)ll : 0.f);
  }
  const int row = PARTS == 2 ? 2 * m : m;
  // ORDER 2: quad l = 8 w + 4 lh + g of window w goes to quad 8 w + 2 g + lh
  const int dq = ORDER == 2 ? (l & ~7) | ((l & 3) << 1) | ((l >> 2) & 1) : l;
  half_t *A = (half_t *)blk + row * kMkLd + 4 * dq;
  *(half4_t *)A = h;
  if (PARTS == 2) *(half4_t *)(A + kMkLd) = lo;
  if constexpr (SUMS) {
    s += dpp<kDppXor1>(s);  // the 8 lanes of a 32-element group
    s += dpp<kDppXor2>(s);
    s += dpp<kDppHalfMirror>(s);
    if ((l & 7) == 0) {
      // group j's sum at K position 4 (j >> 2) + e (hi) and 8 + that (lo), with e
      // the position of j & 3 in the (0, 2, 1, 3) order of the mins operand
      const int j = l >> 3, e = ((j & 1) << 1) | ((j >> 1) & 1), k = 4 * (j >> 2) + e;
      const float xs = s * 0.03125f;
      const half_t xh = (half_t)xs, xl = (half_t)(xs - (float)xh);
      half_t *S = (half_t *)(blk + mk_s_off<MA>()) + row * 16;
      S[k] = xh;
      S[8 + k] = xl;
      if (PARTS == 2) {
        S[16 + k] = (half_t)0.f;
        S[24 + k] = (half_t)0.f;
      }
    }
  }
  if ((NF == 8 && (l & 7) == 0) || l == 0) {
    float *F = (float *)(blk + mk_f_off<MA, SUMS>()) + (NF == 8 ? (l >> 3) * 16 * MA : 0);
    F[row] = pow2f(-ex);
    if (PARTS == 2) F[row + 1] = pow2f(-ex);
  }
}

// The activations' image, once per call: one wave per (unit, activation
// row), four per block; rows M .. ROWS - 1 are written as zeros.
template <typename XT, int MA, int TYPE>
__global__ __launch_bounds__(256) void mk_prep_kernel(const XT *__restrict__ x, int64_t ldx, int M,
                                                      uint8_t *__restrict__ img) {
  constexpr int PARTS = sizeof(XT) == 4 ? 2 : 1;
  const int u = blockIdx.x, m = 4 * blockIdx.y + (threadIdx.x >> 6), l = threadIdx.x & 63;
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  if (m < M) {
    const XT *src = x + (int64_t)m * ldx + 256 * u + 4 * l;
    if constexpr (sizeof(XT) == 4) {
      const float4 t = *(const float4 *)src;
      v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    } else {
      const half4_t t = *(const half4_t *)src;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (float)t[e];
    }
  }
  mk_stage<PARTS, MA, MkFmt<TYPE>::ORDER, MkFmt<TYPE>::SUMS, MkFmt<TYPE>::NF>(
      v, m, l, img + (size_t)u * mk_ub<TYPE, MA>());
}

// The mins operand of lane group g: m_j for j = 4 (g & 1) + (0, 2, 1, 3).
__device__ __forceinline__ half4_t mk_mins_operand(uint32_t mw) {
  constexpr uint32_t nb = neg_base(0);
  return as_h4(f16_codes(mw, 0x00FF00FFu, nb), f16_codes(mw >> 8, 0x00FF00FFu, nb));
}

// sc q for the two codes masked (m) into the halves of w: (base + c) sc' - 1024 sc'
// with base = 1024.0 in both halves, c = q (low nibbles, sc' = sc) or 16 q
// (high nibbles, sc' = sc / 16); scp holds sc' in both halves, nsp -1024 sc'.
// Exact: every product and the result q sc <= 945 are f16 integers.
__device__ __forceinline__ uint32_t mk_scaled(uint32_t w, uint32_t m, uint32_t base, half2_t scp,
                                              half2_t nsp) {
  const half2_t c = __builtin_bit_cast(half2_t, and_or(w, m, base));
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c, scp, nsp));
}

template <int MA, int T>
__device__ __forceinline__ void mk_unit(const Unit<12> (&w)[T], int bo, int lane, bool valid,
                                        float (&acc)[T][MA][4]) {
#pragma clang fp contract(off)
  const int r = lane & 15, g = lane >> 4;
  // 1024.0 x 2 in a register: with both the mask and this as literals the
  // compiler splits every and-or into two instructions
  uint32_t base = kF16Base;
  asm volatile("" : "+v"(base));
  // SC[t][i]: scales (sc0, sc2), (sc1, sc3) / 16, (sc4, sc6), (sc5, sc7) / 16
  // (odd sub-blocks hold high nibbles); NS = -1024 SC
  half2_t SC[T][4], NS[T][4];
  uint32_t ml[T], mh[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    uint32_t scl, sch;
    q4k_scales_packed(w[t].h.y, w[t].h.z, w[t].h.w, scl, sch, ml[t], mh[t]);
    constexpr uint32_t nb = neg_base(0);
    const half2_t h16 = {(half_t)0.0625f, (half_t)0.0625f}, hn = {(half_t)-1024.f, (half_t)-1024.f};
    SC[t][0] = __builtin_bit_cast(half2_t, f16_codes(scl, 0x00FF00FFu, nb));
    SC[t][1] = __builtin_bit_cast(half2_t, f16_codes(scl >> 8, 0x00FF00FFu, nb)) * h16;
    SC[t][2] = __builtin_bit_cast(half2_t, f16_codes(sch, 0x00FF00FFu, nb));
    SC[t][3] = __builtin_bit_cast(half2_t, f16_codes(sch >> 8, 0x00FF00FFu, nb)) * h16;
#pragma unroll
    for (int i = 0; i < 4; ++i) NS[t][i] = SC[t][i] * hn;
  }
  float4_t D[T][MA];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int a = 0; a < MA; ++a) D[t][a] = (float4_t){0.f, 0.f, 0.f, 0.f};
  const int arow = bo + r * (kMkLd * 2) + 16 * g;  // byte offset of the lane's A fragment
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    uint32_t wq[T][4];  // the lane's chunk-c words and their bytes 1, 3 moved down
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint32_t q[8] = {w[t].a.x, w[t].a.y, w[t].a.z, w[t].a.w,
                             w[t].b.x, w[t].b.y, w[t].b.z, w[t].b.w};
      wq[t][0] = q[2 * c];
      wq[t][1] = q[2 * c] >> 8;
      wq[t][2] = q[2 * c + 1];
      wq[t][3] = q[2 * c + 1] >> 8;
    }
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {  // sub-block j = 2c + hb: low (hb 0) / high nibbles
      const int j = 2 * c + hb;
      const uint32_t m = hb ? 0x00F000F0u : 0x000F000Fu;
      half8_t A[MA];
#pragma unroll
      for (int a = 0; a < MA; ++a) A[a] = lds_h8b(arow + a * 16 * (kMkLd * 2) + 2 * (64 * c + 32 * hb));
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int si = (j >> 2) * 2 + hb, sh = (j >> 1) & 1;
        const half2_t scp = {SC[t][si][sh], SC[t][si][sh]}, nsp = {NS[t][si][sh], NS[t][si][sh]};
        const half8_t B = as_h8(mk_scaled(wq[t][0], m, base, scp, nsp), mk_scaled(wq[t][1], m, base, scp, nsp),
                                mk_scaled(wq[t][2], m, base, scp, nsp), mk_scaled(wq[t][3], m, base, scp, nsp));
#pragma unroll
        for (int a = 0; a < MA; ++a)
          D[t][a] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[a], B, D[t][a], 0, 0, 0);
      }
      // wide tiles: one sub-block's operands at a time (unconstrained, the
      // scheduler loads every A fragment of the unit up front and spills)
      if constexpr (MA * T >= 4) __builtin_amdgcn_sched_barrier(0);
    }
  }
  // mins: one 16x16x16 MFMA per activation tile (K = 8 group sums x hi / lo)
  half4_t B2[T];
  float d[T], dm[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    B2[t] = mk_mins_operand((g & 1) ? mh[t] : ml[t]);
    // a slot past the wave's units (valid false) adds exactly zero
    d[t] = valid ? h2f(w[t].h.x) : 0.f;
    dm[t] = valid ? -32.f * h2f(w[t].h.x >> 16) : 0.f;
  }
#pragma unroll
  for (int a = 0; a < MA; ++a) {
    const half4_t A2 = lds_h4b(bo + mk_s_off<MA>() + (16 * a + r) * 32 + 8 * g);
    const float4 F = *(const float4 *)(g_lds + bo + mk_f_off<MA>() + (16 * a + 4 * g) * 4);
    const float f[4] = {F.x, F.y, F.z, F.w};
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const float4_t zero = {0.f, 0.f, 0.f, 0.f};
      const float4_t D2 = __builtin_amdgcn_mfma_f32_16x16x16f16(A2, B2[t], zero, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[t][a][i] = fmaf(f[i], fmaf(d[t], D[t][a][i], dm[t] * D2[i]), acc[t][a][i]);
    }
    if constexpr (MA * T >= 4) __builtin_amdgcn_sched_barrier(0);  // one tile at a time
  }
  // The sums are used only under the output's conditions: without this the
  // compiler sinks every unit's update there and keeps all the units'
  // products alive until the end (spilling them).
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int a = 0; a < MA; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(acc[t][a][i]));
}

template <int TYPE, int MA, int T>
__device__ __forceinline__ void mk_unit_iq(const Unit<TYPE> (&w)[T], int bo, int lane, bool valid,
                                           int tbl, float (&acc)[T][MA][4]) {
#pragma clang fp contract(off)
  const int r = lane & 15, g = lane >> 4;
  float4_t D[T][MA];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int a = 0; a < MA; ++a) D[t][a] = (float4_t){0.f, 0.f, 0.f, 0.f};
  const int arow = bo + r * (kMkLd * 2) + 16 * g;  // byte offset of the lane's A fragment
#pragma unroll
  for (int ib = 0; ib < 8; ++ib) {
    half8_t A[MA];
#pragma unroll
    for (int a = 0; a < MA; ++a) A[a] = lds_h8b(arow + a * 16 * (kMkLd * 2) + 64 * ib);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const half8_t B = iq_b<TYPE>(w[t], ib, g, g_lds + tbl);
#pragma unroll
      for (int a = 0; a < MA; ++a) D[t][a] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[a], B, D[t][a], 0, 0, 0);
    }
    if constexpr (MA * T >= 4) __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int a = 0; a < MA; ++a) {
    const float4 F = *(const float4 *)(g_lds + bo + mk_f_off<MA, false>() + (16 * a + 4 * g) * 4);
    const float f[4] = {F.x, F.y, F.z, F.w};
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const float us = valid ? iq_unit_scale<TYPE>(w[t]) : 0.f;  // a slot past the units adds zero
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[t][a][i] = fmaf(f[i], us * D[t][a][i], acc[t][a][i]);
    }
  }
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int a = 0; a < MA; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(acc[t][a][i]));
}

// Q6_K: each int8 group scale is split as sc = 16 sh + sl (sl in [0, 15], sh
// in [-8, 7]), so that the B operands sl (q - 32) and sh (q - 32) are exact
// f16 integers (|.| <= 480), made as (1024 + q) s - 1056 s by one
// v_pk_fma_f16 per two codes.  Window w = 4 hf + t (32 elements of K) holds
// the groups 8 hf + 2 t + lh, lh = 0, 1 (the image interleaves their quads,
// ORDER 2), so one 16x16x32 MFMA per part covers both groups and the unit's
// 16 MFMAs chain into two accumulators per activation tile:
//     D = Dl + 16 Dh = sum_s sc_s sum_k x (q - 32),  acc += F d D.
template <int MA, int T>
__device__ __forceinline__ void mk_unit_q6k(const Unit<14> (&w)[T], int bo, int lane, bool valid,
                                            float (&acc)[T][MA][4]) {
#pragma clang fp contract(off)
  const int r = lane & 15, g = lane >> 4;
  uint32_t base = kF16Base;  // in a register: one v_and_or_b32 per masked pair
  asm volatile("" : "+v"(base));
  float4_t Dl[T][MA], Dh[T][MA];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int a = 0; a < MA; ++a) Dl[t][a] = Dh[t][a] = (float4_t){0.f, 0.f, 0.f, 0.f};
  const int arow = bo + r * (kMkLd * 2) + 16 * g;  // byte offset of the lane's A fragment
  const half2_t n1056 = {(half_t)-1056.f, (half_t)-1056.f};
#pragma unroll
  for (int q = 0; q < 4; ++q) {  // scale word q: groups 4q .. 4q + 3, windows 2q, 2q + 1
    // SL[t][e] = (sl of group 4q + e, and of 4q + e + 2), SH likewise; NL, NH = -1056 x them
    half2_t SL[T][2], SH[T][2], NL[T][2], NH[T][2];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint32_t sw = q == 0 ? w[t].sc.x : q == 1 ? w[t].sc.y : q == 2 ? w[t].sc.z : w[t].sc.w;
      constexpr uint32_t nb0 = neg_base(0), nb8 = neg_base(8);
      SL[t][0] = __builtin_bit_cast(half2_t, f16_codes(sw, 0x000F000Fu, nb0));
      SL[t][1] = __builtin_bit_cast(half2_t, f16_codes(sw >> 8, 0x000F000Fu, nb0));
      // the high nibble, signed: (nibble ^ 8) = sh + 8
      SH[t][0] = __builtin_bit_cast(half2_t, f16_codes((sw >> 4) ^ 0x00080008u, 0x000F000Fu, nb8));
      SH[t][1] = __builtin_bit_cast(half2_t, f16_codes((sw >> 12) ^ 0x00080008u, 0x000F000Fu, nb8));
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        NL[t][e] = SL[t][e] * n1056;
        NH[t][e] = SH[t][e] * n1056;
      }
    }
#pragma unroll
    for (int tp = 0; tp < 2; ++tp) {  // window 2q + tp: hf = q >> 1, quarter tt = 2 (q & 1) + tp
      const int hf = q >> 1, tt = 2 * (q & 1) + tp;
      half8_t A[MA];
#pragma unroll
      for (int a = 0; a < MA; ++a) A[a] = lds_h8b(arow + a * 16 * (kMkLd * 2) + 64 * (4 * hf + tt));
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const uint32_t dw[12] = {w[t].p0.x, w[t].p0.y, w[t].p0.z, w[t].p0.w, w[t].p1.x, w[t].p1.y,
                                 w[t].p1.z, w[t].p1.w, w[t].p2.x, w[t].p2.y, w[t].p2.z, w[t].p2.w};
        uint32_t bl[4], bh[4];
#pragma unroll
        for (int lh = 0; lh < 2; ++lh) {
          const int i = 2 * hf + lh;
          const uint32_t qa = dw[3 * i], qb = dw[3 * i + 1], qh = dw[3 * i + 2];
          // the lane's 4 codes of group 8 hf + 2 tt + lh (k = 4 g .. 4 g + 3)
          const uint32_t v = tt == 0   ? (qa & 0x0F0F0F0Fu) | ((qh << 4) & 0x30303030u)
                             : tt == 1 ? (qb & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u)
                             : tt == 2 ? ((qa >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u)
                                       : ((qb >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u);
          // scale of the group: byte 2 tp + lh of word q (SL[.][lh] holds bytes lh, lh + 2)
          const half_t sl = SL[t][lh][tp], sh = SH[t][lh][tp];
          const half_t nl = NL[t][lh][tp], nh = NH[t][lh][tp];
          const half2_t c02 = __builtin_bit_cast(half2_t, and_or(v, 0x00FF00FFu, base));
          const half2_t c13 = __builtin_bit_cast(half2_t, and_or(v >> 8, 0x00FF00FFu, base));
          const half2_t sl2 = {sl, sl}, sh2 = {sh, sh}, nl2 = {nl, nl}, nh2 = {nh, nh};
          bl[2 * lh] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c02, sl2, nl2));
          bl[2 * lh + 1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c13, sl2, nl2));
          bh[2 * lh] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c02, sh2, nh2));
          bh[2 * lh + 1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c13, sh2, nh2));
        }
        const half8_t Bl = as_h8(bl[0], bl[1], bl[2], bl[3]), Bh = as_h8(bh[0], bh[1], bh[2], bh[3]);
#pragma unroll
        for (int a = 0; a < MA; ++a) {
          Dl[t][a] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[a], Bl, Dl[t][a], 0, 0, 0);
          Dh[t][a] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[a], Bh, Dh[t][a], 0, 0, 0);
        }
      }
      if constexpr (MA * T >= 4) __builtin_amdgcn_sched_barrier(0);
    }
  }
  float d[T];
#pragma unroll
  for (int t = 0; t < T; ++t) d[t] = valid ? h2f(w[t].d) : 0.f;  // a slot past the units adds zero
#pragma unroll
  for (int a = 0; a < MA; ++a) {
    const float4 F = *(const float4 *)(g_lds + bo + mk_f_off<MA, false>() + (16 * a + 4 * g) * 4);
    const float f[4] = {F.x, F.y, F.z, F.w};
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[t][a][i] = fmaf(f[i], d[t] * fmaf(16.f, Dh[t][a][i], Dl[t][a][i]), acc[t][a][i]);
  }
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int a = 0; a < MA; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(acc[t][a][i]));
}

// Q8_0: eight 32-element blocks per unit, each with its own scale d_b and its
// own inverse activation scale F_b (NF = 8): one MFMA of the exact int8 codes
// per block and activation tile, acc += (F_b d_b) D_b.
template <int MA, int T>
__device__ __forceinline__ void mk_unit_q8(const Q8Super (&w)[T], int bo, int lane, bool valid,
                                           float (&acc)[T][MA][4]) {
#pragma clang fp contract(off)
  const int r = lane & 15, g = lane >> 4;
  const int arow = bo + r * (kMkLd * 2) + 16 * g;  // byte offset of the lane's A fragment
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    half8_t A[MA];
    float4 F[MA];
#pragma unroll
    for (int a = 0; a < MA; ++a) {
      A[a] = lds_h8b(arow + a * 16 * (kMkLd * 2) + 64 * b);
      F[a] = *(const float4 *)(g_lds + bo + mk_f_off<MA, false>() + (16 * MA * b + 16 * a + 4 * g) * 4);
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const half8_t B = q8_operand(w[t].b[b]);
      const float d = valid ? h2f(w[t].b[b].d) : 0.f;  // a slot past the units adds zero
#pragma unroll
      for (int a = 0; a < MA; ++a) {
        const float4_t zero = {0.f, 0.f, 0.f, 0.f};
        const float4_t D = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[a], B, zero, 0, 0, 0);
        const float f[4] = {F[a].x, F[a].y, F[a].z, F[a].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][a][i] = fmaf(f[i] * d, D[i], acc[t][a][i]);
      }
    }
    if constexpr (MA * T >= 4) __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int a = 0; a < MA; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(acc[t][a][i]));
}

// Workgroup (blockIdx.x, blockIdx.y) of TS x KL waves: row tiles
// TS T blockIdx.x .. + TS T - 1 (T per wave; wave w takes tile slot w % TS and
// K-lane w / TS), units blockIdx.y kw .. + kw - 1 of K, of which K-lane kl
// takes every KL-th from kl.
//
// Order of work: every thread requests its share of the range's activations,
// then all of its tiles' units (at most U per tile); it writes the range's
// image to shared memory as the activations land (the weights still in
// flight); after the one barrier each wave consumes its units in order as
// they arrive.  The K-lanes of a tile slot are added in a fixed order through
// shared memory.
//
// SX (MA <= 3, or 4 with K >= 8192): the workgroup converts its own range of x into
// the image (mk_stage, one wave per (unit, activation row)).  Otherwise the
// image comes from the workspace (mk_prep_kernel): through registers for
// MA <= 2, LDS-direct loads for MA 3, 4.
//
// K split over gridDim.y > 1 ranges: each range's partial sums go to `part`
// ([range][M][np]) and mk_reduce_kernel adds them in range order, so the
// result does not depend on which range finishes first.  (The last range of
// a tile group adding the partials itself, behind an agent-scope release /
// acquire counter, measured 1.5-3 us slower per call than the second launch:
// the partial stores, the count and the reads are three dependent memory
// round trips under the weight stream.)
template <int TYPE, typename XT, int MA, int T, int TS, int KL, bool SX>
__global__ __launch_bounds__(64 * TS * KL) void mk_kernel(const uint8_t *__restrict__ img,
                                                          const XT *__restrict__ x, int64_t ldx,
                                                          const uint8_t *__restrict__ W, int N,
                                                          int K, int M, int kw,
                                                          float *__restrict__ y, int64_t ldy,
                                                          float *__restrict__ part) {
  constexpr int PARTS = sizeof(XT) == 4 ? 2 : 1, NW = TS * KL;
  constexpr int UB = mk_ub<TYPE, MA>(), TU = MkFmt<TYPE>::TU;
  constexpr int KWM = SX ? kMkFuseKw : mk_kw_max<TYPE, MA>();  // units a range may hold
  constexpr int CP = SX ? 1 : (KWM * UB / 16 + 64 * NW - 1) / (64 * NW);  // 16 B pieces per thread
  constexpr int U = (KWM + KL - 1) / KL;                                    // unit slots per wave
  constexpr int RW = 16 * MA / PARTS;                  // activation rows of an image block
  constexpr int SP = SX ? (KWM * RW + NW - 1) / NW : 1;  // (unit, row) pairs a wave stages
  constexpr bool IQ = is_iq(TYPE);
  // slots in flight per tile: a few MB over the chip keep the transfer at full
  // rate and the arrivals in order (all at once, they land in no useful order
  // and the decode runs after the transfer instead of under it)
  constexpr int P = (MA > 2 ? GGUF_MK_DEPTH_WIDE : GGUF_MK_DEPTH) < U
                        ? (MA > 2 ? GGUF_MK_DEPTH_WIDE : GGUF_MK_DEPTH) : U;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int ts = wave % TS, kl = wave / TS;
  const int ntiles = (N + 15) >> 4, nu = K >> 8;
  const int t0 = (blockIdx.x * TS + ts) * T;
  const int u0 = blockIdx.y * kw, nun = min(kw, nu - u0);
  const int cnt_u = (nun - kl + KL - 1) / KL;  // the wave's units: kl + KL i, i < cnt_u
  const int tb = nu * TU;
  const int nq = nun * (UB / 16);  // 16-byte pieces of the range's image
  const int tbl = (kw * UB + 1023) & ~1023;  // IQ types: the decode tables, behind the range

  // the range's activations.  SX: x itself, 4 values per lane of each
  // (unit, row) pair the wave converts (rows past M are zeros).  Otherwise the
  // image: narrow tiles (MA <= 2) through registers, requested ahead of the
  // weights and written as it lands (pieces past the range repeat the last
  // one and are not stored); wide tiles by LDS-direct loads in 1 KB pieces
  // (the workspace holds 1 KB of slack past the image), no registers, before
  // the weights are requested (the barrier waits for every load).
  constexpr bool DMA = !SX && MA > 2;
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // a value type: no memcpy copies
  const uint8_t *src = SX ? img : img + (size_t)u0 * UB;
  u32x4 R[DMA || SX ? 1 : CP];
  float xv[SP][4];
  IqTabRegs<TYPE, 64 * NW> tab;
  if constexpr (IQ) iq_get_tables<TYPE, 64 * NW>(tab);
  if constexpr (SX) {
#pragma unroll
    for (int i = 0; i < SP; ++i) {
      const int q = wave + NW * i, ul = q / RW, m = q - ul * RW;
#pragma unroll
      for (int e = 0; e < 4; ++e) xv[i][e] = 0.f;
      if (ul < nun && m < M) {  // uniform
        const XT *p = x + (int64_t)m * ldx + 256 * (u0 + ul) + 4 * lane;
        if constexpr (sizeof(XT) == 4) {
          const float4 t = *(const float4 *)p;
          xv[i][0] = t.x;
          xv[i][1] = t.y;
          xv[i][2] = t.z;
          xv[i][3] = t.w;
        } else {
          const half4_t t = *(const half4_t *)p;
#pragma unroll
          for (int e = 0; e < 4; ++e) xv[i][e] = (float)t[e];
        }
      }
    }
  } else if constexpr (DMA) {
    const int kb = (nun * UB + 1023) >> 10;
    for (int i = wave; i < kb; i += NW)
      __builtin_amdgcn_global_load_lds((const void *)(src + 1024 * i + 16 * lane),
                                       (__attribute__((address_space(3))) void *)(g_lds + 1024 * i),
                                       16, 0, 0);
    if constexpr (IQ) iq_put_tables<TYPE, 64 * NW>(tab, g_lds + tbl);
    __syncthreads();
  } else {
#pragma unroll
    for (int c = 0; c < CP; ++c)
      R[c] = *(const u32x4 *)(src + 16 * min((int)threadIdx.x + 64 * NW * c, nq - 1));
  }
  __amdgpu_buffer_rsrc_t rs[T];
#pragma unroll
  for (int t = 0; t < T; ++t)  // a tile past the weight's end has no records (loads read 0)
    rs[t] = __builtin_amdgcn_make_buffer_rsrc((void *)(W + (int64_t)min(t0 + t, ntiles - 1) * tb), 0,
                                              t0 + t < ntiles ? tb : 0, kRsrcWord3);
  // The wave's U unit slots in straight-line code, P in flight (slot i + P
  // requested once slot i is consumed), branch-free: a slot past the wave's
  // units loads its last unit (an L2 hit) and adds zero.  Under a branch or in
  // a loop the memory-counter waits lose track of the requests and wait for
  // all of them at every unit.
  const int ulast = cnt_u > 0 ? kl + KL * (cnt_u - 1) : 0;  // a unit of the range
  typename MkUnitOf<TYPE>::type wb[P][T];
  // Slots requested before the activations are converted: one per tile for
  // the types other than Q4_K, the rest after the staging barrier, so that
  // the activation loads queue behind less weight traffic (M = 8, graph
  // replays: Q6_K 17.35 -> 16.54 us, IQ2_XXS 14.88 -> 14.02, Q8_0 17.35 ->
  // 17.12); Q4_K measured level (12.11 -> 12.18) and requests them all.
  constexpr int P0 = SX && TYPE != 12 ? 1 : P;
#pragma unroll
  for (int i = 0; i < P0; ++i)
#pragma unroll
    for (int t = 0; t < T; ++t) load_unit(rs[t], (u0 + min(kl + KL * i, ulast)) * TU, r, g, wb[i][t]);
  if constexpr (SX) {
#pragma unroll
    for (int i = 0; i < SP; ++i) {
      const int q = wave + NW * i, ul = q / RW, m = q - ul * RW;
      if (ul < nun)  // uniform
        mk_stage<PARTS, MA, MkFmt<TYPE>::ORDER, MkFmt<TYPE>::SUMS, MkFmt<TYPE>::NF>(
            xv[i], m, lane, g_lds + ul * UB);
    }
    if constexpr (IQ) iq_put_tables<TYPE, 64 * NW>(tab, g_lds + tbl);
    __syncthreads();
#pragma unroll
    for (int i = P0; i < P; ++i)
#pragma unroll
      for (int t = 0; t < T; ++t) load_unit(rs[t], (u0 + min(kl + KL * i, ulast)) * TU, r, g, wb[i][t]);
  } else if constexpr (!DMA) {
#pragma unroll
    for (int c = 0; c < CP; ++c) {
      const int q = (int)threadIdx.x + 64 * NW * c;
      if (q < nq) *(u32x4 *)(g_lds + 16 * q) = R[c];
    }
    if constexpr (IQ) iq_put_tables<TYPE, 64 * NW>(tab, g_lds + tbl);
    __syncthreads();
  }
  float acc[T][MA][4];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int a = 0; a < MA; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[t][a][i] = 0.f;
#pragma unroll
  for (int i = 0; i < U; ++i) {
    // wave priority from the units still to do: the waves of a SIMD otherwise
    // issue oldest first and the youngest finishes last
    {
      const int rem = U - i;
      if (rem >= 4) __builtin_amdgcn_s_setprio(3);
      else if (rem == 3) __builtin_amdgcn_s_setprio(2);
      else if (rem == 2) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
    }
    if constexpr (IQ)
      mk_unit_iq<TYPE, MA, T>(wb[i % P], min(kl + KL * i, ulast) * UB, lane, i < cnt_u, tbl, acc);
    else if constexpr (TYPE == 14)
      mk_unit_q6k<MA, T>(wb[i % P], min(kl + KL * i, ulast) * UB, lane, i < cnt_u, acc);
    else if constexpr (TYPE == 8)
      mk_unit_q8<MA, T>(wb[i % P], min(kl + KL * i, ulast) * UB, lane, i < cnt_u, acc);
    else
      mk_unit<MA, T>(wb[i % P], min(kl + KL * i, ulast) * UB, lane, i < cnt_u, acc);
    if (i + P < U)  // compile-time
#pragma unroll
      for (int t = 0; t < T; ++t)
        load_unit(rs[t], (u0 + min(kl + KL * (i + P), ulast)) * TU, r, g, wb[i % P][t]);
  }
  __builtin_amdgcn_s_setprio(0);
  if constexpr (KL > 1) {  // K-lanes 1 .. KL - 1 hand their sums to lane 0, added in order
    __syncthreads();  // the staged activations are consumed
    float *red = (float *)g_lds;  // [KL - 1][TS][T][MA][4][64]
    if (kl > 0) {
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int a = 0; a < MA; ++a)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            red[(((((kl - 1) * TS + ts) * T + t) * MA + a) * 4 + i) * 64 + lane] = acc[t][a][i];
    }
    __syncthreads();
    if (kl == 0) {
#pragma unroll
      for (int k2 = 1; k2 < KL; ++k2)
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
          for (int a = 0; a < MA; ++a)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              acc[t][a][i] += red[(((((k2 - 1) * TS + ts) * T + t) * MA + a) * 4 + i) * 64 + lane];
    }
  }
  // this range's sums: to y when K is not split, else to the range's partials
  const bool split = gridDim.y > 1;
  const int np = ntiles * 16;
  float *o = split ? part + (int64_t)blockIdx.y * M * np : y;
  const int64_t ldo = split ? (int64_t)np : ldy;
  if (kl == 0) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int n = 16 * (t0 + t) + r;
      if (n >= N) continue;
#pragma unroll
      for (int a = 0; a < MA; ++a) {
        if (PARTS == 2) {
          const int m = 8 * a + 2 * g;
          if (m < M) o[(int64_t)m * ldo + n] = acc[t][a][0] + acc[t][a][1];
          if (m + 1 < M) o[(int64_t)(m + 1) * ldo + n] = acc[t][a][2] + acc[t][a][3];
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int m = 16 * a + 4 * g + i;
            if (m < M) o[(int64_t)m * ldo + n] = acc[t][a][i];
          }
        }
      }
    }
  }
}

// y[m, n] = sum over the S ranges of part[s][m][n] (row stride np), in range
// order: the reduction of K ranges too many for the in-kernel one.  One
// output element per thread; the partials are requested kMkBatch at a time.
__global__ __launch_bounds__(256) void mk_reduce_kernel(const float *__restrict__ part, int S, int M,
                                                        int np, int N, float *__restrict__ y,
                                                        int64_t ldy) {
  const int m = blockIdx.y, n = blockIdx.x * 256 + (int)threadIdx.x;
  if (n >= N) return;
  const float *p = part + (int64_t)m * np + n;
  const int64_t st = (int64_t)M * np;
  float a = p[0];
  for (int s0 = 1; s0 < S; s0 += kMkBatch) {
    float v[kMkBatch];
#pragma unroll
    for (int s = 0; s < kMkBatch; ++s) v[s] = s0 + s < S ? p[(s0 + s) * st] : 0.f;
#pragma unroll
    for (int s = 0; s < kMkBatch; ++s)
      if (s0 + s < S) a += v[s];
  }
  y[(int64_t)m * ldy + n] = a;
}

// Launch shape: MA activation tiles; TS tile slots x KL K-lanes of T tiles
// per workgroup; K split into `ranges` of kw units.
//   SX (MA <= 3, or 4 with K >= 8192): 16 tiles per workgroup, one per wave; ranges of at most
//     kMkFuseKw units (the conversion each workgroup does stays small), more
//     while the grid has fewer than GGUF_MK_MIN_WGS workgroups.
//   Otherwise: as few ranges as the shared memory allows (the image comes
//     from the prep launch), more while the grid has fewer than
//     GGUF_MK_MIN_WGS workgroups.
// Workspace: from kWsPrefix on (the prefix is not used here), the image (not
// SX) and the ranges' partial sums (split K only).
struct MkPlan {
  int ma, ts, kl, t, groups, kw, ranges;
  bool sx;
  size_t lds, part_off, bytes;  // part_off: from the start of the workspace
};
template <int TYPE, typename XT>
MkPlan mk_plan(int M, int N, int K) {
  constexpr int PARTS = sizeof(XT) == 4 ? 2 : 1;
  MkPlan p;
  p.ma = (M * PARTS + 15) / 16;
  // each workgroup converts its own K range up to 3 activation tiles, and at 4
  // when K has at least 32 units (measured: 32 f32 rows at K = 14336 gain 1-2 us
  // per call against the prep launch + image copy, at K = 4096 they lose 1.5 us;
  // 24 rows gain at K = 4096 too), or for Q6_K at any K (32 rows at K = 4096:
  // 28.59 -> 27.13 us; Q8_0 level, the IQ types 2% slower)
  p.sx = GGUF_MK_FUSE && (p.ma <= 3 || (p.ma == 4 && (K / 256 >= 32 || TYPE == 14)));
  const bool wide = p.ma > 2;
  p.ts = p.sx ? 16 : wide ? 16 / GGUF_MK_WIDE_T : 4;
  p.kl = p.sx || wide ? 1 : 4;
  p.t = !p.sx && wide ? GGUF_MK_WIDE_T : 1;
  const size_t ub = p.ma == 1 ? mk_ub<TYPE, 1>() : p.ma == 2 ? mk_ub<TYPE, 2>()
                  : p.ma == 3 ? mk_ub<TYPE, 3>() : mk_ub<TYPE, 4>();
  const int kw_max = p.sx ? kMkFuseKw
                   : p.ma == 1 ? mk_kw_max<TYPE, 1>() : p.ma == 2 ? mk_kw_max<TYPE, 2>()
                   : p.ma == 3 ? mk_kw_max<TYPE, 3>() : mk_kw_max<TYPE, 4>();
  const int ntiles = (N + 15) / 16, nu = K / 256;
  p.groups = (ntiles + p.ts * p.t - 1) / (p.ts * p.t);
  int ranges = (nu + kw_max - 1) / kw_max;
  while (ranges < nu && (int64_t)p.groups * ranges < GGUF_MK_MIN_WGS) ++ranges;
  p.kw = (nu + ranges - 1) / ranges;
  p.ranges = (nu + p.kw - 1) / p.kw;
  const size_t stage = ((size_t)p.kw * ub + 1023) & ~(size_t)1023;
  const size_t red = (size_t)(p.kl - 1) * p.ts * p.t * p.ma * 4 * 64 * 4;
  const size_t used = stage + iq_tbl_bytes<TYPE>();  // the tables sit behind the range
  p.lds = used > red ? used : red;
  // 1 KB slack past the image for the 1 KB copy pieces
  const size_t img = p.sx ? 0 : ((size_t)nu * ub + 1024 + 255) & ~(size_t)255;
  const size_t parts = p.ranges > 1 ? (size_t)p.ranges * M * ntiles * 16 * 4 : 0;
  p.part_off = (size_t)kWsPrefix + img;
  p.bytes = img + parts > 0 ? p.part_off + parts : 0;
  return p;
}

template <int TYPE, typename XT, int MA, int T, int TS, int KL, bool SX>
hipError_t launch_mk_ma(const XT *x, int64_t ldx, const uint8_t *W, int N, int K, float *y,
                        int64_t ldy, int M, float *work, const MkPlan &p, hipStream_t s) {
  constexpr int PARTS = sizeof(XT) == 4 ? 2 : 1;
  uint8_t *ws = (uint8_t *)work, *img = ws + kWsPrefix;
  hipError_t e = hipSuccess;
  if constexpr (!SX) {
    hipLaunchKernelGGL((mk_prep_kernel<XT, MA, TYPE>),
                       dim3((unsigned)(K / 256), (unsigned)(16 * MA / PARTS / 4)), dim3(256), 0, s,
                       x, ldx, M, img);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  auto kern = mk_kernel<TYPE, XT, MA, T, TS, KL, SX>;
  if (p.lds > 65536) {
    e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)p.lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)p.groups, (unsigned)p.ranges), dim3(64 * TS * KL), p.lds, s,
                     img, x, ldx, W, N, K, M, p.kw, y, ldy,
                     p.ranges > 1 ? (float *)(ws + p.part_off) : nullptr);
  e = hipGetLastError();
  if (e != hipSuccess || p.ranges == 1) return e;
  const int np = (N + 15) / 16 * 16;
  hipLaunchKernelGGL(mk_reduce_kernel, dim3((unsigned)((N + 255) / 256), (unsigned)M), dim3(256), 0, s,
                     (const float *)(ws + p.part_off), p.ranges, M, np, N, y, ldy);
  return hipGetLastError();
}

// Workspace bytes of the batched path for M rows of XT activations.
template <int TYPE, typename XT>
size_t mk_work_bytes(int M, int N, int K) {
  return mk_plan<TYPE, XT>(M, N, K).bytes;
}

// hipErrorNotSupported (nothing launched) when the workspace is missing or
// too small: the caller then takes the kernel that stages in every workgroup.
template <int TYPE, typename XT>
hipError_t launch_mk(const XT *x, int64_t ldx, const uint8_t *W, int N, int K, float *y,
                     int64_t ldy, int M, float *work, int64_t work_floats, hipStream_t s) {
  if (K % 256) return hipErrorNotSupported;  // units of 256 elements (Q8_0: eight blocks)
  const MkPlan p = mk_plan<TYPE, XT>(M, N, K);
  if (M > 32 || (p.bytes > 0 && (!work || (size_t)work_floats * 4 < p.bytes)))
    return hipErrorNotSupported;
  if (p.sx) {
    if (p.ma == 1) return launch_mk_ma<TYPE, XT, 1, 1, 16, 1, true>(x, ldx, W, N, K, y, ldy, M, work, p, s);
    if (p.ma == 2) return launch_mk_ma<TYPE, XT, 2, 1, 16, 1, true>(x, ldx, W, N, K, y, ldy, M, work, p, s);
    if (p.ma == 3) return launch_mk_ma<TYPE, XT, 3, 1, 16, 1, true>(x, ldx, W, N, K, y, ldy, M, work, p, s);
    return launch_mk_ma<TYPE, XT, 4, 1, 16, 1, true>(x, ldx, W, N, K, y, ldy, M, work, p, s);
  }
  switch (p.ma) {  // the shapes mk_plan assumes for each MA
    case 1: return launch_mk_ma<TYPE, XT, 1, 1, 4, 4, false>(x, ldx, W, N, K, y, ldy, M, work, p, s);
    case 2: return launch_mk_ma<TYPE, XT, 2, 1, 4, 4, false>(x, ldx, W, N, K, y, ldy, M, work, p, s);
    case 3: return launch_mk_ma<TYPE, XT, 3, GGUF_MK_WIDE_T, 16 / GGUF_MK_WIDE_T, 1, false>(x, ldx, W, N, K, y, ldy, M, work, p, s);
    default: return launch_mk_ma<TYPE, XT, 4, GGUF_MK_WIDE_T, 16 / GGUF_MK_WIDE_T, 1, false>(x, ldx, W, N, K, y, ldy, M, work, p, s);
  }
}
