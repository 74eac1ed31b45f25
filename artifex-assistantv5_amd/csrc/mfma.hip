// MFMA dequant-GEMM: y[m, n] = sum_k x[m, k] * dequant(W)[n, k].
//
// The reference has no GEMM for these types: prefill re-runs its GEMV once
// per activation row (webgpu/src/engine/forward-pass.ts:1536-1539).  Here a
// workgroup owns a BM x BN output tile; per 64-wide K step it stages the
// activation tile (fp16) and the weight tile dequantized to fp16 (one
// rounding of the exact f32 dequant value, RNE) in LDS, and its four waves
// feed v_mfma_f32_16x16x32_f16 with f32 accumulation.  f32 activations are
// rounded to fp16 when staged.
#include "common.hpp"

namespace gguf {

constexpr int kBK = 64;
constexpr int kLd = kBK + 8;  // LDS row stride in halves (144 B, 16-B aligned)

template <typename XT, int BM>
__device__ __forceinline__ void stage_a(const XT *__restrict__ x, int64_t ldx, int M, int K,
                                        int m0, int k0, half_t *As, int tid) {
#pragma unroll
  for (int p = tid; p < BM * 8; p += 256) {
    const int r = p >> 3, cc = p & 7;
    const int m = m0 + r, k = k0 + 8 * cc;
    half8_t v;
    if (m < M && k < K) {
      if constexpr (sizeof(XT) == 4) {
        const float4 *src = (const float4 *)(x + (int64_t)m * ldx + k);
        const float4 a = src[0], b = src[1];
        v = half8_t{(half_t)a.x, (half_t)a.y, (half_t)a.z, (half_t)a.w,
                    (half_t)b.x, (half_t)b.y, (half_t)b.z, (half_t)b.w};
      } else {
        v = *(const half8_t *)(x + (int64_t)m * ldx + k);
      }
    } else {
      v = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
    }
    *(half8_t *)(As + r * kLd + 8 * cc) = v;
  }
}

__device__ __forceinline__ void put16(half_t *dst, const float *v) {
  half8_t a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = (half_t)v[i];
    b[i] = (half_t)v[8 + i];
  }
  *(half8_t *)dst = a;
  *(half8_t *)(dst + 8) = b;
}

__device__ __forceinline__ void zero16(half_t *dst) {
  *(half8_t *)dst = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
  *(half8_t *)(dst + 8) = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
}

// Weight tile: BN rows x 64 columns [k0, k0 + 64) dequantized to fp16.
template <int TYPE, int BN>
__device__ __forceinline__ void stage_b(const uint8_t *__restrict__ W, int64_t trb, int N, int K,
                                        int n0, int k0, half_t *Bs, int tid) {
#pragma unroll
  for (int p = tid; p < BN * 2; p += 256) {
    const int r = p >> 1, u = p & 1;
    const int n = n0 + r;
    half_t *dst = Bs + r * kLd;
    if (TYPE == 12) {  // Q4_K: the window is chunk c of superblock sb; u = half of the chunk
      const int sb = k0 >> 8, c = (k0 >> 6) & 3;
      if (n < N) {
        const uint8_t *blk = W + (int64_t)n * trb + 144 * sb;
        const uint4 hd = ldg16(blk);
        const uint4 qv = ldg16(blk + 16 + 32 * c + 16 * u);
        const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
        uint32_t sc0, m0, sc1, m1;
        q4k_scale_min(2 * c, hd.y, hd.z, hd.w, sc0, m0);
        q4k_scale_min(2 * c + 1, hd.y, hd.z, hd.w, sc1, m1);
        const float d1 = d * (float)sc0, mn1 = dmin * (float)m0;
        const float d2 = d * (float)sc1, mn2 = dmin * (float)m1;
        const uint32_t q[4] = {qv.x, qv.y, qv.z, qv.w};
        float lo[16], hi[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const uint32_t b = (q[i >> 2] >> (8 * (i & 3))) & 0xFFu;
          lo[i] = d1 * (float)(b & 0x0Fu) - mn1;
          hi[i] = d2 * (float)(b >> 4) - mn2;
        }
        put16(dst + 16 * u, lo);
        put16(dst + 32 + 16 * u, hi);
      } else {
        zero16(dst + 16 * u);
        zero16(dst + 32 + 16 * u);
      }
    } else if (TYPE == 8) {  // Q8_0: u selects block k0/32 + u
      const int nb = K >> 5, b = (k0 >> 5) + u;
      if (n < N && b < nb) {
        const uint8_t *row = W + (int64_t)n * trb;
        const uint4 q0 = ldg16(row + 32 * b), q1 = ldg16(row + 32 * b + 16);
        const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const float d = h2f(*(const uint16_t *)(row + K + 2 * b));
        float v[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) v[i] = d * (float)(int8_t)((q[i >> 2] >> (8 * (i & 3))) & 0xFFu);
        put16(dst + 32 * u, v);
        put16(dst + 32 * u + 16, v + 16);
      } else {
        zero16(dst + 32 * u);
        zero16(dst + 32 * u + 16);
      }
    } else {  // Q6_K: window = elements [64p, 64p + 64) of superblock sb; u = lane group g
      const int sb = k0 >> 8, pq = (k0 >> 6) & 3;
      const int h = pq >> 1, hi_nib = pq & 1;  // t = 2*hi_nib (from ql_a) and 2*hi_nib + 1 (ql_b)
      if (n < N) {
        const uint8_t *row = W + (int64_t)n * trb;
        const uint4 a = ldg16(row + 128 * sb + 64 * h + 16 * u);
        const uint4 bq = ldg16(row + 128 * sb + 64 * h + 32 + 16 * u);
        const uint4 hq = ldg16(row + K / 2 + 64 * sb + 32 * h + 16 * u);
        const int8_t *scp = (const int8_t *)(row + K / 2 + K / 4 + 16 * sb + 8 * h + u);
        const float d = h2f(*(const uint16_t *)(row + K / 2 + K / 4 + K / 16 + 2 * sb));
        const float s0 = d * (float)scp[4 * hi_nib], s1 = d * (float)scp[4 * hi_nib + 2];
        const uint32_t qa[4] = {a.x, a.y, a.z, a.w}, qb[4] = {bq.x, bq.y, bq.z, bq.w};
        const uint32_t qh[4] = {hq.x, hq.y, hq.z, hq.w};
        const int hs0 = hi_nib ? 4 : 0, hs1 = hi_nib ? 6 : 2;
        float v0[16], v1[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int w = i >> 2, sh = 8 * (i & 3);
          const uint32_t ab = (qa[w] >> sh) & 0xFFu, bb = (qb[w] >> sh) & 0xFFu;
          const uint32_t hb = (qh[w] >> sh) & 0xFFu;
          const uint32_t na = hi_nib ? (ab >> 4) : (ab & 0x0Fu);
          const uint32_t nbv = hi_nib ? (bb >> 4) : (bb & 0x0Fu);
          const int q0 = (int)(na | (((hb >> hs0) & 3u) << 4)) - 32;
          const int q1 = (int)(nbv | (((hb >> hs1) & 3u) << 4)) - 32;
          v0[i] = s0 * (float)q0;
          v1[i] = s1 * (float)q1;
        }
        put16(dst + 16 * u, v0);
        put16(dst + 32 + 16 * u, v1);
      } else {
        zero16(dst + 16 * u);
        zero16(dst + 32 + 16 * u);
      }
    }
  }
}

template <int TYPE, typename XT, int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(256) void mfma_gemm_kernel(const XT *__restrict__ x, int64_t ldx,
                                                        const uint8_t *__restrict__ W, int64_t trb,
                                                        int M, int N, int K, float *__restrict__ y,
                                                        int64_t ldy) {
  static_assert(WM * WN == 4, "four waves");
  constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
  __shared__ half_t As[BM * kLd];
  __shared__ half_t Bs[BN * kLd];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  float4_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < K; k0 += kBK) {
    stage_a<XT, BM>(x, ldx, M, K, m0, k0, As, tid);
    stage_b<TYPE, BN>(W, trb, N, K, n0, k0, Bs, tid);
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 32) {
      half8_t a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        a[i] = *(const half8_t *)(As + (wm * TM * 16 + i * 16 + (lane & 15)) * kLd + kk + 8 * (lane >> 4));
#pragma unroll
      for (int j = 0; j < TN; ++j)
        b[j] = *(const half8_t *)(Bs + (wn * TN * 16 + j * 16 + (lane & 15)) * kLd + kk + 8 * (lane >> 4));
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * TM * 16 + i * 16 + 4 * (lane >> 4) + r;
        const int n = n0 + wn * TN * 16 + j * 16 + (lane & 15);
        if (m < M && n < N) y[(int64_t)m * ldy + n] = acc[i][j][r];
      }
}

template <int TYPE, typename XT>
static void launch_type(const XT *x, int64_t ldx, const uint8_t *W, int64_t trb, int M, int N, int K,
                        float *y, int64_t ldy, bool skinny, hipStream_t s) {
  if (skinny) {
    constexpr int BM = 32, BN = 128;
    const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
    hipLaunchKernelGGL((mfma_gemm_kernel<TYPE, XT, BM, BN, 1, 4>), grid, dim3(256), 0, s, x, ldx,
                       W, trb, M, N, K, y, ldy);
  } else {
    constexpr int BM = 128, BN = 128;
    const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
    hipLaunchKernelGGL((mfma_gemm_kernel<TYPE, XT, BM, BN, 2, 2>), grid, dim3(256), 0, s, x, ldx,
                       W, trb, M, N, K, y, ldy);
  }
}

template <typename XT>
static hipError_t launch_mfma_t(const XT *x, int64_t ldx, const uint8_t *W, int type, int64_t n,
                                int64_t k, int64_t trb, float *y, int64_t ldy, int64_t m,
                                bool skinny, hipStream_t s) {
  if (type == 12)
    launch_type<12, XT>(x, ldx, W, trb, (int)m, (int)n, (int)k, y, ldy, skinny, s);
  else if (type == 8)
    launch_type<8, XT>(x, ldx, W, trb, (int)m, (int)n, (int)k, y, ldy, skinny, s);
  else
    launch_type<14, XT>(x, ldx, W, trb, (int)m, (int)n, (int)k, y, ldy, skinny, s);
  return hipGetLastError();
}

hipError_t launch_mfma(const void *x, int x_type, int64_t ldx, const uint8_t *tiles, int type,
                       int64_t n, int64_t k, int64_t trb, float *y, int64_t ldy, int64_t m,
                       bool skinny, hipStream_t s) {
  if (x_type == 0)
    return launch_mfma_t<float>((const float *)x, ldx, tiles, type, n, k, trb, y, ldy, m, skinny, s);
  return launch_mfma_t<half_t>((const half_t *)x, ldx, tiles, type, n, k, trb, y, ldy, m, skinny, s);
}

}  // namespace gguf
