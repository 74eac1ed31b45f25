// MFMA dequant-GEMM for prefill: y[m, n] = sum_k x[m, k] * dequant(W)[n, k].
//
// The reference has no GEMM for these types: prefill re-runs its GEMV once
// per activation row (webgpu/src/engine/forward-pass.ts:1536-1539).  Here a
// workgroup owns a BM x BN output tile; per 64-wide K step it stages the
// activation tile (fp16) and the weight tile dequantized to fp16 (one
// rounding of the exact f32 dequant value, RNE) in LDS, and its four waves
// feed v_mfma_f32_16x16x32_f16 with f32 accumulation.  f32 activations are
// rounded to fp16 when staged.  Weight tiles are read from the row-tile
// layout (common.hpp): BN = 128 rows are 8 consecutive row tiles.
#include "common.hpp"

namespace gguf {

namespace {

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

__device__ __forceinline__ void put8(half_t *dst, const float *v) {
  half8_t a;
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = (half_t)v[i];
  *(half8_t *)dst = a;
}
__device__ __forceinline__ void put4(half_t *dst, const float *v) {
  *(half4_t *)dst = half4_t{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
}
__device__ __forceinline__ void zero8(half_t *dst) {
  *(half8_t *)dst = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
}

// Weight tile: BN rows x 64 columns [k0, k0 + 64) dequantized to fp16.
// Work item = (row tile tt, lane slot (r, g)); rows past N are the zero
// padding of the last tile or, for tiles past the end, skipped (written 0).
template <int TYPE, int BN>
__device__ __forceinline__ void stage_b(const uint8_t *__restrict__ W, int N, int K, int n0, int k0,
                                        half_t *Bs, int tid) {
  constexpr int TU = Fmt<TYPE>::TU, UE = Fmt<TYPE>::UE;
  const int nu = K / UE;
  const int ntiles = (N + 15) >> 4;
  if (TYPE == 8) {
    // two blocks per step: items (tt, b, g, r)
#pragma unroll
    for (int p = tid; p < BN * 8; p += 256) {
      const int r = p & 15, g = (p >> 4) & 3, b = (p >> 6) & 1, tt = p >> 7;
      const int tile = (n0 >> 4) + tt, blk = (k0 >> 5) + b;
      half_t *dst = Bs + (16 * tt + r) * kLd + 32 * b + 8 * g;
      if (tile < ntiles && blk < nu) {
        const uint8_t *tu = W + ((int64_t)tile * nu + blk) * TU;
        const uint2 q = *(const uint2 *)(tu + 32 + (16 * g + r) * 8);
        const float d = h2f(*(const uint16_t *)(tu + 2 * r));
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = d * (float)(int8_t)(((i < 4 ? q.x : q.y) >> (8 * (i & 3))) & 0xFFu);
        put8(dst, v);
      } else {
        zero8(dst);
      }
    }
    return;
  }
  const int u = k0 >> 8, wq = (k0 >> 6) & 3;
#pragma unroll
  for (int p = tid; p < BN * 4; p += 256) {
    const int r = p & 15, g = (p >> 4) & 3, tt = p >> 6;
    const int tile = (n0 >> 4) + tt;
    half_t *row = Bs + (16 * tt + r) * kLd;
    if (tile >= ntiles) {
      if (TYPE == 12) {
        zero8(row + 8 * g);
        zero8(row + 32 + 8 * g);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) *(half4_t *)(row + 16 * j + 4 * g) = half4_t{0, 0, 0, 0};
      }
      continue;
    }
    const uint8_t *tu = W + ((int64_t)tile * nu + u) * TU;
    if (TYPE == 12) {  // window = chunk c = wq: lo -> [8g, 8g+8), hi -> [32 + 8g, 32 + 8g + 8)
      const int c = wq, cp = c >> 1, h = c & 1;
      const uint4 hd = ldg16(tu + 16 * r);
      const uint4 pc = ldg16(tu + 256 + ((4 * cp + g) * 16 + r) * 16);
      const uint32_t q0 = h ? pc.z : pc.x, q1 = h ? pc.w : pc.y;
      const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
      uint32_t sc0, m0, sc1, m1;
      q4k_scale_min(2 * c, hd.y, hd.z, hd.w, sc0, m0);
      q4k_scale_min(2 * c + 1, hd.y, hd.z, hd.w, sc1, m1);
      const float d1 = d * (float)sc0, mn1 = dmin * (float)m0;
      const float d2 = d * (float)sc1, mn2 = dmin * (float)m1;
      float lo[8], hi[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t b = ((i < 4 ? q0 : q1) >> (8 * (i & 3))) & 0xFFu;
        lo[i] = d1 * (float)(b & 0x0Fu) - mn1;
        hi[i] = d2 * (float)(b >> 4) - mn2;
      }
      put8(row + 8 * g, lo);
      put8(row + 32 + 8 * g, hi);
    } else {  // Q6_K: window = half hf, quarters t in {2 tp, 2 tp + 1}
      const int hf = wq >> 1, tp = wq & 1;
      const float d = h2f(*(const uint16_t *)(tu + 3328 + 2 * r));
      const int8_t *sc = (const int8_t *)(tu + 3072 + 16 * r);
#pragma unroll
      for (int lh = 0; lh < 2; ++lh) {
        const int i = 2 * hf + lh;  // dwords 3i .. 3i + 2 of the lane's 12
        uint32_t dq[3];
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          const int dwi = 3 * i + j;
          dq[j] = *(const uint32_t *)(tu + ((4 * (dwi >> 2) + g) * 16 + r) * 16 + 4 * (dwi & 3));
        }
#pragma unroll
        for (int tt2 = 0; tt2 < 2; ++tt2) {
          const int t = 2 * tp + tt2;
          const uint32_t ql = (t & 1) ? dq[1] : dq[0];
          const float s = d * (float)sc[8 * hf + 2 * t + lh];
          float v[4];
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const uint32_t qb = (ql >> (8 * b)) & 0xFFu, hb = (dq[2] >> (8 * b)) & 0xFFu;
            const uint32_t nib = (t >> 1) ? (qb >> 4) : (qb & 0x0Fu);
            v[b] = s * (float)((int)(nib | (((hb >> (2 * t)) & 3u) << 4)) - 32);
          }
          // window-local element 32 * tt2 + 16 lh + 4 g + b
          put4(row + 32 * tt2 + 16 * lh + 4 * g, v);
        }
      }
    }
  }
}

template <int TYPE, typename XT, int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(256) void gemm_kernel(const XT *__restrict__ x, int64_t ldx,
                                                   const uint8_t *__restrict__ W, int M, int N,
                                                   int K, float *__restrict__ y, int64_t ldy) {
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
    stage_b<TYPE, BN>(W, N, K, n0, k0, Bs, tid);
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
void launch_type(const XT *x, int64_t ldx, const uint8_t *W, int M, int N, int K, float *y,
                 int64_t ldy, hipStream_t s) {
  constexpr int BM = 128, BN = 128;
  const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
  hipLaunchKernelGGL((gemm_kernel<TYPE, XT, BM, BN, 2, 2>), grid, dim3(256), 0, s, x, ldx, W, M, N,
                     K, y, ldy);
}

template <typename XT>
hipError_t launch_x(const XT *x, int64_t ldx, const uint8_t *W, int type, int64_t n, int64_t k,
                    float *y, int64_t ldy, int64_t m, hipStream_t s) {
  if (type == 12)
    launch_type<12, XT>(x, ldx, W, (int)m, (int)n, (int)k, y, ldy, s);
  else if (type == 8)
    launch_type<8, XT>(x, ldx, W, (int)m, (int)n, (int)k, y, ldy, s);
  else
    launch_type<14, XT>(x, ldx, W, (int)m, (int)n, (int)k, y, ldy, s);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(const void *x, int x_type, int64_t ldx, const uint8_t *tiles, int type,
                       int64_t n, int64_t k, float *y, int64_t ldy, int64_t m, hipStream_t s) {
  const int esize = x_type == 0 ? 4 : 2;
  const int64_t chunk = (int64_t)65535 * 128;  // grid.y cap
  hipError_t e = hipSuccess;
  for (int64_t m0 = 0; m0 < m && e == hipSuccess; m0 += chunk) {
    const int64_t mc = (m - m0) < chunk ? (m - m0) : chunk;
    const char *xb = (const char *)x + m0 * ldx * esize;
    e = x_type == 0 ? launch_x<float>((const float *)xb, ldx, tiles, type, n, k, y + m0 * ldy, ldy,
                                      mc, s)
                    : launch_x<half_t>((const half_t *)xb, ldx, tiles, type, n, k, y + m0 * ldy,
                                       ldy, mc, s);
  }
  return e;
}

}  // namespace gguf
