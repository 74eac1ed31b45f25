// Decode-step glue of a Llama-style layer around the quantized projections:
// RMSNorm (optionally fused with the residual add that precedes it), SwiGLU,
// rotate_half RoPE + KV-cache append + GQA attention for one new position,
// and greedy argmax.  Reference shaders: rmsnorm.wgsl:1-9,58-67,
// rope.wgsl:1-10, elementwise.wgsl:96-102 (gate_silu), argmax.wgsl; the
// layer loop is webgpu/src/engine/forward-pass.ts:2925-3297.
//
// All kernels are f32, one row (or one KV head) per workgroup; they are small
// and latency-bound, so the goal is one launch per op with coalesced 16-byte
// accesses, not occupancy.
#include <mutex>

#include "common.hpp"

namespace gguf {

namespace {

constexpr int kGlueThreads = 256;

// Sum over the workgroup; every thread gets the result.  `red` holds one
// float per wave.
__device__ __forceinline__ float block_sum(float v, float *red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float s = 0.f;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) s += red[w];
  return s;
}

__device__ __forceinline__ float block_max(float v, float *red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float s = red[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) s = fmaxf(s, red[w]);
  return s;
}

// y = x * 1/sqrt(mean(x^2) + eps) * w  (rmsnorm.wgsl:58-67, direct weight);
// with r != null the residual add x += r is applied first and x is updated.
// Rows of up to 4 * 4 * kNormThreads elements are held in registers (one
// read of x); longer rows are read twice.
constexpr int kNormThreads = 1024;
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(float *__restrict__ x,
                                                               const float *__restrict__ r,
                                                               const float *__restrict__ w,
                                                               float eps, float *__restrict__ y,
                                                               int n) {
  __shared__ float red[kNormThreads / 64];
  float *xr = x + (int64_t)blockIdx.x * n;
  const float *rr = r ? r + (int64_t)blockIdx.x * n : nullptr;
  float *yr = y + (int64_t)blockIdx.x * n;
  constexpr int R = 4;
  float4 v[R];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < R; ++c) {
    const int i = 4 * (c * kNormThreads + threadIdx.x);
    v[c] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (i < n) {
      v[c] = *(const float4 *)(xr + i);
      if (rr) {
        const float4 a = *(const float4 *)(rr + i);
        v[c].x += a.x;
        v[c].y += a.y;
        v[c].z += a.z;
        v[c].w += a.w;
        *(float4 *)(xr + i) = v[c];
      }
    }
    ss += v[c].x * v[c].x + v[c].y * v[c].y + v[c].z * v[c].z + v[c].w * v[c].w;
  }
  for (int i = 4 * (R * kNormThreads + threadIdx.x); i < n; i += 4 * kNormThreads) {
    float4 a = *(const float4 *)(xr + i);
    if (rr) {
      const float4 b = *(const float4 *)(rr + i);
      a.x += b.x;
      a.y += b.y;
      a.z += b.z;
      a.w += b.w;
      *(float4 *)(xr + i) = a;
    }
    ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
  }
  const float inv = 1.0f / sqrtf(block_sum(ss, red) / (float)n + eps);
#pragma unroll
  for (int c = 0; c < R; ++c) {
    const int i = 4 * (c * kNormThreads + threadIdx.x);
    if (i < n) {
      const float4 g = *(const float4 *)(w + i);
      *(float4 *)(yr + i) = make_float4(v[c].x * inv * g.x, v[c].y * inv * g.y,
                                        v[c].z * inv * g.z, v[c].w * inv * g.w);
    }
  }
  for (int i = 4 * (R * kNormThreads + threadIdx.x); i < n; i += 4 * kNormThreads) {
    const float4 a = *(const float4 *)(xr + i), g = *(const float4 *)(w + i);
    *(float4 *)(yr + i) = make_float4(a.x * inv * g.x, a.y * inv * g.y, a.z * inv * g.z,
                                      a.w * inv * g.w);
  }
}

// out[i] = up[i] * silu(gate[i]) for a row [gate (ffn) | up (ffn)]
// (elementwise.wgsl:96-102 with a = up, b = gate).
__global__ __launch_bounds__(kGlueThreads) void swiglu_kernel(const float *__restrict__ gu,
                                                              float *__restrict__ out, int ffn) {
  const float *g = gu + (int64_t)blockIdx.y * 2 * ffn, *u = g + ffn;
  float *o = out + (int64_t)blockIdx.y * ffn;
  const int i = 4 * (blockIdx.x * kGlueThreads + threadIdx.x);
  if (i >= ffn) return;
  const float4 a = *(const float4 *)(g + i), b = *(const float4 *)(u + i);
  *(float4 *)(o + i) = make_float4(b.x * (a.x / (1.0f + expf(-a.x))), b.y * (a.y / (1.0f + expf(-a.y))),
                                   b.z * (a.z / (1.0f + expf(-a.z))), b.w * (a.w / (1.0f + expf(-a.w))));
}

// Decode attention in one launch, flash-decoding style.  Workgroup (g, sp)
// takes KV head g and cache slots [64 sp, 64 sp + 64) of the causal range
// 0..p, p = *pos; the n = ceil((p + 1) / 64) workgroups of the range take
// part and the others exit.  The workgroup whose range holds p writes slot p
// (k after rotate_half RoPE, v as is) into the cache.
//
// Every global load of a workgroup (its K / V rows, the new k / v, the first
// query row of each wave, the RoPE rows) is issued before any is consumed,
// so the whole input arrives in one latency round.  The K / V rows are
// staged in LDS (K rows at a stride of HD + 4 floats, so that lane t reading
// row t is free of bank conflicts); wave w takes query heads w, w + 4, ...:
// lane t owns slot t0 + t, a wave computes 64 dot products, one wave-wide
// softmax reduction and sum_t p_t v_t reading V rows from LDS.
//
// With n = 1 the workgroup writes the output.  Otherwise it writes its
// partial-softmax record per query head (layout and merge rule next to
// kAttnSplit), and the last of the n workgroups to finish -- an atomic
// counter per KV head, kept in the workspace and left at zero -- merges the n
// records in split order, so the result does not depend on which workgroup
// finishes last.  With out == nullptr every workgroup writes its records and
// nothing is merged: the consumer (the output projection's merge prologue)
// merges them with the same arithmetic.
constexpr int kSplit = kAttnSplit;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

template <int HD>
__global__ __launch_bounds__(kGlueThreads) void attention_kernel(
    const float *__restrict__ qkv, const int64_t *__restrict__ pos, const float *__restrict__ cs,
    const float *__restrict__ sn, float *__restrict__ kc, float *__restrict__ vc,
    float *__restrict__ out, float *__restrict__ work, unsigned *__restrict__ counters, int nh,
    int nkv, int max_seq) {
  constexpr int half = HD / 2, KLD = HD + 4, C4 = HD / 4;
  constexpr int KV4 = kSplit * C4 / kGlueThreads;  // float4 of K (and of V) per thread
  constexpr int QR = (half + 63) / 64;             // query element pairs per lane
  // K / V rows; row kSplit is a pad that takes the stores of rows outside the range
  __shared__ __align__(16) float ks[(kSplit + 1) * KLD];
  __shared__ __align__(16) float vs[(kSplit + 1) * HD];
  __shared__ __align__(16) float qw[4 * HD];       // per wave: roped, scaled query
  __shared__ float pw[4 * kSplit];                  // per wave: probabilities
  __shared__ int merge;
  const int grp = nh / nkv, g = blockIdx.x, sp = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int S = gridDim.y;
  const int64_t p64 = pos[0];
  if (p64 < 0 || p64 >= max_seq) return;  // no cache slot: write nothing
  const int p = (int)p64, T = p + 1, t0 = sp * kSplit;
  if (t0 >= T) return;                     // beyond the causal range
  const int n = (T + kSplit - 1) / kSplit;
  const int tn = min(kSplit, T - t0);
  const int tp = p - t0;                   // row of slot p in this block when < kSplit
  const bool holds_p = tp < kSplit;
  const bool rec_only = out == nullptr;
  constexpr int RS = attn_record_stride(HD);
  float *kbase = kc + (int64_t)g * max_seq * HD, *vbase = vc + (int64_t)g * max_seq * HD;
  const float *crow = cs + (int64_t)p * half, *srow = sn + (int64_t)p * half;

  // 1. all global loads, straight-line: a row outside [t0, t0 + tn) or slot p
  // (written below) reads row t0 instead (always a valid slot) into the pad
  float4 kr[KV4], vr[KV4];
#pragma unroll
  for (int i = 0; i < KV4; ++i) {
    const int e = tid + i * kGlueThreads, t = e / C4, c = e - t * C4;
    const int row = (t < tn && t != tp) ? t0 + t : t0;
    kr[i] = *(const float4 *)(kbase + (int64_t)row * HD + 4 * c);
    vr[i] = *(const float4 *)(vbase + (int64_t)row * HD + 4 * c);
  }
  const int j0 = wave;
  float qa[QR], qb[QR], qc[QR], qs[QR];
  if (j0 < grp) {
    const float *qin = qkv + (int64_t)(g * grp + j0) * HD;
#pragma unroll
    for (int r = 0; r < QR; ++r) {
      const int i = lane + 64 * r;
      if (i < half) {
        qa[r] = qin[i];
        qb[r] = qin[i + half];
        qc[r] = crow[i];
        qs[r] = srow[i];
      }
    }
  }
  float ka = 0.f, kb = 0.f, kcs = 0.f, ksn = 0.f, vv = 0.f;
  if (holds_p) {
    const float *kin = qkv + (int64_t)nh * HD + g * HD;
    const float *vin = qkv + (int64_t)(nh + nkv) * HD + g * HD;
    if (tid < half) {
      ka = kin[tid];
      kb = kin[tid + half];
      kcs = crow[tid];
      ksn = srow[tid];
    }
    if (tid < HD) vv = vin[tid];
  }

  // keep the loads above ahead of every use below (the scheduler would
  // otherwise sink each load to its store and serialize the round trips)
  __builtin_amdgcn_sched_barrier(0);

  // 2. LDS: the block's K / V rows, slot p (rotate_half RoPE of k, rope.wgsl:1-10;
  // also into the caches) and each wave's first roped, scaled query
#pragma unroll
  for (int i = 0; i < KV4; ++i) {
    const int e = tid + i * kGlueThreads, t = e / C4, c = e - t * C4;
    const int st = (t < tn && t != tp) ? t : kSplit;
    *(float4 *)(ks + st * KLD + 4 * c) = kr[i];
    *(float4 *)(vs + st * HD + 4 * c) = vr[i];
  }
  if (holds_p) {
    float *krow = kbase + (int64_t)p * HD, *vrow = vbase + (int64_t)p * HD;
    if (tid < half) {
      const float k0 = ka * kcs - kb * ksn, k1 = kb * kcs + ka * ksn;
      krow[tid] = k0;
      krow[tid + half] = k1;
      ks[tp * KLD + tid] = k0;
      ks[tp * KLD + tid + half] = k1;
    }
    if (tid < HD) {
      vrow[tid] = vv;
      vs[tp * HD + tid] = vv;
    }
  }
  const float scale = 1.0f / sqrtf((float)HD);
  float *q = qw + wave * HD;
  if (j0 < grp) {
#pragma unroll
    for (int r = 0; r < QR; ++r) {
      const int i = lane + 64 * r;
      if (i < half) {
        q[i] = (qa[r] * qc[r] - qb[r] * qs[r]) * scale;
        q[i + half] = (qb[r] * qc[r] + qa[r] * qs[r]) * scale;
      }
    }
  }
  __syncthreads();

  // 3. per query head: scores, softmax, sum p v
  float *pr = pw + wave * kSplit;
  for (int j = j0; j < grp; j += 4) {
    if (j != j0) {  // later heads of a group larger than four: rope this query now
      const float *qin = qkv + (int64_t)(g * grp + j) * HD;
      for (int i = lane; i < half; i += 64) {
        const float c = crow[i], sv = srow[i], a = qin[i], b = qin[i + half];
        q[i] = (a * c - b * sv) * scale;
        q[i + half] = (b * c + a * sv) * scale;
      }
    }
    // the wave's own LDS writes are visible to it in program order
    float sc = -INFINITY;
    if (lane < tn) {
      const float *kr_ = ks + lane * KLD;
      float a0 = 0.f, a1 = 0.f;
#pragma unroll
      for (int c = 0; c < C4; c += 2) {
        const float4 k0 = *(const float4 *)(kr_ + 4 * c), q0 = *(const float4 *)(q + 4 * c);
        const float4 k1 = *(const float4 *)(kr_ + 4 * c + 4), q1 = *(const float4 *)(q + 4 * c + 4);
        a0 += q0.x * k0.x + q0.y * k0.y + q0.z * k0.z + q0.w * k0.w;
        a1 += q1.x * k1.x + q1.y * k1.y + q1.z * k1.z + q1.w * k1.w;
      }
      sc = a0 + a1;
    }
    const float m = wave_max(sc);
    const float e = lane < tn ? expf(sc - m) : 0.f;
    const float l = wave_sum(e);
    pr[lane] = e;
    const bool direct = n == 1 && !rec_only;
    float *rec = work + ((int64_t)(g * S + sp) * grp + j) * RS;
    float *o_out = direct ? out + (int64_t)(g * grp + j) * HD : rec;
    const float inv = direct ? 1.0f / l : 1.0f;
    for (int i = lane; i < HD; i += 64) {
      float o = 0.f;
#pragma unroll 8
      for (int t = 0; t < tn; ++t) o += pr[t] * vs[t * HD + i];
      o_out[i] = o * inv;
    }
    if (!direct && lane == 0) {
      rec[HD] = m;
      rec[HD + 1] = l;
    }
  }
  if (n == 1 || rec_only) return;

  // 4. the last of the n workgroups of KV head g merges the records
  __threadfence();  // this workgroup's records are visible before it is counted
  __syncthreads();
  if (tid == 0) merge = atomicAdd(counters + g, 1u) == (unsigned)(n - 1);
  __syncthreads();
  if (!merge) return;
  __threadfence();  // every other workgroup's records are visible to the merge
  // wave w merges query heads w, w + 4, ...: lane s reads record s's (m, l),
  // so a chunk of 64 records costs one load round, and the weighted sums of
  // the outputs issue their loads together.  L and the outputs accumulate in
  // split order, as the merge prologue of the output projection does.
  constexpr int QO = HD / 64;  // outputs per lane
  const int64_t stride = (int64_t)grp * RS;
  float *pl = ks;  // the K rows are consumed: per wave, the 64 (w_s, l_s) of a chunk
  for (int j = wave; j < grp; j += 4) {
    const float *base = work + ((int64_t)g * S * grp + j) * RS;
    float M = -INFINITY;
    for (int s0 = 0; s0 < n; s0 += 64)
      if (s0 + lane < n) M = fmaxf(M, base[(s0 + lane) * stride + HD]);
    M = wave_max(M);
    float L = 0.f, o[QO];
#pragma unroll
    for (int r = 0; r < QO; ++r) o[r] = 0.f;
    for (int s0 = 0; s0 < n; s0 += 64) {
      float w = 0.f, lv = 0.f;
      if (s0 + lane < n) {
        const float *rec = base + (s0 + lane) * stride;
        w = expf(rec[HD] - M);
        lv = rec[HD + 1];
      }
      pr[lane] = w;  // wave-local: read back in program order
      pl[wave * 64 + lane] = lv;
      const int cnt = min(64, n - s0);
#pragma unroll 8
      for (int u = 0; u < cnt; ++u) {
        const float wu = pr[u];
        L = fmaf(wu, pl[wave * 64 + u], L);
        const float *ro = base + (s0 + u) * stride + lane;
#pragma unroll
        for (int r = 0; r < QO; ++r) o[r] = fmaf(wu, ro[64 * r], o[r]);
      }
    }
    const float inv = 1.0f / L;
#pragma unroll
    for (int r = 0; r < QO; ++r) out[(int64_t)(g * grp + j) * HD + lane + 64 * r] = o[r] * inv;
  }
  if (tid == 0) counters[g] = 0u;  // ready for the next call
}

// ---------------------------------------------------------------------------
// Prefill attention: M new positions, two launches.
//
// rope_append_kernel: one workgroup per row m.  It applies rotate_half RoPE
// (rope.wgsl:1-10, the same products as the decode kernel) to the row's k
// heads and stores k and v at slot pos[m] of the caches.  A row whose position
// lies outside 0..max_seq-1 writes nothing.
//
// attention_prefill_kernel: causal GQA attention of each row over slots
// 0..pos[m] (attention.wgsl:60-234 with new_seq_len = M), flash-style on the
// f32 matrix cores.
// - A workgroup takes 16 rows and one KV head.  Wave w takes query heads
//   w, w + 4, ... of the group, one per pass over the keys.
// - Keys come in tiles of KT slots: K rows [KT][HD + 4] and V transposed
//   [HD][KT + 4] in LDS.  The next tile's loads are in flight while the
//   current tile is used.
// - Per 16 keys, v_mfma_f32_16x16x4f32 computes S^T = K . Q^T (keys x rows).
//   Its accumulator layout (lane l: keys 4(l/16) + r of row l%16) is exactly
//   the B-operand layout of O^T += V^T . P^T when k-step r takes keys
//   4(l/16) + r.  So the probabilities never leave their registers.
// - Every lane holds one row's running max, running sum and output column,
//   so the online-softmax rescale is lane-local.
// - The head_dim reduction of S^T runs over elements 16a + 4(l/16) + b, a
//   bijection onto 0..HD-1, so each lane's K and Q operands are float4 reads.
// A row whose position lies outside 0..max_seq-1, or past M, attends to
// nothing and is not written.
constexpr int kPfRows = 16;  // rows (positions) per workgroup

template <int HD>
struct PfShape {
  static constexpr int KT = HD <= 128 ? 64 : 32;          // key slots per tile
  static constexpr int KLD = HD + 4, VLD = KT + 4;         // LDS row strides (floats)
  static constexpr int NF = KT * HD / 4 / kGlueThreads;    // float4 of K (and of V) per thread
};

template <int HD>
__global__ __launch_bounds__(kGlueThreads) void rope_append_kernel(
    const float *__restrict__ qkv, int64_t ldq, const int64_t *__restrict__ pos,
    const float *__restrict__ cs, const float *__restrict__ sn, float *__restrict__ kc,
    float *__restrict__ vc, int nh, int nkv, int max_seq) {
  constexpr int half = HD / 2;
  const int64_t m = blockIdx.x;
  const int64_t p = pos[m];
  if (p < 0 || p >= max_seq) return;
  const float *kin = qkv + m * ldq + (int64_t)nh * HD, *vin = kin + (int64_t)nkv * HD;
  const float *crow = cs + p * half, *srow = sn + p * half;
  for (int e = threadIdx.x; e < nkv * half; e += kGlueThreads) {
    const int h = e / half, i = e - h * half;
    const float a = kin[h * HD + i], b = kin[h * HD + i + half], c = crow[i], s = srow[i];
    float *krow = kc + ((int64_t)h * max_seq + p) * HD;
    krow[i] = a * c - b * s;
    krow[i + half] = b * c + a * s;
  }
  for (int e = threadIdx.x; e < nkv * HD; e += kGlueThreads) {
    const int h = e / HD, i = e - h * HD;
    vc[((int64_t)h * max_seq + p) * HD + i] = vin[h * HD + i];
  }
}

__device__ __forceinline__ float4_t mfma_f32(float a, float b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int HD>
__global__ __launch_bounds__(kGlueThreads) void attention_prefill_kernel(
    const float *__restrict__ qkv, int64_t ldq, const int64_t *__restrict__ pos, int64_t M,
    const float *__restrict__ cs, const float *__restrict__ sn, const float *__restrict__ kc,
    const float *__restrict__ vc, float *__restrict__ out, int64_t ldo, int nh, int nkv,
    int max_seq) {
  using Sh = PfShape<HD>;
  constexpr int KT = Sh::KT, KLD = Sh::KLD, VLD = Sh::VLD, NF = Sh::NF, half = HD / 2;
  constexpr int QA = HD / 16;  // float4 of q per lane, and 16-element output tiles
  constexpr int NT = KT / 16;  // 16-key tiles per key tile
  __shared__ __align__(16) float ks[KT * KLD];
  __shared__ __align__(16) float vt[HD * VLD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, g4 = lane >> 4;  // MFMA column (row of the block), k group
  const int grp = nh / nkv, kvh = blockIdx.y;
  const int64_t m = (int64_t)blockIdx.x * kPfRows + col;
  int my = -1;  // the row's position; -1: attends to nothing, not written
  if (m < M) {
    const int64_t p = pos[m];
    if (p >= 0 && p < max_seq) my = (int)p;
  }
  // slots 0 .. kend - 1 hold every key of the block's rows (same in every wave)
  int kend = my + 1;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) kend = max(kend, __shfl_xor(kend, o));
  const int ntile = (kend + KT - 1) / KT;
  const float *kbase = kc + (int64_t)kvh * max_seq * HD;
  const float *vbase = vc + (int64_t)kvh * max_seq * HD;
  const float scale = 1.0f / sqrtf((float)HD);

  // float4 f = i * 256 + tid of a tile: 64-float4 block f / 64 = (16-slot block,
  // 4-chunk block); within it slot f % 16, chunk (f / 16) % 4.  A wave's LDS
  // stores (K rows, V transposed) are then free of bank conflicts.
  float4 kr[NF], vr[NF];
  auto load_tile = [&](int t0) {
#pragma unroll
    for (int i = 0; i < NF; ++i) {
      const int f = i * kGlueThreads + tid, blk = f >> 6;
      const int t = (blk / (HD / 16)) * 16 + (f & 15), c = (blk % (HD / 16)) * 4 + ((f >> 4) & 3);
      const int row = t0 + t;  // < kend <= max_seq when read
      kr[i] = row < kend ? *(const float4 *)(kbase + (int64_t)row * HD + 4 * c)
                         : make_float4(0.f, 0.f, 0.f, 0.f);
      vr[i] = row < kend ? *(const float4 *)(vbase + (int64_t)row * HD + 4 * c)
                         : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < NF; ++i) {
      const int f = i * kGlueThreads + tid, blk = f >> 6;
      const int t = (blk / (HD / 16)) * 16 + (f & 15), c = (blk % (HD / 16)) * 4 + ((f >> 4) & 3);
      *(float4 *)(ks + t * KLD + 4 * c) = kr[i];
      vt[(4 * c + 0) * VLD + t] = vr[i].x;
      vt[(4 * c + 1) * VLD + t] = vr[i].y;
      vt[(4 * c + 2) * VLD + t] = vr[i].z;
      vt[(4 * c + 3) * VLD + t] = vr[i].w;
    }
  };

  for (int hp = 0; hp * 4 < grp; ++hp) {
    const int jh = hp * 4 + wave;  // query head within the group
    const bool act = jh < grp;     // wave-uniform
    const int64_t qcol = (int64_t)(kvh * grp + jh) * HD + 4 * g4;
    // the row's query, roped and scaled: q[a] = elements 16a + 4 g4 + 0..3
    float4 q[QA];
#pragma unroll
    for (int a = 0; a < QA; ++a) q[a] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (act && my >= 0) {
      const float *qin = qkv + m * ldq + qcol;
#pragma unroll
      for (int a = 0; a < QA; ++a) q[a] = *(const float4 *)(qin + 16 * a);
      const float *crow = cs + (int64_t)my * half + 4 * g4, *srow = sn + (int64_t)my * half + 4 * g4;
#pragma unroll
      for (int a = 0; a < QA / 2; ++a) {
        const float4 c = *(const float4 *)(crow + 16 * a), s = *(const float4 *)(srow + 16 * a);
        const float4 x = q[a], y = q[a + QA / 2];
        q[a] = make_float4((x.x * c.x - y.x * s.x) * scale, (x.y * c.y - y.y * s.y) * scale,
                           (x.z * c.z - y.z * s.z) * scale, (x.w * c.w - y.w * s.w) * scale);
        q[a + QA / 2] =
            make_float4((y.x * c.x + x.x * s.x) * scale, (y.y * c.y + x.y * s.y) * scale,
                        (y.z * c.z + x.z * s.z) * scale, (y.w * c.w + x.w * s.w) * scale);
      }
    }
    float4_t o[QA];
#pragma unroll
    for (int a = 0; a < QA; ++a) o[a] = float4_t{0.f, 0.f, 0.f, 0.f};
    float mrun = -INFINITY, lrun = 0.f;

    if (ntile > 0) load_tile(0);
    for (int it = 0; it < ntile; ++it) {
      __syncthreads();  // every wave is done with the previous tile
      store_tile();
      __syncthreads();
      if (it + 1 < ntile) load_tile((it + 1) * KT);
      if (!act) continue;
      // S^T for the tile's keys: s[j][r] = score of key it*KT + 16j + 4 g4 + r
      float4_t s[NT];
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        s[j] = float4_t{0.f, 0.f, 0.f, 0.f};
        const float *kp = ks + (16 * j + col) * KLD + 4 * g4;
#pragma unroll
        for (int a = 0; a < QA; ++a) {
          const float4 kf = *(const float4 *)(kp + 16 * a);
          s[j] = mfma_f32(kf.x, q[a].x, s[j]);
          s[j] = mfma_f32(kf.y, q[a].y, s[j]);
          s[j] = mfma_f32(kf.z, q[a].z, s[j]);
          s[j] = mfma_f32(kf.w, q[a].w, s[j]);
        }
      }
      // causal mask, the block's max over the row (4 lanes share a row)
      const int tb = it * KT + 4 * g4;
      float bm = -INFINITY;
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float v = tb + 16 * j + r <= my ? s[j][r] : -INFINITY;
          s[j][r] = v;
          bm = fmaxf(bm, v);
        }
      bm = fmaxf(bm, __shfl_xor(bm, 16));
      bm = fmaxf(bm, __shfl_xor(bm, 32));
      const float mnew = fmaxf(mrun, bm);
      const float alpha = mnew == -INFINITY ? 1.f : expf(mrun - mnew);
      mrun = mnew;
      float ls = 0.f;
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float e = s[j][r] == -INFINITY ? 0.f : expf(s[j][r] - mnew);
          s[j][r] = e;
          ls += e;
        }
      lrun = lrun * alpha + ls;
#pragma unroll
      for (int a = 0; a < QA; ++a) o[a] *= alpha;
      // O^T[d][row] += sum over the tile's keys of V[key][d] P[row][key]
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const float *vp = vt + col * VLD + 16 * j + 4 * g4;
#pragma unroll
        for (int a = 0; a < QA; ++a) {
          const float4 vf = *(const float4 *)(vp + 16 * a * VLD);
          o[a] = mfma_f32(vf.x, s[j][0], o[a]);
          o[a] = mfma_f32(vf.y, s[j][1], o[a]);
          o[a] = mfma_f32(vf.z, s[j][2], o[a]);
          o[a] = mfma_f32(vf.w, s[j][3], o[a]);
        }
      }
    }
    if (!act) continue;
    float l = lrun + __shfl_xor(lrun, 16);
    l += __shfl_xor(l, 32);
    if (my >= 0) {
      const float inv = 1.0f / l;
      float *orow = out + m * ldo + qcol;
#pragma unroll
      for (int a = 0; a < QA; ++a)
        *(float4 *)(orow + 16 * a) = make_float4(o[a][0] * inv, o[a][1] * inv, o[a][2] * inv,
                                                 o[a][3] * inv);
    }
  }
}

// Argmax, pass 1: workgroup b scans a contiguous chunk and writes its (value,
// index) with the first index on ties and NaN never winning; pass 2 (one
// workgroup) merges the partials the same way.
constexpr int kArgBlocks = 256;

__device__ __forceinline__ void better(float &v, int64_t &i, float ov, int64_t oi) {
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}

__device__ __forceinline__ void block_argmax(float &v, int64_t &idx, float *bv, int64_t *bi) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) better(v, idx, __shfl_xor(v, o), __shfl_xor(idx, o));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    bv[wave] = v;
    bi[wave] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0)
    for (int w2 = 1; w2 < (int)(blockDim.x >> 6); ++w2) better(v, idx, bv[w2], bi[w2]);
}

__global__ __launch_bounds__(kGlueThreads) void argmax_partial_kernel(const float *__restrict__ x,
                                                                      int64_t n,
                                                                      float *__restrict__ pv,
                                                                      int64_t *__restrict__ pi) {
  __shared__ float bv[kGlueThreads / 64];
  __shared__ int64_t bi[kGlueThreads / 64];
  const int64_t chunk = (n + kArgBlocks - 1) / kArgBlocks;
  const int64_t lo = (int64_t)blockIdx.x * chunk, hi = min(n, lo + chunk);
  float v = -INFINITY;
  int64_t idx = INT64_MAX;  // no candidate yet
  for (int64_t i = lo + threadIdx.x; i < hi; i += kGlueThreads) better(v, idx, x[i], i);
  block_argmax(v, idx, bv, bi);
  if (threadIdx.x == 0) {
    pv[blockIdx.x] = v;
    pi[blockIdx.x] = idx;
  }
}

__global__ __launch_bounds__(kGlueThreads) void argmax_merge_kernel(const float *__restrict__ pv,
                                                                    const int64_t *__restrict__ pi,
                                                                    int64_t *__restrict__ out) {
  __shared__ float bv[kGlueThreads / 64];
  __shared__ int64_t bi[kGlueThreads / 64];
  float v = -INFINITY;
  int64_t idx = INT64_MAX;
  for (int b = threadIdx.x; b < kArgBlocks; b += kGlueThreads) better(v, idx, pv[b], pi[b]);
  block_argmax(v, idx, bv, bi);
  if (threadIdx.x == 0) out[0] = idx == INT64_MAX ? 0 : idx;
}

}  // namespace

hipError_t launch_rmsnorm(float *x, const float *r, const float *w, float eps, float *y,
                          int64_t rows, int64_t n, hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(kNormThreads), 0, s, x, r, w, eps,
                     y, (int)n);
  return hipGetLastError();
}

hipError_t launch_swiglu(const float *gu, float *out, int64_t rows, int64_t ffn, hipStream_t s) {
  const unsigned bx = (unsigned)((ffn / 4 + kGlueThreads - 1) / kGlueThreads);
  hipLaunchKernelGGL(swiglu_kernel, dim3(bx, (unsigned)rows), dim3(kGlueThreads), 0, s, gu, out,
                     (int)ffn);
  return hipGetLastError();
}

// Workspace: the records [nkv][S][grp][hd + 4] floats, then nkv counters.
static int64_t attention_record_bytes(int nh, int nkv, int hd, int64_t max_seq) {
  const int64_t S = (max_seq + kSplit - 1) / kSplit;
  return (int64_t)sizeof(float) * nkv * S * (nh / nkv) * attn_record_stride(hd);
}

int64_t attention_work_bytes(int nh, int nkv, int hd, int64_t max_seq) {
  return attention_record_bytes(nh, nkv, hd, max_seq) + ((int64_t)nkv * 4 + 15) / 16 * 16;
}

hipError_t launch_attention_decode(const float *qkv, const int64_t *pos, const float *cs,
                                   const float *sn, float *kc, float *vc, float *out, float *work,
                                   int nh, int nkv, int hd, int64_t max_seq, hipStream_t s) {
  const int S = (int)((max_seq + kSplit - 1) / kSplit);
  unsigned *counters =
      (unsigned *)((char *)work + attention_record_bytes(nh, nkv, hd, max_seq));
  const dim3 grid((unsigned)nkv, (unsigned)S), block(kGlueThreads);
  if (hd == 64)
    hipLaunchKernelGGL(attention_kernel<64>, grid, block, 0, s, qkv, pos, cs, sn, kc, vc, out,
                       work, counters, nh, nkv, (int)max_seq);
  else if (hd == 128)
    hipLaunchKernelGGL(attention_kernel<128>, grid, block, 0, s, qkv, pos, cs, sn, kc, vc, out,
                       work, counters, nh, nkv, (int)max_seq);
  else
    hipLaunchKernelGGL(attention_kernel<256>, grid, block, 0, s, qkv, pos, cs, sn, kc, vc, out,
                       work, counters, nh, nkv, (int)max_seq);
  return hipGetLastError();
}

template <int HD>
static hipError_t launch_prefill_hd(const float *qkv, int64_t ldq, const int64_t *pos, int64_t m,
                                    const float *cs, const float *sn, float *kc, float *vc,
                                    float *out, int64_t ldo, int nh, int nkv, int max_seq,
                                    hipStream_t s) {
  hipLaunchKernelGGL(rope_append_kernel<HD>, dim3((unsigned)m), dim3(kGlueThreads), 0, s, qkv,
                     ldq, pos, cs, sn, kc, vc, nh, nkv, max_seq);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 grid((unsigned)((m + kPfRows - 1) / kPfRows), (unsigned)nkv);
  hipLaunchKernelGGL(attention_prefill_kernel<HD>, grid, dim3(kGlueThreads), 0, s, qkv, ldq, pos,
                     m, cs, sn, kc, vc, out, ldo, nh, nkv, max_seq);
  return hipGetLastError();
}

hipError_t launch_attention_prefill(const float *qkv, int64_t ldq, const int64_t *pos, int64_t m,
                                    const float *cs, const float *sn, float *kc, float *vc,
                                    float *out, int64_t ldo, int nh, int nkv, int hd,
                                    int64_t max_seq, hipStream_t s) {
  if (hd == 64)
    return launch_prefill_hd<64>(qkv, ldq, pos, m, cs, sn, kc, vc, out, ldo, nh, nkv,
                                 (int)max_seq, s);
  if (hd == 128)
    return launch_prefill_hd<128>(qkv, ldq, pos, m, cs, sn, kc, vc, out, ldo, nh, nkv,
                                  (int)max_seq, s);
  return launch_prefill_hd<256>(qkv, ldq, pos, m, cs, sn, kc, vc, out, ldo, nh, nkv,
                                (int)max_seq, s);
}

// ---------------------------------------------------------------------------
// Attention without a caller workspace (gguf_hip_attention_decode_noalloc).
// The records and counters live in `scratch`, a file-scope device array that
// every GPU the library runs on holds until the process ends.  Its address is
// taken once per device with hipGetSymbolAddress (the host-side name is only
// a stand-in, not a device address) and passed to the kernels.  Calls that
// overlap on one GPU race on it; each call clears the counters it uses with a
// fill kernel first (no memset, so the call can be captured in a graph).
// ---------------------------------------------------------------------------
namespace {

__device__ __align__(256) unsigned char scratch[kNoAllocAttentionBytes];

std::mutex g_scratch_mu;
constexpr int kMaxDevices = 64;
void *g_scratch[kMaxDevices];  // per device: the device address of `scratch`

__global__ __launch_bounds__(kGlueThreads) void clear_u32_kernel(unsigned *__restrict__ p, int n) {
  for (int i = threadIdx.x; i < n; i += kGlueThreads) p[i] = 0u;
}

hipError_t scratch_ptr(void **out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return hipSuccess;
}

}  // namespace

hipError_t launch_attention_decode_noalloc(const float *qkv, const int64_t *pos, const float *cs,
                                           const float *sn, float *kc, float *vc, float *out,
                                           int nh, int nkv, int hd, int64_t max_seq,
                                           hipStream_t s) {
  void *ws = nullptr;
  hipError_t e = scratch_ptr(&ws);
  if (e != hipSuccess) return e;
  unsigned *counters = (unsigned *)((char *)ws + attention_record_bytes(nh, nkv, hd, max_seq));
  hipLaunchKernelGGL(clear_u32_kernel, dim3(1), dim3(kGlueThreads), 0, s, counters, nkv);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_attention_decode(qkv, pos, cs, sn, kc, vc, out, (float *)ws, nh, nkv, hd, max_seq,
                                 s);
}

int64_t argmax_work_bytes() { return (int64_t)kArgBlocks * (sizeof(float) + sizeof(int64_t)); }

hipError_t launch_argmax(const float *x, int64_t n, int64_t *out, void *work, hipStream_t s) {
  int64_t *pi = (int64_t *)work;
  float *pv = (float *)(pi + kArgBlocks);
  hipLaunchKernelGGL(argmax_partial_kernel, dim3(kArgBlocks), dim3(kGlueThreads), 0, s, x, n, pv,
                     pi);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(argmax_merge_kernel, dim3(1), dim3(kGlueThreads), 0, s, pv, pi, out);
  return hipGetLastError();
}

}  // namespace gguf
