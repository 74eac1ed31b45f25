// C ABI of libgguf_hip (declared in include/gguf_hip.h).
//
// Every entry point validates its arguments before touching HIP, so the
// error paths (unsupported type, block-size mismatch, byte-length mismatch,
// null or misaligned pointers) behave identically with or without a GPU.
// Error texts follow the reference's throws: gguf.ts:75-79,85-87,
// gguf-dequant.ts:678-680,837, forward-pass.ts:1486-1489,1524.
#include <stdarg.h>
#include <stdio.h>

#include "common.hpp"
#include "gguf_hip.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return GGUF_HIP_OK;
}

// gguf.ts:39-73
bool traits(int t, int *block, int *size) {
  static const int tbl[][3] = {
      {0, 1, 4},     {1, 1, 2},     {30, 1, 2},    {24, 1, 1},    {25, 1, 2},    {26, 1, 4},
      {27, 1, 8},    {28, 1, 8},    {2, 32, 18},   {3, 32, 20},   {6, 32, 22},   {7, 32, 24},
      {8, 32, 34},   {9, 32, 36},   {10, 256, 84}, {11, 256, 110}, {12, 256, 144}, {13, 256, 176},
      {14, 256, 210}, {15, 256, 292}, {16, 256, 66}, {17, 256, 74}, {18, 256, 98},  {19, 256, 50},
      {20, 32, 18},  {21, 256, 110}, {22, 256, 82}, {23, 256, 136}, {29, 256, 56}};
  for (const auto &e : tbl)
    if (e[0] == t) {
      *block = e[1];
      *size = e[2];
      return true;
    }
  return false;
}

// The grid-codebook IQ types.  Their decode variant needs a workspace only
// beyond K = kIqOneShotMaxK (the one-shot kernel's staging limit).
constexpr int64_t kIqOneShotMaxK = 16384;
bool grid_type(int t) {
  return t == GGUF_HIP_IQ2_XXS || t == GGUF_HIP_IQ2_XS || t == GGUF_HIP_IQ2_S ||
         t == GGUF_HIP_IQ3_XXS || t == GGUF_HIP_IQ3_S || t == GGUF_HIP_IQ1_M;
}

bool kernel_type(int t) {
  return t == GGUF_HIP_Q8_0 || t == GGUF_HIP_Q4_K || t == GGUF_HIP_Q5_K || t == GGUF_HIP_Q6_K ||
         t == GGUF_HIP_Q4_0 || t == GGUF_HIP_Q5_0 || t == GGUF_HIP_IQ4_NL || t == GGUF_HIP_IQ4_XS ||
         t == GGUF_HIP_Q2_K || t == GGUF_HIP_Q3_K || grid_type(t);
}

int check_type(int t) {
  int b, s;
  if (!traits(t, &b, &s)) return fail(GGUF_HIP_ERR_TYPE, "[GGUF] Unsupported ggml type %d", t);
  if (!kernel_type(t))
    return fail(GGUF_HIP_ERR_TYPE, "[gguf-hip] no kernel for ggml type %d", t);
  return GGUF_HIP_OK;
}

int check_k(int t, int64_t k) {
  int b, s;
  traits(t, &b, &s);
  if (k <= 0 || k % b != 0)
    return fail(GGUF_HIP_ERR_SHAPE, "[GGUF] ne[0]=%lld not divisible by block size %d for type %d",
                (long long)k, b, t);
  // kernels address 8 row tiles of one K range with 32-bit byte offsets
  if (k > (int64_t)1 << 24)
    return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] K=%lld too large (max 2^24)", (long long)k);
  return GGUF_HIP_OK;
}

// Bytes of one row's GGUF blocks; the row-tile layout stores rows in groups
// of 16 (common.hpp), so a weight of n rows takes round_up(n, 16) rows.
int64_t row_bytes(int t, int64_t k) {
  int b, s;
  traits(t, &b, &s);
  return (k / b) * s;
}

int64_t tiled_bytes(int t, int64_t n_rows, int64_t k) {
  return ((n_rows + 15) / 16) * 16 * row_bytes(t, k);
}

bool aligned(const void *p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

int hip_status(hipError_t e, const char *what) {
  if (e != hipSuccess)
    return fail(GGUF_HIP_ERR_HIP, "[gguf-hip] %s: %s", what, hipGetErrorString(e));
  return ok();
}

}  // namespace

extern "C" {

int gguf_hip_abi_version(void) { return GGUF_HIP_ABI_VERSION; }

const char *gguf_hip_last_error(void) { return g_err; }

int gguf_hip_type_traits(int ggml_type, int *block_elems, int *type_size) {
  int b, s;
  if (!traits(ggml_type, &b, &s))
    return fail(GGUF_HIP_ERR_TYPE, "[GGUF] Unsupported ggml type %d", ggml_type);
  if (block_elems) *block_elems = b;
  if (type_size) *type_size = s;
  return ok();
}

int64_t gguf_hip_raw_bytes(int ggml_type, int64_t n_rows, int64_t k) {
  int b, s;
  if (!traits(ggml_type, &b, &s))
    return fail(GGUF_HIP_ERR_TYPE, "[GGUF] Unsupported ggml type %d", ggml_type);
  if (k <= 0 || k % b != 0)
    return fail(GGUF_HIP_ERR_SHAPE, "[GGUF] ne[0]=%lld not divisible by block size %d for type %d",
                (long long)k, b, ggml_type);
  if (n_rows < 0) return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] negative row count");
  ok();
  return n_rows * (k / b) * s;
}

int64_t gguf_hip_tile_bytes(int ggml_type, int64_t n_rows, int64_t k) {
  int rc = check_type(ggml_type);
  if (rc) return rc;
  if ((rc = check_k(ggml_type, k))) return rc;
  if (n_rows < 0) return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] negative row count");
  ok();
  return tiled_bytes(ggml_type, n_rows, k);
}

int gguf_hip_repack(const void *raw, int64_t raw_bytes, int ggml_type, int64_t n_rows, int64_t k,
                    void *tiles, int64_t tile_bytes, void *stream) {
  int rc = check_type(ggml_type);
  if (rc) return rc;
  if ((rc = check_k(ggml_type, k))) return rc;
  if (n_rows < 0) return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] negative row count");
  int b, s;
  traits(ggml_type, &b, &s);
  const int64_t want_raw = n_rows * (k / b) * s;
  if (raw_bytes != want_raw)
    return fail(GGUF_HIP_ERR_BYTES, "[repackGGUF] byteLength %lld != expected %lld",
                (long long)raw_bytes, (long long)want_raw);
  const int64_t want_tiles = tiled_bytes(ggml_type, n_rows, k);
  if (tile_bytes != want_tiles)
    return fail(GGUF_HIP_ERR_BYTES, "[repackGGUF] output byteLength %lld != expected %lld",
                (long long)tile_bytes, (long long)want_tiles);
  if (n_rows == 0) return ok();
  if (!raw || !tiles) return fail(GGUF_HIP_ERR_NULL, "[gguf-hip] null pointer");
  if (!aligned(tiles, 16))
    return fail(GGUF_HIP_ERR_ALIGN, "[gguf-hip] tile buffer must be 16-byte aligned");
  return hip_status(gguf::launch_repack((const uint8_t *)raw, ggml_type, n_rows, k,
                                        (uint8_t *)tiles, (hipStream_t)stream),
                    "repack launch");
}

int gguf_hip_dequant(const void *tiles, int ggml_type, int64_t n_rows, int64_t k, float *out,
                     int64_t ldo, void *stream) {
  int rc = check_type(ggml_type);
  if (rc) return rc;
  if ((rc = check_k(ggml_type, k))) return rc;
  if (n_rows < 0) return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] negative row count");
  if (n_rows > 1 && ldo < k) return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] ldo < K");
  if (n_rows == 0) return ok();
  if (!tiles || !out) return fail(GGUF_HIP_ERR_NULL, "[gguf-hip] null pointer");
  if (!aligned(tiles, 16))
    return fail(GGUF_HIP_ERR_ALIGN, "[gguf-hip] tile buffer must be 16-byte aligned");
  if (!aligned(out, 4)) return fail(GGUF_HIP_ERR_ALIGN, "[gguf-hip] output must be 4-byte aligned");
  return hip_status(gguf::launch_dequant((const uint8_t *)tiles, ggml_type, n_rows, k, out, ldo,
                                         (hipStream_t)stream),
                    "dequant launch");
}

int gguf_hip_dequant_raw(const void *raw, int ggml_type, int64_t n_elems, float *out,
                         void *stream) {
  int rc = check_type(ggml_type);
  if (rc) return rc;
  int b, s;
  traits(ggml_type, &b, &s);
  if (n_elems < 0 || n_elems % b != 0)
    return fail(GGUF_HIP_ERR_SHAPE, "[GGUF] n=%lld not divisible by %d", (long long)n_elems, b);
  if (n_elems == 0) return ok();
  if (!raw || !out) return fail(GGUF_HIP_ERR_NULL, "[gguf-hip] null pointer");
  if (!aligned(out, 4)) return fail(GGUF_HIP_ERR_ALIGN, "[gguf-hip] output must be 4-byte aligned");
  return hip_status(
      gguf::launch_dequant_raw((const uint8_t *)raw, ggml_type, n_elems, out, (hipStream_t)stream),
      "dequant_raw launch");
}

int gguf_hip_get_rows(const void *raw, int ggml_type, int64_t n_rows, int64_t k,
                      const int64_t *ids, int64_t n_ids, float *out, int64_t ldo, void *stream) {
  int rc = check_type(ggml_type);
  if (rc) return rc;
  if ((rc = check_k(ggml_type, k))) return rc;
  if (n_rows < 0 || n_ids < 0) return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] negative row count");
  if (n_ids > 1 && ldo < k) return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] ldo < K");
  if (n_ids == 0) return ok();
  if (!raw || !ids || !out) return fail(GGUF_HIP_ERR_NULL, "[gguf-hip] null pointer");
  if (!aligned(ids, 8)) return fail(GGUF_HIP_ERR_ALIGN, "[gguf-hip] ids must be 8-byte aligned");
  if (!aligned(out, 4)) return fail(GGUF_HIP_ERR_ALIGN, "[gguf-hip] output must be 4-byte aligned");
  return hip_status(gguf::launch_get_rows((const uint8_t *)raw, ggml_type, n_rows, k, ids, n_ids,
                                          out, ldo, (hipStream_t)stream),
                    "get_rows launch");
}

int gguf_hip_matmul_ws(const void *x, int x_type, int64_t ldx, const void *tiles, int ggml_type,
                       int64_t n, int64_t k, float *y, int64_t ldy, int64_t m, int variant,
                       void *work, int64_t work_bytes, void *stream) {
  int rc = check_type(ggml_type);
  if (rc) return rc;
  if ((rc = check_k(ggml_type, k))) return rc;
  if (x_type != GGUF_HIP_F32 && x_type != GGUF_HIP_F16)
    return fail(GGUF_HIP_ERR_DTYPE, "[gguf-hip] activations must be f32 (0) or f16 (1), got %d",
                x_type);
  if (variant < GGUF_HIP_VARIANT_AUTO || variant > GGUF_HIP_VARIANT_GEMM)
    return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] unknown kernel variant %d", variant);
  if (m < 0 || n < 0) return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] negative M or N");
  if (n > ((int64_t)1 << 30) || m > ((int64_t)1 << 30))
    return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] M or N too large");
  if (m > 1 && ldx < k) return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] ldx < K");
  if (m > 1 && ldy < n) return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] ldy < N");
  if (m == 0 || n == 0) return ok();
  if (!x || !tiles || !y) return fail(GGUF_HIP_ERR_NULL, "[gguf-hip] null pointer");
  const int64_t esize = x_type == GGUF_HIP_F32 ? 4 : 2;
  if (!aligned(tiles, 16))
    return fail(GGUF_HIP_ERR_ALIGN, "[gguf-hip] weight buffer must be 16-byte aligned");
  if (!aligned(x, 16) || (m > 1 && (ldx * esize) % 16 != 0))
    return fail(GGUF_HIP_ERR_ALIGN, "[gguf-hip] activation rows must be 16-byte aligned");
  if (!aligned(y, 4)) return fail(GGUF_HIP_ERR_ALIGN, "[gguf-hip] output must be 4-byte aligned");
  if (work_bytes < 0) return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] negative workspace size");
  if (work && !aligned(work, 16))
    return fail(GGUF_HIP_ERR_ALIGN, "[gguf-hip] workspace must be 16-byte aligned");

  const hipStream_t s = (hipStream_t)stream;
  // f16 activations: the decode path up to 32 rows, the fp16 GEMM above; f32
  // activations keep the f32-grade decode path below GGUF_HIP_F32_GEMM_MIN_M
  // rows (the reference computes in f32) and take the row-scaled fp16 GEMM
  // from there on (prefill)
  if (variant == GGUF_HIP_VARIANT_AUTO)
    variant = m <= (x_type == GGUF_HIP_F32 ? GGUF_HIP_F32_GEMM_MIN_M - 1 : GGUF_HIP_DECODE_MAX_M)
                  ? GGUF_HIP_VARIANT_DECODE
                  : GGUF_HIP_VARIANT_GEMM;
  // grid types: up to K = 16384 the decode variant runs without a workspace
  // (the one-shot kernel, once per row when the workspace is missing); beyond
  // it only the batched kernel serves them, and that needs one
  if (grid_type(ggml_type) && variant == GGUF_HIP_VARIANT_DECODE && k > kIqOneShotMaxK) {
    const int64_t need = 4 * gguf::launch_decode_work(ggml_type, x_type, n, k, m);
    if (need > 0 && (!work || work_bytes < need))
      return fail(GGUF_HIP_ERR_SHAPE,
                  "[gguf-hip] ggml type %d needs a workspace of %lld bytes (gguf_hip_matmul_workspace), "
                  "got %lld", ggml_type, (long long)need, (long long)(work ? work_bytes : 0));
  }
  // the GEMM addresses one 128-row activation block with 32-bit byte offsets
  if (variant == GGUF_HIP_VARIANT_GEMM && (127 * ldx + k) * esize >= ((int64_t)1 << 31))
    return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] ldx too large for the GEMM kernel");
  const hipError_t e =
      variant == GGUF_HIP_VARIANT_DECODE
          ? gguf::launch_decode(x, x_type, ldx, (const uint8_t *)tiles, ggml_type, n, k, y, ldy, m,
                                (float *)work, work ? work_bytes / 4 : 0, s)
          : gguf::launch_gemm(x, x_type, ldx, (const uint8_t *)tiles, ggml_type, n, k, y, ldy, m,
                              work && work_bytes > gguf::kWsPrefix
                                  ? (float *)((char *)work + gguf::kWsPrefix) : nullptr,
                              work && work_bytes > gguf::kWsPrefix
                                  ? (work_bytes - gguf::kWsPrefix) / 4 : 0, s);
  return hip_status(e, "matmul launch");
}

int gguf_hip_matmul_variant(const void *x, int x_type, int64_t ldx, const void *tiles,
                            int ggml_type, int64_t n, int64_t k, float *y, int64_t ldy, int64_t m,
                            int variant, void *stream) {
  return gguf_hip_matmul_ws(x, x_type, ldx, tiles, ggml_type, n, k, y, ldy, m, variant, nullptr, 0,
                            stream);
}

int64_t gguf_hip_matmul_workspace(int ggml_type, int x_type, int64_t n, int64_t k, int64_t m) {
  int rc = check_type(ggml_type);
  if (rc) return rc;
  if ((rc = check_k(ggml_type, k))) return rc;
  if (x_type != GGUF_HIP_F32 && x_type != GGUF_HIP_F16)
    return fail(GGUF_HIP_ERR_DTYPE, "[gguf-hip] activations must be f32 (0) or f16 (1), got %d",
                x_type);
  if (m < 0 || n < 0 || n > ((int64_t)1 << 30) || m > ((int64_t)1 << 30))
    return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] bad M or N");
  ok();
  if (n == 0 || m == 0) return 0;
  // the larger of the decode path's and the GEMM's (AUTO may take either)
  // (M = 1: the one-shot kernel needs none; grid types above K = 16384 still do)
  const int64_t dec = (m < 2 && (!grid_type(ggml_type) || k <= kIqOneShotMaxK))
                          ? 0 : gguf::launch_decode_work(ggml_type, x_type, n, k, m);
  int64_t gem = m > 32 ? gguf::launch_gemm_work(ggml_type, x_type, n, k, m) : 0;
  if (gem > 0) gem += gguf::kWsPrefix / 4;  // the GEMM's partial sums follow the counter prefix
  return 4 * (dec > gem ? dec : gem);
}

int gguf_hip_rmsnorm(const float *x, const float *w, float eps, float *y, int64_t rows,
                     int64_t n, void *stream) {
  return gguf_hip_add_rmsnorm(const_cast<float *>(x), nullptr, w, eps, y, rows, n, stream);
}

int gguf_hip_add_rmsnorm(float *x, const float *res, const float *w, float eps, float *y,
                         int64_t rows, int64_t n, void *stream) {
  if (rows < 0 || n <= 0 || n % 4 || n > ((int64_t)1 << 30) || rows > 65535 * 1024)
    return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] rmsnorm: bad shape rows=%lld n=%lld",
                (long long)rows, (long long)n);
  if (!(eps >= 0.0f)) return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] rmsnorm: eps must be >= 0");
  if (rows == 0) return ok();
  if (!x || !w || !y) return fail(GGUF_HIP_ERR_NULL, "[gguf-hip] null pointer");
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(y, 16) || (res && !aligned(res, 16)))
    return fail(GGUF_HIP_ERR_ALIGN, "[gguf-hip] rmsnorm buffers must be 16-byte aligned");
  if (res && y == x) return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] add_rmsnorm: y aliases x");
  return hip_status(gguf::launch_rmsnorm(x, res, w, eps, y, rows, n, (hipStream_t)stream),
                    "rmsnorm launch");
}

int gguf_hip_swiglu(const float *gate_up, float *out, int64_t rows, int64_t ffn, void *stream) {
  if (rows < 0 || ffn <= 0 || ffn % 4 || ffn > ((int64_t)1 << 30) || rows > 65535)
    return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] swiglu: bad shape rows=%lld ffn=%lld",
                (long long)rows, (long long)ffn);
  if (rows == 0) return ok();
  if (!gate_up || !out) return fail(GGUF_HIP_ERR_NULL, "[gguf-hip] null pointer");
  if (!aligned(gate_up, 16) || !aligned(out, 16))
    return fail(GGUF_HIP_ERR_ALIGN, "[gguf-hip] swiglu buffers must be 16-byte aligned");
  return hip_status(gguf::launch_swiglu(gate_up, out, rows, ffn, (hipStream_t)stream),
                    "swiglu launch");
}

int check_attention(int n_heads, int n_kv_heads, int head_dim, int64_t max_seq) {
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads || n_heads / n_kv_heads > 8)
    return fail(GGUF_HIP_ERR_SHAPE,
                "[gguf-hip] attention: n_heads %d must be 1..8 times n_kv_heads %d", n_heads,
                n_kv_heads);
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] attention: head_dim %d not 64, 128 or 256",
                head_dim);
  if (max_seq <= 0 || max_seq > (1 << 20))
    return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] attention: max_seq %lld out of range",
                (long long)max_seq);
  if ((int64_t)n_kv_heads * max_seq * head_dim > ((int64_t)1 << 31))
    return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] attention: cache of one layer too large");
  return GGUF_HIP_OK;
}

int64_t gguf_hip_attention_workspace(int n_heads, int n_kv_heads, int head_dim, int64_t max_seq) {
  const int rc = check_attention(n_heads, n_kv_heads, head_dim, max_seq);
  if (rc) return rc;
  ok();
  return gguf::attention_work_bytes(n_heads, n_kv_heads, head_dim, max_seq);
}

int gguf_hip_attention_decode(const float *qkv, const int64_t *pos, const float *cos_table,
                              const float *sin_table, float *k_cache, float *v_cache, float *out,
                              int n_heads, int n_kv_heads, int head_dim, int64_t max_seq,
                              void *work, void *stream) {
  int rc = check_attention(n_heads, n_kv_heads, head_dim, max_seq);
  if (rc) return rc;
  if (!qkv || !pos || !cos_table || !sin_table || !k_cache || !v_cache || !work)
    return fail(GGUF_HIP_ERR_NULL, "[gguf-hip] null pointer");
  if (!aligned(qkv, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(out, 4) ||
      !aligned(pos, 8) || !aligned(cos_table, 4) || !aligned(sin_table, 4) || !aligned(work, 16))
    return fail(GGUF_HIP_ERR_ALIGN, "[gguf-hip] attention buffers misaligned");
  return hip_status(gguf::launch_attention_decode(qkv, pos, cos_table, sin_table, k_cache,
                                                  v_cache, out, (float *)work, n_heads,
                                                  n_kv_heads, head_dim, max_seq,
                                                  (hipStream_t)stream),
                    "attention launch");
}

int gguf_hip_attention_decode_noalloc(const float *qkv, const int64_t *pos,
                                      const float *cos_table, const float *sin_table,
                                      float *k_cache, float *v_cache, float *out, int n_heads,
                                      int n_kv_heads, int head_dim, int64_t max_seq,
                                      void *stream) {
  int rc = check_attention(n_heads, n_kv_heads, head_dim, max_seq);
  if (rc) return rc;
  const int64_t need = gguf::attention_work_bytes(n_heads, n_kv_heads, head_dim, max_seq);
  if (need > gguf::kNoAllocAttentionBytes)
    return fail(GGUF_HIP_ERR_SHAPE,
                "[gguf-hip] attention_decode_noalloc: the shape needs %lld bytes of workspace, "
                "more than the library's %lld (use gguf_hip_attention_decode with a workspace)",
                (long long)need, (long long)gguf::kNoAllocAttentionBytes);
  if (!qkv || !pos || !cos_table || !sin_table || !k_cache || !v_cache || !out)
    return fail(GGUF_HIP_ERR_NULL, "[gguf-hip] null pointer");
  if (!aligned(qkv, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(out, 4) ||
      !aligned(pos, 8) || !aligned(cos_table, 4) || !aligned(sin_table, 4))
    return fail(GGUF_HIP_ERR_ALIGN, "[gguf-hip] attention buffers misaligned");
  return hip_status(gguf::launch_attention_decode_noalloc(qkv, pos, cos_table, sin_table, k_cache,
                                                          v_cache, out, n_heads, n_kv_heads,
                                                          head_dim, max_seq, (hipStream_t)stream),
                    "attention launch");
}

int gguf_hip_attention_prefill(const float *qkv, int64_t ldqkv, const int64_t *pos, int64_t m,
                               const float *cos_table, const float *sin_table, float *k_cache,
                               float *v_cache, float *out, int64_t ldo, int n_heads,
                               int n_kv_heads, int head_dim, int64_t max_seq, void *stream) {
  int rc = check_attention(n_heads, n_kv_heads, head_dim, max_seq);
  if (rc) return rc;
  if (m < 0 || m > ((int64_t)1 << 30))
    return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] attention_prefill: M %lld out of range",
                (long long)m);
  const int64_t row = (int64_t)(n_heads + 2 * n_kv_heads) * head_dim;
  if (ldqkv < row || ldqkv % 4 || ldo < (int64_t)n_heads * head_dim || ldo % 4)
    return fail(GGUF_HIP_ERR_SHAPE,
                "[gguf-hip] attention_prefill: ldqkv %lld (row %lld) / ldo %lld (row %lld) must "
                "hold a row and be multiples of 4",
                (long long)ldqkv, (long long)row, (long long)ldo,
                (long long)n_heads * head_dim);
  if (m == 0) return ok();
  if (!qkv || !pos || !cos_table || !sin_table || !k_cache || !v_cache || !out)
    return fail(GGUF_HIP_ERR_NULL, "[gguf-hip] null pointer");
  if (!aligned(qkv, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(out, 16) ||
      !aligned(pos, 8) || !aligned(cos_table, 16) || !aligned(sin_table, 16))
    return fail(GGUF_HIP_ERR_ALIGN, "[gguf-hip] attention_prefill buffers misaligned");
  return hip_status(gguf::launch_attention_prefill(qkv, ldqkv, pos, m, cos_table, sin_table,
                                                   k_cache, v_cache, out, ldo, n_heads,
                                                   n_kv_heads, head_dim, max_seq,
                                                   (hipStream_t)stream),
                    "attention_prefill launch");
}

int64_t gguf_hip_argmax_workspace(void) { return gguf::argmax_work_bytes(); }

int gguf_hip_argmax(const float *x, int64_t n, int64_t *out, void *work, void *stream) {
  if (n <= 0) return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] argmax: n must be positive");
  if (!x || !out || !work) return fail(GGUF_HIP_ERR_NULL, "[gguf-hip] null pointer");
  if (!aligned(x, 4) || !aligned(out, 8) || !aligned(work, 8))
    return fail(GGUF_HIP_ERR_ALIGN, "[gguf-hip] argmax buffers misaligned");
  return hip_status(gguf::launch_argmax(x, n, out, work, (hipStream_t)stream), "argmax launch");
}

int gguf_hip_matmul_fused(const float *x, const void *tiles, int ggml_type, int64_t n, int64_t k,
                          float *y, int prologue, const float *norm_w, float eps, int epilogue,
                          void *stream) {
  int rc = check_type(ggml_type);
  if (rc) return rc;
  if ((rc = check_k(ggml_type, k))) return rc;
  if (prologue < GGUF_HIP_PROLOGUE_NONE || prologue > GGUF_HIP_PROLOGUE_SWIGLU)
    return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] unknown prologue %d", prologue);
  if (epilogue < GGUF_HIP_EPILOGUE_STORE || epilogue > GGUF_HIP_EPILOGUE_SWIGLU)
    return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] unknown epilogue %d", epilogue);
  if (epilogue == GGUF_HIP_EPILOGUE_SWIGLU && n % 32)
    return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] SwiGLU epilogue: N %% 32 != 0");
  if (n < 0 || n > ((int64_t)1 << 30)) return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] bad N");
  if (k > 16384)
    return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] fused matmul: K=%lld above 16384", (long long)k);
  if (k % 16) return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] fused matmul: K %% 16 != 0");
  if (prologue == GGUF_HIP_PROLOGUE_RMSNORM && !(eps >= 0.0f))
    return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] rmsnorm: eps must be >= 0");
  if (n == 0) return ok();
  if (!x || !tiles || !y || (prologue == GGUF_HIP_PROLOGUE_RMSNORM && !norm_w))
    return fail(GGUF_HIP_ERR_NULL, "[gguf-hip] null pointer");
  if (!aligned(x, 16) || !aligned(tiles, 16) || !aligned(y, 4) ||
      (norm_w && prologue == GGUF_HIP_PROLOGUE_RMSNORM && !aligned(norm_w, 16)))
    return fail(GGUF_HIP_ERR_ALIGN, "[gguf-hip] fused matmul buffers misaligned");
  const hipError_t e = gguf::launch_decode_fused(x, (const uint8_t *)tiles, ggml_type, n, k, y,
                                                 prologue, norm_w, eps, epilogue,
                                                 (hipStream_t)stream);
  if (e == hipErrorNotSupported)
    return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] no fused kernel for N=%lld K=%lld type %d",
                (long long)n, (long long)k, ggml_type);
  return hip_status(e, "fused matmul launch");
}

int gguf_hip_matmul_attn_merge(const void *work, const int64_t *pos, int n_heads, int n_kv_heads,
                               int head_dim, int64_t max_seq, const void *tiles, int ggml_type,
                               int64_t n, float *y, int epilogue, void *stream) {
  int rc = check_attention(n_heads, n_kv_heads, head_dim, max_seq);
  if (rc) return rc;
  if ((rc = check_type(ggml_type))) return rc;
  const int64_t k = (int64_t)n_heads * head_dim;
  if ((rc = check_k(ggml_type, k))) return rc;
  if (epilogue != GGUF_HIP_EPILOGUE_STORE && epilogue != GGUF_HIP_EPILOGUE_ACCUMULATE)
    return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] attention merge: epilogue %d not store / accumulate",
                epilogue);
  if (n < 0 || n > ((int64_t)1 << 30)) return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] bad N");
  if (n == 0) return ok();
  if (!work || !pos || !tiles || !y) return fail(GGUF_HIP_ERR_NULL, "[gguf-hip] null pointer");
  if (!aligned(work, 16) || !aligned(pos, 8) || !aligned(tiles, 16) || !aligned(y, 4))
    return fail(GGUF_HIP_ERR_ALIGN, "[gguf-hip] attention merge buffers misaligned");
  const gguf::AttnRecords ar{(const float *)work, pos, n_heads, n_kv_heads, head_dim, (int)max_seq};
  const hipError_t e = gguf::launch_decode_attn_merge(ar, (const uint8_t *)tiles, ggml_type, n, y,
                                                      epilogue, (hipStream_t)stream);
  if (e == hipErrorNotSupported)
    return fail(GGUF_HIP_ERR_SHAPE, "[gguf-hip] no merge kernel for N=%lld K=%lld type %d",
                (long long)n, (long long)k, ggml_type);
  return hip_status(e, "attention merge launch");
}

int gguf_hip_matmul(const void *x, int x_type, int64_t ldx, const void *tiles, int ggml_type,
                    int64_t n, int64_t k, float *y, int64_t ldy, int64_t m, void *stream) {
  return gguf_hip_matmul_variant(x, x_type, ldx, tiles, ggml_type, n, k, y, ldy, m,
                                 GGUF_HIP_VARIANT_AUTO, stream);
}

}  // extern "C"
