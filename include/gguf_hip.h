/*
 * gguf_hip.h — C ABI of the MI355X (gfx950) GGUF dequant-matmul library.
 *
 * Drop-in for the quantized-projection path of the reference WebGPU engine:
 *   dispatchMatmulGGUF(aBuf, gg, cBuf, M, N, K, label, io)
 *       webgpu/src/engine/forward-pass.ts:1496-1544
 *   repackGGUFForGPU(ggmlType, data, n)        webgpu/src/model/gguf-dequant.ts:809-840
 *   dequantGGML(ggmlType, data, n)             webgpu/src/model/gguf-dequant.ts:844-868
 *   ggmlTypeTraits / ggmlTensorBytes           webgpu/src/model/gguf.ts:75-92
 *
 * Conventions
 *  - Plain pointers and sizes only.  Device pointers are HIP device memory;
 *    `stream` is a hipStream_t (NULL = the legacy default stream).
 *  - Every call validates its arguments before any HIP call and returns 0 on
 *    success or a negative GGUF_HIP_ERR_* code; gguf_hip_last_error() then
 *    describes the failure (thread-local string, valid until the next call on
 *    that thread).  Validation failures therefore work without a GPU.
 *  - Work is enqueued on `stream` and the calls return without a host sync,
 *    like the reference's BatchedDispatcher (webgpu/src/engine/compute.ts:146-266).
 *  - No call allocates device memory: weights, activations and outputs are
 *    owned by the caller, as in the reference (forward-pass.ts:1140-1163).
 *  - Weights live in the "row-tile layout": rows are grouped in tiles of 16
 *    (the last tile zero-padded); for each 256-element superblock (Q2_K,
 *    Q3_K, Q4_K, Q5_K, Q6_K, IQ4_XS) or 32-element block (Q8_0, Q4_0, Q5_0, IQ4_NL) of
 *    K, a tile stores the 16 rows' GGUF blocks interleaved at 16-byte
 *    granularity (8 bytes for Q8_0 quants; the 4-bit codes of Q4_0 / Q5_0 /
 *    IQ4_NL and of each IQ4_XS sub-block regrouped into one 4-byte word per
 *    lane), so that one wave-wide load of a matrix-core operand reads
 *    contiguous HBM.  The grid-codebook types (IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS,
 *    IQ3_S, IQ1_M; 256-element superblocks) store per tile and superblock the
 *    16 f16 d fields first (32 bytes), then each row's remaining block bytes
 *    as they are (IQ1_M, which has no d field: the 16 blocks as they are).  The
 *    byte count is exactly round_up(N, 16) rows of GGUF blocks
 *    (gguf_hip_tile_bytes); the interleave is defined in csrc/common.hpp of
 *    the library.  gguf_hip_repack converts raw GGUF bytes.  Row ranges that
 *    start on a multiple of 16 are weights of their own (byte offset
 *    start * row_bytes), which is how gate+up fusion concatenates weights.
 */
#ifndef GGUF_HIP_H
#define GGUF_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The library is built with hidden visibility; only the entry points below
 * are exported (kernels and helpers cannot be interposed across libraries). */
#pragma GCC visibility push(default)

#define GGUF_HIP_ABI_VERSION 18

/* ggml type ids (gguf.ts:24-35); activation dtypes reuse F32 / F16. */
#define GGUF_HIP_F32 0
#define GGUF_HIP_F16 1
#define GGUF_HIP_Q4_0 2
#define GGUF_HIP_Q5_0 6
#define GGUF_HIP_Q8_0 8
#define GGUF_HIP_Q2_K 10
#define GGUF_HIP_Q3_K 11
#define GGUF_HIP_Q4_K 12
#define GGUF_HIP_Q5_K 13
#define GGUF_HIP_Q6_K 14
#define GGUF_HIP_IQ4_NL 20
#define GGUF_HIP_IQ4_XS 23
/* grid-codebook types: the decode variant needs a workspace only for K > 16384 */
#define GGUF_HIP_IQ2_XXS 16
#define GGUF_HIP_IQ2_XS 17
#define GGUF_HIP_IQ3_XXS 18
#define GGUF_HIP_IQ3_S 21
#define GGUF_HIP_IQ2_S 22
#define GGUF_HIP_IQ1_M 29

/* Error codes.  The Python host maps them onto the reference's throws:
 * TYPE -> NotImplementedError ("no pipeline for ggml type", forward-pass.ts:1524;
 *         "Unsupported ggml type", gguf.ts:75-79)
 * SHAPE / NULL / ALIGN / DTYPE / BYTES -> ValueError
 *         ("ne[0] not divisible by block size", gguf.ts:85-87;
 *          "byteLength != expected", gguf-dequant.ts:678-680;
 *          offsets must be aligned, forward-pass.ts:1486-1489)
 * HIP -> RuntimeError. */
#define GGUF_HIP_OK 0
#define GGUF_HIP_ERR_TYPE (-1)
#define GGUF_HIP_ERR_SHAPE (-2)
#define GGUF_HIP_ERR_NULL (-3)
#define GGUF_HIP_ERR_ALIGN (-4)
#define GGUF_HIP_ERR_DTYPE (-5)
#define GGUF_HIP_ERR_BYTES (-6)
#define GGUF_HIP_ERR_HIP (-7)

/* Kernel family for gguf_hip_matmul_variant. */
#define GGUF_HIP_VARIANT_AUTO 0   /* DECODE for f16 x with M <= GGUF_HIP_DECODE_MAX_M and
                                     for f32 x with M < GGUF_HIP_F32_GEMM_MIN_M, GEMM above */
#define GGUF_HIP_VARIANT_DECODE 1 /* matrix-core decode: exact quant codes x f16 hi + lo
                                     parts of the activations scaled by a power of two
                                     per 256- or 32-element unit, f32 scales; one pass
                                     over the weights per 32 activation rows (any M) */
#define GGUF_HIP_VARIANT_GEMM 2   /* MFMA GEMM with dequantized fp16 weight tiles and fp16
                                     activations staged in LDS (prefill); f32 activation
                                     rows are scaled by a power of two each first */
#define GGUF_HIP_DECODE_MAX_M 32
#define GGUF_HIP_F32_GEMM_MIN_M 512

/* ABI version of the loaded library (GGUF_HIP_ABI_VERSION). */
int gguf_hip_abi_version(void);

/* Description of the last error on the calling thread ("" if none). */
const char *gguf_hip_last_error(void);

/* Elements and bytes per block of a ggml type; gguf.ts:75-79 (ggmlTypeTraits). */
int gguf_hip_type_traits(int ggml_type, int *block_elems, int *type_size);

/* Raw GGUF bytes of an [n_rows, k] tensor (gguf.ts:82-92, ggmlTensorBytes);
 * negative error code on failure. */
int64_t gguf_hip_raw_bytes(int ggml_type, int64_t n_rows, int64_t k);

/* Bytes of an [n_rows, k] weight in the row-tile layout, round_up(n_rows, 16)
 * rows of GGUF blocks; replaces the GGUF_GPU_LAYOUT stride table
 * (gguf-dequant.ts:655-672).  Negative on error. */
int64_t gguf_hip_tile_bytes(int ggml_type, int64_t n_rows, int64_t k);

/* Raw GGUF bytes (device, any alignment, exactly raw_bytes long) -> row-tile
 * layout (device, 16-byte aligned, exactly tile_bytes long).  Replaces
 * repackGGUFForGPU (gguf-dequant.ts:809-840) including its byte-length check
 * (assertBytes, :678-680).  Padding rows of the last tile are written as zero. */
int gguf_hip_repack(const void *raw, int64_t raw_bytes, int ggml_type, int64_t n_rows,
                    int64_t k, void *tiles, int64_t tile_bytes, void *stream);

/* Dequantize an [n_rows, k] weight in the row-tile layout to f32
 * out[n * ldo + i].  Bit-exact to dequantGGML (gguf-dequant.ts:844-868). */
int gguf_hip_dequant(const void *tiles, int ggml_type, int64_t n_rows, int64_t k, float *out,
                     int64_t ldo, void *stream);

/* Dequantize n_elems elements of raw GGUF bytes (device, any alignment) to
 * f32 out[0..n_elems).  Same values as dequantGGML (gguf-dequant.ts:844-868);
 * the reference uses it for the CPU embedding row-gather (forward-pass.ts:2171-2186). */
int gguf_hip_dequant_raw(const void *raw, int ggml_type, int64_t n_elems, float *out,
                         void *stream);

/* Row gather of a raw GGUF table: out[i * ldo + j] = dequant(raw row ids[i])[j]
 * for i < n_ids, j < k.  raw: n_rows x k elements of raw GGUF rows (device,
 * any alignment); ids: device int64[n_ids]; out: f32.  Values are those of
 * dequantGGML on the row's bytes.  Replaces the reference's CPU embedding
 * row-gather (webgpu/src/engine/forward-pass.ts:2171-2186, token_embd kept in
 * RAM by webgpu/src/model/gguf-loader.ts:177-187); here the table stays in HBM
 * and the ids are read on the device, so a decode step that gathers its token
 * can be captured in a graph.  An id outside [0, n_rows) yields a row of NaN. */
int gguf_hip_get_rows(const void *raw, int ggml_type, int64_t n_rows, int64_t k,
                      const int64_t *ids, int64_t n_ids, float *out, int64_t ldo, void *stream);

/* y[m * ldy + n] = sum_k x[m * ldx + k] * dequant(W)[n, k] for m < M, n < N.
 * x: f32 or f16 (x_type = GGUF_HIP_F32 / GGUF_HIP_F16), 16-byte aligned rows
 * (ldx * sizeof(x) % 16 == 0), any finite values: the kernels scale blocks of
 * activations by powers of two before they enter the f16 matrix cores, so
 * there is no range limit beyond f32's own (non-finite x gives non-finite y).
 * W: row-tile layout, 16-byte aligned.
 * y: f32, 4-byte aligned.  Accumulation in f32.  Replaces dispatchMatmulGGUF
 * (forward-pass.ts:1496-1544); its io.aOffset / io.cOffset windows are plain
 * pointer offsets here. */
int gguf_hip_matmul(const void *x, int x_type, int64_t ldx, const void *tiles, int ggml_type,
                    int64_t n, int64_t k, float *y, int64_t ldy, int64_t m, void *stream);

/* gguf_hip_matmul with an explicit kernel family (GGUF_HIP_VARIANT_*), the
 * analog of the reference's per-dispatch pipeline choice (forward-pass.ts:1501-1524). */
int gguf_hip_matmul_variant(const void *x, int x_type, int64_t ldx, const void *tiles,
                            int ggml_type, int64_t n, int64_t k, float *y, int64_t ldy,
                            int64_t m, int variant, void *stream);

/* gguf_hip_matmul_variant with a caller workspace (device, 16-byte aligned,
 * work_bytes long; NULL / 0 = none).  With at least gguf_hip_matmul_workspace
 * bytes, a decode pass of 2..32 activation rows, and a GEMM whose output tiles
 * leave most CUs idle (fewer than 192 of 128 x 256; superblock types), split K
 * over the grid and add the slices' partial sums in a fixed order: the same
 * results as without a workspace up to f32 rounding of the sums,
 * deterministic either way, and much faster for weights of few rows (the FFN
 * down projection) and short prefills (M = 512, N = 4096: 258 -> 476
 * TFLOP/s).  Up to 24 f32 (48 f16) rows, and 32 when K >= 8192 or the
 * weight is Q6_K, the batched
 * decode converts the activations in every workgroup (its own K range);
 * otherwise a first launch converts them once.  A last launch adds the K
 * ranges' sums in range order.
 * The workspace's first 65536 bytes are reserved: no call reads or writes
 * them, and one workspace serves calls of any shape and type.
 * The reference engine likewise preallocates its scratch (forward-pass.ts:1140-1163).
 * Calls that share a workspace must not overlap.
 * The grid-codebook IQ types run the decode variant without a workspace up
 * to K = 16384, as every other type does: M = 1 is one launch, and M >= 2
 * without a workspace (or with one smaller than gguf_hip_matmul_workspace)
 * runs the M = 1 kernel once per row; with the workspace the batched kernel
 * reads the weights once for all rows.  Beyond K = 16384 only the batched
 * kernel serves them: without the workspace the call returns
 * GGUF_HIP_ERR_SHAPE before launching anything.
 * The GEMM variant with f32 activations and a workspace of
 * gguf_hip_matmul_workspace bytes stages the rows once: a first launch writes
 * each row times its power of two as an fp16 image (M x K halves after M
 * row scales) and the fp16 kernels run on it, the same bits as without the
 * workspace (where every workgroup scales its rows itself) and 1.2-1.45x
 * faster (Q4_K, N = 14336, K = 4096: M = 512 500 -> 658, M = 2048 567 -> 829
 * TFLOP/s). */
int gguf_hip_matmul_ws(const void *x, int x_type, int64_t ldx, const void *tiles, int ggml_type,
                       int64_t n, int64_t k, float *y, int64_t ldy, int64_t m, int variant,
                       void *work, int64_t work_bytes, void *stream);

/* Bytes of workspace gguf_hip_matmul_ws uses for these shapes (0: none);
 * negative on bad arguments. */
int64_t gguf_hip_matmul_workspace(int ggml_type, int x_type, int64_t n, int64_t k, int64_t m);

/* Prologues of gguf_hip_matmul_fused. */
#define GGUF_HIP_PROLOGUE_NONE 0
#define GGUF_HIP_PROLOGUE_RMSNORM 1 /* x' = x / sqrt(mean(x^2) + eps) * norm_w */
#define GGUF_HIP_PROLOGUE_SWIGLU 2  /* x = [gate (k) | up (k)], x' = up * silu(gate) */

/* Epilogues of gguf_hip_matmul_fused. */
#define GGUF_HIP_EPILOGUE_STORE 0      /* y[n] = r[n] */
#define GGUF_HIP_EPILOGUE_ACCUMULATE 1 /* y[n] += r[n] (the residual add) */
#define GGUF_HIP_EPILOGUE_SWIGLU 2     /* W holds gate / up row tiles interleaved
                                        * (tile 2m = gate rows 16m..16m+15, tile
                                        * 2m + 1 = those up rows; N % 32 == 0):
                                        * y[16m + i] = r[16(2m+1) + i] * silu(r[32m + i]),
                                        * N / 2 outputs */

/* One decode-step projection with its neighbours fused in: the row
 * r[n] = sum_k x'[k] * dequant(W)[n, k] for a single f32 activation row x
 * (16-byte aligned), x' given by the prologue, written by the epilogue.
 * The reference dispatches these as separate rmsnorm, gate_silu, matmul and
 * add shaders in its layer loop (forward-pass.ts:2925-3297).  K <= 16384;
 * shapes without a fused kernel return GGUF_HIP_ERR_SHAPE. */
int gguf_hip_matmul_fused(const float *x, const void *tiles, int ggml_type, int64_t n, int64_t k,
                          float *y, int prologue, const float *norm_w, float eps, int epilogue,
                          void *stream);

/* ---------------------------------------------------------------------------
 * Decode-step glue around the quantized projections (f32, contiguous rows,
 * 16-byte aligned pointers, lengths multiple of 4).  The reference runs these
 * as WGSL shaders inside its layer loop (forward-pass.ts:2925-3297).
 * ------------------------------------------------------------------------- */

/* y[r] = x[r] / sqrt(mean(x[r]^2) + eps) * w for rows r < rows of n elements
 * (rmsnorm.wgsl:1-9,58-67 with use_residual_weight = 0). */
int gguf_hip_rmsnorm(const float *x, const float *w, float eps, float *y, int64_t rows,
                     int64_t n, void *stream);

/* Residual add then RMSNorm: x[r] += res[r] (x updated in place), then
 * y[r] = rmsnorm(x[r]) * w.  The reference's separate add and rmsnorm
 * dispatches of its layer loop, fused.  y must not alias x. */
int gguf_hip_add_rmsnorm(float *x, const float *res, const float *w, float eps, float *y,
                         int64_t rows, int64_t n, void *stream);

/* out[r, i] = up[i] * silu(gate[i]) for rows [gate (ffn) | up (ffn)]
 * (elementwise.wgsl:96-102, gate_silu with a = up, b = gate). */
int gguf_hip_swiglu(const float *gate_up, float *out, int64_t rows, int64_t ffn, void *stream);

/* One decode position p = *pos (device int64): rotate_half RoPE of q and k
 * (rope.wgsl:1-10; cos / sin tables [max_seq, head_dim / 2] at row p), k and
 * v appended to the caches at slot p, then causal GQA attention of each query
 * head h over slots 0..p of KV head h / (n_heads / n_kv_heads), softmax scaled
 * by 1/sqrt(head_dim).  qkv = [q (n_heads*head_dim) | k | v (n_kv*head_dim each)];
 * caches [n_kv, max_seq, head_dim]; out [n_heads * head_dim]; head_dim is 64,
 * 128 or 256 and n_heads / n_kv_heads at most 8.  One launch.  `work`
 * (device, 16-byte aligned, gguf_hip_attention_workspace bytes) holds the
 * per-64-slot partial softmax records and one counter per KV head; it must be
 * zero-filled once before its first use, and every call leaves the counters
 * at zero again.  Calls that share a workspace must not overlap.  The
 * position is read on the device, so the call can be captured in a graph.
 * out == NULL: only the records are written (no merge, counters untouched),
 * for gguf_hip_matmul_attn_merge to merge inside the output projection. */
int gguf_hip_attention_decode(const float *qkv, const int64_t *pos, const float *cos_table,
                              const float *sin_table, float *k_cache, float *v_cache, float *out,
                              int n_heads, int n_kv_heads, int head_dim, int64_t max_seq,
                              void *work, void *stream);

/* Bytes of the gguf_hip_attention_decode workspace; negative on bad shapes. */
int64_t gguf_hip_attention_workspace(int n_heads, int n_kv_heads, int head_dim, int64_t max_seq);

/* gguf_hip_attention_decode that allocates nothing and takes no workspace.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under graph capture, serving loops, harnesses that
 * forbid it).  Same arguments and results as gguf_hip_attention_decode with
 * out != NULL (out is required).  The records and counters live in a device
 * array of GGUF_HIP_NOALLOC_ATTENTION_BYTES inside the library, one per GPU,
 * held until the process ends; shapes whose workspace
 * (gguf_hip_attention_workspace) exceeds it return GGUF_HIP_ERR_SHAPE.  All
 * calls on one GPU share that array: calls that overlap on a GPU race. */
#define GGUF_HIP_NOALLOC_ATTENTION_BYTES 8388608 /* 8 MiB */
int gguf_hip_attention_decode_noalloc(const float *qkv, const int64_t *pos,
                                      const float *cos_table, const float *sin_table,
                                      float *k_cache, float *v_cache, float *out, int n_heads,
                                      int n_kv_heads, int head_dim, int64_t max_seq,
                                      void *stream);

/* Prefill attention over m new rows (attention.wgsl:60-234 with new_seq_len =
 * m, causal, and rope.wgsl:1-10 before it; forward-pass.ts:2925-3297).  For
 * each row r at position pos[r] (device int64 [m]): rotate_half RoPE of q and
 * k with the tables' row pos[r], k and v stored at slot pos[r] of the caches,
 * then causal GQA attention of each query head h over slots 0..pos[r] of KV
 * head h / (n_heads / n_kv_heads), softmax scaled by 1/sqrt(head_dim).
 * qkv rows (stride ldqkv floats) = [q (n_heads*head_dim) | k | v
 * (n_kv*head_dim each)]; out rows (stride ldo) = n_heads*head_dim.  Slots
 * below a row's position that the call does not write must hold keys already
 * (an earlier prefill or decode call).  Positions within a call must be
 * distinct; a position outside 0..max_seq-1 leaves its row's cache slot and
 * output untouched.  out must not overlap qkv or the caches.  Shapes as
 * gguf_hip_attention_decode; ldqkv and ldo multiples of 4; qkv, out, caches
 * and tables 16-byte aligned.  Two launches, no workspace.  m == 0 is a
 * no-op. */
int gguf_hip_attention_prefill(const float *qkv, int64_t ldqkv, const int64_t *pos, int64_t m,
                               const float *cos_table, const float *sin_table, float *k_cache,
                               float *v_cache, float *out, int64_t ldo, int n_heads,
                               int n_kv_heads, int head_dim, int64_t max_seq, void *stream);

/* The attention output projection of one decode position with the attention
 * merge fused in: y (= or +=, epilogue STORE / ACCUMULATE) W . a, where a
 * [n_heads * head_dim] is the attention output merged on the fly from the
 * records that gguf_hip_attention_decode(..., out = NULL, work) wrote for
 * position *pos -- the same arithmetic as that call's own merge, so y equals
 * gguf_hip_matmul_fused(a, W, ..., PROLOGUE_NONE, ...) on its output.  Replaces
 * the reference's attention-output and o-projection dispatches
 * (forward-pass.ts:2925-3297) by one.  The shapes are those of the attention
 * call; K = n_heads * head_dim <= 8192.  A position outside 0..max_seq - 1
 * gives NaN outputs. */
int gguf_hip_matmul_attn_merge(const void *work, const int64_t *pos, int n_heads, int n_kv_heads,
                               int head_dim, int64_t max_seq, const void *tiles, int ggml_type,
                               int64_t n, float *y, int epilogue, void *stream);

/* *out = first index of the maximum of x[0..n) (NaN never wins); greedy
 * sampling.  `work`: gguf_hip_argmax_workspace() bytes of device memory
 * (8-byte aligned) for the per-workgroup partials. */
int gguf_hip_argmax(const float *x, int64_t n, int64_t *out, void *work, void *stream);

/* Bytes of the gguf_hip_argmax workspace. */
int64_t gguf_hip_argmax_workspace(void);

#pragma GCC visibility pop

#ifdef __cplusplus
}
#endif

#endif /* GGUF_HIP_H */
