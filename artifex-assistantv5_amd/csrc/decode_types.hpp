// Per-type entry points of the decode kernels (decode_impl.hpp), one
// translation unit per ggml type (decode_<type>.hip).
#pragma once

#include "common.hpp"

namespace gguf {

#define GGUF_DECODE_DECLARE(NAME)                                                               \
  hipError_t decode_##NAME(const void *x, int x_type, int64_t ldx, const uint8_t *tiles, int n, \
                           int k, float *y, int64_t ldy, int m, float *work,                    \
                           int64_t work_floats, hipStream_t s);                                 \
  int64_t decode_work_##NAME(int x_type, int n, int k, int m);                                  \
  hipError_t decode_fused_##NAME(const float *x, const uint8_t *tiles, int n, int k, float *y,  \
                                 int prologue, const float *pw, float eps, int epi,             \
                                 hipStream_t s);                                                \
  hipError_t decode_merge_##NAME(const AttnRecords &ar, const uint8_t *tiles, int n, float *y,  \
                                 int epi, hipStream_t s);
GGUF_DECODE_DECLARE(q4_0)
GGUF_DECODE_DECLARE(q5_0)
GGUF_DECODE_DECLARE(q8_0)
GGUF_DECODE_DECLARE(q2_k)
GGUF_DECODE_DECLARE(q3_k)
GGUF_DECODE_DECLARE(q4_k)
GGUF_DECODE_DECLARE(q5_k)
GGUF_DECODE_DECLARE(q6_k)
GGUF_DECODE_DECLARE(iq4_nl)
GGUF_DECODE_DECLARE(iq4_xs)
GGUF_DECODE_DECLARE(iq2_xxs)
GGUF_DECODE_DECLARE(iq2_xs)
GGUF_DECODE_DECLARE(iq2_s)
GGUF_DECODE_DECLARE(iq3_xxs)
GGUF_DECODE_DECLARE(iq3_s)
GGUF_DECODE_DECLARE(iq1_m)

#undef GGUF_DECODE_DECLARE

}  // namespace gguf
