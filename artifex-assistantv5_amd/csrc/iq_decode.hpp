// Weight loads and decode-kernel glue of the grid-codebook IQ types (their
// arithmetic is in iq_ops.hpp).  Included by decode_impl.hpp after its buffer
// loads.
#pragma once

template <int TYPE>
__device__ __forceinline__ void load_iq(__amdgpu_buffer_rsrc_t rs, int soff, int r, IqUnit<TYPE> &u) {
  constexpr int RD = iq_rd<TYPE>();
  const int base = iq_rec_off<TYPE>(r);
#pragma unroll
  for (int c = 0; c < RD / 4; ++c) {
    const uint4 v = bload16(rs, base + 16 * c, soff);
    u.w[4 * c] = v.x; u.w[4 * c + 1] = v.y; u.w[4 * c + 2] = v.z; u.w[4 * c + 3] = v.w;
  }
  if constexpr (RD % 4 >= 2) {
    const uint2 v = bload8(rs, base + 16 * (RD / 4), soff);
    u.w[RD / 4 * 4] = v.x;
    u.w[RD / 4 * 4 + 1] = v.y;
  }
  if constexpr (RD % 2 == 1) u.w[RD - 1] = bload4(rs, base + 4 * (RD - 1), soff);
  u.d = IqFmt<TYPE>::HASD ? bload2(rs, 2 * r, soff) : 0u;
}
// the type's grid bytes, as 16-byte chunks
// The per-lane unit of the decode kernels and its load.
#define GGUF_IQ_UNIT(T)                                                                          \
  template <>                                                                                    \
  struct Unit<T> : IqUnit<T> {};                                                                 \
  __device__ __forceinline__ void load_unit(__amdgpu_buffer_rsrc_t rs, int soff, int r, int,     \
                                            Unit<T> &u) {                                        \
    load_iq<T>(rs, soff, r, u);                                                                  \
  }                                                                                              \
  template <>                                                                                    \
  struct Dec<T> {                                                                                \
    static constexpr int GS = 32, P1 = 1;                                                        \
    static constexpr bool SUMS = false, NAT = true;                                              \
  };
GGUF_IQ_UNIT(16)
GGUF_IQ_UNIT(17)
GGUF_IQ_UNIT(18)
GGUF_IQ_UNIT(21)
GGUF_IQ_UNIT(22)
GGUF_IQ_UNIT(29)
#undef GGUF_IQ_UNIT
