// Decode kernels for ggml type 29 (IQ1_M); the kernels are in decode_mk.hpp.
#include "decode_impl.hpp"

namespace gguf {
GGUF_DECODE_DEFINE_IQ(29, iq1_m)
}  // namespace gguf
