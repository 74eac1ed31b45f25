// Decode kernels for ggml type 23 (IQ4_XS); the kernels are in decode_impl.hpp.
#include "decode_impl.hpp"

namespace gguf {
GGUF_DECODE_DEFINE(23, iq4_xs)
}  // namespace gguf
