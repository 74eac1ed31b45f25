// Decode kernels for ggml type 8 (Q8_0); the kernels are in decode_impl.hpp.
#include "decode_impl.hpp"

namespace gguf {
GGUF_DECODE_DEFINE(8, q8_0)
}  // namespace gguf
