// Decode kernels for ggml type 2 (Q4_0); the kernels are in decode_impl.hpp.
#include "decode_impl.hpp"

namespace gguf {
GGUF_DECODE_DEFINE(2, q4_0)
}  // namespace gguf
