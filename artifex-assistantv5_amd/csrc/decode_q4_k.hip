// Decode kernels for ggml type 12 (Q4_K); the kernels are in decode_impl.hpp.
#include "decode_impl.hpp"

namespace gguf {
GGUF_DECODE_DEFINE(12, q4_k)
}  // namespace gguf
