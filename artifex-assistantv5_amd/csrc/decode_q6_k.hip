// Decode kernels for ggml type 14 (Q6_K); the kernels are in decode_impl.hpp.
#include "decode_impl.hpp"

namespace gguf {
GGUF_DECODE_DEFINE(14, q6_k)
}  // namespace gguf
