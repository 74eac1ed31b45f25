// Decode kernels for ggml type 10 (Q2_K); the kernels are in decode_impl.hpp.
#include "decode_impl.hpp"

namespace gguf {
GGUF_DECODE_DEFINE(10, q2_k)
}  // namespace gguf
