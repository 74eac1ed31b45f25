// Decode kernels for ggml type 13 (Q5_K); the kernels are in decode_impl.hpp.
#include "decode_impl.hpp"

namespace gguf {
GGUF_DECODE_DEFINE(13, q5_k)
}  // namespace gguf
