// Decode kernels for ggml type 11 (Q3_K); the kernels are in decode_impl.hpp.
#include "decode_impl.hpp"

namespace gguf {
GGUF_DECODE_DEFINE(11, q3_k)
}  // namespace gguf
