// Decode kernels for ggml type 6 (Q5_0); the kernels are in decode_impl.hpp.
#include "decode_impl.hpp"

namespace gguf {
GGUF_DECODE_DEFINE(6, q5_0)
}  // namespace gguf
