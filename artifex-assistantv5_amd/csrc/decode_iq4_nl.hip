// Decode kernels for ggml type 20 (IQ4_NL); the kernels are in decode_impl.hpp.
#include "decode_impl.hpp"

namespace gguf {
GGUF_DECODE_DEFINE(20, iq4_nl)
}  // namespace gguf
