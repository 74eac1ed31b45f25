// Decode kernels for ggml type 21 (IQ3_S); the kernels are in decode_mk.hpp.
#include "decode_impl.hpp"

namespace gguf {
GGUF_DECODE_DEFINE_IQ(21, iq3_s)
}  // namespace gguf
