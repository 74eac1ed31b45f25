// Decode kernels for ggml type 22 (IQ2_S); the kernels are in decode_mk.hpp.
#include "decode_impl.hpp"

namespace gguf {
GGUF_DECODE_DEFINE_IQ(22, iq2_s)
}  // namespace gguf
