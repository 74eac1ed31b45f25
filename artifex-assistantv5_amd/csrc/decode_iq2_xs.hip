// Decode kernels for ggml type 17 (IQ2_XS); the kernels are in decode_mk.hpp.
#include "decode_impl.hpp"

namespace gguf {
GGUF_DECODE_DEFINE_IQ(17, iq2_xs)
}  // namespace gguf
