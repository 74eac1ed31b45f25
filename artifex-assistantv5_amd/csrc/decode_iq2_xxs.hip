// Decode kernels for ggml type 16 (IQ2_XXS); the kernels are in decode_mk.hpp.
#include "decode_impl.hpp"

namespace gguf {
GGUF_DECODE_DEFINE_IQ(16, iq2_xxs)
}  // namespace gguf
