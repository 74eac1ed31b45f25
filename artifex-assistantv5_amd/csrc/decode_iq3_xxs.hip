// Decode kernels for ggml type 18 (IQ3_XXS); the kernels are in decode_mk.hpp.
#include "decode_impl.hpp"

namespace gguf {
GGUF_DECODE_DEFINE_IQ(18, iq3_xxs)
}  // namespace gguf
