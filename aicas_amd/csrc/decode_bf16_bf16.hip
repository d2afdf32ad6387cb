// Decode-kernel instantiations for q bf16, kv cache bf16.
#include "decode_launch.hpp"

int launch_decode_bf16_bf16(const aicas::DecodeParams& p, int d, int g, bool paged, bool append, bool qk, dim3 grid,
                            hipStream_t s) {
  return aicas::launch_decode_pair<aicas::kBF16, aicas::kBF16>(p, d, g, paged, append, qk, grid, s);
}
