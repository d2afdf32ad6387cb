// Decode-kernel instantiations for q fp16, kv cache fp16.
#include "decode_launch.hpp"

int launch_decode_fp16_fp16(const aicas::DecodeParams& p, int d, int g, bool paged, bool append, bool qk, dim3 grid,
                            hipStream_t s) {
  return aicas::launch_decode_pair<aicas::kFP16, aicas::kFP16>(p, d, g, paged, append, qk, grid, s);
}
