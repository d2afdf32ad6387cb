// Decode-kernel instantiations for q fp16, kv cache fp8.
#include "decode_launch.hpp"

int launch_decode_fp16_fp8(const aicas::DecodeParams& p, int d, int g, bool paged, bool append, bool qk, dim3 grid,
                           hipStream_t s) {
  return aicas::launch_decode_pair<aicas::kFP16, aicas::kFP8E4M3>(p, d, g, paged, append, qk, grid, s);
}
