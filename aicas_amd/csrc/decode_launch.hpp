// Decode-kernel dispatch over head_dim, GQA group size, layout, the fused append and its q/k prologue, for one
// (q dtype, kv dtype) pair. Included once per pair by decode_<q>_<kv>.hip so that the instantiations
// compile in parallel.
#pragma once

#include "decode_attn.hpp"

namespace aicas {

template <int Q, int KV, int D, int G, bool PAGED, bool SPEC>
void launch_decode_dgps(const DecodeParams& p, bool append, bool qk, dim3 grid, hipStream_t s) {
  const dim3 block(kBlockThreads);
  if (qk) hipLaunchKernelGGL((decode_attn_kernel<Q, KV, D, G, PAGED, true, true, SPEC>), grid, block, 0, s, p);
  else if (append)
    hipLaunchKernelGGL((decode_attn_kernel<Q, KV, D, G, PAGED, true, false, SPEC>), grid, block, 0, s, p);
  else hipLaunchKernelGGL((decode_attn_kernel<Q, KV, D, G, PAGED, false, false, SPEC>), grid, block, 0, s, p);
}

// Contiguous caches whose every split is kept busy by the caller's lower bound on the lengths take the variant
// that fetches its first rows before reading the length.
template <int Q, int KV, int D, int G, bool PAGED>
void launch_decode_dgp(const DecodeParams& p, bool append, bool qk, dim3 grid, hipStream_t s) {
  if constexpr (!PAGED) {
    if (p.spec_splits >= p.max_splits) {
      launch_decode_dgps<Q, KV, D, G, false, true>(p, append, qk, grid, s);
      return;
    }
  }
  launch_decode_dgps<Q, KV, D, G, PAGED, false>(p, append, qk, grid, s);
}

template <int Q, int KV, int D, int G>
void launch_decode_dg(const DecodeParams& p, bool paged, bool append, bool qk, dim3 grid, hipStream_t s) {
  if (paged) launch_decode_dgp<Q, KV, D, G, true>(p, append, qk, grid, s);
  else launch_decode_dgp<Q, KV, D, G, false>(p, append, qk, grid, s);
}

template <int Q, int KV, int D>
int launch_decode_d(const DecodeParams& p, int g, bool paged, bool append, bool qk, dim3 grid, hipStream_t s) {
  switch (g) {
    case 1: launch_decode_dg<Q, KV, D, 1>(p, paged, append, qk, grid, s); return 0;
    case 2: launch_decode_dg<Q, KV, D, 2>(p, paged, append, qk, grid, s); return 0;
    case 4: launch_decode_dg<Q, KV, D, 4>(p, paged, append, qk, grid, s); return 0;
    case 8: launch_decode_dg<Q, KV, D, 8>(p, paged, append, qk, grid, s); return 0;
    default: return 1;
  }
}

template <int Q, int KV>
int launch_decode_pair(const DecodeParams& p, int d, int g, bool paged, bool append, bool qk, dim3 grid, hipStream_t s) {
  switch (d) {
    case 16: return launch_decode_d<Q, KV, 16>(p, g, paged, append, qk, grid, s);
    case 32: return launch_decode_d<Q, KV, 32>(p, g, paged, append, qk, grid, s);
    case 64: return launch_decode_d<Q, KV, 64>(p, g, paged, append, qk, grid, s);
    case 128: return launch_decode_d<Q, KV, 128>(p, g, paged, append, qk, grid, s);
    default: return 1;
  }
}

}  // namespace aicas
