// KV gather: the first L_b tokens of every (sequence, kv head) of a cache in any layout the kernels read
// (contiguous or paged, 16-bit or fp8 with per-(token, head) scales), written as dense 16-bit rows
// out[b, h, t, :] for t < out_len; rows at or past L_b are zero. fp8 rows come out as code * scale in fp32,
// rounded once to the output type: the dequantised cache a prefill's attention reads, the counterpart of the
// reference's gather of its paged, quantised cache (new KV cache/evaluation_wrapper.py:428-453 and
// _gather_paged_kv_cache there).
//
// Grid (row blocks, kv heads, sequences): a workgroup writes kGatherPasses passes of 256 / (D / 8) rows of one
// (sequence, head), 16 bytes of K and of V output per lane and row; every pass's source rows are loaded before
// any is converted. Byte work, HBM-bound: read L_b rows (D * e bytes, plus a 4-byte scale for fp8) of K and of
// V, write out_len rows of 2 * D bytes of each.
#pragma once

#include "common.hpp"

namespace aicas {

struct GatherParams {
  KVLayout cache;
  const int32_t* seq_lens;  // [B] tokens of each sequence to copy
  void* k_out;
  void* v_out;
  int64_t out_stride_b, out_stride_h, out_stride_t;  // elements; the head_dim stride is 1
  int32_t out_len;
  int32_t num_kv_heads;
  int32_t* status;
};

constexpr int kGatherPasses = 8;

constexpr int gather_rows_per_workgroup(int head_dim) { return kBlockThreads / (head_dim / 8) * kGatherPasses; }

// KV_DT: cache type; OUT_DT: the output's 16-bit type (the cache's own for 16-bit caches).
template <int KV_DT, int OUT_DT, int D>
__global__ __launch_bounds__(kBlockThreads) void kv_gather_kernel(GatherParams p) {
  constexpr bool FP8 = (KV_DT == kFP8E4M3);
  constexpr int VEC = 8;      // output elements per lane and row (16 bytes)
  constexpr int R = D / VEC;  // lanes per row
  constexpr int ROWS_PER_PASS = kBlockThreads / R;
  static_assert(!FP8 || OUT_DT != kFP8E4M3, "the output is 16-bit");

  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int lane = tid % R;
  const int t0 = blockIdx.x * ROWS_PER_PASS * kGatherPasses + tid / R;

  int L = p.seq_lens[b];
  if (L > p.cache.max_tokens) {
    if (p.status && tid == 0 && blockIdx.x == 0 && h == 0) atomicOr(p.status, kStatusLenClamped);
    L = p.cache.max_tokens;
  }
  L = max(0, min(L, p.out_len));

  // Source rows of every pass, loaded before any conversion. Every load is issued unconditionally (a pass past
  // the length, or behind an invalid block id, reads an in-bounds row and is masked afterwards), so the loads
  // are in flight together: the block ids of all passes first, then the rows.
  int64_t blk[kGatherPasses];
  int tin[kGatherPasses];
  bool ok[kGatherPasses];
  if (p.cache.block_table) {
    const int32_t* const row_ids = p.cache.block_table + static_cast<int64_t>(b) * p.cache.block_table_stride;
#pragma unroll
    for (int k = 0; k < kGatherPasses; ++k) {
      const int tc = min(t0 + k * ROWS_PER_PASS, max(L - 1, 0));
      blk[k] = row_ids[tc / p.cache.page_size];
      tin[k] = tc % p.cache.page_size;
    }
  } else {
#pragma unroll
    for (int k = 0; k < kGatherPasses; ++k) {
      blk[k] = b;
      tin[k] = min(t0 + k * ROWS_PER_PASS, max(L - 1, 0));
    }
  }
  bool bad = false;
#pragma unroll
  for (int k = 0; k < kGatherPasses; ++k) {
    const bool valid = blk[k] >= 0 && blk[k] < p.cache.num_blocks;
    const bool live = t0 + k * ROWS_PER_PASS < L;
    ok[k] = live && valid;
    bad |= live && !valid;
    if (!valid) blk[k] = 0;
  }
  uint4 kw[kGatherPasses], vw[kGatherPasses];  // 16-bit: 8 elements; fp8: 8 codes in .x, .y
  float ks[kGatherPasses], vs[kGatherPasses];
#pragma unroll
  for (int k = 0; k < kGatherPasses; ++k) {
    const int64_t row = blk[k] * p.cache.stride_blk + h * p.cache.stride_h + static_cast<int64_t>(tin[k]) * p.cache.stride_t;
    if constexpr (FP8) {
      const uint2 kc = *reinterpret_cast<const uint2*>(static_cast<const uint8_t*>(p.cache.k) + row + lane * VEC);
      const uint2 vc = *reinterpret_cast<const uint2*>(static_cast<const uint8_t*>(p.cache.v) + row + lane * VEC);
      kw[k] = make_uint4(kc.x, kc.y, 0u, 0u);
      vw[k] = make_uint4(vc.x, vc.y, 0u, 0u);
      const int64_t srow = blk[k] * p.cache.scale_stride_blk + h * p.cache.scale_stride_h + tin[k];
      ks[k] = p.cache.k_scale[srow];
      vs[k] = p.cache.v_scale[srow];
    } else {
      kw[k] = load_stream16(static_cast<const uint16_t*>(p.cache.k) + row + lane * VEC);
      vw[k] = load_stream16(static_cast<const uint16_t*>(p.cache.v) + row + lane * VEC);
    }
  }

  if (bad && p.status && lane == 0) atomicOr(p.status, kStatusBlockOutOfRange);

  // fp8: 8 codes (two dwords) -> 8 values code * scale, rounded to OUT_DT and packed in 4 dwords
  auto dequant = [](uint32_t w0, uint32_t w1, float scale) -> uint4 {
    uint32_t out[4];
    const uint32_t src[2] = {w0, w1};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const uint32_t v2 = half ? e4m3x2_to_16<OUT_DT, true>(src[i]) : e4m3x2_to_16<OUT_DT, false>(src[i]);
        float lo, hi;
        unpack2<OUT_DT>(v2, lo, hi);
        out[2 * i + half] = pack2<OUT_DT>(__fmul_rn(lo, scale), __fmul_rn(hi, scale));
      }
    }
    return make_uint4(out[0], out[1], out[2], out[3]);
  };

  uint16_t* const ko = static_cast<uint16_t*>(p.k_out) + b * p.out_stride_b + h * p.out_stride_h + lane * VEC;
  uint16_t* const vo = static_cast<uint16_t*>(p.v_out) + b * p.out_stride_b + h * p.out_stride_h + lane * VEC;
#pragma unroll
  for (int k = 0; k < kGatherPasses; ++k) {
    const int t = t0 + k * ROWS_PER_PASS;
    if (t >= p.out_len) continue;
    uint4 a = kw[k], c = vw[k];
    if constexpr (FP8) {
      a = dequant(kw[k].x, kw[k].y, ks[k]);
      c = dequant(vw[k].x, vw[k].y, vs[k]);
    }
    if (!ok[k]) a = c = make_uint4(0u, 0u, 0u, 0u);
    store_stream16(ko + static_cast<int64_t>(t) * p.out_stride_t, a);
    store_stream16(vo + static_cast<int64_t>(t) * p.out_stride_t, c);
  }
}

}  // namespace aicas
