// KV append: write each sequence's new K/V rows into its cache at positions[b] .. positions[b]+n_new-1.
//
// Semantics follow the preallocated in-place append of the reference
// (dujunbaoV1/evaluation_wrapper.py:84-100, index_copy_ of the new rows at the current length), which
// is bitwise the same cache content as HF DynamicLayer.update's torch.cat
// (transformers/cache_utils.py:127-146). For fp8 caches the rows are quantized on write with one fp32
// scale per (token, kv-head): scale = amax/448, q = e4m3(clamp(x / scale, -448, 448)), the code from gfx950's
// fp8 conversion instruction (round to nearest even) of the correctly rounded quotient (fp8_quantize).
//
// Grid (row blocks, sequences): a workgroup writes kAppendPasses passes of 256 / (D / 8) rows of one sequence
// (K rows first, then V rows; head-major, then token), with every pass's source rows loaded before
// positions[b] is read. A decode step's append (a few rows per sequence) is one workgroup per sequence, whose
// thread 0 stores positions[b] + n_new into seq_lens_out[b] after every row is written; seq_lens_out may
// therefore alias positions (an in-place length bump that a captured HIP graph can replay step after step).
// When a sequence's rows need several workgroups, the host follows with bump_lens_kernel instead, so that no
// workgroup can read a bumped position.
#pragma once

#include "common.hpp"

namespace aicas {

struct AppendParams {
  KVLayout cache;
  const void* k_src;
  const void* v_src;
  int64_t k_src_stride_b, v_src_stride_b;  // elements; the head_dim stride is 1
  // The per-row strides as 32-bit values (the host checks that they fit), so that each term of a row's offset is
  // one 32 x 32 -> 64-bit multiply-add: [0] K, [1] V.
  uint32_t src_stride_h[2], src_stride_t[2];
  uint32_t dst_stride_blk, dst_stride_h, dst_stride_t;  // cache rows (elements)
  uint32_t scale_stride_blk, scale_stride_h;            // fp8 scales (token stride 1)
  const int32_t* positions;
  int32_t* seq_lens_out;
  int32_t* status;
  int32_t num_kv_heads;
  int32_t n_new;
  FastDiv div_n_new;   // division by n_new
  int32_t page_shift;  // paged caches: log2(page_size)
};

constexpr int kAppendPasses = 8;

// Rows one workgroup writes.
constexpr int append_rows_per_workgroup(int head_dim) { return kBlockThreads / (head_dim / 8) * kAppendPasses; }

// SRC_DT: dtype of the incoming rows (bf16 or fp16). KV_DT: cache dtype (same as SRC_DT, or fp8).
template <int SRC_DT, int KV_DT, int D>
__global__ __launch_bounds__(kBlockThreads) void kv_append_kernel(AppendParams p) {
  constexpr int VEC = 8;      // source elements per thread (16 bytes)
  constexpr int R = D / VEC;  // threads per row
  static_assert(R >= 1 && R <= 16, "a row must fit one DPP row");
  constexpr int ROWS_PER_PASS = kBlockThreads / R;

  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid % R;
  const int rows_per_tensor = p.num_kv_heads * p.n_new;
  const int rows_total = 2 * rows_per_tensor;
  const int first_row = blockIdx.x * ROWS_PER_PASS * kAppendPasses + tid / R;

  // Row r of the launch's 0 <= r < rows_total (K rows first, then V rows; head-major, then token): tensor
  // `which`, kv head h, new row j (a division by n_new with the launch's multiplier: per-lane integer
  // divisions by launch values were most of this kernel's instructions).
  auto row_coords = [&](int r, int& which, int& h, int& j) {
    which = r >= rows_per_tensor ? 1 : 0;
    const int rr = r - which * rows_per_tensor;
    h = fast_div(rr, p.div_n_new);
    j = rr - h * p.n_new;
  };
  const uint16_t* const k_src_b = static_cast<const uint16_t*>(p.k_src) + b * p.k_src_stride_b;
  const uint16_t* const v_src_b = static_cast<const uint16_t*>(p.v_src) + b * p.v_src_stride_b;
  // Every pass's rows are loaded before the position is known, overlapping the reads; rows past the last (a
  // partial last workgroup) load the last row again, unused, so that every load is issued unconditionally.
  uint4 x[kAppendPasses];
#pragma unroll
  for (int k = 0; k < kAppendPasses; ++k) {
    int which, h, j;
    row_coords(min(first_row + k * ROWS_PER_PASS, rows_total - 1), which, h, j);
    // selects between values held in scalar registers (indexing the argument arrays by `which` would load the
    // chosen field per lane)
    const uint32_t sh = which == 0 ? p.src_stride_h[0] : p.src_stride_h[1];
    const uint32_t st = which == 0 ? p.src_stride_t[0] : p.src_stride_t[1];
    const uint16_t* src = (which == 0 ? k_src_b : v_src_b) + (static_cast<uint64_t>(static_cast<uint32_t>(h)) * sh +
                                                              static_cast<uint64_t>(static_cast<uint32_t>(j)) * st);
    x[k] = load_stream16(src + lane * VEC);
  }
  const int pos = p.positions[b];  // uniform: every wave reads it

  // Where every pass's row goes. Paged caches: the block ids of all passes are loaded together (each index
  // clamped into the table), then checked, so that the passes do not wait for them one after another.
  uint64_t dst_row[kAppendPasses], dst_srow[kAppendPasses];
  bool dst_ok[kAppendPasses];
  {
    int tok[kAppendPasses], head[kAppendPasses];
    int32_t blk[kAppendPasses];
#pragma unroll
    for (int k = 0; k < kAppendPasses; ++k) {
      int which, j;
      row_coords(min(first_row + k * ROWS_PER_PASS, rows_total - 1), which, head[k], j);
      tok[k] = pos + j;
    }
    if (p.cache.block_table) {
      const int32_t* const ids = p.cache.block_table + static_cast<int64_t>(b) * p.cache.block_table_stride;
#pragma unroll
      for (int k = 0; k < kAppendPasses; ++k) blk[k] = ids[min(max(tok[k], 0), p.cache.max_tokens - 1) >> p.page_shift];
    } else {
#pragma unroll
      for (int k = 0; k < kAppendPasses; ++k) blk[k] = b;
    }
    const int page_mask = (1 << p.page_shift) - 1;
    int32_t flags = 0;
#pragma unroll
    for (int k = 0; k < kAppendPasses; ++k) {
      const int r = first_row + k * ROWS_PER_PASS;
      const int t = tok[k];
      const bool live = r < rows_total;
      const bool in_cache = t >= 0 && t < p.cache.max_tokens;
      const bool valid = blk[k] >= 0 && blk[k] < p.cache.num_blocks;
      if (live && !in_cache) flags |= kStatusAppendOverflow;
      else if (live && !valid) flags |= kStatusBlockOutOfRange;
      dst_ok[k] = live && in_cache && valid;
      const uint32_t ublk = static_cast<uint32_t>(blk[k]), uh = static_cast<uint32_t>(head[k]);
      const uint32_t tin = static_cast<uint32_t>(p.cache.block_table ? t & page_mask : t);
      dst_row[k] = static_cast<uint64_t>(ublk) * p.dst_stride_blk + static_cast<uint64_t>(uh) * p.dst_stride_h +
                   static_cast<uint64_t>(tin) * p.dst_stride_t;
      dst_srow[k] = static_cast<uint64_t>(ublk) * p.scale_stride_blk + static_cast<uint64_t>(uh) * p.scale_stride_h +
                    tin;
    }
    if (flags && p.status && lane == 0) atomicOr(p.status, flags);
  }
  // 16-bit caches: every load (source rows, block ids) has been issued; wait for all of them once, so that no
  // pass's stores are followed by a wait (behind the conditional stores the compiler's waits would cover the
  // stores too). fp8 caches leave the waits per pass: their quantisation is the larger cost, and converting a
  // pass while the later passes' rows are still arriving is worth more than the stores' waits.
  if constexpr (KV_DT != kFP8E4M3) wait_vmem();

#pragma unroll
  for (int k = 0; k < kAppendPasses; ++k) {
    const int r = first_row + k * ROWS_PER_PASS;
    if (r >= rows_total) continue;  // the whole row group (R lanes) skips together
    const int which = r >= rows_per_tensor ? 1 : 0;
    const uint64_t row = dst_row[k], srow = dst_srow[k];
    const bool ok = dst_ok[k];
    if constexpr (KV_DT == kFP8E4M3) {
      float f[VEC];
      unpack2<SRC_DT>(x[k].x, f[0], f[1]);
      unpack2<SRC_DT>(x[k].y, f[2], f[3]);
      unpack2<SRC_DT>(x[k].z, f[4], f[5]);
      unpack2<SRC_DT>(x[k].w, f[6], f[7]);
      bool nonfinite;
      const float scale = fp8_row_scale<R, VEC>(f, nonfinite);  // every lane of the row takes part
      if (nonfinite && ok && lane == 0 && p.status) atomicOr(p.status, kStatusNonFiniteRow);
      uint32_t packed[2];
      fp8_quantize<VEC>(f, scale, packed);
      if (ok) {
        uint8_t* dst = static_cast<uint8_t*>(which == 0 ? p.cache.k : p.cache.v) + row + lane * VEC;
        *reinterpret_cast<uint2*>(dst) = make_uint2(packed[0], packed[1]);
        if (lane == 0) (which == 0 ? p.cache.k_scale : p.cache.v_scale)[srow] = scale;
      }
    } else {
      static_assert(KV_DT == SRC_DT, "16-bit caches store the incoming rows bit for bit");
      if (ok) {
        uint16_t* dst = static_cast<uint16_t*>(which == 0 ? p.cache.k : p.cache.v) + row + lane * VEC;
        *reinterpret_cast<uint4*>(dst) = x[k];
      }
    }
  }
  if (gridDim.x == 1) {
    __syncthreads();  // every wave has read positions[b] (which seq_lens_out may alias)
    if (tid == 0 && p.seq_lens_out) p.seq_lens_out[b] = pos + p.n_new;
  }
}

// seq_lens_out[b] = positions[b] + n_new, after a multi-workgroup append (positions may alias seq_lens_out).
__global__ __launch_bounds__(kBlockThreads) void bump_lens_kernel(const int32_t* positions, int32_t* seq_lens_out,
                                                                  int32_t n_new, int32_t batch) {
  const int b = blockIdx.x * kBlockThreads + threadIdx.x;
  if (b < batch) seq_lens_out[b] = positions[b] + n_new;
}

}  // namespace aicas
