// Device block allocator for paged KV caches: a stack of free block ids in device memory, handed out to the
// pages an append is about to touch and taken back when a sequence is released, written into the same int32
// block table [B, width] that the append and decode kernels read.
//
// Replaces the reference's page-table growth in Python (new KV cache/evaluation_wrapper.py:141-190: a list of
// {"logical_page_id", "block_id"} dicts per layer, grown by list.append as pages fill, never reused before a
// reset). Here allocation and release are kernels on the caller's stream, so a decode step that allocates its
// next page still needs no host synchronisation and can be captured in a HIP graph.
//
// Both kernels run as a single workgroup that walks the batch in tiles of kPoolThreads sequences with a
// workgroup-wide scan, so the result is the sequential one, in sequence order: sequence b's missing pages, in
// page order, pop the next free ids from the top of the stack (alloc); sequence b's blocks, in page order, are
// pushed onto it (free). No atomics, and a reproducible table.
#pragma once

#include "common.hpp"

namespace aicas {

constexpr int kPoolThreads = 1024;

struct BlockPoolParams {
  int32_t* free_blocks;  // [num_blocks] stack; entries [0, *free_count) are free, the top is the last
  int32_t* free_count;   // [1]
  int32_t num_blocks;
  int32_t* table;        // [batch, width] block table (-1: no block)
  int64_t stride;        // elements between rows
  int32_t width;
  int32_t batch;
  // alloc
  const int32_t* positions;  // first token of the append, per sequence
  int32_t n_new;             // tokens appended per sequence (>= 1)
  int32_t page_shift;        // log2(page_size)
  // free
  const int32_t* release;    // [batch] nonzero: release this sequence
  int32_t* seq_lens;         // [batch] set to 0 for released sequences (may be nullptr)
  int32_t* status;           // may be nullptr
};

// Exclusive scan of v over the workgroup (kPoolThreads threads, every thread calls it); total = sum of all.
__device__ __forceinline__ int pool_exclusive_scan(int v, int& total) {
  constexpr int kWaves = kPoolThreads / kWave;
  __shared__ int s_wave[kWaves];
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  int x = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  if (lane == kWave - 1) s_wave[wave] = x;
  __syncthreads();
  if (wave == 0) {
    int w = lane < kWaves ? s_wave[lane] : 0;
#pragma unroll
    for (int off = 1; off < kWaves; off <<= 1) {
      const int y = __shfl_up(w, off);
      if (lane >= off) w += y;
    }
    if (lane < kWaves) s_wave[lane] = w;
  }
  __syncthreads();
  const int before = wave > 0 ? s_wave[wave - 1] : 0;
  total = s_wave[kWaves - 1];
  __syncthreads();  // s_wave is reused by the next call
  return before + x - v;
}

// Fills the stack so that pops hand out blocks 0, 1, 2, ... in that order.
__global__ __launch_bounds__(kPoolThreads) void block_pool_init_kernel(int32_t* free_blocks, int32_t* free_count,
                                                                       int32_t num_blocks) {
  for (int i = blockIdx.x * kPoolThreads + threadIdx.x; i < num_blocks; i += gridDim.x * kPoolThreads)
    free_blocks[i] = num_blocks - 1 - i;
  if (blockIdx.x == 0 && threadIdx.x == 0) *free_count = num_blocks;
}

// Every page that tokens [positions[b], positions[b] + n_new) of sequence b touch gets a block if its table entry
// is negative. Pages past the row's width set AICAS_STATUS_APPEND_OVERFLOW; an empty stack leaves the entry at -1
// and sets AICAS_STATUS_OUT_OF_BLOCKS (the append then drops those rows, as for any invalid entry).
__global__ __launch_bounds__(kPoolThreads) void block_alloc_kernel(BlockPoolParams p) {
  __shared__ int s_top;
  const int tid = threadIdx.x;
  if (tid == 0) s_top = min(max(*p.free_count, 0), p.num_blocks);
  __syncthreads();
  for (int t0 = 0; t0 < p.batch; t0 += kPoolThreads) {
    const int b = t0 + tid;
    int first = 0, last = -1, need = 0;
    int32_t* row = nullptr;
    if (b < p.batch) {
      row = p.table + static_cast<int64_t>(b) * p.stride;
      const int pos = max(p.positions[b], 0);
      first = pos >> p.page_shift;
      last = (pos + p.n_new - 1) >> p.page_shift;
      if (last >= p.width) {
        if (p.status) atomicOr(p.status, kStatusAppendOverflow);
        last = p.width - 1;
      }
      for (int pg = first; pg <= last; ++pg) need += row[pg] < 0 ? 1 : 0;
    }
    int total;
    const int off = pool_exclusive_scan(need, total);
    const int top = s_top;
    if (need > 0) {
      int k = 0;
      bool short_of_blocks = false;
      for (int pg = first; pg <= last; ++pg) {
        if (row[pg] < 0) {
          const int idx = top - 1 - (off + k);
          if (idx >= 0) {
            row[pg] = p.free_blocks[idx];
          } else {
            short_of_blocks = true;
          }
          ++k;
        }
      }
      if (short_of_blocks && p.status) atomicOr(p.status, kStatusOutOfBlocks);
    }
    __syncthreads();
    if (tid == 0) s_top = max(top - total, 0);
    __syncthreads();
  }
  if (tid == 0) *p.free_count = s_top;
}

// Every sequence with release[b] != 0 gives its blocks (valid entries, in page order) back to the stack; its row
// becomes all -1 and its length 0. Ids outside [0, num_blocks) are dropped (AICAS_STATUS_BLOCK_OUT_OF_RANGE), and
// so is anything that would overfill the stack (a block released twice).
__global__ __launch_bounds__(kPoolThreads) void block_free_kernel(BlockPoolParams p) {
  __shared__ int s_top;
  const int tid = threadIdx.x;
  if (tid == 0) s_top = min(max(*p.free_count, 0), p.num_blocks);
  __syncthreads();
  for (int t0 = 0; t0 < p.batch; t0 += kPoolThreads) {
    const int b = t0 + tid;
    const bool rel = b < p.batch && p.release[b] != 0;
    int32_t* row = rel ? p.table + static_cast<int64_t>(b) * p.stride : nullptr;
    int cnt = 0;
    if (rel) {
      for (int pg = 0; pg < p.width; ++pg) cnt += (row[pg] >= 0 && row[pg] < p.num_blocks) ? 1 : 0;
    }
    int total;
    const int off = pool_exclusive_scan(cnt, total);
    const int top = s_top;
    if (rel) {
      int k = 0;
      bool bad = false;
      for (int pg = 0; pg < p.width; ++pg) {
        const int32_t e = row[pg];
        if (e >= 0 && e < p.num_blocks) {
          const int idx = top + off + k;
          if (idx < p.num_blocks) {
            p.free_blocks[idx] = e;
          } else {
            bad = true;
          }
          ++k;
        } else if (e >= p.num_blocks) {
          bad = true;
        }
        row[pg] = -1;
      }
      if (p.seq_lens) p.seq_lens[b] = 0;
      if (bad && p.status) atomicOr(p.status, kStatusBlockOutOfRange);
    }
    __syncthreads();
    if (tid == 0) s_top = min(top + total, p.num_blocks);
    __syncthreads();
  }
  if (tid == 0) *p.free_count = s_top;
}

}  // namespace aicas
