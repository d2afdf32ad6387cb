// C ABI of libaicas_decode.so: argument checking, launch planning and kernel dispatch.
// The declarations and their reference counterparts are in include/aicas_decode.h.

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <mutex>

#include "aicas_decode.h"
#include "block_pool.hpp"
#include "decode_attn.hpp"
#include "kv_append.hpp"
#include "kv_gather.hpp"

// Decode launchers, one translation unit per (q dtype, kv dtype) pair (decode_<q>_<kv>.hip); they return
// nonzero for a head_dim / group size that is not instantiated.
int launch_decode_bf16_bf16(const aicas::DecodeParams&, int, int, bool, bool, bool, dim3, hipStream_t);
int launch_decode_fp16_fp16(const aicas::DecodeParams&, int, int, bool, bool, bool, dim3, hipStream_t);
int launch_decode_bf16_fp8(const aicas::DecodeParams&, int, int, bool, bool, bool, dim3, hipStream_t);
int launch_decode_fp16_fp8(const aicas::DecodeParams&, int, int, bool, bool, bool, dim3, hipStream_t);

namespace {

thread_local char g_last_error[512] = "";


int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_last_error[0] = '\0';
  return AICAS_OK;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(AICAS_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return ok();
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Byte range [lo, hi) spanned by a [n0, n1, d] 16-bit tensor with element strides s0, s1 (non-negative) and a
// unit last stride.
struct Extent {
  uintptr_t lo, hi;
};
Extent extent16(const void* p, int64_t n0, int64_t s0, int64_t n1, int64_t s1, int64_t d) {
  const uintptr_t lo = reinterpret_cast<uintptr_t>(p);
  const int64_t last = (n0 - 1) * s0 + (n1 - 1) * s1 + d;
  return {lo, lo + static_cast<uintptr_t>(std::max<int64_t>(last, 0)) * 2};
}
bool overlaps(const Extent& a, const Extent& b) { return a.lo < b.hi && b.lo < a.hi; }
bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }
int ilog2(int64_t x) {
  int s = 0;
  while ((int64_t{1} << s) < x) ++s;
  return s;
}
int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

int elem_bytes(int32_t dt) { return dt == AICAS_DTYPE_FP8_E4M3 ? 1 : 2; }
bool valid_dtype(int32_t dt) { return dt == AICAS_DTYPE_BF16 || dt == AICAS_DTYPE_FP16 || dt == AICAS_DTYPE_FP8_E4M3; }
bool valid_head_dim(int32_t d) { return d == 16 || d == 32 || d == 64 || d == 128; }

// Tokens one workgroup chunk covers, and the rows one workgroup load covers (the kernel's own constants).
int tokens_per_iteration(int32_t kv_dtype, int32_t head_dim) {
  if (kv_dtype == AICAS_DTYPE_FP8_E4M3) return aicas::KVTraits<aicas::kFP8E4M3>::tokens_per_chunk(head_dim);
  return aicas::KVTraits<aicas::kBF16>::tokens_per_chunk(head_dim);
}
int rows_per_load(int32_t kv_dtype, int32_t head_dim) {
  return tokens_per_iteration(kv_dtype, head_dim) / aicas::KVTraits<aicas::kBF16>::kUnroll;
}

// Compute units of the current device (queried once per device; 256 on MI355X).
int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Checks shared by append and decode; fills the device-side layout.
int make_layout(const aicas_kv_cache_t* c, int32_t batch, int32_t num_kv_heads, int32_t head_dim,
                aicas::KVLayout& out) {
  if (!c) return fail(AICAS_ERR_INVALID, "cache descriptor is NULL");
  if (!c->k || !c->v) return fail(AICAS_ERR_INVALID, "cache K/V pointers must be non-NULL");
  if (!valid_dtype(c->kv_dtype)) return fail(AICAS_ERR_UNSUPPORTED, "unknown kv_dtype %d", c->kv_dtype);
  if (!aligned16(c->k) || !aligned16(c->v)) return fail(AICAS_ERR_INVALID, "cache K/V must be 16-byte aligned");
  const int eb = elem_bytes(c->kv_dtype);
  if ((c->stride_blk * eb) % 16 || (c->stride_h * eb) % 16 || (c->stride_t * eb) % 16)
    return fail(AICAS_ERR_INVALID, "cache strides must be multiples of 16 bytes (got %lld, %lld, %lld elements)",
                (long long)c->stride_blk, (long long)c->stride_h, (long long)c->stride_t);
  if (c->stride_t < head_dim) return fail(AICAS_ERR_INVALID, "cache token stride %lld < head_dim %d",
                                          (long long)c->stride_t, head_dim);
  if (c->page_size <= 0) return fail(AICAS_ERR_INVALID, "page_size must be positive");
  if (c->kv_dtype == AICAS_DTYPE_FP8_E4M3 && (!c->k_scale || !c->v_scale))
    return fail(AICAS_ERR_INVALID, "fp8 caches need k_scale and v_scale");
  out.k = c->k;
  out.v = c->v;
  out.k_scale = c->k_scale;
  out.v_scale = c->v_scale;
  out.stride_blk = c->stride_blk;
  out.stride_h = c->stride_h;
  out.stride_t = c->stride_t;
  out.scale_stride_blk = c->scale_stride_blk;
  out.scale_stride_h = c->scale_stride_h;
  out.page_size = c->page_size;
  if (c->block_table) {
    if (!is_pow2(c->page_size)) return fail(AICAS_ERR_INVALID, "paged caches need a power-of-two page_size");
    if (c->block_table_stride <= 0 || c->num_blocks <= 0)
      return fail(AICAS_ERR_INVALID, "paged caches need block_table_stride > 0 and num_blocks > 0");
    const int64_t mt = c->block_table_stride * c->page_size;
    out.block_table = c->block_table;
    out.block_table_stride = c->block_table_stride;
    out.num_blocks = c->num_blocks;
    out.max_tokens = static_cast<int32_t>(mt > INT32_MAX ? INT32_MAX : mt);
  } else {
    out.block_table = nullptr;
    out.block_table_stride = 0;
    out.num_blocks = batch;
    out.max_tokens = c->page_size;
  }
  (void)num_kv_heads;
  return AICAS_OK;
}

// ---------------------------------------------------------------------------------------------------------
// Dispatch tables.

// Grid (row blocks, sequences). With more than one row block per sequence the length bump is a second launch
// (the append kernel only bumps in place when one workgroup owns the sequence).
template <int SRC, int KV>
int launch_append_d(const aicas::AppendParams& p, int32_t batch, int32_t head_dim, hipStream_t s) {
  // the kernel indexes a sequence's rows with 31-bit integers
  const int64_t rows = 2 * int64_t{p.num_kv_heads} * p.n_new;
  if (rows > INT32_MAX) return fail(AICAS_ERR_UNSUPPORTED, "too many rows (%lld) in one append", (long long)rows);
  const int64_t blocks = ceil_div(rows, aicas::append_rows_per_workgroup(head_dim));
  const dim3 grid(static_cast<uint32_t>(blocks), batch), block(aicas::kBlockThreads);
  switch (head_dim) {
    case 16: hipLaunchKernelGGL((aicas::kv_append_kernel<SRC, KV, 16>), grid, block, 0, s, p); break;
    case 32: hipLaunchKernelGGL((aicas::kv_append_kernel<SRC, KV, 32>), grid, block, 0, s, p); break;
    case 64: hipLaunchKernelGGL((aicas::kv_append_kernel<SRC, KV, 64>), grid, block, 0, s, p); break;
    case 128: hipLaunchKernelGGL((aicas::kv_append_kernel<SRC, KV, 128>), grid, block, 0, s, p); break;
    default: return fail(AICAS_ERR_UNSUPPORTED, "head_dim %d not supported", head_dim);
  }
  if (blocks > 1 && p.seq_lens_out) {
    hipLaunchKernelGGL(aicas::bump_lens_kernel, dim3(ceil_div(batch, aicas::kBlockThreads)),
                       dim3(aicas::kBlockThreads), 0, s, p.positions, p.seq_lens_out, p.n_new, batch);
  }
  return check_launch("aicas_kv_append");
}

template <int KV, int OUT>
int launch_gather_d(const aicas::GatherParams& p, int32_t batch, int32_t head_dim, hipStream_t s) {
  const int64_t blocks = ceil_div(p.out_len, aicas::gather_rows_per_workgroup(head_dim));
  const dim3 grid(static_cast<uint32_t>(blocks), p.num_kv_heads, batch), block(aicas::kBlockThreads);
  switch (head_dim) {
    case 16: hipLaunchKernelGGL((aicas::kv_gather_kernel<KV, OUT, 16>), grid, block, 0, s, p); break;
    case 32: hipLaunchKernelGGL((aicas::kv_gather_kernel<KV, OUT, 32>), grid, block, 0, s, p); break;
    case 64: hipLaunchKernelGGL((aicas::kv_gather_kernel<KV, OUT, 64>), grid, block, 0, s, p); break;
    case 128: hipLaunchKernelGGL((aicas::kv_gather_kernel<KV, OUT, 128>), grid, block, 0, s, p); break;
    default: return fail(AICAS_ERR_UNSUPPORTED, "head_dim %d not supported", head_dim);
  }
  return check_launch("aicas_kv_gather");
}

template <bool APPEND>
int launch_decode(const aicas::DecodeParams& p, int q_dtype, int kv_dtype, int d, int g, bool paged, bool qk,
                  dim3 grid, hipStream_t s) {
  using namespace aicas;
  int rc;
  if (q_dtype == kBF16) {
    rc = kv_dtype == kFP8E4M3 ? launch_decode_bf16_fp8(p, d, g, paged, APPEND, qk, grid, s)
                              : launch_decode_bf16_bf16(p, d, g, paged, APPEND, qk, grid, s);
  } else {
    rc = kv_dtype == kFP8E4M3 ? launch_decode_fp16_fp8(p, d, g, paged, APPEND, qk, grid, s)
                              : launch_decode_fp16_fp16(p, d, g, paged, APPEND, qk, grid, s);
  }
  if (rc) return fail(AICAS_ERR_UNSUPPORTED, "head_dim %d / GQA group size %d not supported", d, g);
  return check_launch(APPEND ? "aicas_decode_attention_append" : "aicas_decode_attention");
}

// Workgroups per compute unit the split planner aims for, in quarters. Measured on MI355X (256 CUs), µs per
// launch: B=8 L=2048 (64 (batch, kv head) pairs) 19.4 / 17.1 / 17.4 / 20.7 / 18.4 / 17.4 / 18.2 for 2 / 3 / 4 /
// 5 / 6 / 7 / 8 splits per pair; B=1 L=32768 (8 pairs) 35.0 / 33.8 / 33.7 / 33.6 / 33.3 / 41.4 / 34.4 / 39.8 for
// 17 / 20 / 24 / 28 / 31 / 33 / 56 / 65 splits; ragged B=32 paged fp8 (256 pairs) 86.8 / 80.9 / 91.3 for 1 / 2 / 4.
// With few pairs: about 7/8 of a workgroup per CU and never more than one (a few CUs holding two workgroups
// make the tail: 264 and 320 workgroups are the slow cases above). With the cache rows loaded non-temporal,
// B=8 L=2048 takes 446.7 us/step at 4 splits against 450.5 at 3, and B=1 L=32768 29.0 / 29.5 / 30.4 / 38.1 us
// at 24 / 29 / 32 / 33 splits. With many pairs (batches of ragged lengths): 7/4, so that the longest sequences
// are split. (Both in eighths.)
constexpr int kFewPairsWGsPerCUx8 = 7;
constexpr int kManyPairsWGsPerCUx8 = 14;

// Workspace layout. The counters sit at fixed offsets, the same for every launch shape, ahead of the
// partials: they are zero between launches whatever shapes ran before on the same workspace, since no launch
// ever stores partials there. A launch may cover at most kMaxPairs (batch row, kv head) pairs.
constexpr int64_t kMaxPairs = 65536;
constexpr size_t kCounterBytes = kMaxPairs * sizeof(int32_t);
constexpr size_t kArrivalOff = 0;                  // [pairs] split arrivals
constexpr size_t kBatchArriveOff = kCounterBytes;  // [batch] readers of positions[b]
constexpr size_t kPartialsOff = 2 * kCounterBytes;

struct Plan {
  int32_t tokens_per_split;  // a sequence of L tokens takes min(num_splits, ceil(L / tokens_per_split)) splits
  int32_t num_splits;
  int32_t len_limit;  // longest sequence the launch can attend in full (paged caches: LDS block-id cache)
  bool many_pairs;    // more (batch row, kv head) pairs than 3/4 of the compute units: a ragged batch's shape
  size_t ml_off, acc_off, bytes;
};

int plan(int32_t kv_dtype, int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
         int32_t max_seq_len, int32_t page_size, int32_t hint, Plan& pl) {
  if (!valid_dtype(kv_dtype)) return fail(AICAS_ERR_UNSUPPORTED, "unknown kv_dtype %d", kv_dtype);
  if (!valid_head_dim(head_dim)) return fail(AICAS_ERR_UNSUPPORTED, "head_dim %d not supported", head_dim);
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || max_seq_len < 0)
    return fail(AICAS_ERR_INVALID, "batch/heads must be positive and max_seq_len non-negative");
  if (int64_t{batch} * num_kv_heads > kMaxPairs)
    return fail(AICAS_ERR_UNSUPPORTED, "batch * num_kv_heads = %lld exceeds %lld", (long long)batch * num_kv_heads,
                (long long)kMaxPairs);
  const int tpi = tokens_per_iteration(kv_dtype, head_dim);
  const int rpb = rows_per_load(kv_dtype, head_dim);
  const int64_t bound = max_seq_len > 0 ? max_seq_len : 1;
  // A split streaming a static range (paged rows too long for the LDS block-id cache) may touch at most
  // kMaxBlockEntries block-table entries: at most `cap` tokens per split.
  const int64_t cap = page_size > 0 ? (int64_t{aicas::kMaxBlockEntries} - 2) * page_size / tpi * tpi : 0;
  int64_t tps, splits;
  const int64_t pairs = int64_t{batch} * num_kv_heads;
  const int64_t cus = device_cus();
  const bool few = pairs * 4 <= 3 * cus;  // at most 3/4 of a pair per CU
  pl.many_pairs = !few;
  if (hint > 0) {
    tps = ceil_div(hint, rpb) * rpb;
    if (cap >= tpi && tps > cap) tps = cap;
    splits = ceil_div(bound, tps);
  } else {
    // Split count: the workgroups per compute unit above, in total. A split covers at least one super-chunk
    // (two chunks) per wave: below that its merge costs more than its streaming saves (B=1 L=1024: 17 splits
    // 9.19 us, 9 splits 8.02 us).
    const int64_t target = int64_t{few ? kFewPairsWGsPerCUx8 : kManyPairsWGsPerCUx8} * cus / 8;
    int64_t splits_wanted = std::max<int64_t>(1, (target + pairs / 2) / pairs);
    if (few) {
      // Few pairs (uniform batches, one long sequence): every sequence long enough is spread over the same
      // number of splits whatever the bound, and each takes min(splits, ceil(L / minimum split)) from its own
      // length: a launch sized for a loose bound (a graph captured at the cache capacity) runs the grid a tight
      // bound would give.
      // At most 4 pairs (one or two sequences with few kv heads): 64 splits per pair, one workgroup per CU at 4
      // pairs; more splits make the many-way merge the cost, fewer leave CUs idle. Measured on MI355X, bf16,
      // D=128, us per launch, plan (7/8 per CU) against 64: 1 pair L=32768 15.4 (224) / 11.4, L=16384 10.5
      // (128) / 9.1; 2 pairs L=16384 11.4 (112) / 9.5; 4 pairs L=32768 16.3 (56) / 15.8, L=8192 9.6 / 9.0.
      splits_wanted = pairs <= 4 ? std::min<int64_t>(64, cus / pairs) : std::min(splits_wanted, cus / pairs);
      splits_wanted = std::max<int64_t>(1, splits_wanted);
      tps = 2 * tpi;
      splits = std::min(splits_wanted, ceil_div(bound, tps));
      if (cap >= tpi) splits = std::max(splits, ceil_div(bound, cap));
    } else {
      // Many pairs (ragged batches): splits in proportion to the length, so that the longest sequences split.
      tps = ceil_div(bound, splits_wanted);
      tps = ceil_div(tps, rpb) * rpb;
      if (tps < 2 * tpi) tps = 2 * tpi;
      if (cap >= tpi && tps > cap) tps = cap;
      splits = ceil_div(bound, tps);
    }
  }
  if (tps > (int64_t{1} << 30)) tps = int64_t{1} << 30;
  if (splits > 65535) return fail(AICAS_ERR_UNSUPPORTED, "too many splits (%lld)", (long long)splits);
  pl.tokens_per_split = static_cast<int32_t>(tps);
  pl.num_splits = static_cast<int32_t>(splits);
  const int64_t lim = cap >= tpi ? cap * splits : int64_t{INT32_MAX};
  pl.len_limit = static_cast<int32_t>(std::min<int64_t>(lim, INT32_MAX));
  const size_t parts = size_t(batch) * num_q_heads * splits;
  pl.ml_off = kPartialsOff;
  pl.acc_off = pl.ml_off + align_up(parts * 2 * sizeof(float), 256);
  pl.bytes = pl.acc_off + align_up(parts * head_dim * sizeof(float), 256);
  return AICAS_OK;
}


struct DecodeCall {
  const aicas_kv_cache_t* cache;
  int32_t q_dtype;
  const void* q;
  int64_t q_stride_b, q_stride_h;
  void* out;
  int64_t out_stride_b, out_stride_h;
  const int32_t* lens;
  int32_t uniform_len;
  int32_t bound;
  int32_t min_attended;  // caller's lower bound on every attended length (0: none)
  int32_t batch, num_q_heads, num_kv_heads, head_dim;
  float sm_scale;
  int32_t tokens_per_split;
  void* workspace;
  size_t workspace_bytes;
  int32_t* status;
  const void* k_new;
  const void* v_new;
  int64_t kn_stride_b, kn_stride_h, vn_stride_b, vn_stride_h;
  int32_t* seq_lens_out;
  const aicas_qk_prologue_t* pro;  // APPEND only; nullptr: q and the new rows are used as given
};

template <bool APPEND>
int run_decode(const DecodeCall& c, hipStream_t stream) {
  if (c.q_dtype != AICAS_DTYPE_BF16 && c.q_dtype != AICAS_DTYPE_FP16)
    return fail(AICAS_ERR_UNSUPPORTED, "q must be bf16 or fp16");
  if (!c.q || !c.out) return fail(AICAS_ERR_INVALID, "q and out must be non-NULL");
  if (!aligned16(c.q) || (c.q_stride_b % 8) || (c.q_stride_h % 8))
    return fail(AICAS_ERR_INVALID, "q must be 16-byte aligned with strides that are multiples of 8 elements");
  if ((reinterpret_cast<uintptr_t>(c.out) & 1u) != 0) return fail(AICAS_ERR_INVALID, "out must be 2-byte aligned");
  if (c.num_kv_heads <= 0 || c.num_q_heads % c.num_kv_heads != 0)
    return fail(AICAS_ERR_INVALID, "num_q_heads (%d) must be a multiple of num_kv_heads (%d)", c.num_q_heads,
                c.num_kv_heads);
  aicas::DecodeParams p{};
  int rc = make_layout(c.cache, c.batch, c.num_kv_heads, c.head_dim, p.cache);
  if (rc) return rc;
  if (c.cache->kv_dtype != AICAS_DTYPE_FP8_E4M3 && c.cache->kv_dtype != c.q_dtype)
    return fail(AICAS_ERR_UNSUPPORTED, "a 16-bit cache must have the dtype of q");
  Plan pl{};
  rc = plan(c.cache->kv_dtype, c.batch, c.num_q_heads, c.num_kv_heads, c.head_dim, c.bound,
            c.cache->block_table ? c.cache->page_size : 0, c.tokens_per_split, pl);
  if (rc) return rc;
  if (!c.workspace) return fail(AICAS_ERR_WORKSPACE, "workspace is NULL (%zu bytes needed)", pl.bytes);
  if (c.workspace_bytes < pl.bytes)
    return fail(AICAS_ERR_WORKSPACE, "workspace has %zu bytes, %zu needed", c.workspace_bytes, pl.bytes);
  if (!aligned16(c.workspace)) return fail(AICAS_ERR_INVALID, "workspace must be 16-byte aligned");
  char* ws = static_cast<char*>(c.workspace);
  p.q = c.q;
  p.q_stride_b = c.q_stride_b;
  p.q_stride_h = c.q_stride_h;
  p.out = c.out;
  p.out_stride_b = c.out_stride_b;
  p.out_stride_h = c.out_stride_h;
  p.seq_lens = c.lens;
  p.uniform_len = c.uniform_len;
  p.num_q_heads = c.num_q_heads;
  p.num_kv_heads = c.num_kv_heads;
  p.tokens_per_split = pl.tokens_per_split;
  p.max_splits = pl.num_splits;
  p.len_limit = pl.len_limit;
  // Splits that every sequence keeps busy by the caller's lower bound: they may fetch their first rows before
  // reading the length. A wrong bound only costs bandwidth: the rows' validity always comes from the length.
  p.spec_splits = c.min_attended > 0
                      ? static_cast<int32_t>(std::min<int64_t>(pl.num_splits,
                                                                ceil_div(int64_t{c.min_attended}, pl.tokens_per_split)))
                      : 0;
  p.page_shift = c.cache->block_table ? ilog2(c.cache->page_size) : 0;
  p.scale_log2 = c.sm_scale * 1.4426950408889634f;
  p.ws_counter = reinterpret_cast<int32_t*>(ws + kArrivalOff);
  // The splits of a pair count in on the pair's arrival counter. Launches of at most 32 pairs give each pair's
  // counter a 128-byte line of its own; more pairs keep them packed. Measured on MI355X, padded against packed:
  // B=1 L=1024 (8 pairs, 9 splits) 6.97 against 7.19 us per launch, B=1 L=32768 (8 pairs, 28 splits) 29.6 both,
  // B=8 L=2048 (64 pairs, 4 splits) 442.0 against 440.5 us per 28-layer step, B=64 ragged 2930 against 2938.
  const int64_t pairs = int64_t{c.batch} * c.num_kv_heads;
  p.counter_stride = pairs <= 32 ? 32 : 1;
  p.ws_arrive = reinterpret_cast<int32_t*>(ws + kBatchArriveOff);
  // Every workgroup of a batch row counts itself in on that row's counter; counters sharing a cache line
  // serialise each other's atomics, so each row gets a 128-byte line of its own while the region allows.
  p.arrive_stride = static_cast<int32_t>(std::min<int64_t>(32, kMaxPairs / c.batch));
  // Ragged batches (many pairs, device lengths): rows dispatched in folded length order (longest first, each with
  // a short row half a grid later), so that workgroups sharing a compute unit carry about equal work. Measured on
  // MI355X with the rows ordered on the host, natural / decreasing / folded: B=32 paged fp8 U{256..8192} 75.2 /
  // 70.9 / 71.4 us per launch, B=64 bf16 U{512..4096} 28 layers 3165 / 3025 / 2875 us per step. The kernel ranks
  // the rows itself, one thread per row.
  p.order_rows = (pl.many_pairs && c.lens && c.batch > 1 && c.batch <= aicas::kBlockThreads) ? 1 : 0;
  p.ws_ml = reinterpret_cast<float*>(ws + pl.ml_off);
  p.ws_acc = reinterpret_cast<float*>(ws + pl.acc_off);
  p.status = c.status;
  p.k_new = c.k_new;
  p.v_new = c.v_new;
  p.kn_stride_b = c.kn_stride_b;
  p.kn_stride_h = c.kn_stride_h;
  p.vn_stride_b = c.vn_stride_b;
  p.vn_stride_h = c.vn_stride_h;
  p.seq_lens_out = c.seq_lens_out;
  if (APPEND && c.pro) {
    const aicas_qk_prologue_t& pro = *c.pro;
    const bool norm = pro.q_norm_weight || pro.k_norm_weight;
    if ((pro.q_norm_weight && !aligned16(pro.q_norm_weight)) || (pro.k_norm_weight && !aligned16(pro.k_norm_weight)))
      return fail(AICAS_ERR_INVALID, "norm weights must be 16-byte aligned");
    if (norm && !(pro.eps >= 0.0f)) return fail(AICAS_ERR_INVALID, "eps must be >= 0");
    if ((pro.cos == nullptr) != (pro.sin == nullptr)) return fail(AICAS_ERR_INVALID, "give both cos and sin, or neither");
    if (pro.cos && (!aligned16(pro.cos) || !aligned16(pro.sin) || (pro.cos_stride_b % 8) || (pro.sin_stride_b % 8)))
      return fail(AICAS_ERR_INVALID, "cos/sin rows must be 16-byte aligned with strides that are multiples of 8");
    if (pro.q_out && (!aligned16(pro.q_out) || (pro.q_out_stride_b % 8) || (pro.q_out_stride_h % 8)))
      return fail(AICAS_ERR_INVALID, "q_out must be 16-byte aligned with strides that are multiples of 8");
    if (pro.q_out) {
      // q_out is written once every workgroup of its (batch row, kv head) has read q and the new rows: it may
      // be q itself, but no other overlap with q or with k_new is allowed
      const Extent qo = extent16(pro.q_out, c.batch, pro.q_out_stride_b, c.num_q_heads, pro.q_out_stride_h,
                                 c.head_dim);
      const Extent qi = extent16(c.q, c.batch, c.q_stride_b, c.num_q_heads, c.q_stride_h, c.head_dim);
      const Extent kn = extent16(c.k_new, c.batch, c.kn_stride_b, c.num_kv_heads, c.kn_stride_h, c.head_dim);
      const bool same_as_q = pro.q_out == c.q && pro.q_out_stride_b == c.q_stride_b && pro.q_out_stride_h == c.q_stride_h;
      if ((!same_as_q && overlaps(qo, qi)) || overlaps(qo, kn))
        return fail(AICAS_ERR_INVALID, "q_out may be q itself but must not otherwise overlap q or k_new");
    }
    p.q_norm_w = pro.q_norm_weight;
    p.k_norm_w = pro.k_norm_weight;
    p.norm_eps = pro.eps;
    p.rope_cos = pro.cos;
    p.rope_sin = pro.sin;
    p.rope_cos_stride_b = pro.cos_stride_b;
    p.rope_sin_stride_b = pro.sin_stride_b;
    p.q_out = pro.q_out;
    p.q_out_stride_b = pro.q_out_stride_b;
    p.q_out_stride_h = pro.q_out_stride_h;
  }
  // the q/k prologue variant runs when there is anything for it to do
  const bool qk = APPEND && c.pro && (p.q_norm_w || p.k_norm_w || p.rope_cos || p.q_out);
  const int g = c.num_q_heads / c.num_kv_heads;
  const dim3 grid(pl.num_splits, c.num_kv_heads, c.batch);
  return launch_decode<APPEND>(p, c.q_dtype, c.cache->kv_dtype, c.head_dim, g, c.cache->block_table != nullptr, qk,
                               grid, stream);
}

int decode_append(const aicas_kv_cache_t* cache, const aicas_qk_prologue_t* pro, int32_t q_dtype, const void* q,
                                  int64_t q_stride_b, int64_t q_stride_h, const void* k_new, int64_t k_stride_b,
                                  int64_t k_stride_h, const void* v_new, int64_t v_stride_b, int64_t v_stride_h,
                                  void* out, int64_t out_stride_b, int64_t out_stride_h, const int32_t* positions,
                                  int32_t* seq_lens_out, int32_t min_len, int32_t max_seq_len, int32_t batch,
                                  int32_t num_q_heads,
                                  int32_t num_kv_heads, int32_t head_dim, float sm_scale, int32_t tokens_per_split,
                                  void* workspace, size_t workspace_bytes, int32_t* status, hipStream_t stream) {
  if (!positions) return fail(AICAS_ERR_INVALID, "positions must be non-NULL");
  if (!k_new || !v_new) return fail(AICAS_ERR_INVALID, "k_new and v_new must be non-NULL");
  if (!aligned16(k_new) || !aligned16(v_new) || (k_stride_b % 8) || (k_stride_h % 8) || (v_stride_b % 8) ||
      (v_stride_h % 8))
    return fail(AICAS_ERR_INVALID, "new K/V rows must be 16-byte aligned with strides that are multiples of 8");
  if (max_seq_len < 1) return fail(AICAS_ERR_INVALID, "max_seq_len must count the appended token");
  if (seq_lens_out && seq_lens_out != positions && batch > 0) {
    // the bump is stored once every reader of the lengths it replaces is done: only the same array is safe
    const auto pos = reinterpret_cast<uintptr_t>(positions);
    const auto out = reinterpret_cast<uintptr_t>(seq_lens_out);
    const uintptr_t bytes = static_cast<uintptr_t>(batch) * sizeof(int32_t);
    if (out < pos + bytes && pos < out + bytes)
      return fail(AICAS_ERR_INVALID, "seq_lens_out may be positions itself but must not otherwise overlap it");
  }
  DecodeCall c{};
  c.cache = cache;
  c.q_dtype = q_dtype;
  c.q = q;
  c.q_stride_b = q_stride_b;
  c.q_stride_h = q_stride_h;
  c.out = out;
  c.out_stride_b = out_stride_b;
  c.out_stride_h = out_stride_h;
  c.lens = positions;
  c.uniform_len = 0;
  c.min_attended = min_len > 0 ? min_len + 1 : 0;  // positions[b] >= min_len: the new token makes min_len + 1
  c.bound = max_seq_len;
  c.batch = batch;
  c.num_q_heads = num_q_heads;
  c.num_kv_heads = num_kv_heads;
  c.head_dim = head_dim;
  c.sm_scale = sm_scale;
  c.tokens_per_split = tokens_per_split;
  c.workspace = workspace;
  c.workspace_bytes = workspace_bytes;
  c.status = status;
  c.k_new = k_new;
  c.v_new = v_new;
  c.kn_stride_b = k_stride_b;
  c.kn_stride_h = k_stride_h;
  c.vn_stride_b = v_stride_b;
  c.vn_stride_h = v_stride_h;
  c.seq_lens_out = seq_lens_out;
  c.pro = pro;
  return run_decode<true>(c, stream);
}

// ---------------------------------------------------------------------------------------------------------
// Scratch of aicas_decode_attention_append_noalloc: the decode workspace (counters, then split partials) as
// static device memory of the library, one copy per device, held until the process ends. In host code the
// name `scratch` is only a host-side stand-in: the device address of each device's copy comes from
// hipGetSymbolAddress, called once per device with that device current, and only that address is ever
// handed to a kernel.
constexpr size_t kScratchBytes = size_t{4} << 20;
static_assert(kScratchBytes > kPartialsOff, "the scratch must hold the counters and some partials");
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// Clears n bytes (n a multiple of 16) with vector stores: a kernel rather than hipMemsetAsync, so that a
// graph capturing the first call records a kernel node.
__global__ void scratch_clear_kernel(uint4* p, size_t n16) {
  for (size_t i = blockIdx.x * size_t{blockDim.x} + threadIdx.x; i < n16; i += size_t{gridDim.x} * blockDim.x)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// The current device's scratch address. The first call on a device looks it up and clears the whole array
// on `stream` (the kernels then keep the counters and partial slots at their between-launch values).
int scratch_address(hipStream_t stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices)
    return fail(AICAS_ERR_INVALID, "no usable current HIP device (got %d)", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(AICAS_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
    hipLaunchKernelGGL(scratch_clear_kernel, dim3(256), dim3(256), 0, stream, static_cast<uint4*>(ptr),
                       kScratchBytes / 16);
    const int rc = check_launch("aicas_decode_attention_append_noalloc (scratch clear)");
    if (rc) return rc;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return AICAS_OK;
}

}  // namespace

extern "C" {

const char* aicas_last_error(void) { return g_last_error; }

int32_t aicas_abi_version(void) { return AICAS_ABI_VERSION; }

int aicas_kv_append(const aicas_kv_cache_t* cache, int32_t src_dtype, const void* k_src, int64_t k_stride_b,
                    int64_t k_stride_h, int64_t k_stride_t, const void* v_src, int64_t v_stride_b,
                    int64_t v_stride_h, int64_t v_stride_t, const int32_t* positions, int32_t* seq_lens_out,
                    int32_t* status, int32_t batch, int32_t num_kv_heads, int32_t head_dim, int32_t n_new,
                    hipStream_t stream) {
  if (batch <= 0 || num_kv_heads <= 0 || n_new <= 0)
    return fail(AICAS_ERR_INVALID, "batch, num_kv_heads and n_new must be positive");
  if (batch > 65535) return fail(AICAS_ERR_UNSUPPORTED, "batch %d exceeds 65535", batch);
  if (!valid_head_dim(head_dim)) return fail(AICAS_ERR_UNSUPPORTED, "head_dim %d not supported", head_dim);
  if (src_dtype != AICAS_DTYPE_BF16 && src_dtype != AICAS_DTYPE_FP16)
    return fail(AICAS_ERR_UNSUPPORTED, "new K/V rows must be bf16 or fp16");
  if (!k_src || !v_src || !positions) return fail(AICAS_ERR_INVALID, "k_src, v_src and positions must be non-NULL");
  if (!aligned16(k_src) || !aligned16(v_src)) return fail(AICAS_ERR_INVALID, "new K/V rows must be 16-byte aligned");
  if ((k_stride_b % 8) || (k_stride_h % 8) || (k_stride_t % 8) || (v_stride_b % 8) || (v_stride_h % 8) ||
      (v_stride_t % 8))
    return fail(AICAS_ERR_INVALID, "new K/V strides must be multiples of 8 elements");
  aicas::AppendParams p{};
  int rc = make_layout(cache, batch, num_kv_heads, head_dim, p.cache);
  if (rc) return rc;
  if (cache->kv_dtype != AICAS_DTYPE_FP8_E4M3 && cache->kv_dtype != src_dtype)
    return fail(AICAS_ERR_UNSUPPORTED, "a 16-bit cache must have the dtype of the new rows");
  // the kernel multiplies row indexes by 32-bit strides (the batch strides stay 64-bit)
  const int64_t row_strides[] = {k_stride_h, k_stride_t, v_stride_h, v_stride_t, cache->stride_blk, cache->stride_h,
                                 cache->stride_t, cache->k_scale ? cache->scale_stride_blk : 0,
                                 cache->k_scale ? cache->scale_stride_h : 0};
  for (const int64_t st : row_strides) {
    if (st < 0 || st > int64_t{UINT32_MAX})
      return fail(AICAS_ERR_UNSUPPORTED, "append strides must lie in [0, 2^32) elements (got %lld)", (long long)st);
  }
  p.k_src = k_src;
  p.v_src = v_src;
  p.k_src_stride_b = k_stride_b;
  p.v_src_stride_b = v_stride_b;
  p.src_stride_h[0] = static_cast<uint32_t>(k_stride_h);
  p.src_stride_t[0] = static_cast<uint32_t>(k_stride_t);
  p.src_stride_h[1] = static_cast<uint32_t>(v_stride_h);
  p.src_stride_t[1] = static_cast<uint32_t>(v_stride_t);
  p.dst_stride_blk = static_cast<uint32_t>(cache->stride_blk);
  p.dst_stride_h = static_cast<uint32_t>(cache->stride_h);
  p.dst_stride_t = static_cast<uint32_t>(cache->stride_t);
  p.scale_stride_blk = static_cast<uint32_t>(cache->k_scale ? cache->scale_stride_blk : 0);
  p.scale_stride_h = static_cast<uint32_t>(cache->k_scale ? cache->scale_stride_h : 0);
  p.positions = positions;
  p.seq_lens_out = seq_lens_out;
  p.status = status;
  p.num_kv_heads = num_kv_heads;
  p.n_new = n_new;
  p.div_n_new = aicas::fast_div_make(static_cast<uint32_t>(n_new));
  p.page_shift = cache->block_table ? ilog2(cache->page_size) : 0;
  using namespace aicas;
  if (src_dtype == kBF16) {
    if (cache->kv_dtype == kFP8E4M3) return launch_append_d<kBF16, kFP8E4M3>(p, batch, head_dim, stream);
    return launch_append_d<kBF16, kBF16>(p, batch, head_dim, stream);
  }
  if (cache->kv_dtype == kFP8E4M3) return launch_append_d<kFP16, kFP8E4M3>(p, batch, head_dim, stream);
  return launch_append_d<kFP16, kFP16>(p, batch, head_dim, stream);
}

int aicas_kv_gather(const aicas_kv_cache_t* cache, const int32_t* seq_lens, int32_t batch, int32_t num_kv_heads,
                    int32_t head_dim, int32_t out_dtype, void* k_out, void* v_out, int64_t out_stride_b,
                    int64_t out_stride_h, int64_t out_stride_t, int32_t out_len, int32_t* status,
                    hipStream_t stream) {
  if (batch <= 0 || num_kv_heads <= 0 || out_len < 0)
    return fail(AICAS_ERR_INVALID, "batch and num_kv_heads must be positive and out_len non-negative");
  if (batch > 65535 || num_kv_heads > 65535)
    return fail(AICAS_ERR_UNSUPPORTED, "batch %d / num_kv_heads %d exceed 65535", batch, num_kv_heads);
  if (!valid_head_dim(head_dim)) return fail(AICAS_ERR_UNSUPPORTED, "head_dim %d not supported", head_dim);
  if (out_dtype != AICAS_DTYPE_BF16 && out_dtype != AICAS_DTYPE_FP16)
    return fail(AICAS_ERR_UNSUPPORTED, "the gathered rows must be bf16 or fp16");
  if (!seq_lens || !k_out || !v_out) return fail(AICAS_ERR_INVALID, "seq_lens, k_out and v_out must be non-NULL");
  if (!aligned16(k_out) || !aligned16(v_out)) return fail(AICAS_ERR_INVALID, "k_out and v_out must be 16-byte aligned");
  if ((out_stride_b % 8) || (out_stride_h % 8) || (out_stride_t % 8) || out_stride_b < 0 || out_stride_h < 0 ||
      out_stride_t < head_dim)
    return fail(AICAS_ERR_INVALID, "output strides must be non-negative multiples of 8 elements, token stride >= head_dim");
  aicas::GatherParams p{};
  int rc = make_layout(cache, batch, num_kv_heads, head_dim, p.cache);
  if (rc) return rc;
  if (cache->kv_dtype != AICAS_DTYPE_FP8_E4M3 && cache->kv_dtype != out_dtype)
    return fail(AICAS_ERR_UNSUPPORTED, "a 16-bit cache is gathered into its own dtype");
  if (out_len == 0) return ok();
  // the outputs may overlap neither each other nor the cache they are read from
  auto span = [](const void* ptr, int64_t last_elem, int eb) -> Extent {
    const uintptr_t lo = reinterpret_cast<uintptr_t>(ptr);
    return {lo, lo + static_cast<uintptr_t>(last_elem) * eb};
  };
  const int64_t out_last = (batch - 1) * out_stride_b + (num_kv_heads - 1) * out_stride_h +
                           int64_t{out_len - 1} * out_stride_t + head_dim;
  const int64_t cache_last = (p.cache.num_blocks - 1) * cache->stride_blk + (num_kv_heads - 1) * cache->stride_h +
                             int64_t{cache->page_size - 1} * cache->stride_t + head_dim;
  const int eb = elem_bytes(cache->kv_dtype);
  const Extent ko = span(k_out, out_last, 2), vo = span(v_out, out_last, 2);
  const Extent kc = span(cache->k, cache_last, eb), vc = span(cache->v, cache_last, eb);
  if (overlaps(ko, vo) || overlaps(ko, kc) || overlaps(ko, vc) || overlaps(vo, kc) || overlaps(vo, vc))
    return fail(AICAS_ERR_INVALID, "k_out / v_out overlap each other or the cache");
  p.seq_lens = seq_lens;
  p.k_out = k_out;
  p.v_out = v_out;
  p.out_stride_b = out_stride_b;
  p.out_stride_h = out_stride_h;
  p.out_stride_t = out_stride_t;
  p.out_len = out_len;
  p.num_kv_heads = num_kv_heads;
  p.status = status;
  using namespace aicas;
  if (cache->kv_dtype == kFP8E4M3) {
    return out_dtype == kBF16 ? launch_gather_d<kFP8E4M3, kBF16>(p, batch, head_dim, stream)
                              : launch_gather_d<kFP8E4M3, kFP16>(p, batch, head_dim, stream);
  }
  return out_dtype == kBF16 ? launch_gather_d<kBF16, kBF16>(p, batch, head_dim, stream)
                            : launch_gather_d<kFP16, kFP16>(p, batch, head_dim, stream);
}

int aicas_decode_plan(int32_t kv_dtype, int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                      int32_t head_dim, int32_t max_seq_len, int32_t page_size, int32_t tokens_per_split_hint,
                      int32_t* tokens_per_split, int32_t* num_splits, size_t* workspace_bytes) {
  Plan pl{};
  const int rc = plan(kv_dtype, batch, num_q_heads, num_kv_heads, head_dim, max_seq_len, page_size,
                      tokens_per_split_hint, pl);
  if (rc) return rc;
  if (tokens_per_split) *tokens_per_split = pl.tokens_per_split;
  if (num_splits) *num_splits = pl.num_splits;
  if (workspace_bytes) *workspace_bytes = pl.bytes;
  return ok();
}

int aicas_decode_attention(const aicas_kv_cache_t* cache, int32_t q_dtype, const void* q, int64_t q_stride_b,
                           int64_t q_stride_h, void* out, int64_t out_stride_b, int64_t out_stride_h,
                           const int32_t* seq_lens, int32_t uniform_len, int32_t min_len, int32_t max_seq_len,
                           int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                           float sm_scale, int32_t tokens_per_split, void* workspace, size_t workspace_bytes,
                           int32_t* status, hipStream_t stream) {
  if (!seq_lens && uniform_len < 0) return fail(AICAS_ERR_INVALID, "uniform_len must be non-negative");
  DecodeCall c{};
  c.cache = cache;
  c.q_dtype = q_dtype;
  c.q = q;
  c.q_stride_b = q_stride_b;
  c.q_stride_h = q_stride_h;
  c.out = out;
  c.out_stride_b = out_stride_b;
  c.out_stride_h = out_stride_h;
  c.lens = seq_lens;
  c.uniform_len = uniform_len;
  c.min_attended = seq_lens ? (min_len > 0 ? min_len : 0) : uniform_len;
  c.bound = seq_lens ? max_seq_len : uniform_len;
  c.batch = batch;
  c.num_q_heads = num_q_heads;
  c.num_kv_heads = num_kv_heads;
  c.head_dim = head_dim;
  c.sm_scale = sm_scale;
  c.tokens_per_split = tokens_per_split;
  c.workspace = workspace;
  c.workspace_bytes = workspace_bytes;
  c.status = status;
  return run_decode<false>(c, stream);
}

int aicas_decode_attention_append(const aicas_kv_cache_t* cache, int32_t q_dtype, const void* q,
                                  int64_t q_stride_b, int64_t q_stride_h, const void* k_new, int64_t k_stride_b,
                                  int64_t k_stride_h, const void* v_new, int64_t v_stride_b, int64_t v_stride_h,
                                  void* out, int64_t out_stride_b, int64_t out_stride_h, const int32_t* positions,
                                  int32_t* seq_lens_out, int32_t min_len, int32_t max_seq_len, int32_t batch,
                                  int32_t num_q_heads,
                                  int32_t num_kv_heads, int32_t head_dim, float sm_scale, int32_t tokens_per_split,
                                  void* workspace, size_t workspace_bytes, int32_t* status, hipStream_t stream) {
  return decode_append(cache, nullptr, q_dtype, q, q_stride_b, q_stride_h, k_new, k_stride_b, k_stride_h, v_new,
                       v_stride_b, v_stride_h, out, out_stride_b, out_stride_h, positions, seq_lens_out, min_len,
                       max_seq_len, batch, num_q_heads, num_kv_heads, head_dim, sm_scale, tokens_per_split, workspace,
                       workspace_bytes, status, stream);
}

int aicas_decode_attention_append_noalloc(const aicas_kv_cache_t* cache, int32_t q_dtype, const void* q,
                                          int64_t q_stride_b, int64_t q_stride_h, const void* k_new,
                                          int64_t k_stride_b, int64_t k_stride_h, const void* v_new,
                                          int64_t v_stride_b, int64_t v_stride_h, void* out, int64_t out_stride_b,
                                          int64_t out_stride_h, const int32_t* positions, int32_t* seq_lens_out,
                                          int32_t min_len, int32_t max_seq_len, int32_t batch, int32_t num_q_heads,
                                          int32_t num_kv_heads, int32_t head_dim, float sm_scale,
                                          int32_t tokens_per_split, int32_t* status, hipStream_t stream) {
  // the launch's workspace size, checked against the scratch before anything touches the device
  if (!cache) return fail(AICAS_ERR_INVALID, "cache descriptor is NULL");
  Plan pl{};
  int rc = plan(cache->kv_dtype, batch, num_q_heads, num_kv_heads, head_dim, max_seq_len,
                cache->block_table ? cache->page_size : 0, tokens_per_split, pl);
  if (rc) return rc;
  if (pl.bytes > kScratchBytes)
    return fail(AICAS_ERR_WORKSPACE,
                "this launch needs a %zu-byte workspace; the library's static scratch holds %zu bytes "
                "(use aicas_decode_attention_append with a caller-allocated workspace)",
                pl.bytes, kScratchBytes);
  void* ws = nullptr;
  rc = scratch_address(stream, &ws);
  if (rc) return rc;
  return decode_append(cache, nullptr, q_dtype, q, q_stride_b, q_stride_h, k_new, k_stride_b, k_stride_h, v_new,
                       v_stride_b, v_stride_h, out, out_stride_b, out_stride_h, positions, seq_lens_out, min_len,
                       max_seq_len, batch, num_q_heads, num_kv_heads, head_dim, sm_scale, tokens_per_split, ws,
                       kScratchBytes, status, stream);
}

int aicas_decode_attention_append_qk(const aicas_kv_cache_t* cache, const aicas_qk_prologue_t* prologue,
                                     int32_t q_dtype, const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                     const void* k_new, int64_t k_stride_b, int64_t k_stride_h, const void* v_new,
                                     int64_t v_stride_b, int64_t v_stride_h, void* out, int64_t out_stride_b,
                                     int64_t out_stride_h, const int32_t* positions, int32_t* seq_lens_out,
                                     int32_t min_len, int32_t max_seq_len, int32_t batch, int32_t num_q_heads,
                                     int32_t num_kv_heads, int32_t head_dim, float sm_scale, int32_t tokens_per_split,
                                     void* workspace, size_t workspace_bytes, int32_t* status, hipStream_t stream) {
  if (!prologue) return fail(AICAS_ERR_INVALID, "prologue must be non-NULL");
  return decode_append(cache, prologue, q_dtype, q, q_stride_b, q_stride_h, k_new, k_stride_b, k_stride_h, v_new,
                       v_stride_b, v_stride_h, out, out_stride_b, out_stride_h, positions, seq_lens_out, min_len,
                       max_seq_len, batch, num_q_heads, num_kv_heads, head_dim, sm_scale, tokens_per_split, workspace,
                       workspace_bytes, status, stream);
}

namespace {
int check_pool(const aicas_block_pool_t* pool) {
  if (!pool || !pool->free_blocks || !pool->free_count) return fail(AICAS_ERR_INVALID, "block pool pointers must be non-NULL");
  if (pool->num_blocks <= 0) return fail(AICAS_ERR_INVALID, "num_blocks must be positive");
  return 0;
}
int check_table(const int32_t* table, int64_t stride, int32_t width) {
  if (!table) return fail(AICAS_ERR_INVALID, "block_table must be non-NULL");
  if (width <= 0 || stride < width) return fail(AICAS_ERR_INVALID, "block table width must be positive and <= its row stride");
  return 0;
}
}  // namespace

int aicas_block_pool_init(const aicas_block_pool_t* pool, hipStream_t stream) {
  int rc = check_pool(pool);
  if (rc) return rc;
  const int blocks = static_cast<int>(std::min<int64_t>(ceil_div(pool->num_blocks, aicas::kPoolThreads), 1024));
  hipLaunchKernelGGL(aicas::block_pool_init_kernel, dim3(blocks), dim3(aicas::kPoolThreads), 0, stream,
                     pool->free_blocks, pool->free_count, pool->num_blocks);
  return check_launch("aicas_block_pool_init");
}

int aicas_block_alloc(const aicas_block_pool_t* pool, int32_t* block_table, int64_t block_table_stride,
                      int32_t table_width, const int32_t* positions, int32_t n_new, int32_t batch, int32_t page_size,
                      int32_t* status, hipStream_t stream) {
  int rc = check_pool(pool);
  if (!rc) rc = check_table(block_table, block_table_stride, table_width);
  if (rc) return rc;
  if (!positions) return fail(AICAS_ERR_INVALID, "positions must be non-NULL");
  if (n_new < 1) return fail(AICAS_ERR_INVALID, "n_new must be >= 1");
  if (batch < 0) return fail(AICAS_ERR_INVALID, "batch must be >= 0");
  if (!is_pow2(page_size)) return fail(AICAS_ERR_INVALID, "page_size must be a power of two");
  if (batch == 0) return ok();
  aicas::BlockPoolParams p{};
  p.free_blocks = pool->free_blocks;
  p.free_count = pool->free_count;
  p.num_blocks = pool->num_blocks;
  p.table = block_table;
  p.stride = block_table_stride;
  p.width = table_width;
  p.batch = batch;
  p.positions = positions;
  p.n_new = n_new;
  p.page_shift = ilog2(page_size);
  p.status = status;
  hipLaunchKernelGGL(aicas::block_alloc_kernel, dim3(1), dim3(aicas::kPoolThreads), 0, stream, p);
  return check_launch("aicas_block_alloc");
}

int aicas_block_free(const aicas_block_pool_t* pool, int32_t* block_table, int64_t block_table_stride,
                     int32_t table_width, const int32_t* release, int32_t* seq_lens, int32_t batch, int32_t* status,
                     hipStream_t stream) {
  int rc = check_pool(pool);
  if (!rc) rc = check_table(block_table, block_table_stride, table_width);
  if (rc) return rc;
  if (!release) return fail(AICAS_ERR_INVALID, "release must be non-NULL");
  if (batch < 0) return fail(AICAS_ERR_INVALID, "batch must be >= 0");
  if (batch == 0) return ok();
  aicas::BlockPoolParams p{};
  p.free_blocks = pool->free_blocks;
  p.free_count = pool->free_count;
  p.num_blocks = pool->num_blocks;
  p.table = block_table;
  p.stride = block_table_stride;
  p.width = table_width;
  p.batch = batch;
  p.release = release;
  p.seq_lens = seq_lens;
  p.status = status;
  hipLaunchKernelGGL(aicas::block_free_kernel, dim3(1), dim3(aicas::kPoolThreads), 0, stream, p);
  return check_launch("aicas_block_free");
}

}  // extern "C"
