// Split-K GQA decode attention for q_len == 1 (flash-decoding), VALU only, with an optional fused KV append.
//
// Computes, for every batch row b and query head hq (kv head hq / G):
//   out[b, hq, :] = softmax(q[b, hq] . K[b, hq/G, :L_b]^T * sm_scale) . V[b, hq/G, :L_b]
// which is what the reference decode path returns (triton_qwen3vl/gqa_decode_attention.py:46-141 and its
// oracle, SDPA over repeat_kv, triton_qwen3vl/fallback.py:7-64), with per-sequence lengths L_b.
//
// Work decomposition: one 256-thread workgroup per (split, kv head, batch row); a sequence of L tokens gets
// n = ceil(L / tokens_per_split) active workgroups. Every K/V row is read once and serves all G query heads of
// the group. A row of D elements is spread over R = D / VEC lanes (16 bytes per lane), so one wave load
// instruction covers 64 / R consecutive tokens (1 KiB). Each wave streams its own super-chunks of 2 x U such
// loads (16 KiB of K and V), double-buffered in registers: one chunk of U loads is in flight while the other
// is consumed.
//
// Scheduling (striped mode): the super-chunks of a sequence are dealt round-robin to the 4 * n waves of its
// workgroups (wave slot w takes super-chunks w, w + 4n, w + 8n, ...), so that every wave carries the same work
// to one super-chunk and the waves of the sequence sweep its K/V together. Paged caches whose block-table
// row does not fit the LDS cache use range mode: each split streams a static range of equal size (to a load
// group), its 4 waves taking super-chunks of it in turn.
//
// Each R-lane row group keeps its own online-softmax state (running max m, sum l, accumulator acc) in fp32
// in the exp2 domain; the states are merged across the row groups of a wave with lane shuffles and across the
// 4 waves through LDS.
//
// Split merge: a split writes its unnormalised (m, l, acc) to the workspace with agent-scope stores (these
// write through to the device coherence point, so no L2 writeback is needed), waits for them to complete,
// and bumps the (b, kv head) arrival counter. The split that arrives last reads every split's partial with
// agent-scope loads and combines them: M = max m_i, l = sum l_i 2^(m_i - M), out = sum acc_i 2^(m_i - M) / l;
// it then re-arms the counter to zero. Nothing ever waits on another workgroup. Sequences that need one
// split write the output directly. Up to 8 splits the merging workgroup reads one output cell per thread; above
// that it reads the partials in 16-byte pieces, several threads per group of 4 cells, so that its loads stay
// one or two round trips deep.
//
// Prologue: q, the new rows (APPEND) and the q/k preparation's inputs, weights and rotary rows (QK) are fetched
// before the lengths are read, so that their latencies overlap; every wave reads its sequence's length with a
// scalar load. The wave's first super-chunk (both buffers) is in flight before any other prologue work (the q/k
// preparation, the new rows' staging) starts: with SPEC (contiguous caches whose every split has work by the
// caller's bound) it is issued before the length arrives, since in the striped schedule it does not depend on
// it. Every load before the token loop is issued on every path, and no loaded register is written before it is
// consumed, so that the compiler's waits are exact: waiting for one buffer never drains the other.
//
// Fused append (APPEND): positions[b] is the length before this step; the kernel attends over
// L_b = positions[b] + 1 tokens, of which token L_b - 1 comes from the new rows (k_new / v_new) instead of the
// cache: every workgroup stages the rows in LDS and the wave that streams the token selects them in before
// consuming its chunk, and split 0 writes the row into the cache (quantized on write for fp8 caches, with the
// attention then using the dequantised row, exactly what a separate append followed by attention would read).
// Every workgroup of batch row b counts itself in on its way out, once all its waves have read positions[b];
// the last one to do so stores positions[b] + 1 to seq_lens_out[b] (which may alias positions), so no workgroup
// can read a bumped length. With the rows in length order (order_rows), where every workgroup reads every row's
// length, the count covers the whole launch and its last workgroup bumps every row.
#pragma once

#include <type_traits>

#include "common.hpp"

namespace aicas {

struct DecodeParams {
  KVLayout cache;
  const void* q;
  int64_t q_stride_b, q_stride_h;  // elements; head_dim stride is 1
  void* out;
  int64_t out_stride_b, out_stride_h;
  const int32_t* seq_lens;  // nullptr: every sequence has uniform_len tokens (APPEND: positions)
  int32_t uniform_len;
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t tokens_per_split;  // a sequence of L tokens takes min(max_splits, ceil(L / tokens_per_split)) splits
  int32_t max_splits;  // == gridDim.x
  int32_t len_limit;   // longest sequence a launch attends in full (with the cache capacity)
  int32_t spec_splits; // splits every sequence keeps busy by the caller's lower bound on the lengths
  int32_t page_shift;  // log2(page_size) for paged caches
  float scale_log2;    // sm_scale * log2(e)
  float* ws_ml;        // [B * Hq * max_splits][2]  (m, l)
  float* ws_acc;       // [B * Hq * max_splits][D]
  int32_t* ws_counter; // [B * Hkv * counter_stride] split arrivals, zero between launches
  int32_t counter_stride;  // int32 slots between (batch row, kv head) arrival counters (32: one 128-byte line each)
  int32_t* ws_arrive;  // [B * arrive_stride] APPEND: readers of positions[b], zero between launches
  int32_t arrive_stride;  // int32 slots between batch rows' counters (32: one 128-byte line each)
  int32_t order_rows;     // nonzero: grid slots take the batch rows in folded length order (see the kernel);
                          // needs seq_lens and B <= kBlockThreads
  int32_t* status;
  // APPEND only
  const void* k_new;
  const void* v_new;
  int64_t kn_stride_b, kn_stride_h, vn_stride_b, vn_stride_h;
  int32_t* seq_lens_out;
  // APPEND only, optional: the model's q/k preparation applied to q and to the new K rows before use —
  // RMSNorm over head_dim with weights q_norm_w / k_norm_w ([D], q dtype; nullptr: no norm) and the rotary
  // embedding with rows rope_cos / rope_sin ([B, D], q dtype; nullptr: none) — and the prepared q written to
  // q_out ([B, Hq, D], nullptr: not written).
  const void* q_norm_w;
  const void* k_norm_w;
  float norm_eps;
  const void* rope_cos;
  const void* rope_sin;
  int64_t rope_cos_stride_b, rope_sin_stride_b;
  void* q_out;
  int64_t q_out_stride_b, q_out_stride_h;
};

constexpr int kMaxBlockEntries = 2048;  // block-table entries a workgroup can hold in LDS
constexpr float kNegBig = -1.0e30f;     // finite "minus infinity" for running maxima

template <int KV_DT>
struct KVTraits {
  static constexpr int kElemBytes = (KV_DT == kFP8E4M3) ? 1 : 2;
  static constexpr int kVec = 16 / kElemBytes;  // elements per lane per row
  static constexpr int kUnroll = 4;             // tokens per lane per chunk
  // tokens one workgroup chunk covers; the host rounds tokens_per_split to a multiple of this
  static constexpr int tokens_per_chunk(int head_dim) {
    return (kWave / (head_dim / kVec)) * kWavesPerBlock * kUnroll;
  }
};

__device__ __forceinline__ void store_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Cache-policy operand of the buffer-load builtin that sets sc1: the bit a relaxed agent-scope atomic load
// carries (global_load_dword ... sc1), here on 16-byte loads.
constexpr int kAuxSc1 = 16;

// The model's q/k preparation for one pair of adjacent elements (d0, d0 + 1) of a head row whose D/2 pairs are
// held by D/2 consecutive lanes of one wave (every lane of the row must take part): RMSNorm over head_dim in
// fp32, rounded to the storage type DT and multiplied by the weight (Qwen3VLTextRMSNorm.forward,
// transformers/models/qwen3_vl/modeling_qwen3_vl.py:391-404), then the rotary embedding x * cos + rotate_half(x)
// * sin with both products and the sum rounded to DT (apply_rotary_pos_emb and rotate_half,
// modeling_qwen3_vl.py:412-438 and :138-142). rotate_half pairs element d with d +- D/2: the same slot of the
// lane D/4 away. `norm` may differ between rows; `rope` is the same for all.
template <int DT, int D>
__device__ __forceinline__ void qk_pair(float& x0, float& x1, int d0, uint32_t weight, bool norm, uint32_t cos2,
                                        uint32_t sin2, bool rope, float eps) {
  constexpr int P = D / 2;  // lanes per row
  static_assert(P <= kWave && kWave % P == 0, "a row's pairs must fit one wave");
  float ss = __fadd_rn(__fmul_rn(x0, x0), __fmul_rn(x1, x1));
#pragma unroll
  for (int off = P / 2; off >= 1; off >>= 1) ss = __fadd_rn(ss, __shfl_xor(ss, off));
  if (norm) {
    const float r = rsqrtf(__fadd_rn(ss * (1.0f / D), eps));
    float w0, w1;
    unpack2<DT>(weight, w0, w1);
    x0 = round_to<DT>(__fmul_rn(w0, round_to<DT>(__fmul_rn(x0, r))));
    x1 = round_to<DT>(__fmul_rn(w1, round_to<DT>(__fmul_rn(x1, r))));
  }
  if (rope) {
    float p0 = __shfl_xor(x0, P / 2);
    float p1 = __shfl_xor(x1, P / 2);
    if (d0 < D / 2) {
      p0 = -p0;
      p1 = -p1;
    }
    float c0, c1, s0, s1;
    unpack2<DT>(cos2, c0, c1);
    unpack2<DT>(sin2, s0, s1);
    x0 = round_to<DT>(__fadd_rn(round_to<DT>(__fmul_rn(x0, c0)), round_to<DT>(__fmul_rn(p0, s0))));
    x1 = round_to<DT>(__fadd_rn(round_to<DT>(__fmul_rn(x1, c1)), round_to<DT>(__fmul_rn(p1, s1))));
  }
}

// A pointer into global memory that is the same in every lane, taken through readfirstlane: a per-lane choice
// between two such pointers then selects between registers, where a choice between two kernel-argument fields
// would otherwise become a per-lane load of the chosen field. The value is rebuilt as a global (address space
// 1) pointer and cast back, so that accesses through it stay global_* instructions: flat_* accesses, which a
// pointer rebuilt from an integer would otherwise get, turn every wait for a load into a wait for all of them.
template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* ptr) {
  const uint64_t v = reinterpret_cast<uint64_t>(ptr);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  __attribute__((address_space(1))) T* g =
      reinterpret_cast<__attribute__((address_space(1))) T*>((static_cast<uint64_t>(hi) << 32) | lo);
  return (T*)g;
}

// U loads of K and of V rows per lane, the rows' validity and, for fp8 caches, the chunk's per-token scales
// (NSW words per lane, see load_rows).
template <int U, int NSW>
struct Chunk {
  uint4 k[U];
  uint4 v[U];
  float sc[NSW];
  bool ok[U];
};

template <int Q_DT, int KV_DT, int D, int G, bool PAGED, bool APPEND, bool QK, bool SPEC>
__global__ __launch_bounds__(kBlockThreads) void decode_attn_kernel(DecodeParams p) {
  static_assert(APPEND || !QK, "the q/k prologue belongs to the fused append");
  static_assert(!(SPEC && PAGED), "only contiguous caches fetch rows before the length is known");
  using Tr = KVTraits<KV_DT>;
  constexpr int EB = Tr::kElemBytes;
  constexpr int VEC = Tr::kVec;
  constexpr int U = Tr::kUnroll;
  constexpr int R = D / VEC;            // lanes per row
  constexpr int RPW = kWave / R;        // rows per wave per load
  constexpr int RPB = RPW * kWavesPerBlock;
  static_assert(R >= 1 && R <= 16, "a row must fit one DPP row");
  constexpr bool FP8 = (KV_DT == kFP8E4M3);
  constexpr int NS = U * RPW;                                 // tokens per wave chunk
  constexpr int NSW = FP8 ? (2 * NS + kWave - 1) / kWave : 1;  // fp8: scale words per lane per chunk
  using ChunkT = Chunk<U, NSW>;

  __shared__ float s_m[kWavesPerBlock][G];
  __shared__ float s_l[kWavesPerBlock][G];
  // the 4 waves' accumulators; later, in the workgroup that merges many splits, the merge's per-thread states
  constexpr int kPoolFloats = kWavesPerBlock * G * D > 6 * kBlockThreads ? kWavesPerBlock * G * D : 6 * kBlockThreads;
  __shared__ __align__(16) float s_pool[kPoolFloats];
  auto& s_acc = *reinterpret_cast<float (*)[kWavesPerBlock][G][D]>(s_pool);
  __shared__ int32_t s_bt[PAGED ? kMaxBlockEntries : 1];
  __shared__ int32_t s_last;
  // order_rows: every batch row's length as read at the start (APPEND: before any bump), and this slot's row
  __shared__ int32_t s_row_len[kBlockThreads];
  __shared__ __align__(16) uint32_t s_row_key[kBlockThreads];
  __shared__ int32_t s_row;
  __shared__ int32_t s_bump;
  // APPEND: the new token's rows as the attention must see them (dequantised codes for fp8 caches)
  __shared__ uint4 s_new[APPEND ? 2 * R : 1];
  __shared__ float s_new_scale[APPEND && FP8 ? 2 : 1];
  // QK: the prepared q rows and K row, as pairs of DT values
  __shared__ uint32_t s_qk[QK ? (G + 1) * (D / 2) : 1];

  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int tid = threadIdx.x;
  // Row order (ragged batches): the rows ranked by decreasing length (ties in row order) are folded over the grid:
  // slot z < h = ceil(B / 2) takes rank z and slot h + i takes rank B - 1 - i, so that the longest rows go out
  // first, each with a short row h slots later — the grid's workgroups that share a compute unit then carry
  // about equal work. Every workgroup reads all the lengths and ranks them the same way (none is bumped before
  // every workgroup has counted in, see count_in), so the slots cover every row exactly once.
  int b = blockIdx.z;
  if (p.order_rows) {
    const int nb = gridDim.z;
    const int z = blockIdx.z;
    const int h = (nb + 1) / 2;
    const int want = z < h ? z : nb - 1 - (z - h);
    const int len_t = tid < nb ? p.seq_lens[tid] : 0;
    s_row_len[tid] = len_t;
    // one 32-bit key per row, distinct and ordered like (length, -row): the length clamped to [0, 2^23) (lengths
    // outside it are clamped by the kernel anyway), then 255 - row; the rows past nb hold 0, below every key
    // they are compared with. A row's rank is the number of larger keys.
    const uint32_t key_t = tid < nb ? (static_cast<uint32_t>(min(max(len_t, 0), (1 << 23) - 1)) << 8) |
                                          static_cast<uint32_t>(255 - tid)
                                    : 0u;
    s_row_key[tid] = key_t;
    __syncthreads();
    if (tid < nb) {
      int rank = 0;
      const uint4* keys = reinterpret_cast<const uint4*>(s_row_key);
#pragma unroll 4
      for (int j = 0; j < (nb + 3) / 4; ++j) {
        const uint4 k4 = keys[j];
        rank += (k4.x > key_t ? 1 : 0) + (k4.y > key_t ? 1 : 0) + (k4.z > key_t ? 1 : 0) + (k4.w > key_t ? 1 : 0);
      }
      if (rank == want) s_row = tid;
    }
    __syncthreads();
    b = __builtin_amdgcn_readfirstlane(s_row);
  }
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // uniform across the wave: scalar control flow
  const int lane = tid % kWave;
  const int row = lane / R;
  const int li = lane % R;

  // Query slices of the G heads served by this kv head (independent of the lengths: issued first).
  const uint16_t* qb = static_cast<const uint16_t*>(p.q) + b * p.q_stride_b;
  // (VEC / 2 pairs of q's 16-bit type per lane; fp8 caches take their K codes to the same type, exactly, so
  // that both dot products run on v_dot2)
  uint32_t qp[G][VEC / 2];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const uint16_t* qh = qb + (kvh * G + h) * p.q_stride_h + li * VEC;
#pragma unroll
    for (int c = 0; c < VEC / 8; ++c) {
      const uint4 w = *reinterpret_cast<const uint4*>(qh + 8 * c);
      qp[h][4 * c + 0] = w.x;
      qp[h][4 * c + 1] = w.y;
      qp[h][4 * c + 2] = w.z;
      qp[h][4 * c + 3] = w.w;
    }
  }

  const uint8_t* kbase = static_cast<const uint8_t*>(p.cache.k);
  const uint8_t* vbase = static_cast<const uint8_t*>(p.cache.v);
  const int64_t head_off = static_cast<int64_t>(kvh) * p.cache.stride_h;
  const int64_t shead_off = static_cast<int64_t>(kvh) * p.cache.scale_stride_h;
  const int page_mask = (1 << p.page_shift) - 1;
  const int tps = p.tokens_per_split;
  // Clamp so that no access leaves the cache (and, paged, no split's range outgrows the LDS block-id cache).
  const int limit = min(p.cache.max_tokens, p.len_limit);
  // A wave streams chunks of CW consecutive tokens (U loads of RPW rows); its unit of work is a super-chunk of
  // two chunks, one per register buffer. Super-chunk j covers tokens [j * SCW, (j + 1) * SCW).
  constexpr int CW = U * RPW;
  constexpr int SCW = 2 * CW;
  const int wave_slot = split * kWavesPerBlock + wave;  // this wave's first super-chunk in striped mode
  // Range mode: the n splits of an L-token sequence cover [begin(s), begin(s + 1)), whole groups of RPB tokens
  // each, so that their sizes differ by at most one group and none exceeds tps rounded up to a group.
  auto split_begin = [](int s, int n, int len) {
    const int64_t groups = (len + RPB - 1) / RPB;
    return min(len, static_cast<int>(static_cast<int64_t>(s) * groups / n) * RPB);
  };

  // APPEND: the new token's source rows, fetched now: they do not depend on the lengths. Lanes tid < R take the
  // K row's slices and lanes R <= tid < 2R the V row's; every other lane fetches a copy of one of them, never
  // used, so that the load is issued on every path and the waits on it stay exact.
  uint4 new_raw[FP8 ? 2 : 1];
  if constexpr (APPEND) {
    const int c = tid % R;
    // both row addresses as uniform values before the per-lane choice (otherwise the choice becomes a per-lane
    // load of the pointer from the kernel arguments, one more round trip ahead of every load)
    const uint16_t* kn = uniform_ptr(static_cast<const uint16_t*>(p.k_new) + b * p.kn_stride_b + kvh * p.kn_stride_h);
    const uint16_t* vn = uniform_ptr(static_cast<const uint16_t*>(p.v_new) + b * p.vn_stride_b + kvh * p.vn_stride_h);
    const uint16_t* src = ((tid / R) & 1) == 0 ? kn : vn;
    new_raw[0] = *reinterpret_cast<const uint4*>(src + c * VEC);
    if constexpr (FP8) new_raw[1] = *reinterpret_cast<const uint4*>(src + c * VEC + 8);
  }
  // QK: the q/k preparation is spread over the workgroup, one pair of adjacent elements (d0, d0 + 1) per thread
  // and round: the G q rows of this kv head, then the new K row, D/2 pairs each. This thread's pairs, their
  // weights and the sequence's cos/sin pairs are fetched with the first loads (a part that is not given reads
  // the q row instead, never used), so that the waits on them stay exact.
  constexpr int kQKPairs = (G + 1) * (D / 2);
  constexpr int kQKRounds = QK ? (kQKPairs + kBlockThreads - 1) / kBlockThreads : 1;
  uint32_t qk_x[kQKRounds], qk_w[kQKRounds], qk_c[kQKRounds], qk_s[kQKRounds];
  const bool qk_norm_q = QK && p.q_norm_w != nullptr;
  const bool qk_norm_k = QK && p.k_norm_w != nullptr;
  const bool qk_rope = QK && p.rope_cos != nullptr;
  if constexpr (QK) {
    const uint16_t* qrow = uniform_ptr(qb + kvh * G * p.q_stride_h);
    const uint16_t* krow =
        uniform_ptr(static_cast<const uint16_t*>(p.k_new) + b * p.kn_stride_b + kvh * p.kn_stride_h);
    const uint16_t* wq = qk_norm_q ? uniform_ptr(static_cast<const uint16_t*>(p.q_norm_w)) : qrow;
    const uint16_t* wk = qk_norm_k ? uniform_ptr(static_cast<const uint16_t*>(p.k_norm_w)) : qrow;
    const uint16_t* cr =
        qk_rope ? uniform_ptr(static_cast<const uint16_t*>(p.rope_cos) + b * p.rope_cos_stride_b) : qrow;
    const uint16_t* sr =
        qk_rope ? uniform_ptr(static_cast<const uint16_t*>(p.rope_sin) + b * p.rope_sin_stride_b) : qrow;
#pragma unroll
    for (int i = 0; i < kQKRounds; ++i) {
      const int pp = min(tid + i * kBlockThreads, kQKPairs - 1);
      const int r = pp / (D / 2);
      const int d0 = 2 * (pp % (D / 2));
      const uint16_t* x = r < G ? qrow + r * p.q_stride_h : krow;
      qk_x[i] = *reinterpret_cast<const uint32_t*>(x + d0);
      qk_w[i] = *reinterpret_cast<const uint32_t*>((r < G ? wq : wk) + d0);
      qk_c[i] = *reinterpret_cast<const uint32_t*>(cr + d0);
      qk_s[i] = *reinterpret_cast<const uint32_t*>(sr + d0);
    }
  }

  // Issues the loads of rows t0 + u * RPW + row of this wave (hi >= 1). Rows at or past hi, the row `skip`
  // and rows on invalid pages come out with ok = false; they still load, from row min(t, hi - 1) (block 0 for
  // an invalid page), so that every load is issued on every path and the compiler can wait for one buffer
  // while the other stays in flight. Their words are never let through by consume. A chunk that is not
  // `valid` (no such chunk) loads row t_dummy of block 0 / of the sequence in every lane, all masked.
  const float* const kscale = FP8 ? uniform_ptr(p.cache.k_scale) : nullptr;
  const float* const vscale = FP8 ? uniform_ptr(p.cache.v_scale) : nullptr;
  auto load_rows = [&](ChunkT& c, int t0, int hi, int skip, int first_entry, bool valid, int t_dummy) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = t0 + u * RPW + row;
      const int tc = valid ? min(t, hi - 1) : t_dummy;
      bool ok = valid && t < hi && t != skip;
      int64_t blk = b;
      int tin = tc;
      if constexpr (PAGED) {
        const int32_t e = s_bt[(tc >> p.page_shift) - first_entry];
        ok = ok && e >= 0;
        blk = valid && e >= 0 ? e : 0;
        tin = tc & page_mask;
      }
      const int64_t off = blk * p.cache.stride_blk + head_off + static_cast<int64_t>(tin) * p.cache.stride_t;
      c.k[u] = load_stream16(kbase + off * EB + li * 16);
      c.v[u] = load_stream16(vbase + off * EB + li * 16);
      c.ok[u] = ok;
    }
    // fp8: the chunk's scales in one load per lane (not one per row and lane): word j of lane l holds entry
    // j * 64 + l of [the K scales of tokens t0 .. t0 + NS - 1, then their V scales] (entries past 2 NS repeat
    // the last one, unused); consume fetches each row's pair from the lanes holding them with a shuffle.
    if constexpr (FP8) {
#pragma unroll
      for (int j = 0; j < NSW; ++j) {
        const int i = min(j * kWave + lane, 2 * NS - 1);
        const bool is_v = i >= NS;
        const int t = t0 + (is_v ? i - NS : i);
        const int tc = valid ? min(t, hi - 1) : t_dummy;
        int64_t blk = b;
        int tin = tc;
        if constexpr (PAGED) {
          const int32_t e = s_bt[(tc >> p.page_shift) - first_entry];
          blk = valid && e >= 0 ? e : 0;
          tin = tc & page_mask;
        }
        c.sc[j] = (is_v ? vscale : kscale)[blk * p.cache.scale_stride_blk + shead_off + tin];
      }
    }
  };

  ChunkT ca, cb;

  // Sequence length (cached tokens before this step's append for APPEND), read by every wave: a uniform load,
  // so its wait does not cover the vector loads issued after it.
  int L = p.seq_lens ? p.seq_lens[b] : p.uniform_len;
  const int len_read = L;
  // SPEC (contiguous caches, launched when the caller's lower bound on the lengths keeps every split busy): a
  // wave's first super-chunk in the striped schedule (super-chunk wave_slot) does not depend on the length, so
  // both buffers go out now, rows clamped to the capacity (always inside the cache), and the rows' validity is
  // settled once the length is known. Otherwise (and for paged caches, which need the block table first) the
  // first rows are fetched once the length is known.
  const int spec_t0 = wave_slot * SCW;
  if constexpr (SPEC) {
    load_rows(ca, spec_t0, p.cache.max_tokens, -1, 0, true, 0);
    load_rows(cb, spec_t0 + CW, p.cache.max_tokens, -1, 0, true, 0);
  }
  // APPEND with seq_lens_out: every workgroup counts itself in on its way out, after a barrier that each of its
  // waves passes once it has read positions[b] (every wave used the value to plan its work); the last of the
  // batch row's workgroups stores the bumped length, so no workgroup can read it. Counting in at exit keeps the
  // contended atomic off the start of the stream.
  auto count_in = [&]() {
    if constexpr (APPEND) {
      if (p.order_rows) {
        // every workgroup has read every row's length: the last of the whole launch bumps them all (from the
        // values read at the start, as the per-row counters below would)
        if (p.seq_lens_out) {
          if (tid == 0) {
            const int readers = gridDim.x * gridDim.y * gridDim.z;
            const int prev = __hip_atomic_fetch_add(p.ws_arrive, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_bump = prev == readers - 1 ? 1 : 0;
            if (prev == readers - 1) __hip_atomic_store(p.ws_arrive, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
          __syncthreads();
          if (s_bump && tid < static_cast<int>(gridDim.z)) p.seq_lens_out[tid] = s_row_len[tid] + 1;
        }
        return;
      }
      if (tid == 0 && p.seq_lens_out) {
        const int readers = gridDim.x * gridDim.y;
        int32_t* const arrive = p.ws_arrive + static_cast<int64_t>(b) * p.arrive_stride;
        const int prev = __hip_atomic_fetch_add(arrive, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (prev == readers - 1) {
          p.seq_lens_out[b] = len_read + 1;
          __hip_atomic_store(arrive, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
  };
  if (L < 0) L = 0;
  int t_new = -1;  // APPEND: token served from the new rows
  if constexpr (APPEND) {
    if (L + 1 > limit) {
      // no slot for the new token: it is dropped (and reported), attention covers the existing tokens
      if (p.status && split == 0 && tid == 0) atomicOr(p.status, kStatusAppendOverflow);
    } else {
      L += 1;
      t_new = L - 1;
    }
  }
  if (L > limit) {
    if (p.status && split == 0 && tid == 0) atomicOr(p.status, kStatusLenClamped);
    L = limit;
  }
  const int n_active = L > 0 ? min(p.max_splits, (L + tps - 1) / tps) : 1;
  if (split >= n_active) {
    __syncthreads();  // every wave has read positions[b]
    count_in();
    return;
  }
  // APPEND, paged: the new token's block id (for the cache write), read before any cache load so that waiting
  // for it leaves those in flight.
  int32_t blk_new = 0;
  if constexpr (APPEND && PAGED) {
    blk_new = p.cache.block_table[static_cast<int64_t>(b) * p.cache.block_table_stride + (max(t_new, 0) >> p.page_shift)];
  }
  // Schedule: striped mode unless a paged sequence's whole block-table row does not fit the LDS cache.
  bool striped = true;
  if constexpr (PAGED) striped = ((L + page_mask) >> p.page_shift) <= kMaxBlockEntries;
  const int n_super = (L + SCW - 1) / SCW;
  const int stripe = n_active * kWavesPerBlock;  // striped mode: waves sharing the sequence
  const int t_begin = striped ? 0 : split_begin(split, n_active, L);
  const int t_end = striped ? L : split_begin(split + 1, n_active, L);

  // Paged caches: stage the block ids this workgroup may touch in LDS (invalid ids become -1 and their tokens
  // are skipped): the whole row in striped mode, the split's range otherwise.
  int first_entry = 0;
  if constexpr (PAGED) {
    first_entry = t_begin >> p.page_shift;
    const int n_ent = t_end > t_begin ? ((t_end - 1) >> p.page_shift) - first_entry + 1 : 0;
    const int32_t* bt = p.cache.block_table + static_cast<int64_t>(b) * p.cache.block_table_stride + first_entry;
    // up to four of a thread's entries in flight at once (one round trip for rows of up to 1024 entries), then
    // the checks and the LDS writes
    constexpr int kBatch = 4;
    const int rounds = (n_ent + kBlockThreads - 1) / kBlockThreads;  // <= kMaxBlockEntries / kBlockThreads
    for (int k0 = 0; k0 < rounds; k0 += kBatch) {
      int32_t ent[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        if (k0 + k < rounds) ent[k] = bt[min(tid + (k0 + k) * kBlockThreads, n_ent - 1)];
      }
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int i = tid + (k0 + k) * kBlockThreads;
        if (k0 + k < rounds && i < n_ent) {
          int32_t blk = ent[k];
          if (blk < 0 || blk >= p.cache.num_blocks) {
            if (p.status) atomicOr(p.status, kStatusBlockOutOfRange);
            blk = -1;
          }
          s_bt[i] = blk;
        }
      }
    }
    __syncthreads();
  }
  // Super-chunk i of this wave starts at super_start(i) (-1: none). A chunk of rows comes from the cache; the
  // new token's row (t_new) is masked there and swapped in from the staged rows before the chunk is consumed.
  auto super_start = [&](int i) -> int {
    if (striped) {
      const int j = wave_slot + i * stripe;
      return j < n_super ? j * SCW : -1;
    }
    const int t = t_begin + (wave + i * kWavesPerBlock) * SCW;
    return t < t_end ? t : -1;
  };
  // The wave's first super-chunk goes out now, before the prologue work below; a wave without one loads a
  // masked dummy (every row reads token t_begin, whose block entry is staged whenever a chunk could exist),
  // so that every load is issued on every path and the waits on the buffers stay exact.
  auto load_chunk = [&](ChunkT& c, int t0, bool valid) {
    load_rows(c, valid ? t0 : t_begin, t_end, t_new, first_entry, valid, t_begin);
  };
  const int sc0 = super_start(0);
  if constexpr (SPEC) {
    // striped: sc0 is spec_t0 when the wave has a first super-chunk; its rows count if they lie below the length
    // and are not the new token's (whose row is swapped in before the chunk is consumed)
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = spec_t0 + u * RPW + row;
      ca.ok[u] = sc0 >= 0 && t < t_end && t != t_new;
      cb.ok[u] = sc0 >= 0 && t + CW < t_end && t + CW != t_new;
    }
  } else {
    load_chunk(ca, sc0, sc0 >= 0);
    load_chunk(cb, sc0 + CW, sc0 >= 0);
  }

  float m[G], l[G], acc[G][VEC];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = kNegBig;
    l[h] = 0.0f;
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[h][i] = 0.0f;
  }

  auto consume = [&](const ChunkT& c) {
    // fp8: each row's K and V scales, from the lanes that loaded them (see load_rows)
    float ks[U], vs[U];
    if constexpr (FP8) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        ks[u] = __shfl(c.sc[(u * RPW) / kWave], (u * RPW + row) % kWave);
        vs[u] = __shfl(c.sc[(NS + u * RPW) / kWave], (NS + u * RPW + row) % kWave);
      }
    }
    // Scores (log2 domain) for U tokens x G heads.
    float s[U][G];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if constexpr (!FP8) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
          float d = 0.0f;
          d = dot2<KV_DT>(qp[h][0], c.k[u].x, d);
          d = dot2<KV_DT>(qp[h][1], c.k[u].y, d);
          d = dot2<KV_DT>(qp[h][2], c.k[u].z, d);
          d = dot2<KV_DT>(qp[h][3], c.k[u].w, d);
          s[u][h] = group_sum<R>(d) * p.scale_log2;
        }
      } else {
        // the 16 codes as 8 exact pairs of q's type, then v_dot2 as for 16-bit caches
        const uint32_t kw[4] = {c.k[u].x, c.k[u].y, c.k[u].z, c.k[u].w};
        uint32_t k2[VEC / 2];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          k2[2 * w] = e4m3x2_to_16<Q_DT, false>(kw[w]);
          k2[2 * w + 1] = e4m3x2_to_16<Q_DT, true>(kw[w]);
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
          float d = 0.0f;
#pragma unroll
          for (int j = 0; j < VEC / 2; ++j) d = dot2<Q_DT>(qp[h][j], k2[j], d);
          s[u][h] = group_sum<R>(d) * (p.scale_log2 * ks[u]);
        }
      }
#pragma unroll
      for (int h = 0; h < G; ++h) s[u][h] = c.ok[u] ? s[u][h] : -__builtin_inff();
    }
    // Online softmax update, values converted once per token and shared by the G heads.
    float mnew[G], alpha[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float mx = s[0][h];
#pragma unroll
      for (int u = 1; u < U; ++u) mx = fmaxf(mx, s[u][h]);
      mnew[h] = fmaxf(m[h], mx);
      alpha[h] = fast_exp2(m[h] - mnew[h]);
      l[h] *= alpha[h];
#pragma unroll
      for (int i = 0; i < VEC; ++i) acc[h][i] *= alpha[h];
      m[h] = mnew[h];
    }
    // P.V on v_dot2, two tokens at a time: each element's two values (one per token) form one operand and the
    // two tokens' probabilities, rounded to q's 16-bit type (as the reference's Triton kernel rounds P before
    // its product with V), the other; products are exact and accumulate in fp32. fp8 rows are first taken to
    // q's type exactly, their per-row scales folded into P.
    static_assert(U % 2 == 0, "tokens are paired");
#pragma unroll
    for (int u = 0; u < U; u += 2) {
      // a masked row's weight is 0, but its registers hold stale words that must not reach the product as NaN/Inf
      const uint32_t wa[4] = {c.ok[u] ? c.v[u].x : 0u, c.ok[u] ? c.v[u].y : 0u, c.ok[u] ? c.v[u].z : 0u,
                              c.ok[u] ? c.v[u].w : 0u};
      const uint32_t wb[4] = {c.ok[u + 1] ? c.v[u + 1].x : 0u, c.ok[u + 1] ? c.v[u + 1].y : 0u,
                              c.ok[u + 1] ? c.v[u + 1].z : 0u, c.ok[u + 1] ? c.v[u + 1].w : 0u};
      // xs[j] / ys[j]: elements 2j / 2j + 1 of both tokens as a pair of q's 16-bit type (token u in the low half)
      uint32_t xs[VEC / 2], ys[VEC / 2];
      if constexpr (!FP8) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          xs[w] = __builtin_amdgcn_perm(wb[w], wa[w], 0x05040100u);
          ys[w] = __builtin_amdgcn_perm(wb[w], wa[w], 0x07060302u);
        }
      } else {
        // the two tokens' codes interleaved first ([a0, b0, a1, b1] and [a2, b2, a3, b3] of codes 4w .. 4w + 3),
        // so that each conversion yields one pair: 2 byte permutes and 4 conversions per word pair instead of
        // 4 conversions and 4 permutes of the converted halves
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t lo = __builtin_amdgcn_perm(wb[w], wa[w], 0x05010400u);
          const uint32_t hi = __builtin_amdgcn_perm(wb[w], wa[w], 0x07030602u);
          xs[2 * w] = e4m3x2_to_16<Q_DT, false>(lo);
          ys[2 * w] = e4m3x2_to_16<Q_DT, true>(lo);
          xs[2 * w + 1] = e4m3x2_to_16<Q_DT, false>(hi);
          ys[2 * w + 1] = e4m3x2_to_16<Q_DT, true>(hi);
        }
      }
      uint32_t pp[G];
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float p0 = fast_exp2(s[u][h] - mnew[h]);
        const float p1 = fast_exp2(s[u + 1][h] - mnew[h]);
        l[h] += p0;
        l[h] += p1;
        const float pv0 = FP8 ? (c.ok[u] ? p0 * vs[u] : 0.0f) : p0;
        const float pv1 = FP8 ? (c.ok[u + 1] ? p1 * vs[u + 1] : 0.0f) : p1;
        pp[h] = pack2<Q_DT>(pv0, pv1);
      }
#pragma unroll
      for (int j = 0; j < VEC / 2; ++j) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
          acc[h][2 * j] = dot2<Q_DT>(xs[j], pp[h], acc[h][2 * j]);
          acc[h][2 * j + 1] = dot2<Q_DT>(ys[j], pp[h], acc[h][2 * j + 1]);
        }
      }
    }
  };

  // The prologue work that needs the length: q's preparation (QK) and the staging of the new rows (APPEND). It
  // runs once the wave's first super-chunk is in flight, so that its latency covers the work.
  auto prologue_work = [&]() {
    // QK: q and the new K row as the model prepares them, one pair per thread and round (their loads were
    // issued before every load of the cache, so waiting for them leaves the first super-chunk in flight), into
    // LDS (the workgroup that writes the output also writes the prepared q to q_out from there). Then every
    // lane takes its q slices from there.
    if constexpr (QK) {
#pragma unroll
      for (int i = 0; i < kQKRounds; ++i) {
        const int pp = tid + i * kBlockThreads;
        const int r = min(pp, kQKPairs - 1) / (D / 2);
        const int d0 = 2 * (pp % (D / 2));
        float x0, x1;
        unpack2<Q_DT>(qk_x[i], x0, x1);
        qk_pair<Q_DT, D>(x0, x1, d0, qk_w[i], r < G ? qk_norm_q : qk_norm_k, qk_c[i], qk_s[i], qk_rope,
                         p.norm_eps);
        if (pp < kQKPairs) s_qk[pp] = pack2<Q_DT>(x0, x1);
      }
      __syncthreads();
#pragma unroll
      for (int h = 0; h < G; ++h) {
#pragma unroll
        for (int j = 0; j < VEC / 2; ++j) {
          qp[h][j] = s_qk[h * (D / 2) + li * (VEC / 2) + j];
        }
      }
    }

    // APPEND: every workgroup stages the new token's rows in LDS as the attention must see them (whichever wave
    // streams token t_new takes them from there); split 0 also writes them into the cache. For fp8 caches the
    // rows are quantized on write exactly as aicas_kv_append does, and the attention uses the dequantised
    // codes.
    if constexpr (APPEND) {
      if (t_new >= 0 && tid < 2 * R) {
        const int which = tid / R;  // 0 = K, 1 = V
        const int c = tid % R;
        // QK: the new K row as prepared above
        if (QK && which == 0) {
          constexpr int NW = FP8 ? 2 : 1;
#pragma unroll
          for (int n = 0; n < NW; ++n) {
            const uint32_t* kp = s_qk + G * (D / 2) + c * (VEC / 2) + 4 * n;
            new_raw[n] = make_uint4(kp[0], kp[1], kp[2], kp[3]);
          }
        }
        int64_t blk = b;
        int tin = t_new;
        bool ok = split == 0;
        if constexpr (PAGED) {
          blk = blk_new;
          tin = t_new & page_mask;
          ok = ok && blk >= 0 && blk < p.cache.num_blocks;
        }
        const int64_t off = blk * p.cache.stride_blk + head_off + static_cast<int64_t>(tin) * p.cache.stride_t;
        uint8_t* const kdst = uniform_ptr(static_cast<uint8_t*>(p.cache.k));
        uint8_t* const vdst = uniform_ptr(static_cast<uint8_t*>(p.cache.v));
        uint8_t* dst_base = which == 0 ? kdst : vdst;
        if constexpr (!FP8) {
          if (ok) *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(dst_base) + off + c * VEC) = new_raw[0];
          s_new[tid] = new_raw[0];
        } else {
          // VEC = 16 source elements (32 bytes) per lane -> 16 codes
          float f[VEC];
          const uint32_t w[8] = {new_raw[0].x, new_raw[0].y, new_raw[0].z, new_raw[0].w,
                                 new_raw[1].x, new_raw[1].y, new_raw[1].z, new_raw[1].w};
#pragma unroll
          for (int i = 0; i < 8; ++i) unpack2<Q_DT>(w[i], f[2 * i], f[2 * i + 1]);
          bool nonfinite;
          const float scale = fp8_row_scale<R, VEC>(f, nonfinite);
          if (nonfinite && ok && c == 0 && p.status) atomicOr(p.status, kStatusNonFiniteRow);
          uint32_t packed[4];
          fp8_quantize<VEC>(f, scale, packed);  // the codes kv_append_kernel writes
          const uint4 codes = make_uint4(packed[0], packed[1], packed[2], packed[3]);
          if (ok) {
            *reinterpret_cast<uint4*>(dst_base + off + c * VEC) = codes;
            if (c == 0) {
              const int64_t soff = blk * p.cache.scale_stride_blk + shead_off + tin;
              (which == 0 ? uniform_ptr(p.cache.k_scale) : uniform_ptr(p.cache.v_scale))[soff] = scale;
            }
          }
          s_new[tid] = codes;
          if (c == 0) s_new_scale[which] = scale;
        }
      }
    }
  };

  prologue_work();
  if constexpr (APPEND) __syncthreads();  // the staged new rows are visible to every wave

  // APPEND: token t_new of a chunk (masked when the chunk was loaded) comes from the staged new rows, selected
  // into a copy of the chunk just before it is consumed, when its loads have landed anyway (only the chunk
  // holding it takes this branch). The token is thus attended to at its place in the stream, exactly as a
  // separate append followed by attention would. The buffer itself is never written here: overwriting it in
  // place (a second definition of the loop-carried registers) made the compiler copy both buffers at the loop
  // head on every round, each copy waiting for its loads, down to vmcnt(0), in the variants without SPEC.
  auto consume_chunk = [&](const ChunkT& c, int t0) {
    if constexpr (APPEND) {
      if (t_new >= t0 && t_new < t0 + CW) {
        ChunkT cs = c;
        const uint4 nk = s_new[li];
        const uint4 nv = s_new[R + li];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const bool isn = t0 + u * RPW + row == t_new;
          cs.k[u] = isn ? nk : c.k[u];
          cs.v[u] = isn ? nv : c.v[u];
          cs.ok[u] = isn || c.ok[u];
        }
        if constexpr (FP8) {
          const int ik = t_new - t0;
#pragma unroll
          for (int j = 0; j < NSW; ++j) {
            if (j * kWave + lane == ik) cs.sc[j] = s_new_scale[0];
            if (j * kWave + lane == NS + ik) cs.sc[j] = s_new_scale[1];
          }
        }
        consume(cs);
        return;
      }
    }
    consume(c);
  };
  // first token of the chunk each buffer holds (far below 0 for a dummy, which holds none)
  int ca_t0 = sc0 >= 0 ? sc0 : -(1 << 30);
  int cb_t0 = sc0 >= 0 ? sc0 + CW : -(1 << 30);

  // Token loop, double-buffered: while one buffer is consumed the other is in flight, and each is reloaded
  // two chunks on as soon as it has been consumed. settle() pins the softmax state after a consume: the empty
  // asm statements take every state register as an operand and the last one orders memory, so the whole
  // consume (its last use of the buffer) precedes the reload that follows, and the new rows land in the
  // registers of the old ones. Without it the compiler sinks the P.V half of a consume past the next loads
  // and copies the buffers on every round, each copy waiting for its load. The scheduling barrier after each
  // reload keeps its loads from sinking into the consume that follows. The last super-chunk is consumed after
  // the loop, so that no load is issued past the end.
  auto settle = [&]() {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      asm volatile("" : "+v"(m[h]), "+v"(l[h]));
#pragma unroll
      for (int i = 0; i < VEC; ++i) asm volatile("" : "+v"(acc[h][i]));
    }
    asm volatile("" ::: "memory");
  };
  int k = 0;  // super-chunks of this wave taken so far
  for (int nsc = super_start(++k); nsc >= 0; nsc = super_start(++k)) {
    consume_chunk(ca, ca_t0);
    settle();
    load_chunk(ca, nsc, true);
    ca_t0 = nsc;
    __builtin_amdgcn_sched_barrier(0);
    consume_chunk(cb, cb_t0);
    settle();
    load_chunk(cb, nsc + CW, true);
    cb_t0 = nsc + CW;
    __builtin_amdgcn_sched_barrier(0);
  }
  consume_chunk(ca, ca_t0);
  consume_chunk(cb, cb_t0);

  // Merge the row groups of this wave (lanes li, li + R, li + 2R, ... hold the same head_dim slice).
#pragma unroll
  for (int off = R; off < kWave; off <<= 1) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float mo = __shfl_xor(m[h], off);
      const float lo = __shfl_xor(l[h], off);
      const float mn = fmaxf(m[h], mo);
      const float c1 = fast_exp2(m[h] - mn);
      const float c2 = fast_exp2(mo - mn);
      l[h] = l[h] * c1 + lo * c2;
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        const float ao = __shfl_xor(acc[h][i], off);
        acc[h][i] = acc[h][i] * c1 + ao * c2;
      }
      m[h] = mn;
    }
  }
  if (row == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) s_acc[wave][h][li * VEC + i] = acc[h][i];
      if (li == 0) {
        s_m[wave][h] = m[h];
        s_l[wave][h] = l[h];
      }
    }
  }
  __syncthreads();

  // Merge the 4 waves into this split's partial state (m, l, acc), one (head, d) cell per thread and round.
  constexpr int CPT = (G * D + kBlockThreads - 1) / kBlockThreads;
  float pm[CPT], pl[CPT], pa[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int idx = min(tid + c * kBlockThreads, G * D - 1);
    const int h = idx / D;
    const int d = idx % D;
    float M = s_m[0][h];
#pragma unroll
    for (int w = 1; w < kWavesPerBlock; ++w) M = fmaxf(M, s_m[w][h]);
    float ls = 0.0f, a = 0.0f;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) {
      const float cw = fast_exp2(s_m[w][h] - M);
      ls = fmaf(s_l[w][h], cw, ls);
      a = fmaf(s_acc[w][h][d], cw, a);
    }
    pm[c] = M;
    pl[c] = ls;
    pa[c] = a;
  }

  uint16_t* outb = static_cast<uint16_t*>(p.out) + b * p.out_stride_b;
  // QK: the prepared q goes out from the workgroup that writes the output, after every split of the pair has
  // read q (q_out may be q itself)
  auto write_out = [&](const float* ls, const float* a) {
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int idx = tid + c * kBlockThreads;
      if (idx < G * D) {
        const int hq = kvh * G + idx / D;
        // an empty sequence (l exactly 0) gives zeros; a NaN l (a poisoned fp8 row) stays NaN
        outb[hq * p.out_stride_h + idx % D] = from_f32<Q_DT>(ls[c] == 0.0f ? 0.0f : a[c] / ls[c]);
      }
    }
    if constexpr (QK) {
      if (p.q_out) {
        for (int pp = tid; pp < G * (D / 2); pp += kBlockThreads) {
          *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(p.q_out) + b * p.q_out_stride_b +
                                       (kvh * G + pp / (D / 2)) * p.q_out_stride_h + 2 * (pp % (D / 2))) = s_qk[pp];
        }
      }
    }
  };
  if (n_active == 1) {
    write_out(pl, pa);
    count_in();
    return;
  }

  // Publish this split's partial with agent-scope stores, wait until they have completed (vmcnt(0): on gfx950
  // an agent-scope store writes through to the device coherence point and is acknowledged from there), then
  // count in on the pair's arrival counter. The split that arrives last reads every split's partial with
  // agent-scope loads (which miss in the non-coherent caches and read that same point), combines them and
  // re-arms the counter. No workgroup ever waits for another.
  const int64_t pair_base = (static_cast<int64_t>(b) * p.num_q_heads + kvh * G) * p.max_splits;  // head h: + h * max_splits
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int idx = tid + c * kBlockThreads;
    if (idx < G * D) {
      const int64_t pidx = pair_base + (idx / D) * p.max_splits + split;
      store_agent(p.ws_acc + pidx * D + idx % D, pa[c]);
      if (idx % D == 0) {
        store_agent(p.ws_ml + 2 * pidx, pm[c]);
        store_agent(p.ws_ml + 2 * pidx + 1, pl[c]);
      }
    }
  }
  wait_vmem();
  __syncthreads();
  int32_t* const counter = p.ws_counter + (static_cast<int64_t>(b) * p.num_kv_heads + kvh) * p.counter_stride;
  if (tid == 0) {
    const int prev = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == n_active - 1) ? 1 : 0;
  }
  __syncthreads();
  if (!s_last) {
    count_in();
    return;
  }

  // The last arriver combines the n_active partials, in split order for every output cell.
  float rl[CPT], ra[CPT];
  if (n_active <= 8) {
    // Few splits: one (head, d) cell per thread and round, a batch of MB splits at a time for all of the thread's
    // cells: the batch's loads are issued unconditionally (past the last split they repeat it, masked below), so
    // they are in flight together and the merge costs ceil(n_active / MB) memory round trips (one unless a
    // thread has four cells); loads behind per-split branches would each end in a wait of their own.
    auto merge_cells = [&](auto mb_tag) {
      constexpr int MB = decltype(mb_tag)::value;
      float M[CPT], ls[CPT], a[CPT];
      int64_t hbase[CPT];
      int dcol[CPT];
#pragma unroll
      for (int c = 0; c < CPT; ++c) {
        const int idx = min(tid + c * kBlockThreads, G * D - 1);
        hbase[c] = pair_base + (idx / D) * p.max_splits;
        dcol[c] = idx % D;
        M[c] = kNegBig;
        ls[c] = 0.0f;
        a[c] = 0.0f;
      }
      for (int i0 = 0; i0 < n_active; i0 += MB) {
        float mi[CPT][MB], li[CPT][MB], ai[CPT][MB];
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
#pragma unroll
          for (int j = 0; j < MB; ++j) {
            const int i = min(i0 + j, n_active - 1);
            mi[c][j] = load_agent(p.ws_ml + 2 * (hbase[c] + i));
            li[c][j] = load_agent(p.ws_ml + 2 * (hbase[c] + i) + 1);
            ai[c][j] = load_agent(p.ws_acc + (hbase[c] + i) * D + dcol[c]);
          }
        }
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
#pragma unroll
          for (int j = 0; j < MB; ++j) {
            if (i0 + j < n_active) {
              const float mn = fmaxf(M[c], mi[c][j]);
              const float c_old = fast_exp2(M[c] - mn);
              const float c_new = fast_exp2(mi[c][j] - mn);
              ls[c] = ls[c] * c_old + li[c][j] * c_new;
              a[c] = a[c] * c_old + ai[c][j] * c_new;
              M[c] = mn;
            }
          }
        }
      }
#pragma unroll
      for (int c = 0; c < CPT; ++c) {
        rl[c] = ls[c];
        ra[c] = a[c];
      }
    };
    merge_cells(std::integral_constant<int, (CPT >= 4 ? 4 : 8)>{});
  } else {
    // Many splits: the partials' acc rows are read in 16-byte pieces. Thread t takes the 4 accumulator columns of
    // cell quad t % Q (Q = G * D / 4 quads: a head and 4 consecutive d) for the splits t / Q, t / Q + S, ...
    // (S = 256 / Q threads per quad): one 16-byte acc load and one 8-byte (m, l) load per split, both
    // agent-scope, a batch of MB of its splits at a time (issued unconditionally, as above), so the merge costs
    // ceil(ceil(n_active / S) / MB) memory round trips. Each thread combines its splits in order; the S states
    // of a quad are then combined in sub order through LDS.
    constexpr int Q = G * D / 4;
    constexpr int S = kBlockThreads / Q;
    static_assert(Q * 4 == G * D && S * Q == kBlockThreads, "cell quads must tile the workgroup");
    const int quad = tid % Q;
    const int sub = tid / Q;  // uniform across a wave whenever Q >= 64
    const int qh = quad / (D / 4);
    const auto acc_rsrc = __builtin_amdgcn_make_buffer_rsrc(p.ws_acc + pair_base * D, static_cast<short>(0),
                                                            0x7fffffff, 0x00020000);
    const uint64_t* const ml_base =
        reinterpret_cast<const uint64_t*>(p.ws_ml + 2 * (pair_base + static_cast<int64_t>(qh) * p.max_splits));
    const int acc_off = (qh * p.max_splits * D + (quad % (D / 4)) * 4) * 4;  // bytes, split 0
    float wm = kNegBig, wl = 0.0f, wa[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto merge_quads = [&](auto mb_tag) {
      constexpr int MB = decltype(mb_tag)::value;
      for (int i0 = sub; i0 < n_active; i0 += MB * S) {
        float4 ai[MB];
        uint64_t mli[MB];
#pragma unroll
        for (int j = 0; j < MB; ++j) {
          const int i = min(i0 + j * S, n_active - 1);
          ai[j] = __builtin_bit_cast(
              float4, __builtin_amdgcn_raw_buffer_load_b128(acc_rsrc, acc_off + i * D * 4, 0, kAuxSc1));
          mli[j] = __hip_atomic_load(const_cast<uint64_t*>(ml_base) + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int j = 0; j < MB; ++j) {
          if (i0 + j * S < n_active) {
            const float mi = __uint_as_float(static_cast<uint32_t>(mli[j]));
            const float li = __uint_as_float(static_cast<uint32_t>(mli[j] >> 32));
            const float mn = fmaxf(wm, mi);
            const float c_old = fast_exp2(wm - mn);
            const float c_new = fast_exp2(mi - mn);
            wl = wl * c_old + li * c_new;
            wa[0] = wa[0] * c_old + ai[j].x * c_new;
            wa[1] = wa[1] * c_old + ai[j].y * c_new;
            wa[2] = wa[2] * c_old + ai[j].z * c_new;
            wa[3] = wa[3] * c_old + ai[j].w * c_new;
            wm = mn;
          }
        }
      }
    };
    // batch: the thread's split count rounded up to a power of two, from 4 to 16 (96 registers of loads)
    const int per_thread = (n_active + S - 1) / S;
    if (per_thread > 8) merge_quads(std::integral_constant<int, 16>{});
    else if (per_thread > 4) merge_quads(std::integral_constant<int, 8>{});
    else merge_quads(std::integral_constant<int, 4>{});
    // LDS (the wave-merge area: every thread is past its last read of it): [thread] (m, l), then [thread] acc
    // quad; thread sub * Q + quad holds sub's state of the quad
    s_pool[2 * tid] = wm;
    s_pool[2 * tid + 1] = wl;
    reinterpret_cast<float4*>(s_pool + 2 * kBlockThreads)[tid] = make_float4(wa[0], wa[1], wa[2], wa[3]);
    __syncthreads();
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int idx = min(tid + c * kBlockThreads, G * D - 1);
      const int qd = idx / 4, col = idx % 4;
      float M = kNegBig, ls = 0.0f, a = 0.0f;
#pragma unroll
      for (int u = 0; u < S; ++u) {
        const int e = u * Q + qd;
        const float mi = s_pool[2 * e];
        const float mn = fmaxf(M, mi);
        const float c_old = fast_exp2(M - mn);
        const float c_new = fast_exp2(mi - mn);
        ls = ls * c_old + s_pool[2 * e + 1] * c_new;
        a = a * c_old + s_pool[2 * kBlockThreads + 4 * e + col] * c_new;
        M = mn;
      }
      rl[c] = ls;
      ra[c] = a;
    }
  }
  write_out(rl, ra);
  if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  count_in();
}

}  // namespace aicas
