// Split-K GQA decode attention for q_len == 1 (flash-decoding), VALU only, with an optional fused KV append.
//
// Computes, for every batch row b and query head hq (kv head hq / G):
//   out[b, hq, :] = softmax(q[b, hq] . K[b, hq/G, :L_b]^T * sm_scale) . V[b, hq/G, :L_b]
// which is what the reference decode path returns (triton_qwen3vl/gqa_decode_attention.py:46-141 and its
// oracle, SDPA over repeat_kv, triton_qwen3vl/fallback.py:7-64), with per-sequence lengths L_b.
//
// Work decomposition: one 256-thread workgroup per (split, kv head, batch row); a split is a range of
// tokens_per_split tokens. Every K/V row is read once and serves all G query heads of the group. A row of D
// elements is spread over R = D / VEC lanes (16 bytes per lane), so one wave load instruction covers 64 / R
// consecutive tokens (1 KiB). Loads are double-buffered in registers: the next chunk of U tokens per lane is
// in flight while the current one is consumed, which keeps ~16 KiB per wave outstanding.
//
// Each R-lane row group keeps its own online-softmax state (running max m, sum l, accumulator acc) in fp32
// in the exp2 domain; the states are merged across the row groups of a wave with lane shuffles and across the
// 4 waves through LDS.
//
// Split merge: a split writes its unnormalised (m, l, acc) to the workspace with agent-scope stores (these
// write through to the device coherence point, so no L2 writeback is needed), waits for them to complete,
// and bumps the (b, kv head) arrival counter. The split that arrives last reads every split's partial with
// agent-scope loads and combines them: M = max m_i, l = sum l_i 2^(m_i - M), out = sum acc_i 2^(m_i - M) / l;
// it then re-arms the counter to zero. Nothing ever waits on another workgroup. Sequences that need one split
// write the output directly.
//
// Prologue: q and, for contiguous caches whose lengths the caller bounds from below (spec_len), the first
// chunk of K/V are fetched before the lengths are read, so that their latencies overlap.
//
// Fused append (APPEND): positions[b] is the length before this step; the kernel attends over
// L_b = positions[b] + 1 tokens, takes token L_b - 1 from the new rows (k_new / v_new) instead of the cache,
// and the workgroup that owns that token writes the row into the cache (quantized on write for fp8 caches,
// with the attention then using the dequantised row, exactly what a separate append followed by attention
// would read). Every workgroup of batch row b counts itself in when it exits (it read positions[b] at the
// start); the last one to do so stores positions[b] + 1 to seq_lens_out[b] (which may alias positions), so
// no workgroup can read a bumped length.
#pragma once

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
  int32_t tokens_per_split;
  int32_t max_splits;  // == gridDim.x
  int32_t page_shift;  // log2(page_size) for paged caches
  float scale_log2;    // sm_scale * log2(e)
  float* ws_ml;        // [B * Hq * max_splits][2]  (m, l)
  float* ws_acc;       // [B * Hq * max_splits][D]
  int32_t* ws_counter; // [B * Hkv] split arrivals, zero between launches
  int32_t* ws_arrive;  // [B] APPEND: workgroups that have read positions[b], zero between launches
  int32_t* status;
  // APPEND only
  const void* k_new;
  const void* v_new;
  int64_t kn_stride_b, kn_stride_h, vn_stride_b, vn_stride_h;
  int32_t* seq_lens_out;
  int32_t spec_len;  // caller-guaranteed lower bound on every sequence's cached length (0: none)
};

constexpr int kMaxBlockEntries = 1024;  // block-table entries one split may touch (LDS cache)
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

// vmcnt(0): wait until this wave's vector memory operations (loads and stores) have completed.
__device__ __forceinline__ void wait_vmem() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__device__ __forceinline__ void store_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int KV_DT, int U>
struct Chunk {
  uint4 k[U];
  uint4 v[U];
  float ks[U];
  float vs[U];
  bool ok[U];
};

template <int Q_DT, int KV_DT, int D, int G, bool PAGED, bool APPEND>
__global__ __launch_bounds__(kBlockThreads) void decode_attn_kernel(DecodeParams p) {
  using Tr = KVTraits<KV_DT>;
  constexpr int EB = Tr::kElemBytes;
  constexpr int VEC = Tr::kVec;
  constexpr int U = Tr::kUnroll;
  constexpr int R = D / VEC;            // lanes per row
  constexpr int RPW = kWave / R;        // rows per wave per load
  constexpr int RPB = RPW * kWavesPerBlock;
  constexpr int TPI = RPB * U;          // tokens per workgroup chunk
  static_assert(R >= 1 && R <= 16, "a row must fit one DPP row");
  constexpr bool FP8 = (KV_DT == kFP8E4M3);

  __shared__ float s_m[kWavesPerBlock][G];
  __shared__ float s_l[kWavesPerBlock][G];
  __shared__ float s_acc[kWavesPerBlock][G][D];
  __shared__ int32_t s_bt[PAGED ? kMaxBlockEntries : 1];
  __shared__ int32_t s_len;
  __shared__ int32_t s_last;
  // APPEND: the new token's rows as the attention must see them (dequantised codes for fp8 caches)
  __shared__ uint4 s_new[APPEND ? 2 * R : 1];
  __shared__ float s_new_scale[APPEND && FP8 ? 2 : 1];

  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int row = lane / R;
  const int li = lane % R;

  // Query slices of the G heads served by this kv head (independent of the lengths: issued first).
  const uint16_t* qb = static_cast<const uint16_t*>(p.q) + b * p.q_stride_b;
  uint32_t qp[G][FP8 ? 1 : VEC / 2];
  float qf[G][FP8 ? VEC : 1];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const uint16_t* qh = qb + (kvh * G + h) * p.q_stride_h + li * VEC;
    if constexpr (!FP8) {
      const uint4 w = *reinterpret_cast<const uint4*>(qh);
      qp[h][0] = w.x;
      qp[h][1] = w.y;
      qp[h][2] = w.z;
      qp[h][3] = w.w;
    } else {
#pragma unroll
      for (int c = 0; c < VEC / 8; ++c) {
        const uint4 w = *reinterpret_cast<const uint4*>(qh + 8 * c);
        unpack2<Q_DT>(w.x, qf[h][8 * c + 0], qf[h][8 * c + 1]);
        unpack2<Q_DT>(w.y, qf[h][8 * c + 2], qf[h][8 * c + 3]);
        unpack2<Q_DT>(w.z, qf[h][8 * c + 4], qf[h][8 * c + 5]);
        unpack2<Q_DT>(w.w, qf[h][8 * c + 6], qf[h][8 * c + 7]);
      }
    }
  }

  const uint8_t* kbase = static_cast<const uint8_t*>(p.cache.k);
  const uint8_t* vbase = static_cast<const uint8_t*>(p.cache.v);
  const int64_t head_off = static_cast<int64_t>(kvh) * p.cache.stride_h;
  const int64_t shead_off = static_cast<int64_t>(kvh) * p.cache.scale_stride_h;
  const int page_mask = (1 << p.page_shift) - 1;
  const int tps = p.tokens_per_split;
  const int t_begin = split * tps;
  // Clamp so that no access leaves the cache or the launched split range.
  const int limit = min(p.cache.max_tokens, tps * p.max_splits);

  // Contiguous caches whose every sequence is known (spec_len, from the caller) to hold the first chunk of this
  // split: fetch that chunk now, so that it overlaps the read of the lengths.
  Chunk<KV_DT, U> ca, cb;
  const bool spec = !PAGED && t_begin + TPI <= p.spec_len && t_begin + TPI <= limit;
  if (spec) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = t_begin + u * RPB + wave * RPW + row;
      const int64_t off = static_cast<int64_t>(b) * p.cache.stride_blk + head_off +
                          static_cast<int64_t>(t) * p.cache.stride_t;
      ca.k[u] = *reinterpret_cast<const uint4*>(kbase + off * EB + li * 16);
      ca.v[u] = *reinterpret_cast<const uint4*>(vbase + off * EB + li * 16);
      if constexpr (FP8) {
        const int64_t soff = static_cast<int64_t>(b) * p.cache.scale_stride_blk + shead_off + t;
        ca.ks[u] = p.cache.k_scale[soff];
        ca.vs[u] = p.cache.v_scale[soff];
      } else {
        ca.ks[u] = 0.0f;
        ca.vs[u] = 0.0f;
      }
      ca.ok[u] = true;
    }
  }

  // Sequence length (cached tokens before this step's append for APPEND).
  if (tid == 0) s_len = p.seq_lens ? p.seq_lens[b] : p.uniform_len;
  __syncthreads();
  int L = s_len;
  const int len_read = L;
  // APPEND with seq_lens_out: every workgroup counts itself in on its way out (thread 0's read of positions[b]
  // completed long before: its value went to LDS ahead of the barrier above); the last of the batch row's
  // workgroups stores the bumped length, so no workgroup can read it. Counting in at exit keeps the
  // contended atomic off the start of the stream.
  auto count_in = [&]() {
    if constexpr (APPEND) {
      if (tid == 0 && p.seq_lens_out) {
        const int readers = gridDim.x * gridDim.y;
        const int prev = __hip_atomic_fetch_add(p.ws_arrive + b, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (prev == readers - 1) {
          p.seq_lens_out[b] = len_read + 1;
          __hip_atomic_store(p.ws_arrive + b, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
  const int n_active = L > 0 ? (L + tps - 1) / tps : 1;
  if (split >= n_active) {
    count_in();
    return;
  }
  const int t_end = min(t_begin + tps, L);

  // Paged caches: stage this split's block ids in LDS (invalid ids become -1 and their tokens are skipped).
  int first_entry = 0;
  if constexpr (PAGED) {
    first_entry = t_begin >> p.page_shift;
    const int n_ent = t_end > t_begin ? ((t_end - 1) >> p.page_shift) - first_entry + 1 : 0;
    const int32_t* bt = p.cache.block_table + static_cast<int64_t>(b) * p.cache.block_table_stride + first_entry;
    for (int i = tid; i < n_ent; i += kBlockThreads) {
      int32_t blk = bt[i];
      if (blk < 0 || blk >= p.cache.num_blocks) {
        if (p.status) atomicOr(p.status, kStatusBlockOutOfRange);
        blk = -1;
      }
      s_bt[i] = blk;
    }
  }
  // APPEND: the workgroup owning the new token writes its rows into the cache and stages them in LDS.
  if constexpr (APPEND) {
    if (t_new >= t_begin && t_new < t_end && tid < 2 * R) {
      const int which = tid / R;  // 0 = K, 1 = V
      const int c = tid % R;
      const uint16_t* src = which == 0
          ? static_cast<const uint16_t*>(p.k_new) + b * p.kn_stride_b + kvh * p.kn_stride_h
          : static_cast<const uint16_t*>(p.v_new) + b * p.vn_stride_b + kvh * p.vn_stride_h;
      int64_t blk = b;
      int tin = t_new;
      bool ok = true;
      if constexpr (PAGED) {
        blk = p.cache.block_table[static_cast<int64_t>(b) * p.cache.block_table_stride + (t_new >> p.page_shift)];
        tin = t_new & page_mask;
        ok = blk >= 0 && blk < p.cache.num_blocks;
      }
      const int64_t off = blk * p.cache.stride_blk + head_off + static_cast<int64_t>(tin) * p.cache.stride_t;
      void* dst_base = which == 0 ? p.cache.k : p.cache.v;
      if constexpr (!FP8) {
        const uint4 x = *reinterpret_cast<const uint4*>(src + c * VEC);
        if (ok) *reinterpret_cast<uint4*>(static_cast<uint16_t*>(dst_base) + off + c * VEC) = x;
        s_new[tid] = x;
      } else {
        // VEC = 16 source elements (32 bytes) per lane -> 16 codes
        float f[VEC];
        const uint4 x0 = *reinterpret_cast<const uint4*>(src + c * VEC);
        const uint4 x1 = *reinterpret_cast<const uint4*>(src + c * VEC + 8);
        const uint32_t w[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) unpack2<Q_DT>(w[i], f[2 * i], f[2 * i + 1]);
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < VEC; ++i) amax = fmaxf(amax, fabsf(f[i]));
        amax = group_max<R>(amax);
        const float scale = amax / 448.0f;
        uint32_t packed[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          uint32_t code = 0u;
          if (scale > 0.0f) code = f32_to_e4m3(fminf(fmaxf(f[i] / scale, -448.0f), 448.0f));
          packed[i / 4] |= code << (8 * (i % 4));
        }
        const uint4 codes = make_uint4(packed[0], packed[1], packed[2], packed[3]);
        if (ok) {
          *reinterpret_cast<uint4*>(static_cast<uint8_t*>(dst_base) + off + c * VEC) = codes;
          if (c == 0) {
            const int64_t soff = blk * p.cache.scale_stride_blk + shead_off + tin;
            (which == 0 ? p.cache.k_scale : p.cache.v_scale)[soff] = scale;
          }
        }
        s_new[tid] = codes;
        if (c == 0) s_new_scale[which] = scale;
      }
    }
  }
  __syncthreads();

  auto load_chunk = [&](Chunk<KV_DT, U>& c, int t0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = t0 + u * RPB + wave * RPW + row;
      bool ok = t < t_end;
      c.k[u] = make_uint4(0u, 0u, 0u, 0u);
      c.v[u] = make_uint4(0u, 0u, 0u, 0u);
      c.ks[u] = 0.0f;
      c.vs[u] = 0.0f;
      // only the split that owns the new token (t < t_end) staged its rows in LDS
      if (APPEND && ok && t == t_new) {
        c.k[u] = s_new[li];
        c.v[u] = s_new[R + li];
        if constexpr (FP8) {
          c.ks[u] = s_new_scale[0];
          c.vs[u] = s_new_scale[1];
        }
        c.ok[u] = true;
        continue;
      }
      int64_t blk = b;
      int tin = t;
      if constexpr (PAGED) {
        if (ok) {
          blk = s_bt[(t >> p.page_shift) - first_entry];
          tin = t & page_mask;
          ok = blk >= 0;
        }
      }
      if (ok) {
        const int64_t off = blk * p.cache.stride_blk + head_off + static_cast<int64_t>(tin) * p.cache.stride_t;
        c.k[u] = *reinterpret_cast<const uint4*>(kbase + off * EB + li * 16);
        c.v[u] = *reinterpret_cast<const uint4*>(vbase + off * EB + li * 16);
        if constexpr (FP8) {
          const int64_t soff = blk * p.cache.scale_stride_blk + shead_off + tin;
          c.ks[u] = p.cache.k_scale[soff];
          c.vs[u] = p.cache.v_scale[soff];
        }
      }
      c.ok[u] = ok;
    }
  };

  float m[G], l[G], acc[G][VEC];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = kNegBig;
    l[h] = 0.0f;
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[h][i] = 0.0f;
  }

  auto consume = [&](const Chunk<KV_DT, U>& c) {
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
        float kf[VEC];
        const uint32_t kw[4] = {c.k[u].x, c.k[u].y, c.k[u].z, c.k[u].w};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(kw[w]), false);
          const f32x2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(kw[w]), true);
          kf[4 * w + 0] = lo.x;
          kf[4 * w + 1] = lo.y;
          kf[4 * w + 2] = hi.x;
          kf[4 * w + 3] = hi.y;
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
          float d = 0.0f;
#pragma unroll
          for (int i = 0; i < VEC; ++i) d = fmaf(qf[h][i], kf[i], d);
          s[u][h] = group_sum<R>(d) * (p.scale_log2 * c.ks[u]);
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
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float vf[VEC];
      const uint32_t vw[4] = {c.v[u].x, c.v[u].y, c.v[u].z, c.v[u].w};
      if constexpr (!FP8) {
#pragma unroll
        for (int w = 0; w < 4; ++w) unpack2<KV_DT>(vw[w], vf[2 * w], vf[2 * w + 1]);
      } else {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(vw[w]), false);
          const f32x2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(vw[w]), true);
          vf[4 * w + 0] = lo.x;
          vf[4 * w + 1] = lo.y;
          vf[4 * w + 2] = hi.x;
          vf[4 * w + 3] = hi.y;
        }
      }
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float pu = fast_exp2(s[u][h] - mnew[h]);
        l[h] += pu;
        const float pv = FP8 ? pu * c.vs[u] : pu;
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[h][i] = fmaf(pv, vf[i], acc[h][i]);
      }
    }
  };

  // Double-buffered token loop: chunk j+1 is in flight while chunk j is consumed.
  {
    int t0 = t_begin;
    if (!spec && t0 < t_end) load_chunk(ca, t0);
    while (t0 < t_end) {
      const int t1 = t0 + TPI;
      if (t1 < t_end) load_chunk(cb, t1);
      consume(ca);
      if (t1 >= t_end) break;
      const int t2 = t1 + TPI;
      if (t2 < t_end) load_chunk(ca, t2);
      consume(cb);
      t0 = t2;
    }
  }

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

  // Merge the 4 waves; either finish the output (one split) or publish this split's partial state.
  const bool single = (n_active == 1);
  uint16_t* outb = static_cast<uint16_t*>(p.out) + b * p.out_stride_b;
  for (int idx = tid; idx < G * D; idx += kBlockThreads) {
    const int h = idx / D;
    const int d = idx % D;
    float M = s_m[0][h];
#pragma unroll
    for (int w = 1; w < kWavesPerBlock; ++w) M = fmaxf(M, s_m[w][h]);
    float ls = 0.0f, a = 0.0f;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) {
      const float c = fast_exp2(s_m[w][h] - M);
      ls = fmaf(s_l[w][h], c, ls);
      a = fmaf(s_acc[w][h][d], c, a);
    }
    const int hq = kvh * G + h;
    if (single) {
      outb[hq * p.out_stride_h + d] = from_f32<Q_DT>(ls > 0.0f ? a / ls : 0.0f);
    } else {
      const int64_t pidx = (static_cast<int64_t>(b) * p.num_q_heads + hq) * p.max_splits + split;
      store_agent(p.ws_acc + pidx * D + d, a);
      if (d == 0) {
        store_agent(p.ws_ml + 2 * pidx, M);
        store_agent(p.ws_ml + 2 * pidx + 1, ls);
      }
    }
  }
  if (single) {
    count_in();
    return;
  }

  // Arrival: the partial stores above are complete (device-visible) before the counter moves.
  wait_vmem();
  __syncthreads();
  int32_t* counter = p.ws_counter + static_cast<int64_t>(b) * p.num_kv_heads + kvh;
  if (tid == 0) {
    const int prev = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == n_active - 1) ? 1 : 0;
  }
  __syncthreads();
  if (!s_last) {
    count_in();
    return;
  }

  // One online pass over the splits, MB at a time: the MB partials' loads are independent and in flight
  // together, so the merge costs about n_active / MB memory round trips.
  constexpr int MB = 8;
  for (int idx = tid; idx < G * D; idx += kBlockThreads) {
    const int h = idx / D;
    const int d = idx % D;
    const int hq = kvh * G + h;
    const int64_t base = (static_cast<int64_t>(b) * p.num_q_heads + hq) * p.max_splits;
    float M = kNegBig, ls = 0.0f, a = 0.0f;
    for (int i0 = 0; i0 < n_active; i0 += MB) {
      float mi[MB], li[MB], ai[MB];
#pragma unroll
      for (int j = 0; j < MB; ++j) {
        const int i = min(i0 + j, n_active - 1);  // duplicates of the last split are masked below
        mi[j] = load_agent(p.ws_ml + 2 * (base + i));
        li[j] = load_agent(p.ws_ml + 2 * (base + i) + 1);
        ai[j] = load_agent(p.ws_acc + (base + i) * D + d);
      }
#pragma unroll
      for (int j = 0; j < MB; ++j) {
        if (i0 + j < n_active) {
          const float mn = fmaxf(M, mi[j]);
          const float c_old = fast_exp2(M - mn);
          const float c_new = fast_exp2(mi[j] - mn);
          ls = ls * c_old + li[j] * c_new;
          a = a * c_old + ai[j] * c_new;
          M = mn;
        }
      }
    }
    outb[hq * p.out_stride_h + d] = from_f32<Q_DT>(ls > 0.0f ? a / ls : 0.0f);
  }
  if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  count_in();
}

}  // namespace aicas
