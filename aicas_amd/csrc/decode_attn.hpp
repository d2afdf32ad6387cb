// Split-K GQA decode attention for q_len == 1 (flash-decoding), VALU only.
//
// Computes, for every batch row b and query head hq (kv head hq / G):
//   out[b, hq, :] = softmax(q[b, hq] . K[b, hq/G, :L_b]^T * sm_scale) . V[b, hq/G, :L_b]
// which is what the reference decode path returns (triton_qwen3vl/gqa_decode_attention.py:46-141 and its
// oracle, SDPA over repeat_kv, triton_qwen3vl/fallback.py:7-64), with per-sequence lengths L_b.
//
// Work decomposition: one 256-thread workgroup per (split, kv head, batch row). A split is a range of
// tokens_per_split tokens. Inside a workgroup every K/V row is read once and serves all G query heads of
// the group. A row of D elements is spread over R = D / VEC lanes (16 bytes per lane), so one wave load
// instruction covers 64 / R consecutive tokens. Each R-lane group keeps its own online-softmax state
// (running max m, sum l, accumulator acc) in fp32, in the exp2 domain; the states are merged across the
// groups of a wave with lane shuffles and across the 4 waves through LDS.
//
// A split writes its unnormalised (m, l, acc) to the workspace; the last split of a (b, kv head) to finish
// (an atomic arrival counter) merges all of them: M = max m_i, l = sum l_i 2^(m_i - M),
// out = sum acc_i 2^(m_i - M) / l, and re-arms the counter to zero for the next launch. Sequences that need
// only one split write the output directly.
#pragma once

#include "common.hpp"

namespace aicas {

struct DecodeParams {
  KVLayout cache;
  const void* q;
  int64_t q_stride_b, q_stride_h;  // elements; head_dim stride is 1
  void* out;
  int64_t out_stride_b, out_stride_h;
  const int32_t* seq_lens;  // nullptr: every sequence has uniform_len tokens
  int32_t uniform_len;
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t tokens_per_split;
  int32_t max_splits;  // == gridDim.x
  int32_t page_shift;  // log2(page_size) for paged caches
  float scale_log2;    // sm_scale * log2(e)
  float* ws_ml;        // [B * Hq * max_splits][2]  (m, l)
  float* ws_acc;       // [B * Hq * max_splits][D]
  int32_t* ws_counter; // [B * Hkv], zero between launches
  int32_t* status;
};

constexpr int kMaxBlockEntries = 1024;  // block-table entries one split may touch (LDS cache)
constexpr float kNegBig = -1.0e30f;     // finite "minus infinity" for running maxima

template <int KV_DT>
struct KVTraits {
  static constexpr int kElemBytes = (KV_DT == kFP8E4M3) ? 1 : 2;
  static constexpr int kVec = 16 / kElemBytes;      // elements per lane per row
  static constexpr int kUnroll = (KV_DT == kFP8E4M3) ? 2 : 4;  // tokens per lane per iteration
};

template <int Q_DT, int KV_DT, int D, int G, bool PAGED>
__global__ __launch_bounds__(kBlockThreads) void decode_attn_kernel(DecodeParams p) {
  using Tr = KVTraits<KV_DT>;
  constexpr int EB = Tr::kElemBytes;
  constexpr int VEC = Tr::kVec;
  constexpr int U = Tr::kUnroll;
  constexpr int R = D / VEC;            // lanes per row
  constexpr int RPW = kWave / R;        // rows per wave per load
  constexpr int RPB = RPW * kWavesPerBlock;
  constexpr int TPI = RPB * U;          // tokens per workgroup iteration
  static_assert(R >= 1 && R <= 16, "a row must fit one DPP row");
  constexpr bool FP8 = (KV_DT == kFP8E4M3);

  __shared__ float s_m[kWavesPerBlock][G];
  __shared__ float s_l[kWavesPerBlock][G];
  __shared__ float s_acc[kWavesPerBlock][G][D];
  __shared__ int32_t s_bt[PAGED ? kMaxBlockEntries : 1];
  __shared__ int32_t s_last;

  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int row = lane / R;
  const int li = lane % R;

  // Sequence length, clamped so that no access leaves the cache or the launched split range.
  int L = p.seq_lens ? p.seq_lens[b] : p.uniform_len;
  const int limit = min(p.cache.max_tokens, p.tokens_per_split * p.max_splits);
  if (L > limit) {
    if (p.status && split == 0 && tid == 0) atomicOr(p.status, kStatusLenClamped);
    L = limit;
  }
  if (L < 0) L = 0;
  const int tps = p.tokens_per_split;
  const int n_active = L > 0 ? (L + tps - 1) / tps : 1;
  if (split >= n_active) return;
  const int t_begin = split * tps;
  const int t_end = min(t_begin + tps, L);

  // Query slices of the G heads served by this kv head.
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
    __syncthreads();
  }

  const uint8_t* kbase = static_cast<const uint8_t*>(p.cache.k);
  const uint8_t* vbase = static_cast<const uint8_t*>(p.cache.v);
  const int64_t head_off = static_cast<int64_t>(kvh) * p.cache.stride_h;
  const int64_t shead_off = static_cast<int64_t>(kvh) * p.cache.scale_stride_h;
  const int page_mask = (1 << p.page_shift) - 1;

  float m[G], l[G], acc[G][VEC];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = kNegBig;
    l[h] = 0.0f;
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[h][i] = 0.0f;
  }

  for (int t0 = t_begin; t0 < t_end; t0 += TPI) {
    uint4 kr[U], vr[U];
    float ks[U], vs[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = t0 + u * RPB + wave * RPW + row;
      ok[u] = t < t_end;
      kr[u] = make_uint4(0u, 0u, 0u, 0u);
      vr[u] = make_uint4(0u, 0u, 0u, 0u);
      ks[u] = 0.0f;
      vs[u] = 0.0f;
      int64_t blk = b;
      int tin = t;
      if constexpr (PAGED) {
        if (ok[u]) {
          blk = s_bt[(t >> p.page_shift) - first_entry];
          tin = t & page_mask;
          ok[u] = blk >= 0;
        }
      }
      if (ok[u]) {
        const int64_t off = blk * p.cache.stride_blk + head_off + static_cast<int64_t>(tin) * p.cache.stride_t;
        kr[u] = *reinterpret_cast<const uint4*>(kbase + off * EB + li * 16);
        vr[u] = *reinterpret_cast<const uint4*>(vbase + off * EB + li * 16);
        if constexpr (FP8) {
          const int64_t soff = blk * p.cache.scale_stride_blk + shead_off + tin;
          ks[u] = p.cache.k_scale[soff];
          vs[u] = p.cache.v_scale[soff];
        }
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
          d = dot2<KV_DT>(qp[h][0], kr[u].x, d);
          d = dot2<KV_DT>(qp[h][1], kr[u].y, d);
          d = dot2<KV_DT>(qp[h][2], kr[u].z, d);
          d = dot2<KV_DT>(qp[h][3], kr[u].w, d);
          s[u][h] = group_sum<R>(d) * p.scale_log2;
        }
      } else {
        float kf[VEC];
        const uint32_t kw[4] = {kr[u].x, kr[u].y, kr[u].z, kr[u].w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(kw[c]), false);
          const f32x2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(kw[c]), true);
          kf[4 * c + 0] = lo.x;
          kf[4 * c + 1] = lo.y;
          kf[4 * c + 2] = hi.x;
          kf[4 * c + 3] = hi.y;
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
          float d = 0.0f;
#pragma unroll
          for (int i = 0; i < VEC; ++i) d = fmaf(qf[h][i], kf[i], d);
          s[u][h] = group_sum<R>(d) * (p.scale_log2 * ks[u]);
        }
      }
#pragma unroll
      for (int h = 0; h < G; ++h) s[u][h] = ok[u] ? s[u][h] : -__builtin_inff();
    }

    // Values as fp32.
    float vf[U][VEC];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t vw[4] = {vr[u].x, vr[u].y, vr[u].z, vr[u].w};
      if constexpr (!FP8) {
#pragma unroll
        for (int c = 0; c < 4; ++c) unpack2<KV_DT>(vw[c], vf[u][2 * c], vf[u][2 * c + 1]);
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(vw[c]), false);
          const f32x2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(vw[c]), true);
          vf[u][4 * c + 0] = lo.x;
          vf[u][4 * c + 1] = lo.y;
          vf[u][4 * c + 2] = hi.x;
          vf[u][4 * c + 3] = hi.y;
        }
      }
    }

    // Online softmax update.
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float mx = s[0][h];
#pragma unroll
      for (int u = 1; u < U; ++u) mx = fmaxf(mx, s[u][h]);
      const float mnew = fmaxf(m[h], mx);
      const float alpha = fast_exp2(m[h] - mnew);
      l[h] *= alpha;
#pragma unroll
      for (int i = 0; i < VEC; ++i) acc[h][i] *= alpha;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float pu = fast_exp2(s[u][h] - mnew);
        l[h] += pu;
        const float pv = FP8 ? pu * vs[u] : pu;
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[h][i] = fmaf(pv, vf[u][i], acc[h][i]);
      }
      m[h] = mnew;
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
      p.ws_acc[pidx * D + d] = a;
      if (d == 0) {
        p.ws_ml[2 * pidx] = M;
        p.ws_ml[2 * pidx + 1] = ls;
      }
    }
  }
  if (single) return;

  // Arrival: the last split of this (b, kv head) merges every split's partial state.
  __threadfence();
  __syncthreads();
  int32_t* counter = p.ws_counter + static_cast<int64_t>(b) * p.num_kv_heads + kvh;
  if (tid == 0) {
    const int prev = atomicAdd(counter, 1);
    s_last = (prev == n_active - 1) ? 1 : 0;
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  for (int idx = tid; idx < G * D; idx += kBlockThreads) {
    const int h = idx / D;
    const int d = idx % D;
    const int hq = kvh * G + h;
    const int64_t base = (static_cast<int64_t>(b) * p.num_q_heads + hq) * p.max_splits;
    float M = kNegBig;
    for (int i = 0; i < n_active; ++i) M = fmaxf(M, p.ws_ml[2 * (base + i)]);
    float ls = 0.0f, a = 0.0f;
    for (int i = 0; i < n_active; ++i) {
      const float c = fast_exp2(p.ws_ml[2 * (base + i)] - M);
      ls = fmaf(p.ws_ml[2 * (base + i) + 1], c, ls);
      a = fmaf(p.ws_acc[(base + i) * D + d], c, a);
    }
    outb[hq * p.out_stride_h + d] = from_f32<Q_DT>(ls > 0.0f ? a / ls : 0.0f);
  }
  if (tid == 0) *counter = 0;
}

}  // namespace aicas
