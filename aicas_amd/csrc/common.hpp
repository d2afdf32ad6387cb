// Shared device helpers for the KV-append and decode-attention kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace aicas {

// Element types understood by the kernels. The numeric values are part of the C ABI.
enum DType : int32_t { kBF16 = 0, kFP16 = 1, kFP8E4M3 = 2 };

// Status bits that kernels OR into an optional device status word when they had to clamp an
// out-of-range length, position or block id instead of touching memory they do not own.
enum StatusBits : int32_t {
  kStatusLenClamped = 1,      // seq_len exceeded what the cache (or the block table) can hold
  kStatusBlockOutOfRange = 2, // a block-table entry was outside [0, num_blocks)
  kStatusAppendOverflow = 4,  // an append position was outside the cache; the row was dropped
  kStatusOutOfBlocks = 8,     // the block pool ran out: a page was left without a block
  kStatusNonFiniteRow = 16,   // an fp8 cache received a row holding NaN or +-Inf (stored poisoned)
};

constexpr int kWave = 64;
constexpr int kBlockThreads = 256;
constexpr int kWavesPerBlock = kBlockThreads / kWave;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float f16lo(uint32_t w) {
  return static_cast<float>(__builtin_bit_cast(f16x2_t, w).x);
}
__device__ __forceinline__ float f16hi(uint32_t w) {
  return static_cast<float>(__builtin_bit_cast(f16x2_t, w).y);
}

// Two 16-bit values packed in one dword -> two floats.
template <int DT>
__device__ __forceinline__ void unpack2(uint32_t w, float& lo, float& hi) {
  if constexpr (DT == kBF16) {
    lo = bf16lo(w);
    hi = bf16hi(w);
  } else {
    lo = f16lo(w);
    hi = f16hi(w);
  }
}

// acc + a.lo*b.lo + a.hi*b.hi with both products exact (16-bit inputs) and fp32 accumulation.
template <int DT>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
  if constexpr (DT == kBF16) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b),
                                           acc, false);
  } else {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b), acc, false);
  }
}

// Two OCP e4m3 codes of w (bytes 0-1, or 2-3 when HI) -> the same two values in the 16-bit type DT, packed
// lo in the low half. Exact: every e4m3 value (subnormals included) is a bf16 and an fp16 value. One
// v_cvt_scalef32_pk_{bf16,f16}_fp8 with unit scale on gfx950.
template <int DT, bool HI>
__device__ __forceinline__ uint32_t e4m3x2_to_16(uint32_t w) {
  if constexpr (DT == kBF16) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI));
  }
}

// float -> bf16 bits, round to nearest even, NaN kept NaN (torch's float->bfloat16 rule): one
// v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f)); }

template <int DT>
__device__ __forceinline__ uint16_t from_f32(float f) {
  if constexpr (DT == kBF16) {
    return f32_to_bf16(f);
  } else {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  }
}

// f rounded to the 16-bit type DT (nearest even) and widened back: the value a DT tensor stores for f.
template <int DT>
__device__ __forceinline__ float round_to(float f) {
  if constexpr (DT == kBF16) {
    return static_cast<float>(static_cast<__bf16>(f));
  } else {
    return static_cast<float>(static_cast<_Float16>(f));
  }
}

// Two floats rounded to DT (nearest even) and packed into one dword, lo in the low half (bf16: one
// v_cvt_pk_bf16_f32 for both).
template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (DT == kBF16) {
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
  } else {
    return static_cast<uint32_t>(from_f32<DT>(lo)) | (static_cast<uint32_t>(from_f32<DT>(hi)) << 16);
  }
}

// OCP FP8 E4M3 ("e4m3fn": bias 7, no infinities, S.1111.111 is NaN, max finite 448).
// Encoder written out from the format: round to nearest even; |x| is expected to be <= 448 already (callers
// clamp), and NaN maps to 0x7f with the sign kept. The kernels encode with e4m3x4 (the hardware conversion);
// this is what aicas_calib_fp8_encoder_check holds it to.
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t mag = u & 0x7fffffffu;
  if (mag > 0x7f800000u) return sign | 0x7fu;
  if (mag >= 0x43e00000u) return sign | 0x7eu;  // |x| >= 448
  if (mag < 0x3c800000u) {
    // |x| < 2^-6: subnormal range, value = m * 2^-9 with m in [0, 8]; m == 8 is the smallest normal.
    const float scaled = __uint_as_float(mag) * 512.0f;  // exact (power-of-two scaling)
    return sign | static_cast<uint32_t>(__builtin_rintf(scaled));  // rint = round half to even
  }
  const uint32_t exp = (mag >> 23) - 127u + 7u;  // in [1, 15]
  const uint32_t man = mag & 0x7fffffu;
  uint32_t m3 = man >> 20;
  const uint32_t rem = man & 0xfffffu;
  if (rem > 0x80000u || (rem == 0x80000u && (m3 & 1u))) m3 += 1u;
  return sign | ((exp << 3) + m3);  // a mantissa carry rolls into the exponent field
}

// Four floats with |x| <= 448 -> their OCP e4m3 codes (round to nearest even), byte i the code of the i-th: two
// gfx950 v_cvt_pk_fp8_f32. On that domain (both zeros and the subnormals included) it gives f32_to_e4m3's codes
// for every float; libaicas_calib.so's aicas_calib_fp8_encoder_check compares the two over all of them.
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false));
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(c, d, static_cast<int>(lo), true));
}

// Cross-lane reductions inside aligned groups of N lanes (N <= 16, one DPP row), result in every lane.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

template <int N>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (N >= 2) x += dpp_f32<0xB1>(x);   // quad_perm [1,0,3,2]
  if constexpr (N >= 4) x += dpp_f32<0x4E>(x);   // quad_perm [2,3,0,1]
  if constexpr (N >= 8) x += dpp_f32<0x141>(x);  // row_half_mirror
  if constexpr (N >= 16) x += dpp_f32<0x140>(x); // row_mirror
  return x;
}

template <int N>
__device__ __forceinline__ uint32_t group_max_u32(uint32_t x) {
  if constexpr (N >= 2) x = max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0xB1, 0xF, 0xF, false)));
  if constexpr (N >= 4) x = max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x4E, 0xF, 0xF, false)));
  if constexpr (N >= 8) x = max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x141, 0xF, 0xF, false)));
  if constexpr (N >= 16) x = max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x140, 0xF, 0xF, false)));
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// amax / 448 correctly rounded: for amax >= 2^-100 from the constant y = 1 / 448 (correctly rounded at compile
// time), q0 = amax * y and one correction q0 + (amax - 448 q0) y (Markstein's theorem, the residual exact in an
// FMA); below that by the IEEE division. aicas_calib_fp8_divide_check compares it with the division for every
// 16-bit row maximum.
__device__ __forceinline__ float fp8_scale_of(float amax) {
  constexpr float kInv448 = 1.0f / 448.0f;
  if (amax >= 0x1p-100f) {
    const float q0 = amax * kInv448;
    return fmaf(fmaf(-q0, 448.0f, amax), kInv448, q0);
  }
  return amax / 448.0f;
}

// Scale of one fp8 cache row spread over N aligned lanes (VEC values each; every lane of the row takes part):
// amax / 448, 0 for an all-zero row. A row holding any NaN or +-Inf gets a NaN scale (and, from the caller's
// `scale > 0` test, all-zero codes), so that it dequantises to NaN everywhere, as the unquantised row would make
// every score that touches it non-finite; `nonfinite` reports it. The maximum is taken over the magnitudes' bit
// patterns, which order like the magnitudes, with Inf and every NaN above all finite values: one reduction
// finds both.
template <int N, int VEC>
__device__ __forceinline__ float fp8_row_scale(const float* f, bool& nonfinite) {
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < VEC; ++i) m = max(m, __float_as_uint(f[i]) & 0x7fffffffu);
  m = group_max_u32<N>(m);
  nonfinite = m >= 0x7f800000u;
  return nonfinite ? __builtin_nanf("") : fp8_scale_of(__uint_as_float(m));
}

// Row scales at or above this take the one-reciprocal division in fp8_quantize.
constexpr float kFp8FastDivMinScale = 0x1p-90f;

// 1 / s for a row scale s >= kFp8FastDivMinScale: the hardware reciprocal (v_rcp_f32) and one Newton step. It is
// the correctly rounded reciprocal for every scale a 16-bit row maximum gives (fp8_scale_of of every positive
// bf16 and fp16 value), which aicas_calib_fp8_divide_check compares with 1.0f / s.
__device__ __forceinline__ float fp8_reciprocal(float s) {
  const float r0 = __builtin_amdgcn_rcpf(s);
  return fmaf(fmaf(-s, r0, 1.0f), r0, r0);
}

// The e4m3 codes of VEC finite values of one fp8 cache row with scale s (fp8_row_scale): clamp(x / s, +-448)
// encoded by e4m3x4, code i in byte i % 4 of packed[i / 4]; a zero or poisoned row (s not > 0) gets zero codes.
// The quotient is x / s correctly rounded, from one reciprocal per row: y = 1 / s (fp8_reciprocal), then per value
// q0 = x * y and one correction q = q0 + (x - s q0) y with the residual exact in an FMA — Markstein's theorem
// (y the correctly rounded reciprocal and q0 within an ulp of x / s make q the correctly rounded quotient) —
// provided the residual does not underflow. For s >= 2^-90 that holds whenever |x / s| >= 2^-11, and smaller
// quotients encode to a zero of x's sign whatever their last bits; smaller scales divide value by value (and
// clamp: a subnormal s can be far from amax / 448). So the codes are
// those of the IEEE quotient for every input, which libaicas_calib.so's aicas_calib_fp8_divide_check compares
// over every (row maximum, value) pair of both 16-bit source types.
template <int VEC>
__device__ __forceinline__ void fp8_quantize(const float* f, float s, uint32_t* packed) {
  float y[VEC];
  if (s >= kFp8FastDivMinScale) {
    const float r = fp8_reciprocal(s);
    // The residual enters negated, q = q0 - (q0 s - x) r: the same rounded value as q0 + (x - q0 s) r for every
    // nonzero quotient, and a zero quotient keeps x's sign (the other order turns -0 into +0). No clamp: with s
    // a normal number |x / s| <= 448 (1 + 2^-23) < 464, which e4m3 rounds to at most 448.
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      const float q0 = f[i] * r;
      y[i] = fmaf(-fmaf(q0, s, -f[i]), r, q0);
    }
  } else if (s > 0.0f) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) y[i] = fminf(fmaxf(f[i] / s, -448.0f), 448.0f);
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) y[i] = 0.0f;
  }
#pragma unroll
  for (int i = 0; i < VEC / 4; ++i) packed[i] = e4m3x4(y[4 * i], y[4 * i + 1], y[4 * i + 2], y[4 * i + 3]);
}

// Division by a divisor d >= 1 fixed for a launch, for dividends 0 <= x < 2^31 (Granlund and Montgomery's
// round-up method): with l = ceil(log2 d) and m = floor(2^32 (2^l - d) / d) + 1, x / d = (umulhi(x, m) + x) >> l,
// where the sum stays below 2^32 because x < 2^31. libaicas_calib.so's aicas_calib_fast_div_check compares it
// with the division on the GPU.
struct FastDiv {
  uint32_t m;
  uint32_t l;
};

inline FastDiv fast_div_make(uint32_t d) {
  uint32_t l = 0;
  while ((uint64_t{1} << l) < d) ++l;
  const uint64_t m = ((uint64_t{1} << 32) * ((uint64_t{1} << l) - d)) / d + 1;
  return FastDiv{static_cast<uint32_t>(m), l};
}

__device__ __forceinline__ int fast_div(int x, FastDiv f) {
  const uint32_t u = static_cast<uint32_t>(x);
  return static_cast<int>((__umulhi(u, f.m) + u) >> f.l);
}

// A 16-byte load of data read once per launch (cache rows): non-temporal (global_load_dwordx4 ... nt), so the
// stream does not allocate in the caches on its way through. The decode kernel's access pattern as a pure read
// (B=8 L=2112, 69 MB): 12.4 us per launch with these loads, 13.5 with plain ones.
__device__ __forceinline__ uint4 load_stream16(const void* p) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 w = __builtin_nontemporal_load(static_cast<const u32x4*>(p));
  return make_uint4(w.x, w.y, w.z, w.w);
}

// vmcnt(0): wait until this wave's vector memory operations (loads and stores) have completed.
__device__ __forceinline__ void wait_vmem() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// 16 bytes stored non-temporal: a stream written once, kept from allocating in L2 and the memory-side cache.
__device__ __forceinline__ void store_stream16(void* p, uint4 v) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, static_cast<u32x4*>(p));
}

// Where a token's K/V row lives. Contiguous caches are the one-block-per-sequence case:
// block id = batch index, page_size = capacity, and the token stride may be any multiple of 16 bytes.
struct KVLayout {
  void* k;
  void* v;
  float* k_scale;
  float* v_scale;
  const int32_t* block_table;  // nullptr for contiguous caches
  int64_t block_table_stride;
  int64_t num_blocks;
  int64_t stride_blk;  // elements
  int64_t stride_h;
  int64_t stride_t;
  int64_t scale_stride_blk;
  int64_t scale_stride_h;
  int32_t page_size;
  int32_t max_tokens;  // tokens one sequence can hold: capacity, or block_table_stride * page_size
};

}  // namespace aicas
