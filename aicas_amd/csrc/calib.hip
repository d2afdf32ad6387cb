// Calibration and self-check kernels (libaicas_calib.so; not part of the decode ABI).
//
// aicas_calib_fp8_encoder_check: the fp8 encoding the kernels use (e4m3x4, gfx950's v_cvt_pk_fp8_f32) against
// the encoder written out from the format (f32_to_e4m3) on every float with |x| <= 448;
// aicas_calib_fp8_divide_check: the kernels' fp8 row scale (fp8_scale_of), reciprocal (fp8_reciprocal) and
// quantiser (fp8_quantize: one reciprocal per row and a corrected product per value) against the IEEE
// divisions, for every row maximum and every (row maximum, value) pair of a 16-bit source type;
// aicas_calib_fast_div_check: the launch-constant integer division (fast_div) against the division.
// GPU tests require zero mismatches from each.
//
// Bandwidth calibration for bench.py --config calib:
// They read exactly the bytes one decode launch of a contiguous bf16 cache reads (K and V rows of B sequences x
// Hkv heads x L tokens, head_dim 128) and compute nothing but an xor of the words, so that their time is the
// streaming ceiling the attention launch is compared with:
//   aicas_calib_stream_read  the attention's own grid and access pattern: (splits, Hkv, B) workgroups of 4 waves,
//                            the sequence's 32-token super-chunks dealt round-robin to its 4 * splits waves, each
//                            super-chunk 2 x 4 non-temporal 16-byte loads of K and of V per lane;
//   aicas_calib_flat_read    the same bytes as one flat range per tensor in `blocks` workgroups (grid-stride,
//                            16 bytes per lane per load): what a finely balanced plain read achieves;
//   aicas_calib_empty        an empty launch (dispatch and completion cost).
// Every thread stores its xor to `sink`, so no load is dead.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "common.hpp"

namespace {

constexpr int kD = 128;          // head_dim
constexpr int kLanesPerRow = 16; // 16 bytes per lane per bf16 row of 128
constexpr int kRowsPerLoad = aicas::kWave / kLanesPerRow;
constexpr int kChunk = 4 * kRowsPerLoad;  // tokens per wave chunk (4 loads)
constexpr int kSuper = 2 * kChunk;        // tokens per super-chunk

__device__ __forceinline__ uint32_t fold(uint4 w) { return w.x ^ w.y ^ w.z ^ w.w; }

__global__ __launch_bounds__(aicas::kBlockThreads) void stream_read_kernel(const uint16_t* k, const uint16_t* v,
                                                                          int64_t stride_b, int64_t stride_h, int L,
                                                                          uint32_t* sink) {
  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / aicas::kWave);
  const int lane = threadIdx.x % aicas::kWave;
  const int row = lane / kLanesPerRow, li = lane % kLanesPerRow;
  const int stripe = gridDim.x * aicas::kWavesPerBlock;
  const int n_super = (L + kSuper - 1) / kSuper;
  const int64_t base = b * stride_b + h * stride_h + li * 8;
  uint32_t acc = 0;
  for (int j = split * aicas::kWavesPerBlock + wave; j < n_super; j += stripe) {
    uint4 kw[8], vw[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int t = min(j * kSuper + u * kRowsPerLoad + row, L - 1);
      kw[u] = aicas::load_stream16(k + base + static_cast<int64_t>(t) * kD);
      vw[u] = aicas::load_stream16(v + base + static_cast<int64_t>(t) * kD);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) acc ^= fold(kw[u]) ^ fold(vw[u]);
  }
  sink[((static_cast<int64_t>(b) * gridDim.y + h) * gridDim.x + split) * blockDim.x + threadIdx.x] = acc;
}

__global__ __launch_bounds__(aicas::kBlockThreads) void flat_read_kernel(const uint4* k, const uint4* v, int64_t n16,
                                                                        uint32_t* sink) {
  uint32_t acc = 0;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += 2 * stride) {
    const uint4 a = aicas::load_stream16(k + i), c = aicas::load_stream16(v + i);
    uint4 a2 = make_uint4(0, 0, 0, 0), c2 = a2;
    if (i + stride < n16) {
      a2 = aicas::load_stream16(k + i + stride);
      c2 = aicas::load_stream16(v + i + stride);
    }
    acc ^= fold(a) ^ fold(c) ^ fold(a2) ^ fold(c2);
  }
  sink[static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x] = acc;
}

__global__ void empty_kernel() {}

// Thread gid of a launch covers the 16 bit patterns (slice << 28) | (16 * gid + i); 2^24 threads cover a slice.
__global__ __launch_bounds__(aicas::kBlockThreads) void fp8_encoder_check_kernel(uint32_t slice,
                                                                                unsigned long long* mismatches,
                                                                                uint32_t* first) {
  const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
  unsigned long long bad = 0;
#pragma unroll
  for (int i = 0; i < 16; i += 4) {
    float x[4];
    uint32_t sw = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t u = (slice << 28) | (16u * gid + static_cast<uint32_t>(i + j));
      x[j] = __uint_as_float(u);
      if (!(fabsf(x[j]) <= 448.0f)) x[j] = 0.0f;  // outside the domain: compare zeros
      sw |= aicas::f32_to_e4m3(x[j]) << (8 * j);
    }
    const uint32_t hw = aicas::e4m3x4(x[0], x[1], x[2], x[3]);
    if (hw != sw) {
      ++bad;
      atomicCAS(first, 0xffffffffu, (slice << 28) | (16u * gid + static_cast<uint32_t>(i)));
    }
  }
  if (bad) atomicAdd(mismatches, bad);
}

// Block i takes the row maximum amax = the (i + 1)-th positive 16-bit pattern of DT (every one is finite for the
// grid the host launches); thread 0 compares the row scale (fp8_scale_of) with amax / 448 and, where the scale
// takes the one-reciprocal path, fp8_reciprocal with 1 / s; thread t then compares the codes of the 256 values
// with patterns 256 t .. 256 t + 255, 4 at a time (those not finite or above amax in magnitude taken as 0), with
// those of the IEEE quotient. mismatches[0] counts code groups, [1] scales, [2] reciprocals.
template <int DT>
__global__ __launch_bounds__(aicas::kBlockThreads) void fp8_divide_check_kernel(unsigned long long* mismatches,
                                                                               uint32_t* first) {
  const uint32_t amax_bits = blockIdx.x + 1;
  float amax, unused;
  aicas::unpack2<DT>(amax_bits, amax, unused);
  const float s_ref = amax / 448.0f;
  const float s = aicas::fp8_scale_of(amax);
  if (threadIdx.x == 0) {
    if (__float_as_uint(s) != __float_as_uint(s_ref)) {
      atomicAdd(mismatches + 1, 1ull);
      atomicCAS(first, 0xffffffffu, amax_bits << 16);
    }
    if (s_ref >= aicas::kFp8FastDivMinScale &&
        __float_as_uint(aicas::fp8_reciprocal(s_ref)) != __float_as_uint(1.0f / s_ref)) {
      atomicAdd(mismatches + 2, 1ull);
      atomicCAS(first, 0xffffffffu, amax_bits << 16);
    }
  }
  unsigned long long bad = 0;
  for (int g = 0; g < 64; ++g) {
    const uint32_t base = threadIdx.x * 256u + 4u * g;
    float x[4], y[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v;
      aicas::unpack2<DT>(base + j, v, unused);
      x[j] = fabsf(v) <= amax ? v : 0.0f;
      y[j] = fminf(fmaxf(x[j] / s_ref, -448.0f), 448.0f);
    }
    uint32_t codes;
    aicas::fp8_quantize<4>(x, s, &codes);
    if (codes != aicas::e4m3x4(y[0], y[1], y[2], y[3])) {
      ++bad;
      atomicCAS(first, 0xffffffffu, (amax_bits << 16) | base);
    }
  }
  if (bad) atomicAdd(mismatches, bad);
}

// Thread g of 2^24 divides g and 2^31 - 1 - 127 g (the whole non-negative 31-bit range, sparsely) by d.
__global__ __launch_bounds__(aicas::kBlockThreads) void fast_div_check_kernel(int32_t d, aicas::FastDiv f,
                                                                             unsigned long long* mismatches,
                                                                             uint32_t* first) {
  const uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
  const int32_t xs[2] = {static_cast<int32_t>(g), static_cast<int32_t>(0x7fffffffu - 127u * g)};
  unsigned long long bad = 0;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (aicas::fast_div(xs[i], f) != xs[i] / d) {
      ++bad;
      atomicCAS(first, 0xffffffffu, static_cast<uint32_t>(d));
    }
  }
  if (bad) atomicAdd(mismatches, bad);
}

}  // namespace

extern "C" {

// k, v: [B, Hkv, capacity, 128] bf16 (element strides stride_b, stride_h; token stride 128); reads the first L
// tokens of every (b, h). sink: splits * Hkv * B * 256 words.
int aicas_calib_stream_read(const void* k, const void* v, int64_t stride_b, int64_t stride_h, int32_t batch,
                            int32_t num_kv_heads, int32_t L, int32_t splits, uint32_t* sink, hipStream_t stream) {
  if (!k || !v || !sink || batch <= 0 || num_kv_heads <= 0 || L <= 0 || splits <= 0) return 1;
  hipLaunchKernelGGL(stream_read_kernel, dim3(splits, num_kv_heads, batch), dim3(aicas::kBlockThreads), 0, stream,
                     static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v), stride_b, stride_h, L, sink);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// k, v: contiguous buffers of n_bytes each (a multiple of 16). sink: blocks * 256 words.
int aicas_calib_flat_read(const void* k, const void* v, int64_t n_bytes, int32_t blocks, uint32_t* sink,
                          hipStream_t stream) {
  if (!k || !v || !sink || n_bytes <= 0 || (n_bytes % 16) || blocks <= 0) return 1;
  hipLaunchKernelGGL(flat_read_kernel, dim3(blocks), dim3(aicas::kBlockThreads), 0, stream,
                     static_cast<const uint4*>(k), static_cast<const uint4*>(v), n_bytes / 16, sink);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// Every float with |x| <= 448 through both encoders, 4 at a time; *mismatches (zeroed here) counts the groups of
// 4 whose codes differ, *first_pattern (set to 0xffffffff here) the first bit pattern of one of them.
// Synchronous: returns after the 16 launches have finished.
int aicas_calib_fp8_encoder_check(unsigned long long* mismatches, uint32_t* first_pattern, hipStream_t stream) {
  if (!mismatches || !first_pattern) return 1;
  if (hipMemsetAsync(mismatches, 0, sizeof(unsigned long long), stream) != hipSuccess) return 2;
  if (hipMemsetAsync(first_pattern, 0xff, sizeof(uint32_t), stream) != hipSuccess) return 2;
  for (uint32_t slice = 0; slice < 16; ++slice) {
    hipLaunchKernelGGL(fp8_encoder_check_kernel, dim3((1u << 24) / aicas::kBlockThreads), dim3(aicas::kBlockThreads),
                       0, stream, slice, mismatches, first_pattern);
    if (hipGetLastError() != hipSuccess) return 2;
  }
  return hipStreamSynchronize(stream) == hipSuccess ? 0 : 2;
}

// src_dtype 0 (bf16) or 1 (fp16): every positive finite row maximum and every value of that type through the
// kernels' row scale, reciprocal and quantiser, against the IEEE divisions; mismatches[3] (zeroed here): groups
// of 4 values whose codes differ, scales that differ, reciprocals that differ; *first_pattern (0xffffffff here)
// holds (amax pattern << 16 | value pattern) of the first difference. Synchronous.
int aicas_calib_fp8_divide_check(int32_t src_dtype, unsigned long long* mismatches, uint32_t* first_pattern,
                                 hipStream_t stream) {
  if (!mismatches || !first_pattern || (src_dtype != aicas::kBF16 && src_dtype != aicas::kFP16)) return 1;
  if (hipMemsetAsync(mismatches, 0, 3 * sizeof(unsigned long long), stream) != hipSuccess) return 2;
  if (hipMemsetAsync(first_pattern, 0xff, sizeof(uint32_t), stream) != hipSuccess) return 2;
  // positive finite patterns: bf16 0x0001 .. 0x7f7f, fp16 0x0001 .. 0x7bff
  if (src_dtype == aicas::kBF16)
    hipLaunchKernelGGL(fp8_divide_check_kernel<aicas::kBF16>, dim3(0x7f7f), dim3(aicas::kBlockThreads), 0, stream,
                       mismatches, first_pattern);
  else
    hipLaunchKernelGGL(fp8_divide_check_kernel<aicas::kFP16>, dim3(0x7bff), dim3(aicas::kBlockThreads), 0, stream,
                       mismatches, first_pattern);
  if (hipGetLastError() != hipSuccess) return 2;
  return hipStreamSynchronize(stream) == hipSuccess ? 0 : 2;
}

// Each of the n divisors (host array, each >= 1) with its multiplier from fast_div_make, against the division on
// 2^25 dividends; *mismatches (zeroed here) counts the differences, *first_divisor (0xffffffff here) the first
// divisor that had one. Synchronous.
int aicas_calib_fast_div_check(const int32_t* divisors, int32_t n, unsigned long long* mismatches,
                               uint32_t* first_divisor, hipStream_t stream) {
  if (!divisors || n <= 0 || !mismatches || !first_divisor) return 1;
  if (hipMemsetAsync(mismatches, 0, sizeof(unsigned long long), stream) != hipSuccess) return 2;
  if (hipMemsetAsync(first_divisor, 0xff, sizeof(uint32_t), stream) != hipSuccess) return 2;
  for (int32_t i = 0; i < n; ++i) {
    if (divisors[i] < 1) return 1;
    hipLaunchKernelGGL(fast_div_check_kernel, dim3((1u << 24) / aicas::kBlockThreads), dim3(aicas::kBlockThreads), 0,
                       stream, divisors[i], aicas::fast_div_make(static_cast<uint32_t>(divisors[i])), mismatches,
                       first_divisor);
    if (hipGetLastError() != hipSuccess) return 2;
  }
  return hipStreamSynchronize(stream) == hipSuccess ? 0 : 2;
}

int aicas_calib_empty(hipStream_t stream) {
  hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, stream);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"
