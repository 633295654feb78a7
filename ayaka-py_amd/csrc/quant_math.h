// Element-level arithmetic of the activation quantizers (e4m3 and UE8M0 encoders,
// magnitude-bit maxima, the Markstein quotient), shared by the quantizer kernels and the
// fused quantize-and-multiply small-batch GEMM so that both produce the same bytes.
#pragma once

#include "ayk_common.h"

namespace ayk {
namespace {

constexpr int kQuantThreads = 256;

// 16-byte vector of activation elements.
template <typename T>
struct Vec16 {
  static constexpr int N = 16 / sizeof(typename T::storage);
};

template <typename T>
__device__ inline void unpack16(const uint4& v, float* f);
template <>
__device__ inline void unpack16<BF16T>(const uint4& v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = u2f(w[i] << 16);
    f[2 * i + 1] = u2f(w[i] & 0xFFFF0000u);
  }
}
template <>
__device__ inline void unpack16<F16T>(const uint4& v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = f16_bits_to_f32((uint16_t)(w[i] & 0xFFFFu));
    f[2 * i + 1] = f16_bits_to_f32((uint16_t)(w[i] >> 16));
  }
}
template <>
__device__ inline void unpack16<F32T>(const uint4& v, float* f) {
  f[0] = u2f(v.x);
  f[1] = u2f(v.y);
  f[2] = u2f(v.z);
  f[3] = u2f(v.w);
}

template <int N>
__device__ inline float absmax_n(const float* f, float m) {
#pragma unroll
  for (int i = 0; i < N; ++i) m = nanmax(m, fabsf(f[i]));
  return m;
}

// Quantize N floats with scale d.s (q = e4m3(clamp(f / s)), f / s correctly rounded)
// and store N bytes.
template <int N>
__device__ inline void store_quant(uint8_t* dst, const float* f, const Divisor& d) {
  static_assert(N % 4 == 0, "16-byte vectors hold 4 or 8 elements");
  float q[N];
  if (d.fast) {  // per row or group; a wavefront whose lanes agree runs one path
#pragma unroll
    for (int i = 0; i < N; ++i) q[i] = clamp_e4m3(divide_fast(d, f[i]));
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) q[i] = clamp_e4m3(f[i] / d.s);
  }
  uint32_t w[N / 4];
#pragma unroll
  for (int i = 0; i < N / 4; ++i) w[i] = e4m3x4_encode(q[4 * i], q[4 * i + 1], q[4 * i + 2], q[4 * i + 3]);
  if constexpr (N == 8) {
    *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
  } else {
    static_assert(N == 4, "16-byte vectors hold 4 or 8 elements");
    *reinterpret_cast<uint32_t*>(dst) = w[0];
  }
}

// ------------------------------------------------------------ finite fast path
// The magnitude bits of a non-negative float (or NaN) order like the values as
// unsigned integers, NaN above infinity: the amax of a row or group is an integer max
// over |x|'s bits, and it is NaN exactly when the row or group holds a NaN. Rows and
// groups whose amax is finite (the rule; infinity and NaN are the exception) take a
// path with no per-element special cases; the others keep the exact element-wise one.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Running max of |x| bits over one 16-byte vector (16-bit floats: two lanes of packed
// 16-bit magnitudes; fp32: one 32-bit magnitude).
template <typename T>
__device__ inline uint32_t absbits_max(const uint4& v, uint32_t acc);
template <>
__device__ inline uint32_t absbits_max<BF16T>(const uint4& v, uint32_t acc) {
  u16x2 m = __builtin_bit_cast(u16x2, acc);
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w[i] & 0x7FFF7FFFu));
  return __builtin_bit_cast(uint32_t, m);
}
template <>
__device__ inline uint32_t absbits_max<F16T>(const uint4& v, uint32_t acc) {
  return absbits_max<BF16T>(v, acc);  // the same packed 16-bit magnitudes
}
template <>
__device__ inline uint32_t absbits_max<F32T>(const uint4& v, uint32_t acc) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) acc = max(acc, w[i] & 0x7FFFFFFFu);
  return acc;
}
// The accumulated magnitude bits as the fp32 bit pattern of the amax (whose integer
// order is the value order, NaN above infinity).
template <typename T>
__device__ inline uint32_t absbits_f32(uint32_t acc);
template <>
__device__ inline uint32_t absbits_f32<BF16T>(uint32_t acc) {
  const uint32_t lo = acc & 0xFFFFu, hi = acc >> 16;
  return (lo > hi ? lo : hi) << 16;
}
template <>
__device__ inline uint32_t absbits_f32<F16T>(uint32_t acc) {
  const uint32_t lo = acc & 0xFFFFu, hi = acc >> 16;
  return f2u(f16_bits_to_f32((uint16_t)(lo > hi ? lo : hi)));
}
template <>
__device__ inline uint32_t absbits_f32<F32T>(uint32_t acc) {
  return acc;
}
template <int WIDTH>
__device__ inline uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int off = WIDTH / 2; off > 0; off >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, off, WIDTH));
  return v;
}
constexpr uint32_t kInfBits = 0x7F800000u;

// Quantize N floats of a row or group with a finite amax by scale s (r = RN(1 / s),
// s and r normal): |x| / s by Markstein's correction (see Divisor), which here needs no
// special case -- |x| <= amax keeps every quotient finite, and the sign, applied
// afterwards, keeps a zero's -- clamped to 448 and encoded without the NaN patch.
template <int N>
__device__ inline void store_quant_finite(uint8_t* dst, const float* f, float s, float r) {
  static_assert(N % 4 == 0, "16-byte vectors hold 4 or 8 elements");
  float q[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float ax = fabsf(f[i]);
    const float q0 = ax * r;
    const float qa = fminf(fmaf(fmaf(-s, q0, ax), r, q0), kE4M3Max);
    q[i] = __builtin_copysignf(qa, f[i]);
  }
  uint32_t w[N / 4];
#pragma unroll
  for (int i = 0; i < N / 4; ++i) {
    w[i] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[4 * i], q[4 * i + 1], 0, false);
    w[i] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[4 * i + 2], q[4 * i + 3], (int)w[i], true);
  }
  if constexpr (N == 8) {
    *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
  } else {
    *reinterpret_cast<uint32_t*>(dst) = w[0];
  }
}
// MX: |x| times the power of two inv (exact but for fp32 subnormals, which round as
// the reference's division by the same power of two), clamped to 448 (the fp32 log2
// can round the exponent one short), sign restored; finite groups only.
template <int N>
__device__ inline void store_mx_finite(uint8_t* dst, const float* f, float inv) {
  float q[N];
#pragma unroll
  for (int i = 0; i < N; ++i) q[i] = __builtin_copysignf(fminf(fabsf(f[i]) * inv, kE4M3Max), f[i]);
  uint32_t w[N / 4];
#pragma unroll
  for (int i = 0; i < N / 4; ++i) {
    w[i] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[4 * i], q[4 * i + 1], 0, false);
    w[i] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[4 * i + 2], q[4 * i + 3], (int)w[i], true);
  }
  if constexpr (N == 8) {
    *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
  } else {
    *reinterpret_cast<uint32_t*>(dst) = w[0];
  }
}

// Block-wide NaN-propagating max over 256 threads; every thread gets the result.
__device__ inline float block_max256(float v, float* red) {
  v = wave_max<kWave>(v);
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x % kWave) == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < kQuantThreads / kWave; ++i) r = nanmax(r, red[i]);
  return r;
}

// The same over magnitude bits (unsigned max, NaN above infinity).
__device__ inline uint32_t block_max256_u32(uint32_t v, uint32_t* red) {
  v = wave_max_u32<kWave>(v);
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x % kWave) == 0) red[wave] = v;
  __syncthreads();
  uint32_t r = red[0];
#pragma unroll
  for (int i = 1; i < kQuantThreads / kWave; ++i) r = max(r, red[i]);
  return r;
}

__device__ inline float floor_amax(float amax) {
  // clamp_min(1e-10) with NaN kept (reference quant.py:26, :63)
  return amax < 1e-10f ? 1e-10f : amax;
}

}  // namespace
}  // namespace ayk
