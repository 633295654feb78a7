// Shared device helpers of libayaka_fp8: number codecs, typed loads/stores,
// wavefront reductions and the error/launch plumbing of the C ABI.
//
// Everything here targets gfx950 (CDNA4): 64-lane wavefronts, OCP fp8 formats.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <string.h>

#include "ayaka_fp8.h"

namespace ayk {

constexpr float kE4M3Max = 448.0f;
constexpr int kWave = 64;

// ------------------------------------------------------------------ bit casts
__host__ __device__ inline uint32_t f2u(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __float_as_uint(f);
#else
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
#endif
}
__host__ __device__ inline float u2f(uint32_t u) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __uint_as_float(u);
#else
  float f;
  memcpy(&f, &u, 4);
  return f;
#endif
}

// --------------------------------------------------------------- e4m3fn codec
// OCP e4m3fn: 1 sign, 4 exponent (bias 7), 3 mantissa bits; no infinities; the
// all-ones magnitude 0x7F is NaN; largest finite value 448 = 1.75 * 2^8; the
// subnormal grid is 2^-9. Encoding rounds to nearest, ties to even, and maps NaN
// and every magnitude that rounds above 448 (>= 464 after the tie rule) to NaN,
// i.e. the IEEE-style result in a format whose only "overflow" value is NaN.
__host__ __device__ inline uint8_t e4m3_encode(float v) {
  const uint32_t bits = f2u(v);
  const uint8_t sign = (uint8_t)((bits >> 24) & 0x80u);
  const uint32_t mag = bits & 0x7FFFFFFFu;
  if (mag >= 0x43F00000u) return sign | 0x7F;  // NaN, inf, >= 480
  if (mag < 0x3C800000u) {                     // below 2^-6: subnormal range
    // mag * 2^9 is exact; rounding it to an integer in [0, 8] is the subnormal
    // code (8 == 2^-6, the smallest normal, whose code is also 8).
    const float scaled = u2f(mag) * 512.0f;
    return sign | (uint8_t)rintf(scaled);
  }
  // Normal range: keep 3 of the 23 mantissa bits with round-half-even; a carry out
  // of the mantissa bumps the exponent, which is the correct rounding.
  const uint32_t lsb = (mag >> 20) & 1u;
  const uint32_t rounded = (mag + 0x7FFFFu + lsb) >> 20;
  return sign | (uint8_t)(rounded - ((127u - 7u) << 3));
}

// OCP e5m2 (1 sign, 5 exponent bits with bias 15, 2 mantissa bits; infinities; largest
// finite 57344): IEEE round to nearest even, so magnitudes from 61440 (the midpoint to
// the next binade) become infinity and NaN stays NaN (0x7F with the sign), as torch's
// float -> float8_e5m2 cast.
__host__ __device__ inline uint8_t e5m2_encode(float v) {
  const uint32_t bits = f2u(v);
  const uint8_t sign = (uint8_t)((bits >> 24) & 0x80u);
  const uint32_t mag = bits & 0x7FFFFFFFu;
  if (mag > 0x7F800000u) return sign | 0x7F;   // NaN
  if (mag >= 0x47700000u) return sign | 0x7C;  // >= 61440 and infinity
  if (mag < 0x38800000u) {                     // below 2^-14: subnormal range
    // mag * 2^16 is exact; rounding it to an integer in [0, 4] is the code (4 == 2^-14).
    return sign | (uint8_t)rintf(u2f(mag) * 65536.0f);
  }
  const uint32_t lsb = (mag >> 21) & 1u;
  const uint32_t rounded = (mag + 0xFFFFFu + lsb) >> 21;
  return sign | (uint8_t)(rounded - ((127u - 15u) << 2));
}
__host__ __device__ inline float e5m2_decode(uint8_t c) {
  // e5m2 is the top byte of an IEEE half.
  const uint16_t h = (uint16_t)c << 8;
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1F, m = (h >> 8) & 3;
  if (e == 0x1F) return u2f(sign | 0x7F800000u | (m ? 0x400000u : 0u));
  if (e == 0) return u2f(sign | f2u((float)m * (1.0f / 65536.0f)));
  return u2f(sign | ((e + 112u) << 23) | (m << 21));
}

// Exact decode of one e4m3fn byte (host and device; the device hot loops use the
// gfx950 hardware converter instead, see e4m3x4_to_f32).
__host__ __device__ inline float e4m3_decode(uint8_t c) {
  const uint32_t sign = (uint32_t)(c & 0x80) << 24;
  const uint32_t e = (c >> 3) & 0xF;
  const uint32_t m = c & 0x7;
  if (e == 0xF && m == 0x7) return u2f(sign | 0x7FC00000u);
  if (e == 0) return u2f(sign | f2u((float)m * (1.0f / 512.0f)));
  return u2f(sign | ((e + 120u) << 23) | (m << 20));
}

// UE8M0 exponent code: value 2^(c-127) built as the fp32 bit pattern c << 23, so
// code 0 is +0.0 and 0xFF is NaN.
__host__ __device__ inline float e8m0_decode(uint32_t c) {
  return c == 0xFFu ? u2f(0x7FC00000u) : u2f(c << 23);
}

// ------------------------------------------------------------------ 16-bit floats
// fp32 -> bf16, round to nearest even; every NaN becomes the canonical 0x7FC0.
__host__ __device__ inline uint16_t f32_to_bf16_bits(float f) {
  const uint32_t u = f2u(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0;
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
__host__ __device__ inline float bf16_bits_to_f32(uint32_t b) { return u2f(b << 16); }

__device__ inline float f16_bits_to_f32(uint16_t h) {
  return __half2float(__ushort_as_half(h));
}
__device__ inline uint16_t f32_to_f16_bits(float f) {
  return __half_as_ushort(__float2half_rn(f));
}

// Element-type tags used to template kernels on the activation / output type.
struct F32T { using storage = float; static constexpr int id = AYK_F32; };
struct F16T { using storage = uint16_t; static constexpr int id = AYK_F16; };
struct BF16T { using storage = uint16_t; static constexpr int id = AYK_BF16; };

template <typename T>
__device__ inline float to_f32(typename T::storage v);
template <>
__device__ inline float to_f32<F32T>(float v) { return v; }
template <>
__device__ inline float to_f32<F16T>(uint16_t v) { return f16_bits_to_f32(v); }
template <>
__device__ inline float to_f32<BF16T>(uint16_t v) { return bf16_bits_to_f32(v); }

// Runtime-typed scalar load / store (epilogues, scales, biases).
__device__ inline float load_f32(const void* p, int dtype, int64_t i) {
  switch (dtype) {
    case AYK_F32: return reinterpret_cast<const float*>(p)[i];
    case AYK_F16: return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
    case AYK_BF16: return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
    case AYK_U8: return e8m0_decode(reinterpret_cast<const uint8_t*>(p)[i]);
    default: return 0.0f;
  }
}
// The same load split in two: the raw dword now, the conversion later. A value that
// is only used after later loads were issued does not make the wavefront wait for
// those loads (the vector-memory counter retires in issue order). The load is a single
// branch-free instruction: the aligned dword that contains element i (it lies in the
// same page as the element, so it is always readable); bits_to_f32 extracts and
// converts it.
struct RawBits {
  uint32_t word;
  uint32_t shift;
};
__device__ inline int dtype_size(int dtype) { return dtype == AYK_F32 ? 4 : (dtype == AYK_U8 ? 1 : 2); }
__device__ inline RawBits load_bits(const void* p, int dtype, int64_t i) {
  // Pointer arithmetic stays on `p` so the compiler keeps the global address space
  // (a flat load would be waited for conservatively).
  const int64_t byte = i * dtype_size(dtype);
  const uint32_t mis = (uint32_t)((reinterpret_cast<uintptr_t>(p) + (uintptr_t)byte) & 3);
  return {*reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(p) + byte - mis), mis * 8};
}
// Branch-free: every decoding is computed and one is selected (a branch here would
// cost the compiler its exact wait counts for loads still in flight).
__device__ inline float bits_to_f32(RawBits r, int dtype) {
  const uint32_t b = r.word >> r.shift;
  const float f32 = u2f(r.word);
  const float f16 = f16_bits_to_f32((uint16_t)b);
  const float bf16 = bf16_bits_to_f32(b & 0xFFFFu);
  const float u8 = e8m0_decode(b & 0xFFu);
  return dtype == AYK_F32 ? f32 : (dtype == AYK_F16 ? f16 : (dtype == AYK_BF16 ? bf16 : u8));
}
__device__ inline void store_f32(void* p, int dtype, int64_t i, float v) {
  switch (dtype) {
    case AYK_F32: reinterpret_cast<float*>(p)[i] = v; break;
    case AYK_F16: reinterpret_cast<uint16_t*>(p)[i] = f32_to_f16_bits(v); break;
    case AYK_BF16: reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v); break;
    default: break;
  }
}

// Fixed-order sum of `split` fp32 partial planes ([split][M][N], 16-byte aligned,
// N % 4 == 0) at elements i .. i + 3 of one row, plus bias, rounded once into out:
// bit for bit the sum v = 0, v += plane 0, v += plane 1, ..., with the planes' loads
// issued four at a time (a load-add chain per plane serialises their latencies).
__device__ inline void split_sum_store4(const float* __restrict__ part, int64_t M, int64_t N, int split, int64_t i,
                                        const void* __restrict__ bias, int bias_dtype, void* __restrict__ out,
                                        int out_dtype, int64_t ldo) {
  const float4* p = reinterpret_cast<const float4*>(part + i);
  const int64_t st = M * N / 4;
  float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  auto add = [&](const float4& a) { v.x += a.x; v.y += a.y; v.z += a.z; v.w += a.w; };
  int s = 0;
  for (; s + 4 <= split; s += 4) {
    const float4 a = p[s * st], b = p[(s + 1) * st], c = p[(s + 2) * st], d = p[(s + 3) * st];
    add(a); add(b); add(c); add(d);
  }
  for (; s < split; ++s) add(p[s * st]);
  const int64_t m = i / N, n = i - m * N;
  const float o[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) store_f32(out, out_dtype, m * ldo + n + q, bias ? o[q] + load_f32(bias, bias_dtype, n + q) : o[q]);
}

// Four e4m3 bytes packed in one dword -> four floats (hardware OCP converter).
__device__ inline void e4m3x4_to_f32(uint32_t w, float* out) {
  typedef float v2f __attribute__((ext_vector_type(2)));
  const v2f lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  const v2f hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  out[0] = lo.x;
  out[1] = lo.y;
  out[2] = hi.x;
  out[3] = hi.y;
}

// Four fp32 values -> four fp8 codes in one dword (byte i holds value i), with the
// hardware round-to-nearest-even converters v_cvt_pk_fp8_f32 (e4m3) and
// v_cvt_pk_bf8_f32 (e5m2). For every non-NaN fp32 input they give exactly
// e4m3_encode / e5m2_encode (compared over all 2^32 bit patterns on gfx950); a NaN
// comes out as 0xFF / 0xFE whatever its sign, so NaN inputs are re-encoded as
// sign | 0x7F, torch's NaN code, on a branch that finite data never takes.
__device__ inline uint32_t fp8_nan_patch(uint32_t w, const float* v) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (v[i] != v[i]) {
      const uint32_t code = ((f2u(v[i]) >> 24) & 0x80u) | 0x7Fu;
      w = (w & ~(0xFFu << (8 * i))) | (code << (8 * i));
    }
  }
  return w;
}
__device__ inline uint32_t e4m3x4_encode(float a, float b, float c, float d) {
  uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, (int)w, true);
  if (__builtin_expect((a != a) | (b != b) | (c != c) | (d != d), 0)) {
    const float v[4] = {a, b, c, d};
    w = fp8_nan_patch(w, v);
  }
  return w;
}
__device__ inline uint32_t e5m2x4_encode(float a, float b, float c, float d) {
  uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(a, b, 0, false);
  w = (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(c, d, (int)w, true);
  if (__builtin_expect((a != a) | (b != b) | (c != c) | (d != d), 0)) {
    const float v[4] = {a, b, c, d};
    w = fp8_nan_patch(w, v);
  }
  return w;
}

// x / s for many x and one s: the correctly rounded quotient from a reciprocal computed
// once, by Markstein's correction (P. W. Markstein, "Computation of elementary functions
// on the IBM RISC System/6000 processor", IBM J. Res. Dev. 34(1), 1990; Muller et al.,
// Handbook of Floating-Point Arithmetic, "Markstein's theorem"): with r = RN(1/s),
// q0 = RN(x r) is within one ulp of x/s, the residual x - s q0 is exact under an FMA,
// and RN(q0 + residual r) = RN(x / s) when nothing underflows. Used only when s and r
// are both normal; q0 itself is returned when it is zero (keeping the sign of a zero x)
// or not finite (x infinite or NaN). For subnormal x the last bit can differ from the
// IEEE quotient, whose magnitude is then below 2^-100 and below every fp8 code.
struct Divisor {
  float s, r;
  bool fast;
};
__device__ inline Divisor make_divisor(float s) {
  Divisor d;
  d.s = s;
  d.r = 1.0f / s;
  const float as = fabsf(s), ar = fabsf(d.r);
  d.fast = as >= 1.17549435e-38f && as <= 3.40282347e38f && ar >= 1.17549435e-38f && ar <= 3.40282347e38f;
  return d;
}
// The quotient of a fast divisor (d.fast), without the IEEE fallback.
__device__ inline float divide_fast(const Divisor& d, float x) {
  const float q0 = x * d.r;
  const float q = fmaf(fmaf(-d.s, q0, x), d.r, q0);
  return (q0 == 0.0f || !(fabsf(q0) <= 3.40282347e38f)) ? q0 : q;
}
__device__ inline float divide(const Divisor& d, float x) { return d.fast ? divide_fast(d, x) : x / d.s; }

// NaN-propagating max of magnitudes, the semantics of torch's amax.
__device__ inline float nanmax(float a, float b) { return (a > b || a != a) ? a : b; }

// Clamp to the finite e4m3 range, keeping NaN (torch.clamp semantics).
__host__ __device__ inline float clamp_e4m3(float v) {
  return v > kE4M3Max ? kE4M3Max : (v < -kE4M3Max ? -kE4M3Max : v);
}

// -------------------------------------------------------------- wave reductions
template <int WIDTH>
__device__ inline float wave_max(float v) {
#pragma unroll
  for (int off = WIDTH / 2; off > 0; off >>= 1) v = nanmax(v, __shfl_xor(v, off, WIDTH));
  return v;
}
template <int WIDTH>
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = WIDTH / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, WIDTH);
  return v;
}

// Full-wavefront sum with DPP moves instead of LDS permutes: pairwise and quad swaps,
// rotations within each 16-lane row, then the row broadcasts 15 and 31 carry row
// totals upward; lane 63 ends with the sum, which is returned to every lane. The
// addition order is fixed, so results are deterministic.
template <int CTRL, int ROW_MASK>
__device__ inline float dpp_move(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, ROW_MASK, 0xF, false));
}
__device__ inline float wave_sum_dpp(float v) {
  v += dpp_move<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
  v += dpp_move<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
  v += dpp_move<0x124, 0xF>(v);  // row_ror:4
  v += dpp_move<0x128, 0xF>(v);  // row_ror:8
  v += dpp_move<0x142, 0xA>(v);  // row_bcast:15 into rows 1, 3
  v += dpp_move<0x143, 0xC>(v);  // row_bcast:31 into rows 2, 3
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// ---------------------------------------------------------------- misc helpers
__host__ __device__ constexpr int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The K-split reduce four elements per thread (split_sum_store4).
namespace {
__global__ __launch_bounds__(256) void split_reduce4_kernel(const float* __restrict__ part, int64_t M, int64_t N, int split,
                                                           const void* __restrict__ bias, int bias_dtype,
                                                           void* __restrict__ out, int out_dtype, int64_t ldo) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= M * N) return;
  split_sum_store4(part, M, N, split, i, bias, bias_dtype, out, out_dtype, ldo);
}
}  // namespace
// Launch the fixed-order reduce of [split][M][N] fp32 partials: four elements per
// thread when N % 4 == 0 and the partials are 16-byte aligned, else `scalar` (one
// element per thread, the same sum).
template <typename ScalarKernel>
inline void launch_split_reduce(ScalarKernel scalar, const float* part, int64_t M, int64_t N, int split, const void* bias,
                                int bias_dtype, void* out, int out_dtype, int64_t ldo, hipStream_t st) {
  if (N % 4 == 0 && aligned16(part)) {
    hipLaunchKernelGGL(split_reduce4_kernel, dim3((unsigned)((M * N / 4 + 255) / 256)), dim3(256), 0, st, part, M, N, split,
                       bias, bias_dtype, out, out_dtype, ldo);
  } else {
    hipLaunchKernelGGL(scalar, dim3((unsigned)((M * N + 255) / 256)), dim3(256), 0, st, part, M, N, split, bias, bias_dtype,
                       out, out_dtype, ldo);
  }
}

// Error state of the C ABI (defined in capi.hip).
int fail(int status, const char* fmt, ...);
int check_launch(const char* what);
int check_device();
// Records which kernels and split the last GEMM launch on this thread used (read back
// through ayk_last_plan; tests assert that a case reaches the kernel it targets).
void note_plan(const char* fmt, ...);

}  // namespace ayk
