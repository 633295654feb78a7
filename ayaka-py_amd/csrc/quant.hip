// Dynamic and static activation quantizers to OCP e4m3fn (gfx950).
//
// Semantics follow the reference's plain-torch quantizers
// (python/ayaka/kernel/triton/reference/quant.py:19-79): fp32 amax, IEEE fp32
// division x / s, clamp to +-448 (NaN kept), round-to-nearest-even e4m3 encode.
// These kernels are HBM-bound (3 bytes/element for bf16 in, e4m3 out), so the
// layout work is about coalescing: every lane moves 16-byte vectors and the
// per-row / per-group reductions are wavefront shuffles, with the row kept in
// registers so x is read from HBM exactly once.
#include "ayk_common.h"
#include "quant_math.h"

namespace ayk {
namespace {

// A 16-byte vector of an activation row read once and not again: a nontemporal load, so
// that the stream does not displace from the caches what the GEMM reads next (its
// weights, and the quantized activation this kernel writes). Per-token K = 3584 at
// M = 4096 over 1 GiB of inputs: 3.15 -> 3.54 TB/s; through the layer (quantizer, then
// GEMM): Qwen2 down at M = 4096 289 -> 236 us, DeepSeek-V3 down 628 -> 597 us.
__device__ inline uint4 load_stream(const uint4* p) {
  typedef int nt4 __attribute__((ext_vector_type(4)));
  const nt4 t = __builtin_nontemporal_load(reinterpret_cast<const nt4*>(p));
  return make_uint4((uint32_t)t[0], (uint32_t)t[1], (uint32_t)t[2], (uint32_t)t[3]);
}
// ------------------------------------------------------------ rowwise (a1)
// One 256-thread block per row. VPT > 0 keeps VPT 16-byte vectors per thread in
// registers (one HBM read of x); VPT == 0 walks the row twice (very long rows).
template <typename T, int VPT>
__global__ __launch_bounds__(kQuantThreads) void per_token_quant_vec_kernel(
    const typename T::storage* __restrict__ x, int64_t k, int64_t ldx,
    uint8_t* __restrict__ q, int64_t ldq, float* __restrict__ scale) {
  constexpr int V = Vec16<T>::N;
  __shared__ float red[kQuantThreads / kWave];
  const int64_t row = blockIdx.x;
  const int64_t nvec = k / V;
  const uint4* xr = reinterpret_cast<const uint4*>(x + row * ldx);
  uint8_t* qr = q + row * ldq;
  float amax = 0.0f;
  float f[V];
  if constexpr (VPT > 0) {
    uint4 cache[VPT];
    uint32_t bits = 0;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int64_t v = threadIdx.x + (int64_t)i * kQuantThreads;
      if (v < nvec) {
        cache[i] = load_stream(xr + v);
        bits = absbits_max<T>(cache[i], bits);
      }
    }
    bits = block_max256_u32(absbits_f32<T>(bits), reinterpret_cast<uint32_t*>(red));
    const float s = floor_amax(u2f(bits)) / kE4M3Max;
    if (threadIdx.x == 0) scale[row] = s;
    if (bits < kInfBits) {  // workgroup-uniform
      const float r = 1.0f / s;
#pragma unroll
      for (int i = 0; i < VPT; ++i) {
        const int64_t v = threadIdx.x + (int64_t)i * kQuantThreads;
        if (v < nvec) {
          unpack16<T>(cache[i], f);
          store_quant_finite<V>(qr + v * V, f, s, r);
        }
      }
      return;
    }
    const Divisor dv = make_divisor(s);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int64_t v = threadIdx.x + (int64_t)i * kQuantThreads;
      if (v < nvec) {
        unpack16<T>(cache[i], f);
        store_quant<V>(qr + v * V, f, dv);
      }
    }
  } else {
    for (int64_t v = threadIdx.x; v < nvec; v += kQuantThreads) {
      unpack16<T>(xr[v], f);
      amax = absmax_n<V>(f, amax);
    }
    amax = floor_amax(block_max256(amax, red));
    const float s = amax / kE4M3Max;
    if (threadIdx.x == 0) scale[row] = s;
    const Divisor dv = make_divisor(s);
    for (int64_t v = threadIdx.x; v < nvec; v += kQuantThreads) {
      unpack16<T>(xr[v], f);
      store_quant<V>(qr + v * V, f, dv);
    }
  }
}

// One wavefront per row (kQuantThreads / 64 rows per workgroup) for rows of at most
// 64 VPT vectors: lane l keeps vectors l, l + 64, ... in registers, the amax is a wave
// reduction, and no workgroup barrier separates a row's read from its store.
template <typename T, int VPT>
__global__ __launch_bounds__(kQuantThreads) void per_token_quant_wave_kernel(
    const typename T::storage* __restrict__ x, int64_t rows, int64_t k, int64_t ldx,
    uint8_t* __restrict__ q, int64_t ldq, float* __restrict__ scale) {
  constexpr int V = Vec16<T>::N;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * (kQuantThreads / kWave) + (threadIdx.x / kWave);
  if (row >= rows) return;  // the whole wavefront leaves together
  const int64_t nvec = k / V;
  const uint4* xr = reinterpret_cast<const uint4*>(x + row * ldx);
  uint8_t* qr = q + row * ldq;
  uint4 cache[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int64_t v = lane + (int64_t)i * kWave;
    if (v < nvec) cache[i] = load_stream(xr + v);
  }
  float f[V];
  uint32_t bits = 0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    if (lane + (int64_t)i * kWave < nvec) bits = absbits_max<T>(cache[i], bits);
  }
  bits = wave_max_u32<kWave>(absbits_f32<T>(bits));
  const float amax = floor_amax(u2f(bits));
  const float sc = amax / kE4M3Max;
  if (lane == 0) scale[row] = sc;
  if (bits < kInfBits) {  // wavefront-uniform
    const float r = 1.0f / sc;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int64_t v = lane + (int64_t)i * kWave;
      if (v < nvec) {
        unpack16<T>(cache[i], f);
        store_quant_finite<V>(qr + v * V, f, sc, r);
      }
    }
    return;
  }
  const Divisor dv = make_divisor(sc);
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int64_t v = lane + (int64_t)i * kWave;
    if (v < nvec) {
      unpack16<T>(cache[i], f);
      store_quant<V>(qr + v * V, f, dv);
    }
  }
}

// Any K, any alignment: scalar loads, two passes over the row.
template <typename T>
__global__ __launch_bounds__(kQuantThreads) void per_token_quant_scalar_kernel(
    const typename T::storage* __restrict__ x, int64_t k, int64_t ldx,
    uint8_t* __restrict__ q, int64_t ldq, float* __restrict__ scale) {
  __shared__ float red[kQuantThreads / kWave];
  const int64_t row = blockIdx.x;
  const typename T::storage* xr = x + row * ldx;
  float amax = 0.0f;
  for (int64_t i = threadIdx.x; i < k; i += kQuantThreads) amax = nanmax(amax, fabsf(to_f32<T>(xr[i])));
  amax = floor_amax(block_max256(amax, red));
  const float s = amax / kE4M3Max;
  if (threadIdx.x == 0) scale[row] = s;
  for (int64_t i = threadIdx.x; i < k; i += kQuantThreads) {
    q[row * ldq + i] = e4m3_encode(clamp_e4m3(to_f32<T>(xr[i]) / s));
  }
}

// ------------------------------------------------- per-(row, group) quantizers
// MX rule (reference quant.py:47-55): e = clamp(ceil(log2(max(amax/448, 1e-38))),
// -126, 127) with log2 evaluated in fp32. The fp32 log2 is formed as the fp32
// rounding of a double-precision log2, i.e. the correctly rounded fp32 result; the
// only inputs where rounding decides the ceiling are r just above a power of two,
// where log2(r) lies within half an fp32 ulp of an integer.
struct MxScale {
  float inv;     // 2^-e (e <= 120 for every finite fp32 amax); NaN for a NaN group
  uint8_t code;  // 0 for an all-zero group, else e + 127
  bool zero;
};
// The ceiling read from the bits of ratio = 2^k (1 + M / 2^23): an exact power of two
// (M == 0) gives k. For M >= 64, log2(1 + M / 2^23) >= 1.1e-5 exceeds half an fp32 ulp
// of every integer |k| <= 127 (at most 2^-18), so the rounded log2 lies above k and the
// ceiling is k + 1. A subnormal ratio (at least 1e-38, below 2^-126) has its log2 in
// (-126.2, -126): the clamped result is -126. Only 1 <= M < 64, and NaN or infinity,
// evaluate the rounded log2.
__device__ inline float mx_ceil_log2(float ratio) {
  const uint32_t b = f2u(ratio);
  const uint32_t ef = (b >> 23) & 0xFFu, m = b & 0x7FFFFFu;
  if (ef == 0u) return -126.0f;
  if (ef != 0xFFu && (m == 0u || m >= 64u)) return (float)((int)ef - 127 + (m != 0u ? 1 : 0));
  return ceilf((float)log2((double)ratio));
}
__device__ inline MxScale mx_scale(float amax) {
  MxScale r;
  if (amax != amax) {
    // A NaN group: the reference's NaN exponent converts to code 0 and every quotient
    // by its NaN scale is NaN.
    r.zero = false;
    r.code = 0;
    r.inv = amax;
    return r;
  }
  float ratio = amax / kE4M3Max;
  ratio = ratio < 1e-38f ? 1e-38f : ratio;
  float e = mx_ceil_log2(ratio);
  e = e < -126.0f ? -126.0f : (e > 127.0f ? 127.0f : e);
  const int ei = (int)e;
  r.zero = (amax == 0.0f);
  r.code = r.zero ? (uint8_t)0 : (uint8_t)(ei + 127);
  // 2^-e; 2^-127 (e = 127, only for an infinite amax) is the subnormal 2^-127, so an
  // infinite element still divides to infinity and clamps to 448 as in the reference.
  r.inv = ei <= 126 ? u2f((uint32_t)(127 - ei) << 23) : u2f(0x00400000u);
  return r;
}

// GL lanes cooperate on one group; each lane holds VPL 16-byte vectors of it. A thread
// works on kGroupSlots such lane slots, one grid span apart (a multiple of 64 threads,
// so the GL lanes of a group stay together in one wavefront), with every slot's loads
// issued before the first reduction.
constexpr int kGroupSlots = 2;
template <typename T, int GL, int VPL, bool MX>
__global__ __launch_bounds__(kQuantThreads) void group_quant_vec_kernel(
    const typename T::storage* __restrict__ x, int64_t rows, int64_t k, int64_t ldx,
    int64_t group, uint8_t* __restrict__ q, int64_t ldq, void* __restrict__ scale_out, int64_t srs, int64_t sgs) {
  constexpr int V = Vec16<T>::N;
  const int64_t gpr = k / group;
  const int64_t span = (int64_t)gridDim.x * kQuantThreads;
  uint4 cache[kGroupSlots][VPL];
  int64_t row[kGroupSlots], g[kGroupSlots];
  bool live[kGroupSlots];
  const int lig = (int)(((int64_t)blockIdx.x * kQuantThreads + threadIdx.x) % GL);
#pragma unroll
  for (int u = 0; u < kGroupSlots; ++u) {
    const int64_t t = (int64_t)blockIdx.x * kQuantThreads + threadIdx.x + u * span;
    const int64_t gi = t / GL;
    live[u] = gi < rows * gpr;
    row[u] = live[u] ? gi / gpr : 0;
    g[u] = live[u] ? gi % gpr : 0;
    // Loaded unconditionally (a slot past the end re-reads group 0 of row 0 and is
    // never stored): a load inside a branch makes the compiler wait for it before the
    // next slot's, which serializes the slots' latencies.
    const uint4* xg = reinterpret_cast<const uint4*>(x + row[u] * ldx + g[u] * group);
#pragma unroll
    for (int j = 0; j < VPL; ++j) cache[u][j] = load_stream(xg + lig + j * GL);
  }
  float f[V];
#pragma unroll
  for (int u = 0; u < kGroupSlots; ++u) {
    uint32_t bits = 0;
#pragma unroll
    for (int j = 0; j < VPL; ++j) bits = absbits_max<T>(cache[u][j], bits);
    bits = absbits_f32<T>(bits);
    // every lane of the group takes part (GL divides 64); a slot past the end is
    // reduced like the others and then left
    bits = wave_max_u32<GL>(live[u] ? bits : 0u);
    if (!live[u]) continue;
    const float amax = u2f(bits);
    const bool finite = bits < kInfBits;
    uint8_t* qg = q + row[u] * ldq + g[u] * group;
    if constexpr (MX) {
      const MxScale ms = mx_scale(amax);
      if (lig == 0) reinterpret_cast<uint8_t*>(scale_out)[row[u] * srs + g[u] * sgs] = ms.code;
      if (finite && !ms.zero) {  // an all-zero group is written as +0 codes below
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
          unpack16<T>(cache[u][j], f);
          store_mx_finite<V>(qg + (int64_t)(lig + j * GL) * V, f, ms.inv);
        }
        continue;
      }
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        unpack16<T>(cache[u][j], f);
        uint32_t w[V / 4] = {};
        if (!ms.zero) {
          float qv[V];
#pragma unroll
          for (int i = 0; i < V; ++i) qv[i] = clamp_e4m3(f[i] * ms.inv);
#pragma unroll
          for (int i = 0; i < V / 4; ++i) w[i] = e4m3x4_encode(qv[4 * i], qv[4 * i + 1], qv[4 * i + 2], qv[4 * i + 3]);
        }
        uint8_t* dst = qg + (int64_t)(lig + j * GL) * V;
        if constexpr (V == 8) {
          *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
        } else {
          *reinterpret_cast<uint32_t*>(dst) = w[0];
        }
      }
    } else {
      const float sc = floor_amax(amax) / kE4M3Max;
      if (lig == 0) reinterpret_cast<float*>(scale_out)[row[u] * srs + g[u] * sgs] = sc;
      if (finite) {
        const float r = 1.0f / sc;
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
          unpack16<T>(cache[u][j], f);
          store_quant_finite<V>(qg + (int64_t)(lig + j * GL) * V, f, sc, r);
        }
        continue;
      }
      const Divisor dv{sc, 0.0f, false};  // IEEE division for infinite / NaN groups
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        unpack16<T>(cache[u][j], f);
        store_quant<V>(qg + (int64_t)(lig + j * GL) * V, f, dv);
      }
    }
  }
}

// Any group size / alignment: one thread per group, two passes.
template <typename T, bool MX>
__global__ __launch_bounds__(kQuantThreads) void group_quant_scalar_kernel(
    const typename T::storage* __restrict__ x, int64_t rows, int64_t k, int64_t ldx,
    int64_t group, uint8_t* __restrict__ q, int64_t ldq, void* __restrict__ scale_out, int64_t srs, int64_t sgs) {
  const int64_t gpr = k / group;
  const int64_t gi = (int64_t)blockIdx.x * kQuantThreads + threadIdx.x;
  if (gi >= rows * gpr) return;
  const int64_t row = gi / gpr, g = gi % gpr;
  const typename T::storage* xg = x + row * ldx + g * group;
  uint8_t* qg = q + row * ldq + g * group;
  float amax = 0.0f;
  for (int64_t i = 0; i < group; ++i) amax = nanmax(amax, fabsf(to_f32<T>(xg[i])));
  if constexpr (MX) {
    const MxScale ms = mx_scale(amax);
    reinterpret_cast<uint8_t*>(scale_out)[row * srs + g * sgs] = ms.code;
    for (int64_t i = 0; i < group; ++i) {
      qg[i] = ms.zero ? (uint8_t)0 : e4m3_encode(clamp_e4m3(to_f32<T>(xg[i]) * ms.inv));
    }
  } else {
    const float s = floor_amax(amax) / kE4M3Max;
    reinterpret_cast<float*>(scale_out)[row * srs + g * sgs] = s;
    for (int64_t i = 0; i < group; ++i) qg[i] = e4m3_encode(clamp_e4m3(to_f32<T>(xg[i]) / s));
  }
}

// ------------------------------------------------------------- static (a4)
template <typename T>
__global__ __launch_bounds__(kQuantThreads) void static_quant_kernel(
    const typename T::storage* __restrict__ x, int64_t n, const void* __restrict__ scale,
    int scale_dtype, uint8_t* __restrict__ q) {
  const float s = load_f32(scale, scale_dtype, 0);
  const int64_t stride = (int64_t)gridDim.x * kQuantThreads;
  for (int64_t i = (int64_t)blockIdx.x * kQuantThreads + threadIdx.x; i < n; i += stride) {
    q[i] = e4m3_encode(clamp_e4m3(to_f32<T>(x[i]) / s));
  }
}

template <typename T>
__global__ __launch_bounds__(kQuantThreads) void static_quant_vec_kernel(
    const typename T::storage* __restrict__ x, int64_t nvec, const void* __restrict__ scale,
    int scale_dtype, uint8_t* __restrict__ q) {
  constexpr int V = Vec16<T>::N;
  const float s = load_f32(scale, scale_dtype, 0);
  const Divisor dv = make_divisor(s);
  const uint4* xv = reinterpret_cast<const uint4*>(x);
  const int64_t stride = (int64_t)gridDim.x * kQuantThreads;
  float f[V];
  // Two vectors in flight per thread: both loads are issued before either is converted.
  for (int64_t v = (int64_t)blockIdx.x * kQuantThreads + threadIdx.x; v < nvec; v += 2 * stride) {
    const bool second = v + stride < nvec;
    const uint4 a = xv[v];
    uint4 b{};
    if (second) b = xv[v + stride];
    unpack16<T>(a, f);
    store_quant<V>(q + v * V, f, dv);
    if (second) {
      unpack16<T>(b, f);
      store_quant<V>(q + (v + stride) * V, f, dv);
    }
  }
}

// ------------------------------------------------------------ host launchers
template <typename T>
int launch_per_token(const void* x, int64_t rows, int64_t k, int64_t ldx, void* q, int64_t ldq,
                     float* scale, hipStream_t st) {
  using S = typename T::storage;
  constexpr int V = Vec16<T>::N;
  const S* xs = static_cast<const S*>(x);
  uint8_t* qb = static_cast<uint8_t*>(q);
  const bool vec_ok = aligned16(x) && (k % V == 0) && ((ldx * (int64_t)sizeof(S)) % 16 == 0) &&
                      ((reinterpret_cast<uintptr_t>(q) % V) == 0) && (ldq % V == 0);
  const dim3 grid((unsigned)rows), block(kQuantThreads);
  if (!vec_ok) {
    hipLaunchKernelGGL(per_token_quant_scalar_kernel<T>, grid, block, 0, st, xs, k, ldx, qb, ldq, scale);
    return check_launch("per_token_quant_fp8");
  }
  const int64_t per_lane = cdiv(k / V, kWave);
  if (per_lane <= 16) {
    const dim3 wgrid((unsigned)cdiv(rows, kQuantThreads / kWave));
#define AYK_PW(VPT) \
  hipLaunchKernelGGL((per_token_quant_wave_kernel<T, VPT>), wgrid, block, 0, st, xs, rows, k, ldx, qb, ldq, scale)
    if (per_lane <= 1) AYK_PW(1);
    else if (per_lane <= 2) AYK_PW(2);
    else if (per_lane <= 4) AYK_PW(4);
    else if (per_lane <= 8) AYK_PW(8);
    else AYK_PW(16);
#undef AYK_PW
    return check_launch("per_token_quant_fp8");
  }
  const int64_t per_thread = cdiv(k / V, kQuantThreads);
#define AYK_PT(VPT) \
  hipLaunchKernelGGL((per_token_quant_vec_kernel<T, VPT>), grid, block, 0, st, xs, k, ldx, qb, ldq, scale)
  if (per_thread <= 1) AYK_PT(1);
  else if (per_thread <= 2) AYK_PT(2);
  else if (per_thread <= 4) AYK_PT(4);
  else if (per_thread <= 8) AYK_PT(8);
  else if (per_thread <= 16) AYK_PT(16);
  else AYK_PT(0);
#undef AYK_PT
  return check_launch("per_token_quant_fp8");
}

template <typename T, bool MX>
// Scale of (row, group g) at scale[row * srs + g * sgs].
int launch_group(const void* x, int64_t rows, int64_t k, int64_t ldx, int64_t group, void* q,
                 int64_t ldq, void* scale, int64_t srs, int64_t sgs, hipStream_t st) {
  using S = typename T::storage;
  constexpr int V = Vec16<T>::N;
  const S* xs = static_cast<const S*>(x);
  uint8_t* qb = static_cast<uint8_t*>(q);
  const int64_t groups = rows * (k / group);
  const int64_t vecs = group / V;
  const bool vec_ok = (group % V == 0) && aligned16(x) && ((ldx * (int64_t)sizeof(S)) % 16 == 0) &&
                      ((reinterpret_cast<uintptr_t>(q) % V) == 0) && (ldq % V == 0) &&
                      (vecs & (vecs - 1)) == 0 && vecs <= 64 * 8;
  if (!vec_ok) {
    const dim3 grid((unsigned)cdiv(groups, kQuantThreads));
    hipLaunchKernelGGL((group_quant_scalar_kernel<T, MX>), grid, dim3(kQuantThreads), 0, st, xs,
                       rows, k, ldx, group, qb, ldq, scale, srs, sgs);
    return check_launch(MX ? "per_token_group_quant_mxfp8" : "per_token_group_quant_fp8");
  }
  const int gl = (int)(vecs < 64 ? vecs : 64);
  const int vpl = (int)(vecs / gl);
  const dim3 grid((unsigned)cdiv(groups * gl, (int64_t)kQuantThreads * kGroupSlots)), block(kQuantThreads);
#define AYK_GQ(GL, VPL)                                                                          \
  hipLaunchKernelGGL((group_quant_vec_kernel<T, GL, VPL, MX>), grid, block, 0, st, xs, rows, k, \
                     ldx, group, qb, ldq, scale, srs, sgs)
  switch (gl) {
    case 1: AYK_GQ(1, 1); break;
    case 2: AYK_GQ(2, 1); break;
    case 4: AYK_GQ(4, 1); break;
    case 8: AYK_GQ(8, 1); break;
    case 16: AYK_GQ(16, 1); break;
    case 32: AYK_GQ(32, 1); break;
    default:
      switch (vpl) {
        case 1: AYK_GQ(64, 1); break;
        case 2: AYK_GQ(64, 2); break;
        case 4: AYK_GQ(64, 4); break;
        default: AYK_GQ(64, 8); break;
      }
  }
#undef AYK_GQ
  return check_launch(MX ? "per_token_group_quant_mxfp8" : "per_token_group_quant_fp8");
}

template <typename T>
int launch_static(const void* x, int64_t n, const void* scale, int sdt, void* q, hipStream_t st) {
  using S = typename T::storage;
  constexpr int V = Vec16<T>::N;
  const S* xs = static_cast<const S*>(x);
  uint8_t* qb = static_cast<uint8_t*>(q);
  if (aligned16(x) && n % V == 0 && (reinterpret_cast<uintptr_t>(q) % V) == 0) {
    const int64_t nvec = n / V;
    const int64_t blocks = cdiv(nvec, kQuantThreads);
    const dim3 grid((unsigned)(blocks < 8192 ? blocks : 8192));
    hipLaunchKernelGGL(static_quant_vec_kernel<T>, grid, dim3(kQuantThreads), 0, st, xs, nvec, scale, sdt, qb);
  } else {
    const int64_t blocks = cdiv(n, kQuantThreads);
    const dim3 grid((unsigned)(blocks < 8192 ? blocks : 8192));
    hipLaunchKernelGGL(static_quant_kernel<T>, grid, dim3(kQuantThreads), 0, st, xs, n, scale, sdt, qb);
  }
  return check_launch("static_quant_fp8");
}

int check_act_dtype(int dt, const char* op) {
  if (dt != AYK_F32 && dt != AYK_F16 && dt != AYK_BF16) {
    return fail(AYK_EINVAL, "%s: x dtype must be float32, float16 or bfloat16 (got %d)", op, dt);
  }
  return AYK_OK;
}

}  // namespace
}  // namespace ayk

using namespace ayk;

extern "C" {

int ayk_per_token_quant_fp8(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx,
                            void* q, int64_t ldq, float* scale, ayk_stream_t stream) {
  if (int rc = check_act_dtype(x_dtype, "per_token_quant_fp8")) return rc;
  if (rows < 0 || k < 1 || ldx < k || ldq < k) {
    return fail(AYK_EINVAL, "per_token_quant_fp8: bad shape rows=%lld k=%lld ldx=%lld ldq=%lld",
                (long long)rows, (long long)k, (long long)ldx, (long long)ldq);
  }
  if (rows > 0x7FFFFFFF) return fail(AYK_EINVAL, "per_token_quant_fp8: rows=%lld exceeds the grid", (long long)rows);
  if (rows == 0) return AYK_OK;
  if (int rc = check_device()) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (x_dtype) {
    case AYK_BF16: return launch_per_token<BF16T>(x, rows, k, ldx, q, ldq, scale, st);
    case AYK_F16: return launch_per_token<F16T>(x, rows, k, ldx, q, ldq, scale, st);
    default: return launch_per_token<F32T>(x, rows, k, ldx, q, ldq, scale, st);
  }
}

static int group_args(const char* op, int x_dtype, int64_t rows, int64_t k, int64_t ldx,
                      int64_t group, int64_t ldq, bool pow2) {
  if (int rc = check_act_dtype(x_dtype, op)) return rc;
  if (group < 1 || (pow2 && (group & (group - 1)))) {
    return fail(AYK_EINVAL, "%s: group_size=%lld must be a positive%s", op, (long long)group,
                pow2 ? " power of two" : " integer");
  }
  if (rows < 0 || k < 1 || k % group || ldx < k || ldq < k) {
    return fail(AYK_EINVAL, "%s: bad shape rows=%lld k=%lld group=%lld", op, (long long)rows,
                (long long)k, (long long)group);
  }
  if (rows * (k / group) > (int64_t)0x7FFFFFFF * 8) return fail(AYK_EINVAL, "%s: too many groups", op);
  return AYK_OK;
}

int ayk_per_token_group_quant_fp8(const void* x, int x_dtype, int64_t rows, int64_t k,
                                  int64_t ldx, int64_t group, void* q, int64_t ldq,
                                  float* scale, ayk_stream_t stream) {
  return ayk_per_token_group_quant_fp8_strided(x, x_dtype, rows, k, ldx, group, q, ldq, scale, group > 0 ? k / group : 0, 1,
                                               stream);
}

int ayk_per_token_group_quant_fp8_strided(const void* x, int x_dtype, int64_t rows, int64_t k,
                                          int64_t ldx, int64_t group, void* q, int64_t ldq,
                                          float* scale, int64_t scale_row_stride, int64_t scale_group_stride,
                                          ayk_stream_t stream) {
  if (int rc = group_args("per_token_group_quant_fp8", x_dtype, rows, k, ldx, group, ldq, true)) return rc;
  const int64_t gpr = k / group;
  const bool rowmajor = scale_group_stride == 1 && scale_row_stride >= gpr;
  const bool colmajor = scale_row_stride == 1 && scale_group_stride >= rows;
  if (!rowmajor && !colmajor) {
    return fail(AYK_EINVAL, "per_token_group_quant_fp8: scale strides (%lld, %lld) must lay out [rows, k/group] or [k/group, rows]",
                (long long)scale_row_stride, (long long)scale_group_stride);
  }
  if (rows == 0) return AYK_OK;
  if (int rc = check_device()) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t srs = scale_row_stride, sgs = scale_group_stride;
  switch (x_dtype) {
    case AYK_BF16: return launch_group<BF16T, false>(x, rows, k, ldx, group, q, ldq, scale, srs, sgs, st);
    case AYK_F16: return launch_group<F16T, false>(x, rows, k, ldx, group, q, ldq, scale, srs, sgs, st);
    default: return launch_group<F32T, false>(x, rows, k, ldx, group, q, ldq, scale, srs, sgs, st);
  }
}

int ayk_per_token_group_quant_mxfp8(const void* x, int x_dtype, int64_t rows, int64_t k,
                                    int64_t ldx, int64_t group, void* q, int64_t ldq,
                                    uint8_t* code, ayk_stream_t stream) {
  if (int rc = group_args("per_token_group_quant_mxfp8", x_dtype, rows, k, ldx, group, ldq, false)) return rc;
  if (rows == 0) return AYK_OK;
  if (int rc = check_device()) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (x_dtype) {
    case AYK_BF16: return launch_group<BF16T, true>(x, rows, k, ldx, group, q, ldq, code, k / group, 1, st);
    case AYK_F16: return launch_group<F16T, true>(x, rows, k, ldx, group, q, ldq, code, k / group, 1, st);
    default: return launch_group<F32T, true>(x, rows, k, ldx, group, q, ldq, code, k / group, 1, st);
  }
}

int ayk_static_quant_fp8(const void* x, int x_dtype, int64_t n, const void* scale,
                         int scale_dtype, void* q, ayk_stream_t stream) {
  if (int rc = check_act_dtype(x_dtype, "static_quant_fp8")) return rc;
  if (scale_dtype != AYK_F32 && scale_dtype != AYK_F16 && scale_dtype != AYK_BF16) {
    return fail(AYK_EINVAL, "static_quant_fp8: scale dtype must be float32, float16 or bfloat16");
  }
  if (n < 0) return fail(AYK_EINVAL, "static_quant_fp8: negative size");
  if (n == 0) return AYK_OK;
  if (int rc = check_device()) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (x_dtype) {
    case AYK_BF16: return launch_static<BF16T>(x, n, scale, scale_dtype, q, st);
    case AYK_F16: return launch_static<F16T>(x, n, scale, scale_dtype, q, st);
    default: return launch_static<F32T>(x, n, scale, scale_dtype, q, st);
  }
}

}  // extern "C"
