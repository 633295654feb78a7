// KV-cache writes and gathers with static per-tensor FP8 quantization (the attention
// side of the FP8 path): reference python/ayaka/kernel/triton/cache/cache_ops.py
// (write_kv :160, scatter_cache :65, gather_cache :230; their PyTorch oracles
// _write_reference :40, _write_kv_reference :97, _gather_reference :206) and the
// per-tensor policy of kvcache/storage/quantization.py:127-212.
//
// HBM-bound row copies: one workgroup per token row (and plane), each thread a
// 16-byte source chunk, fp8 rows written as 8- or 4-byte chunks. Slots are int64 row
// indices of the flattened [pages * page_size, heads * head_dim] cache.
#include "ayk_common.h"

namespace ayk {
namespace {

constexpr int kKvThreads = 128;
constexpr int kKvVecThreads = 256;
// Chunks per thread in the vector kernels, one grid span apart (all loads issued first).
constexpr int kKvUnroll = 2;

__device__ inline float load_elem(const void* p, int dtype, int64_t i) {
  switch (dtype) {
    case AYK_F32: return reinterpret_cast<const float*>(p)[i];
    case AYK_F16: return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
    case AYK_BF16: return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
    case AYK_E4M3: return e4m3_decode(reinterpret_cast<const uint8_t*>(p)[i]);
    default: return e5m2_decode(reinterpret_cast<const uint8_t*>(p)[i]);
  }
}

__host__ __device__ inline float clamp_e5m2(float y) {
  return y > 57344.0f ? 57344.0f : (y < -57344.0f ? -57344.0f : y);
}

// One element into a cache row: fp8 caches take round-to-nearest-even of the clamped
// scaled value (clamp keeps NaN, as torch.clamp), float caches a plain cast.
__device__ inline void store_elem(void* p, int dtype, int64_t i, float x, float inverse) {
  if (dtype == AYK_E4M3) {
    reinterpret_cast<uint8_t*>(p)[i] = e4m3_encode(clamp_e4m3(x * inverse));
  } else if (dtype == AYK_E5M2) {
    reinterpret_cast<uint8_t*>(p)[i] = e5m2_encode(clamp_e5m2(x * inverse));
  } else {
    store_f32(p, dtype, i, x);
  }
}

// x * scale rounded to fp32 and kept there: left to itself the compiler fuses the
// multiply with a later fp16 conversion into one mixed-precision fma with a +0 addend,
// which turns -0 into +0.
__device__ inline float scaled(float x, float scale) {
  float y = x * scale;
  asm volatile("" : "+v"(y));
  return y;
}

// ---------------------------------------------------------------- 8-element vectors
// Element i (a multiple of 8) of a row: 8 values as one 32-, 16- or 8-byte access.
constexpr int elem_bytes(int dt) { return dt == AYK_F32 ? 4 : (dt == AYK_F16 || dt == AYK_BF16 ? 2 : 1); }

// The raw bytes of 8 elements (up to 32 bytes).
struct Raw8 {
  uint4 lo, hi;
};

template <int DT>
__device__ inline Raw8 load_raw8(const void* p, int64_t i) {
  Raw8 r{};
  const uint8_t* b = static_cast<const uint8_t*>(p) + i * elem_bytes(DT);
  if constexpr (elem_bytes(DT) == 4) {
    r.lo = reinterpret_cast<const uint4*>(b)[0];
    r.hi = reinterpret_cast<const uint4*>(b)[1];
  } else if constexpr (elem_bytes(DT) == 2) {
    r.lo = *reinterpret_cast<const uint4*>(b);
  } else {
    const uint2 w = *reinterpret_cast<const uint2*>(b);
    r.lo.x = w.x;
    r.lo.y = w.y;
  }
  return r;
}

template <int DT>
__device__ inline void store_raw8(void* p, int64_t i, const Raw8& r) {
  uint8_t* b = static_cast<uint8_t*>(p) + i * elem_bytes(DT);
  if constexpr (elem_bytes(DT) == 4) {
    reinterpret_cast<uint4*>(b)[0] = r.lo;
    reinterpret_cast<uint4*>(b)[1] = r.hi;
  } else if constexpr (elem_bytes(DT) == 2) {
    *reinterpret_cast<uint4*>(b) = r.lo;
  } else {
    *reinterpret_cast<uint2*>(b) = make_uint2(r.lo.x, r.lo.y);
  }
}

__device__ inline uint32_t raw_word(const Raw8& r, int w) {
  const uint32_t v[8] = {r.lo.x, r.lo.y, r.lo.z, r.lo.w, r.hi.x, r.hi.y, r.hi.z, r.hi.w};
  return v[w];
}

template <int DT>
__device__ inline void decode8(const Raw8& r, float* x) {
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    if constexpr (DT == AYK_F32) {
      x[q] = u2f(raw_word(r, q));
    } else if constexpr (DT == AYK_F16 || DT == AYK_BF16) {
      const uint16_t h = (uint16_t)(raw_word(r, q / 2) >> (16 * (q % 2)));
      x[q] = DT == AYK_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
    } else {
      const uint8_t c = (uint8_t)(raw_word(r, q / 4) >> (8 * (q % 4)));
      x[q] = DT == AYK_E4M3 ? e4m3_decode(c) : e5m2_decode(c);
    }
  }
}

// fp8: clamp(x * inverse) rounded to nearest even; 16/32-bit floats: plain cast.
template <int DT>
__device__ inline Raw8 encode8(const float* x, float inverse) {
  Raw8 r{};
  uint32_t w[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
  if constexpr (DT == AYK_E4M3 || DT == AYK_E5M2) {
    float y[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) y[q] = DT == AYK_E4M3 ? clamp_e4m3(x[q] * inverse) : clamp_e5m2(x[q] * inverse);
#pragma unroll
    for (int h = 0; h < 2; ++h)
      w[h] = DT == AYK_E4M3 ? e4m3x4_encode(y[4 * h], y[4 * h + 1], y[4 * h + 2], y[4 * h + 3])
                            : e5m2x4_encode(y[4 * h], y[4 * h + 1], y[4 * h + 2], y[4 * h + 3]);
  } else {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      if constexpr (DT == AYK_F32) {
        w[q] = f2u(x[q]);
      } else {
        const uint32_t h = DT == AYK_BF16 ? f32_to_bf16_bits(x[q]) : f32_to_f16_bits(x[q]);
        w[q / 2] |= h << (16 * (q % 2));
      }
    }
  }
  r.lo = make_uint4(w[0], w[1], w[2], w[3]);
  r.hi = make_uint4(w[4], w[5], w[6], w[7]);
  return r;
}

// Vector write: chunk c is elements 8 * (c % cpr) .. + 7 of token c / cpr; a thread
// takes kKvUnroll chunks one grid span apart; blockIdx.y
// is the plane (0 key, 1 value). The host checks width % 8 == 0, 16-byte aligned rows
// and chunk counts below 2^31.
template <int SRC, int DST>
__global__ __launch_bounds__(kKvVecThreads) void kv_write_vec_kernel(
    const void* __restrict__ key, const void* __restrict__ value, uint32_t cpr, uint32_t chunks, int64_t width,
    int64_t src_stride, void* __restrict__ key_cache, void* __restrict__ value_cache, int64_t num_slots,
    const int64_t* __restrict__ slots, float k_inv, float v_inv) {
  const uint32_t span = gridDim.x * kKvVecThreads;
  const bool v_plane = blockIdx.y == 1;
  const void* src = v_plane ? value : key;
  void* dst = v_plane ? value_cache : key_cache;
  Raw8 in[kKvUnroll];
  int64_t slot[kKvUnroll], e[kKvUnroll];
#pragma unroll
  for (int u = 0; u < kKvUnroll; ++u) {
    const uint32_t c = blockIdx.x * kKvVecThreads + threadIdx.x + u * span;
    slot[u] = -1;
    if (c < chunks) {
      const uint32_t t = c / cpr;
      e[u] = (int64_t)(c - t * cpr) * 8;
      slot[u] = slots[t];
      in[u] = load_raw8<SRC>(src, (int64_t)t * src_stride + e[u]);
    }
  }
#pragma unroll
  for (int u = 0; u < kKvUnroll; ++u) {
    if (slot[u] < 0 || slot[u] >= num_slots) continue;  // past the end, masked or invalid: nothing written
    if constexpr (SRC == DST) {
      store_raw8<DST>(dst, slot[u] * width + e[u], in[u]);
    } else {
      float x[8];
      decode8<SRC>(in[u], x);
      store_raw8<DST>(dst, slot[u] * width + e[u], encode8<DST>(x, v_plane ? v_inv : k_inv));
    }
  }
}

// Vector gather: out-of-range slots give zero rows; DEQ multiplies by `scale` in fp32.
template <int SRC, int DST, bool DEQ>
__global__ __launch_bounds__(kKvVecThreads) void kv_gather_vec_kernel(const void* __restrict__ cache, uint32_t cpr,
                                                                       uint32_t chunks, int64_t width, int64_t num_slots,
                                                                       const int64_t* __restrict__ slots,
                                                                       void* __restrict__ dest, float scale) {
  const uint32_t span = gridDim.x * kKvVecThreads;
  Raw8 in[kKvUnroll];
  int64_t d[kKvUnroll];
  bool live[kKvUnroll], ok[kKvUnroll];
#pragma unroll
  for (int u = 0; u < kKvUnroll; ++u) {
    const uint32_t c = blockIdx.x * kKvVecThreads + threadIdx.x + u * span;
    live[u] = c < chunks;
    ok[u] = false;
    in[u] = Raw8{};
    if (live[u]) {
      const uint32_t i = c / cpr;
      const int64_t e = (int64_t)(c - i * cpr) * 8;
      const int64_t slot = slots[i];
      d[u] = (int64_t)i * width + e;
      ok[u] = slot >= 0 && slot < num_slots;
      if (ok[u]) in[u] = load_raw8<SRC>(cache, slot * width + e);
    }
  }
#pragma unroll
  for (int u = 0; u < kKvUnroll; ++u) {
    if (!live[u]) continue;
    if (!ok[u]) {
      store_raw8<DST>(dest, d[u], Raw8{});  // all-zero bits are +0 in every dtype here
    } else if constexpr (SRC == DST && !DEQ) {
      store_raw8<DST>(dest, d[u], in[u]);
    } else {
      float x[8];
      decode8<SRC>(in[u], x);
      if constexpr (DEQ) {
#pragma unroll
        for (int q = 0; q < 8; ++q) x[q] = scaled(x[q], scale);
      }
      store_raw8<DST>(dest, d[u], encode8<DST>(x, 1.0f));
    }
  }
}

// fp8 cache -> 16-bit destination with rows of whole 16-element chunks (16 cache bytes,
// 32 destination bytes): one 16-byte load and two 16-byte stores per chunk. A thread
// takes kKvWide chunks one grid span apart and loads every slot index before any cache
// row, so it waits two memory latencies in all (the row address depends on the slot).
// One chunk per thread measured fastest (16384 Llama-3-8B tokens: 14.6 us against
// 15.4 / 17.0 / 19.7 us for 2 / 4 / 8): more resident wavefronts beat more loads per
// wavefront here.
constexpr int kKvWide = 1;
template <int SRC, int DST, bool DEQ>
__global__ __launch_bounds__(kKvVecThreads) void kv_gather_wide_kernel(const uint8_t* __restrict__ cache, uint32_t cpr,
                                                                        uint32_t chunks, int64_t width, int64_t num_slots,
                                                                        const int64_t* __restrict__ slots,
                                                                        void* __restrict__ dest, float scale) {
  static_assert(elem_bytes(SRC) == 1 && elem_bytes(DST) == 2, "fp8 cache, 16-bit destination");
  const uint32_t span = gridDim.x * kKvVecThreads;
  // Branch-free up to the stores: a load inside a branch makes the compiler wait for
  // it before the next one, which serializes the chunks' latencies. Chunks past the end
  // re-read the last chunk; slots outside the cache read cache row 0 and are zeroed.
  int64_t src[kKvWide], d[kKvWide];
  bool live[kKvWide], ok[kKvWide];
#pragma unroll
  for (int u = 0; u < kKvWide; ++u) {
    const uint32_t c0 = blockIdx.x * kKvVecThreads + threadIdx.x + u * span;
    live[u] = c0 < chunks;
    const uint32_t c = live[u] ? c0 : chunks - 1;
    const uint32_t i = c / cpr;
    const int64_t e = (int64_t)(c - i * cpr) * 16;
    d[u] = (int64_t)i * width + e;
    const int64_t slot = slots[i];
    ok[u] = slot >= 0 && slot < num_slots;
    src[u] = (ok[u] ? slot : 0) * width + e;
  }
  uint4 in[kKvWide];
#pragma unroll
  for (int u = 0; u < kKvWide; ++u) {
    const uint4 v = *reinterpret_cast<const uint4*>(cache + src[u]);
    in[u] = ok[u] ? v : make_uint4(0u, 0u, 0u, 0u);
  }
#pragma unroll
  for (int u = 0; u < kKvWide; ++u) {
    if (!live[u]) continue;
    uint4* out = reinterpret_cast<uint4*>(static_cast<uint8_t*>(dest) + d[u] * 2);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      Raw8 r{};
      r.lo.x = h ? in[u].z : in[u].x;
      r.lo.y = h ? in[u].w : in[u].y;
      float x[8];
      decode8<SRC>(r, x);
      if constexpr (DEQ) {
#pragma unroll
        for (int q = 0; q < 8; ++q) x[q] = scaled(x[q], scale);
      }
      // An out-of-range slot gives a zero row: its zero bytes decode to +0.
      out[h] = encode8<DST>(x, 1.0f).lo;
    }
  }
}

// Scalar fallbacks for rows that are not 8-element / 16-byte aligned.
// blockIdx.x: token; blockIdx.y: plane (0 key, 1 value).
__global__ __launch_bounds__(kKvThreads) void kv_write_kernel(const void* __restrict__ key, const void* __restrict__ value,
                                                               int src_dtype, int64_t width, int64_t src_stride,
                                                               void* __restrict__ key_cache, void* __restrict__ value_cache,
                                                               int cache_dtype, int64_t num_slots,
                                                               const int64_t* __restrict__ slots, float k_inv, float v_inv) {
  const int64_t t = blockIdx.x;
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= num_slots) return;
  const bool v_plane = blockIdx.y == 1;
  const void* src = v_plane ? value : key;
  void* dst = v_plane ? value_cache : key_cache;
  const float inv = v_plane ? v_inv : k_inv;
  const int64_t s0 = t * src_stride, d0 = slot * width;
  const bool same = src_dtype == cache_dtype;  // bit copy, as a same-dtype .to() is
  for (int64_t i = threadIdx.x; i < width; i += kKvThreads) {
    if (same && src_dtype == AYK_F32)
      static_cast<uint32_t*>(dst)[d0 + i] = static_cast<const uint32_t*>(src)[s0 + i];
    else if (same)
      static_cast<uint16_t*>(dst)[d0 + i] = static_cast<const uint16_t*>(src)[s0 + i];
    else
      store_elem(dst, cache_dtype, d0 + i, load_elem(src, src_dtype, s0 + i), inv);
  }
}

__global__ __launch_bounds__(kKvThreads) void kv_gather_kernel(const void* __restrict__ cache, int cache_dtype,
                                                                int64_t num_slots, int64_t width,
                                                                const int64_t* __restrict__ slots, void* __restrict__ dest,
                                                                int dest_dtype, float scale, int dequantize) {
  const int64_t i = blockIdx.x;
  const int64_t slot = slots[i];
  const bool ok = slot >= 0 && slot < num_slots;
  for (int64_t e = threadIdx.x; e < width; e += kKvThreads) {
    float x = ok ? load_elem(cache, cache_dtype, slot * width + e) : 0.0f;
    if (dequantize) x = scaled(x, scale);
    if (dest_dtype == AYK_E4M3 || dest_dtype == AYK_E5M2) {
      // Raw fp8 copy (no dequantization, same dtype).
      static_cast<uint8_t*>(dest)[i * width + e] = ok ? static_cast<const uint8_t*>(cache)[slot * width + e] : (uint8_t)0;
    } else if (!dequantize && dest_dtype == cache_dtype) {
      // Same float dtype: copy the bits (NaN payloads included), as index_select does.
      const int sz = dtype_size(dest_dtype);
      if (sz == 4) {
        static_cast<uint32_t*>(dest)[i * width + e] = ok ? static_cast<const uint32_t*>(cache)[slot * width + e] : 0u;
      } else {
        static_cast<uint16_t*>(dest)[i * width + e] = ok ? static_cast<const uint16_t*>(cache)[slot * width + e] : (uint16_t)0;
      }
    } else {
      store_f32(dest, dest_dtype, i * width + e, x);
    }
  }
}

// ---------------------------------------------------------------- host dispatch
template <int SRC>
void launch_write_vec(int dst, dim3 grid, hipStream_t st, const void* key, const void* value, uint32_t cpr,
                            uint32_t chunks, int64_t width, int64_t stride, void* kc, void* vc, int64_t num_slots,
                            const int64_t* slots, float ki, float vi) {
#define AYK_KVW(D)                                                                                                      \
  hipLaunchKernelGGL((kv_write_vec_kernel<SRC, D>), grid, dim3(kKvVecThreads), 0, st, key, value, cpr, chunks, width, \
                     stride, kc, vc, num_slots, slots, ki, vi)
  switch (dst) {
    case AYK_F32: AYK_KVW(AYK_F32); break;
    case AYK_F16: AYK_KVW(AYK_F16); break;
    case AYK_BF16: AYK_KVW(AYK_BF16); break;
    case AYK_E4M3: AYK_KVW(AYK_E4M3); break;
    default: AYK_KVW(AYK_E5M2); break;
  }
#undef AYK_KVW
}

template <int SRC, bool DEQ>
void launch_gather_vec(int dst, dim3 grid, hipStream_t st, const void* cache, uint32_t cpr, uint32_t chunks,
                       int64_t width, int64_t num_slots, const int64_t* slots, void* dest, float scale) {
#define AYK_KVG(D)                                                                                                   \
  hipLaunchKernelGGL((kv_gather_vec_kernel<SRC, D, DEQ>), grid, dim3(kKvVecThreads), 0, st, cache, cpr, chunks, width, \
                     num_slots, slots, dest, scale)
  switch (dst) {
    case AYK_F32: AYK_KVG(AYK_F32); break;
    case AYK_F16: AYK_KVG(AYK_F16); break;
    case AYK_BF16: AYK_KVG(AYK_BF16); break;
    default:
      // fp8 destinations are only raw copies of the same dtype (checked by the caller).
      if constexpr (!DEQ && (SRC == AYK_E4M3 || SRC == AYK_E5M2)) AYK_KVG(SRC);
      break;
  }
#undef AYK_KVG
}

bool is_kv_dtype(int dt) {
  return dt == AYK_F32 || dt == AYK_F16 || dt == AYK_BF16 || dt == AYK_E4M3 || dt == AYK_E5M2;
}

}  // namespace
}  // namespace ayk

using namespace ayk;

extern "C" {

int ayk_kv_cache_write(const void* key, const void* value, int src_dtype, int64_t num_tokens, int64_t width,
                       int64_t src_row_stride, void* key_cache, void* value_cache, int cache_dtype,
                       int64_t num_slots, const int64_t* slots, float k_inverse, float v_inverse,
                       ayk_stream_t stream) {
  const char* op = "kv_cache_write";
  if (num_tokens < 0 || width < 1 || num_slots < 0 || src_row_stride < width)
    return fail(AYK_EINVAL, "%s: bad shape tokens=%lld width=%lld slots=%lld stride=%lld", op, (long long)num_tokens,
                (long long)width, (long long)num_slots, (long long)src_row_stride);
  if (src_dtype != AYK_F32 && src_dtype != AYK_F16 && src_dtype != AYK_BF16)
    return fail(AYK_EINVAL, "%s: key/value must be float32, float16 or bfloat16", op);
  if (!is_kv_dtype(cache_dtype)) return fail(AYK_EINVAL, "%s: unsupported cache dtype %d", op, cache_dtype);
  if (!(k_inverse > 0.0f) || !(v_inverse > 0.0f) || k_inverse == INFINITY || v_inverse == INFINITY)
    return fail(AYK_EINVAL, "%s: KV inverse scales must be finite and positive", op);
  if (num_tokens == 0) return AYK_OK;
  if (key == nullptr || key_cache == nullptr || slots == nullptr || (value != nullptr) != (value_cache != nullptr))
    return fail(AYK_EINVAL, "%s: missing operand", op);
  if (num_tokens > 0x7FFFFFFF) return fail(AYK_EINVAL, "%s: too many tokens", op);
  if (int rc = check_device()) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned planes = value ? 2u : 1u;
  const int64_t cpr = width / 8, chunks = num_tokens * cpr;
  const bool vec = width % 8 == 0 && src_row_stride % 8 == 0 && chunks < 0x7FFFFFFFll && aligned16(key) &&
                   aligned16(key_cache) && (!value || (aligned16(value) && aligned16(value_cache)));
  if (vec) {
    const dim3 grid((unsigned)cdiv(chunks, kKvVecThreads * kKvUnroll), planes);
    const uint32_t c32 = (uint32_t)cpr, n32 = (uint32_t)chunks;
    switch (src_dtype) {
      case AYK_F32:
        launch_write_vec<AYK_F32>(cache_dtype, grid, st, key, value, c32, n32, width, src_row_stride, key_cache,
                                  value_cache, num_slots, slots, k_inverse, v_inverse);
        break;
      case AYK_F16:
        launch_write_vec<AYK_F16>(cache_dtype, grid, st, key, value, c32, n32, width, src_row_stride, key_cache,
                                  value_cache, num_slots, slots, k_inverse, v_inverse);
        break;
      default:
        launch_write_vec<AYK_BF16>(cache_dtype, grid, st, key, value, c32, n32, width, src_row_stride, key_cache,
                                   value_cache, num_slots, slots, k_inverse, v_inverse);
        break;
    }
  } else {
    hipLaunchKernelGGL(kv_write_kernel, dim3((unsigned)num_tokens, planes), dim3(kKvThreads), 0, st, key, value,
                       src_dtype, width, src_row_stride, key_cache, value_cache, cache_dtype, num_slots, slots,
                       k_inverse, v_inverse);
  }
  return check_launch(op);
}

int ayk_kv_cache_gather(const void* cache, int cache_dtype, int64_t num_slots, int64_t width, const int64_t* slots,
                        int64_t n, void* dest, int dest_dtype, float scale, int dequantize, ayk_stream_t stream) {
  const char* op = "kv_cache_gather";
  if (n < 0 || width < 1 || num_slots < 0) return fail(AYK_EINVAL, "%s: bad shape", op);
  if (!is_kv_dtype(cache_dtype) || !is_kv_dtype(dest_dtype)) return fail(AYK_EINVAL, "%s: unsupported dtype", op);
  const bool fp8_src = cache_dtype == AYK_E4M3 || cache_dtype == AYK_E5M2;
  const bool fp8_dst = dest_dtype == AYK_E4M3 || dest_dtype == AYK_E5M2;
  if (dequantize && (!fp8_src || fp8_dst)) return fail(AYK_EINVAL, "%s: dequantize needs an fp8 cache and a float destination", op);
  if (!dequantize && fp8_dst && dest_dtype != cache_dtype) return fail(AYK_EINVAL, "%s: fp8 destination must match the cache dtype", op);
  if (n == 0) return AYK_OK;
  if (cache == nullptr || slots == nullptr || dest == nullptr) return fail(AYK_EINVAL, "%s: missing operand", op);
  if (n > 0x7FFFFFFF) return fail(AYK_EINVAL, "%s: too many rows", op);
  if (int rc = check_device()) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t cpr = width / 8, chunks = n * cpr;
  const bool dst16 = dest_dtype == AYK_F16 || dest_dtype == AYK_BF16;
  // (The wide kernel reads cache row 0 for out-of-range slots: it needs a non-empty cache.)
  if (fp8_src && dst16 && num_slots > 0 && width % 16 == 0 && chunks / 2 < 0x7FFFFFFFll && aligned16(cache) &&
      aligned16(dest)) {
    const uint32_t c32 = (uint32_t)(width / 16), n32 = (uint32_t)(chunks / 2);
    const dim3 grid((unsigned)cdiv(chunks / 2, kKvVecThreads * kKvWide));
#define AYK_KVW16(S, D, Q)                                                                                      \
  hipLaunchKernelGGL((kv_gather_wide_kernel<S, D, Q>), grid, dim3(kKvVecThreads), 0, st,                     \
                     static_cast<const uint8_t*>(cache), c32, n32, width, num_slots, slots, dest, scale)
    const bool e4 = cache_dtype == AYK_E4M3, bf = dest_dtype == AYK_BF16;
    if (dequantize) {
      if (e4) { if (bf) AYK_KVW16(AYK_E4M3, AYK_BF16, true); else AYK_KVW16(AYK_E4M3, AYK_F16, true); }
      else { if (bf) AYK_KVW16(AYK_E5M2, AYK_BF16, true); else AYK_KVW16(AYK_E5M2, AYK_F16, true); }
    } else {
      if (e4) { if (bf) AYK_KVW16(AYK_E4M3, AYK_BF16, false); else AYK_KVW16(AYK_E4M3, AYK_F16, false); }
      else { if (bf) AYK_KVW16(AYK_E5M2, AYK_BF16, false); else AYK_KVW16(AYK_E5M2, AYK_F16, false); }
    }
#undef AYK_KVW16
  } else if (width % 8 == 0 && chunks < 0x7FFFFFFFll && aligned16(cache) && aligned16(dest)) {
    const dim3 grid((unsigned)cdiv(chunks, kKvVecThreads * kKvUnroll));
    const uint32_t c32 = (uint32_t)cpr, n32 = (uint32_t)chunks;
#define AYK_KVG_SRC(S)                                                                                        \
  case S:                                                                                                     \
    if (dequantize)                                                                                           \
      launch_gather_vec<S, true>(dest_dtype, grid, st, cache, c32, n32, width, num_slots, slots, dest, scale); \
    else                                                                                                      \
      launch_gather_vec<S, false>(dest_dtype, grid, st, cache, c32, n32, width, num_slots, slots, dest, scale); \
    break;
    switch (cache_dtype) {
      AYK_KVG_SRC(AYK_F32)
      AYK_KVG_SRC(AYK_F16)
      AYK_KVG_SRC(AYK_BF16)
      AYK_KVG_SRC(AYK_E4M3)
      AYK_KVG_SRC(AYK_E5M2)
      default: break;
    }
#undef AYK_KVG_SRC
  } else {
    hipLaunchKernelGGL(kv_gather_kernel, dim3((unsigned)n), dim3(kKvThreads), 0, st, cache, cache_dtype, num_slots,
                       width, slots, dest, dest_dtype, scale, dequantize);
  }
  return check_launch(op);
}

}  // extern "C"
