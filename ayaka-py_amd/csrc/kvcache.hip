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

__device__ inline float load_elem(const void* p, int dtype, int64_t i) {
  switch (dtype) {
    case AYK_F32: return reinterpret_cast<const float*>(p)[i];
    case AYK_F16: return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
    case AYK_BF16: return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
    case AYK_E4M3: return e4m3_decode(reinterpret_cast<const uint8_t*>(p)[i]);
    default: return e5m2_decode(reinterpret_cast<const uint8_t*>(p)[i]);
  }
}

// One element into a cache row: fp8 caches take round-to-nearest-even of the clamped
// scaled value (clamp keeps NaN, as torch.clamp), float caches a plain cast.
__device__ inline void store_elem(void* p, int dtype, int64_t i, float x, float inverse) {
  if (dtype == AYK_E4M3) {
    reinterpret_cast<uint8_t*>(p)[i] = e4m3_encode(clamp_e4m3(x * inverse));
  } else if (dtype == AYK_E5M2) {
    const float y = x * inverse;
    const float c = y > 57344.0f ? 57344.0f : (y < -57344.0f ? -57344.0f : y);
    reinterpret_cast<uint8_t*>(p)[i] = e5m2_encode(c);
  } else {
    store_f32(p, dtype, i, x);
  }
}

// blockIdx.x: token; blockIdx.y: plane (0 key, 1 value).
__global__ __launch_bounds__(kKvThreads) void kv_write_kernel(const void* __restrict__ key, const void* __restrict__ value,
                                                               int src_dtype, int64_t width, int64_t src_stride,
                                                               void* __restrict__ key_cache, void* __restrict__ value_cache,
                                                               int cache_dtype, int64_t num_slots,
                                                               const int64_t* __restrict__ slots, float k_inv, float v_inv) {
  const int64_t t = blockIdx.x;
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= num_slots) return;  // masked / invalid: nothing written
  const bool v_plane = blockIdx.y == 1;
  const void* src = v_plane ? value : key;
  void* dst = v_plane ? value_cache : key_cache;
  const float inv = v_plane ? v_inv : k_inv;
  const int64_t s0 = t * src_stride, d0 = slot * width;
  // 8 elements per thread and step: one 16-byte load for 16-bit sources.
  for (int64_t e = (int64_t)threadIdx.x * 8; e < width; e += (int64_t)kKvThreads * 8) {
    if (e + 8 <= width && cache_dtype == AYK_E4M3 && src_dtype != AYK_F32) {
      const uint4 raw = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(src) + s0 + e);
      const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
      uint32_t packed[2] = {0u, 0u};
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const uint16_t b = (uint16_t)(w[q / 2] >> (16 * (q % 2)));
        const float x = src_dtype == AYK_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
        packed[q / 4] |= (uint32_t)e4m3_encode(clamp_e4m3(x * inv)) << (8 * (q % 4));
      }
      *reinterpret_cast<uint2*>(static_cast<uint8_t*>(dst) + d0 + e) = make_uint2(packed[0], packed[1]);
    } else {
      const int64_t end = e + 8 < width ? e + 8 : width;
      for (int64_t i = e; i < end; ++i) store_elem(dst, cache_dtype, d0 + i, load_elem(src, src_dtype, s0 + i), inv);
    }
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
    if (dequantize) x = x * scale;
    if (dest_dtype == AYK_E4M3 || dest_dtype == AYK_E5M2) {
      // Raw fp8 copy (no dequantization, same dtype).
      static_cast<uint8_t*>(dest)[i * width + e] = ok ? static_cast<const uint8_t*>(cache)[slot * width + e] : (uint8_t)0;
    } else {
      store_f32(dest, dest_dtype, i * width + e, x);
    }
  }
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
  if (src_dtype != AYK_F32 && (reinterpret_cast<uintptr_t>(key) & 15 || (value && reinterpret_cast<uintptr_t>(value) & 15) ||
                               src_row_stride % 8))
    return fail(AYK_EINVAL, "%s: 16-bit key/value rows must be 16-byte aligned", op);
  if (num_tokens > 0x7FFFFFFF) return fail(AYK_EINVAL, "%s: too many tokens", op);
  if (int rc = check_device()) return rc;
  const dim3 grid((unsigned)num_tokens, value ? 2u : 1u);
  hipLaunchKernelGGL(kv_write_kernel, grid, dim3(kKvThreads), 0, static_cast<hipStream_t>(stream), key, value, src_dtype,
                     width, src_row_stride, key_cache, value_cache, cache_dtype, num_slots, slots, k_inverse, v_inverse);
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
  hipLaunchKernelGGL(kv_gather_kernel, dim3((unsigned)n), dim3(kKvThreads), 0, static_cast<hipStream_t>(stream), cache,
                     cache_dtype, num_slots, width, slots, dest, dest_dtype, scale, dequantize);
  return check_launch(op);
}

}  // extern "C"
