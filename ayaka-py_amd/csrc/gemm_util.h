// Device helpers shared by the GEMM translation units (gemm.hip, gemm_block.hip).
#pragma once

#include "ayk_common.h"

namespace ayk {
namespace {

// Word 3 of a raw (unstructured, stride 0) buffer resource on gfx9-family GPUs.
constexpr int kBufferFlags = 0x00020000;

// s_waitcnt with only the vector-memory count constrained (gfx9 encoding: vmcnt in
// bits [3:0] and [15:14], expcnt [6:4] and lgkmcnt [11:8] left at their maxima).
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// Workgroup barrier after this wavefront's LDS accesses completed (lgkmcnt(0)); unlike
// __syncthreads it does not wait for outstanding global loads.
__device__ inline void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
}

// A raw buffer resource from wave-uniform values, forced into SGPRs: a descriptor the
// compiler cannot prove uniform is wrapped in a readfirstlane loop at every load.
__device__ inline __amdgpu_buffer_rsrc_t uniform_rsrc(const void* base, int32_t records) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)p);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(p >> 32));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0,
                                           __builtin_amdgcn_readfirstlane(records), kBufferFlags);
}

// Two floats -> two bf16 (round to nearest even) in one dword, with the gfx950
// packed converter.
__device__ inline uint32_t pack_bf16x2(float a, float b) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{a, b}), bf2));
}

}  // namespace
}  // namespace ayk
