// Block-scaled (128 x 128 weight blocks, 1 x 128 activation groups) fp8 GEMM with
// 256 x 256 tiles: the launcher that gemm.hip's fp8_blockwise_mm dispatch calls.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime.h>

namespace ayk {

struct Block256Args {
  const uint8_t* a;  // [M, K] e4m3, row stride lda
  int64_t lda;
  const uint8_t* w;  // [N, K] e4m3, row stride ldw
  int64_t ldw;
  int64_t M, N, K;
  const float* sa;   // fp32 activation scales: [M, ld_sa] (sa_col_major = 0) or [KB, ld_sa]
  int64_t ld_sa;     // row stride of sa in elements (row-major), or K-block stride (column-major)
  int sa_col_major;
  const void* sb;    // weight scales [ceil(N / 128), ld_sb], fp32 / fp16 / bf16
  int sb_dtype;
  int64_t ld_sb;
  const void* bias;  // [N] or nullptr
  int bias_dtype;
  void* out;         // [M, N], row stride ldo
  int out_dtype;
  int64_t ldo;
  float* ws;         // split-K partials [split, M, N] fp32
  size_t ws_bytes;
  int nt_stores;     // store final outputs nontemporally (set by the kernels, not callers)
};

// Grouped (MoE) problem: expert e owns activation rows [expert_offsets[e], + M_e) of
// a [m_total, k] and weights b[e] = [n, k]; scales sa [m_total, k / 128], sb[e]
// [n / 128, k / 128] fp32; out [m_total, n]. problem_sizes [E, 3] = (M_e, N_e, K_e) and
// expert_offsets [E] are read on the device.
struct Grouped256Args {
  const uint8_t* a;
  const uint8_t* b;
  const float* sa;    // [m_total, k / 128]
  const float* sa_t;  // nullptr, or the same table transposed: [k / 128, m_total]
  const float* sb;
  void* out;
  int out_dtype;
  const int32_t* problem_sizes;
  const int32_t* expert_offsets;
  int num_experts;
  int64_t m_total, n, k;
};

// Whether the 256 x 256 kernel takes this problem (shape, alignment and dtype rules).
bool block256_supported(const Block256Args& g);
// K splits the 256 x 256 kernel uses (1: none); a function of the shape only.
int64_t block256_split(int64_t M, int64_t N, int64_t K);
// Launch (the kernel and, with a K split, the reduce). Returns an ayk_status.
int block256_launch(const Block256Args& g, hipStream_t st, const char* op);
// Grouped launch (n and k multiples of 128, 16-byte aligned operands, checked by the
// caller). Returns an ayk_status.
int grouped_block256_launch(const Grouped256Args& ga, hipStream_t st, const char* op);

}  // namespace ayk
