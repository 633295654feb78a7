// FP8 x FP8 GEMM for decode batches (M <= 64): the launcher that gemm.hip's
// fp8_scaled_mm / mxfp8_scaled_mm dispatch calls.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime.h>

namespace ayk {

struct SkinnyFp8Args {
  int mode;          // 0: fp32 per-row / per-tensor scales; 1: UE8M0 codes per 32 K;
                     // 2: fp32 block-128 scales (sa [M, ld_sa] or, with sa_vec, [KB, M];
                     //    sb [ceil(N / 128), ld_sb])
  const uint8_t* a;  // [M, K] e4m3, row stride lda
  int64_t lda;
  const uint8_t* w;  // [N, K] e4m3, row stride ldw
  int64_t ldw;
  int64_t M, N, K;
  const void* sa;    // fp32 scalar / [M] (sa_vec), or u8 codes [M, ld_sa]
  int sa_vec;
  int64_t ld_sa;
  const void* sb;    // fp32 scalar / [N] (sb_vec), or u8 codes [N, ld_sb]
  int sb_vec;
  int64_t ld_sb;
  const void* bias;  // [N] or nullptr
  int bias_dtype;
  void* out;         // [M, N], row stride ldo
  int out_dtype;
  int64_t ldo;
  float* ws;         // K-split partials [split, M, N] fp32
  size_t ws_bytes;
};

// Whether the kernel takes this problem (shape, alignment and scale-layout rules).
bool skinny_fp8_supported(const SkinnyFp8Args& g);
// Bytes of K-split partials a launch of this shape needs (0: none); shape only.
size_t skinny_fp8_workspace(int64_t M, int64_t N, int64_t K, int mode);
// Launch (the kernel and, with a K split, the fixed-order reduce). Returns an ayk_status.
int skinny_fp8_launch(const SkinnyFp8Args& g, hipStream_t st, const char* op);
// Per-token quantization of a bf16 / fp16 / fp32 activation (x, row stride ldx in
// elements) fused with the 2-8-row GEMM (g.a, g.lda, g.sa unused). Returns an ayk_status.
bool rows_gemv_quant_supported(const SkinnyFp8Args& g, int x_dtype, int64_t ldx, const void* x);
int rows_gemv_quant_launch(const SkinnyFp8Args& g, const void* x, int x_dtype, int64_t ldx, hipStream_t st,
                           const char* op);

}  // namespace ayk
