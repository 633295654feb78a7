/*
 * ayaka_fp8.h -- C ABI of the MI355X (gfx950) FP8 linear library `libayaka_fp8.so`.
 *
 * One entry point per `torch.ops.ayaka.*` operator of the reference's FP8 linear
 * path. Every pointer is a raw device pointer (HIP memory on the current device),
 * every size an int64, every element type a value of `ayk_dtype`, and every call is
 * enqueued on the given stream without host synchronisation. No entry point
 * allocates device memory: the split-K GEMVs take a caller-provided workspace whose
 * size is returned by the matching `*_workspace_bytes` query.
 *
 * Return value: AYK_OK (0), or a nonzero `ayk_status` with a message retrievable by
 * `ayk_last_error()` (thread-local, valid until the next failing call on the thread).
 *
 * Layout conventions (all row-major, innermost stride 1):
 *   activations a / x : [M, K], row stride lda/ldx elements
 *   weights w / b     : [N, K] e4m3 bytes, row stride ldw/ldb bytes
 *   outputs out       : [M, N], row stride ldo elements
 */
#ifndef AYAKA_FP8_H
#define AYAKA_FP8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Opaque stream handle: a hipStream_t (0 = the legacy default stream). */
typedef void* ayk_stream_t;

typedef enum ayk_dtype {
  AYK_F32 = 0,
  AYK_F16 = 1,
  AYK_BF16 = 2,
  AYK_E4M3 = 3, /* OCP float8 e4m3fn */
  AYK_U8 = 4,   /* raw bytes; as a scale: UE8M0 exponent codes */
  AYK_E5M2 = 5  /* OCP float8 e5m2 (KV caches) */
} ayk_dtype;

typedef enum ayk_status {
  AYK_OK = 0,
  AYK_EINVAL = 1,     /* bad argument: shape, stride, dtype or alignment */
  AYK_EARCH = 2,      /* the current device is not gfx950 */
  AYK_ELAUNCH = 3,    /* the HIP launch failed */
  AYK_EWORKSPACE = 4  /* workspace missing or too small */
} ayk_status;

/* Message of the last failing call on this thread ("" if none). */
const char* ayk_last_error(void);

/* Which kernels (and K split) the last GEMM launch on this thread ran, e.g.
 * "skinny fn=2 fm=2 ks=1 g=2 ch=4 split=1" or "pair tail=4": a diagnostic string,
 * not a stable format. No counterpart in the reference (its Triton launches pick
 * configurations inside Triton's autotuner); tests and profilers read it to assert
 * that a shape reaches the kernel it targets. */
const char* ayk_last_plan(void);

/* Library ABI version (major * 100 + minor). */
int ayk_abi_version(void);

/* 1 if `device` is a gfx950 GPU this library has code for, else 0. */
int ayk_device_supported(int device);

/* ---------------------------------------------------------------- quantizers
 * All quantizers write OCP e4m3fn with round-to-nearest-even after clamping the
 * fp32 quotient to [-448, 448]. `x_dtype` is AYK_F32, AYK_F16 or AYK_BF16.     */

/* Replaces ayaka::per_token_quant_fp8
 * (python/ayaka/kernel/triton/quant/fp8_quant.py:452; oracle reference/quant.py:59-66).
 * scale[m] = max(max|x[m,:]|, 1e-10) / 448 ; q = e4m3(clamp(x / scale[m])). */
int ayk_per_token_quant_fp8(const void* x, int x_dtype, int64_t rows, int64_t k,
                            int64_t ldx, void* q, int64_t ldq, float* scale,
                            ayk_stream_t stream);

/* Replaces ayaka::per_token_group_quant_fp8 (fp8_quant.py:297; oracle quant.py:19-29).
 * One fp32 scale per (row, group) stored [rows, k/group] row-major.
 * group: positive power of two dividing k. */
int ayk_per_token_group_quant_fp8(const void* x, int x_dtype, int64_t rows, int64_t k,
                                  int64_t ldx, int64_t group, void* q, int64_t ldq,
                                  float* scale, ayk_stream_t stream);

/* per_token_group_quant_fp8 with the scale table's layout given by strides: the scale of
 * (row m, group g) is stored at scale[m * scale_row_stride + g * scale_group_stride],
 * which must describe [rows, k/group] (group stride 1) or [k/group, rows] (row stride 1).
 * No counterpart in the reference, whose quantizer writes row-major scales only: the
 * column-major table is the layout the block-128 GEMM reads fastest at prefill sizes
 * (fp8_blockwise_mm's sa_col_major), written directly instead of transposed afterwards. */
int ayk_per_token_group_quant_fp8_strided(const void* x, int x_dtype, int64_t rows, int64_t k,
                                          int64_t ldx, int64_t group, void* q, int64_t ldq,
                                          float* scale, int64_t scale_row_stride, int64_t scale_group_stride,
                                          ayk_stream_t stream);

/* Replaces ayaka::per_token_group_quant_mxfp8 (fp8_quant.py:374; oracle quant.py:40-56).
 * code[m, g] = 0 for an all-zero group, else clamp(ceil(log2(amax/448)), -126, 127) + 127.
 * group: positive, divides k. */
int ayk_per_token_group_quant_mxfp8(const void* x, int x_dtype, int64_t rows, int64_t k,
                                    int64_t ldx, int64_t group, void* q, int64_t ldq,
                                    uint8_t* code, ayk_stream_t stream);

/* Replaces ayaka::static_quant_fp8 (fp8_quant.py:517; oracle quant.py:69-79).
 * q[i] = e4m3(clamp(x[i] / scale[0])) over n contiguous elements; the scale is read
 * on the device (`scale_dtype` F32/F16/BF16). */
int ayk_static_quant_fp8(const void* x, int x_dtype, int64_t n, const void* scale,
                         int scale_dtype, void* q, ayk_stream_t stream);

/* ------------------------------------------------------------------ GEMMs
 * Output dtype `out_dtype` is AYK_F32, AYK_F16 or AYK_BF16; `bias` may be NULL.
 * fp32 accumulation everywhere; one rounding to the output dtype.             */

/* Replaces ayaka::fp8_scaled_mm (gemm/fp8_gemm.py:246; oracle reference/gemm.py:17-37).
 * out = (a @ b^T) * scale_a * scale_b + bias, with b the [N, K] weight.
 * scale_a: scalar (sa_per_row = 0) or [M]; scale_b: scalar (sb_per_col = 0) or [N].
 * Requires K % 16 == 0, lda/ldb multiples of 16 and 16-byte aligned a/b. */
int ayk_fp8_scaled_mm(const void* a, int64_t lda, const void* b, int64_t ldb,
                      int64_t M, int64_t N, int64_t K,
                      const void* scale_a, int sa_dtype, int sa_per_row,
                      const void* scale_b, int sb_dtype, int sb_per_col,
                      const void* bias, int bias_dtype,
                      void* out, int out_dtype, int64_t ldo,
                      void* workspace, size_t workspace_bytes, ayk_stream_t stream);
/* Bytes of split-K partials ayk_fp8_scaled_mm may need for this shape (0: none). A
 * launch short of one full round of tiles splits K; a launch whose last round of
 * 256 x 256 tiles is at most a third full splits that round's tiles over K; a decode
 * batch (M <= 64) on a narrow projection splits K across workgroups. Each piece writes
 * its fp32 partial and a fixed-order sum adds the bias and rounds once. The size is
 * the largest any of these needs for the shape. */
size_t ayk_fp8_scaled_mm_workspace_bytes(int64_t M, int64_t N, int64_t K);

/* fp8_rowwise_linear (gemm/fp8_linear.py:168) for 2 to 8 activation rows in one launch:
 * per-token quantization of x (bf16 / fp16 / fp32, row stride ldx in elements) with the
 * arithmetic of ayk_per_token_quant_fp8, then out = (q @ w^T) * s_token * scale_b + bias,
 * the same result bit for bit as the two launches. No counterpart in the reference,
 * which launches the quantizer and the GEMM separately. Requires 2 <= M <= 8,
 * N * K <= 2^24, K % 16 == 0, M * K <= 64 KiB, 16-byte aligned rows of x and w.
 * scale_b: fp32 scalar (sb_per_col = 0) or [N]. */
int ayk_fp8_rowwise_linear_small(const void* x, int x_dtype, int64_t ldx, int64_t M,
                                 const void* w, int64_t ldw, int64_t N, int64_t K,
                                 const float* scale_b, int sb_per_col, const void* bias,
                                 int bias_dtype, void* out, int out_dtype, int64_t ldo,
                                 ayk_stream_t stream);

/* Replaces ayaka::int8_scaled_mm (gemm/int8_gemm.py:134; oracle reference/gemm.py:192-211).
 * out = float(a @ b^T, int32 accumulation) * scale_a[m] * scale_b[n] + bias, with a the
 * [M, K] int8 activation and b the [N, K] int8 weight; scale_a [M] and scale_b [N] fp32.
 * Requires K % 16 == 0, lda/ldb multiples of 16 and 16-byte aligned a/b. */
int ayk_int8_scaled_mm(const void* a, int64_t lda, const void* b, int64_t ldb,
                       int64_t M, int64_t N, int64_t K,
                       const float* scale_a, const float* scale_b,
                       const void* bias, int bias_dtype,
                       void* out, int out_dtype, int64_t ldo,
                       void* workspace, size_t workspace_bytes, ayk_stream_t stream);
/* Bytes of split-K partials ayk_int8_scaled_mm may need for this shape (0: none); the
 * same rule as ayk_fp8_scaled_mm_workspace_bytes. */
size_t ayk_int8_scaled_mm_workspace_bytes(int64_t M, int64_t N, int64_t K);

/* Replaces ayaka::fp8_blockwise_mm (gemm/fp8_gemm.py:370; oracle reference/gemm.py:40-70).
 * out = sum_kb (a[:, kb] @ b[:, kb]^T) * scale_a[m, kb] * scale_b[n / 128, kb] + bias.
 * scale_a: [M, ceil(K/128)] (or [ceil(K/128), M] when sa_col_major), scale_b:
 * [ceil(N/128), ceil(K/128)], both contiguous. Same alignment rules as above. */
int ayk_fp8_blockwise_mm(const void* a, int64_t lda, const void* b, int64_t ldb,
                         int64_t M, int64_t N, int64_t K,
                         const void* scale_a, int sa_dtype, int sa_col_major,
                         const void* scale_b, int sb_dtype,
                         const void* bias, int bias_dtype,
                         void* out, int out_dtype, int64_t ldo,
                         void* workspace, size_t workspace_bytes, ayk_stream_t stream);
/* Bytes of split-K partials ayk_fp8_blockwise_mm may need for this shape (0: none). A
 * launch with fewer tiles than fill the machine (or, for M <= 64, fewer row groups)
 * splits K and sums fp32 partials in a fixed order before the single rounding. */
size_t ayk_fp8_blockwise_mm_workspace_bytes(int64_t M, int64_t N, int64_t K);

/* Replaces fp8_blockwise_scaled_grouped_mm (kernel/triton/moe/moe_grouped_gemm.py:599,
 * kernel :472-585): the MoE grouped block-128 GEMM. Expert e computes rows
 * [expert_offsets[e], + problem_sizes[e][0]) of out:
 *   out[m, n] = sum_kb scales_a[m, kb] * scales_b[e][n / 128][kb] * (a[m, kb] . b[e][n, kb])
 * with a [m_total, k] e4m3, b memory [E][n][k] e4m3, scales_a [m_total, k/128] fp32,
 * scales_a_t nullptr or the same table transposed, [k/128, m_total] (no counterpart in
 * the reference: experts over the whole k read it, at one cache line per 32 rows),
 * scales_b [E][n/128][k/128] fp32, out [m_total, n] bf16/fp16 (row stride n); rows of no
 * expert are not written. problem_sizes [E, 3] int32 (M_e, N_e, K_e) and expert_offsets
 * [E] int32 are read on the device (clamped to the operands). n % 128 == 0,
 * k % 128 == 0, 16-byte aligned a/b/out. */
int ayk_fp8_grouped_blockwise_mm(const void* a, const void* b, const float* scales_a, const float* scales_a_t,
                                 const float* scales_b,
                                 const int32_t* problem_sizes, const int32_t* expert_offsets, int64_t num_experts,
                                 int64_t m_total, int64_t n, int64_t k, void* out, int out_dtype,
                                 ayk_stream_t stream);

/* Replaces ayaka::mxfp8_scaled_mm (gemm/fp8_mxfp8_gemm.py:163; oracle reference/gemm.py:73-92).
 * out = sum_g (a[:, g] @ w[:, g]^T) * 2^(a_scale[m,g]-127) * 2^(w_scale[n,g]-127) + bias
 * over 32-wide K groups g; UE8M0 code 0 decodes to 0 and 0xFF to NaN.
 * K % 32 == 0; a_scale [M, K/32] (row stride ld_as), w_scale [N, K/32] (ld_ws). */
int ayk_mxfp8_scaled_mm(const void* a, int64_t lda, const uint8_t* a_scale, int64_t ld_as,
                        const void* w, int64_t ldw, const uint8_t* w_scale, int64_t ld_ws,
                        int64_t M, int64_t N, int64_t K,
                        const void* bias, int bias_dtype,
                        void* out, int out_dtype, int64_t ldo,
                        void* workspace, size_t workspace_bytes, ayk_stream_t stream);
/* Bytes of split-K partials ayk_mxfp8_scaled_mm may need for this shape (0: none);
 * the same rule as ayk_fp8_scaled_mm_workspace_bytes. */
size_t ayk_mxfp8_scaled_mm_workspace_bytes(int64_t M, int64_t N, int64_t K);

/* Replaces ayaka::fp8_weight_only_gemv (gemm/fp8_gemv.py:323; oracle reference/gemm.py:129-157).
 * out[n] = sum_k x[k] * w[n, k] * scale[(n / by) * scale_row_stride + k / bx]
 * x: [K] F16/BF16; scale_dtype: AYK_U8 (UE8M0), AYK_F32 or AYK_BF16; out dtype == x dtype.
 * The workspace holds split-K partials (see ayk_fp8_weight_only_gemv_workspace_bytes). */
int ayk_fp8_weight_only_gemv(const void* x, int x_dtype, const void* w, int64_t ldw,
                             int64_t N, int64_t K, const void* scale, int scale_dtype,
                             int64_t scale_row_stride, int64_t block_size_y,
                             int64_t block_size_x, void* out,
                             void* workspace, size_t workspace_bytes, ayk_stream_t stream);
size_t ayk_fp8_weight_only_gemv_workspace_bytes(int64_t N, int64_t K);

/* No counterpart in the reference. ayk_fp8_weight_only_gemv without a workspace
 * argument, for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc): the split-K partials live
 * in a static per-device array of ayk_fp8_weight_only_gemv_static_max_bytes() bytes
 * (64 KiB, enough for every shape; a shape needing more is rejected with
 * AYK_EWORKSPACE). Allocates nothing. All calls on one GPU share that array, so calls
 * that overlap on one GPU (different streams, or host threads) race. */
int ayk_fp8_weight_only_gemv_static(const void* x, int x_dtype, const void* w, int64_t ldw,
                                    int64_t N, int64_t K, const void* scale, int scale_dtype,
                                    int64_t scale_row_stride, int64_t block_size_y,
                                    int64_t block_size_x, void* out, ayk_stream_t stream);
size_t ayk_fp8_weight_only_gemv_static_max_bytes(void);

/* Replaces ayaka::fp8_weight_only_gemm (gemm/fp8_w8a16_gemm.py:144; oracle
 * reference/gemm.py:95-126). The [M, K] form of ayk_fp8_weight_only_gemv; out dtype ==
 * x dtype. Each dequantized weight w * scale is rounded to the activation dtype before
 * the product, as the reference does (with a per-row scale, block_size_x >= K, the
 * exact fp8 weight enters the product and the scale multiplies the fp32 sum).
 * Decode batches (M <= 32) may use a K split whose partials live in the workspace;
 * ayk_fp8_weight_only_gemm_workspace_bytes(M, N, K, block_size_x) gives its size
 * (0: none needed). */
int ayk_fp8_weight_only_gemm(const void* x, int x_dtype, int64_t ldx, int64_t M,
                             const void* w, int64_t ldw, int64_t N, int64_t K,
                             const void* scale, int scale_dtype, int64_t scale_row_stride,
                             int64_t block_size_y, int64_t block_size_x,
                             void* out, int64_t ldo, void* workspace, size_t workspace_bytes,
                             ayk_stream_t stream);
size_t ayk_fp8_weight_only_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K,
                                                int64_t block_size_x);

/* Replaces ayaka::fp8_blockwise_gemv (gemm/fp8_gemv.py:433; oracle reference/gemm.py:160-189).
 * out[n] = sum_kb (a[kb] . b[n, kb]) * scale_a[kb] * scale_b[n / 128, kb] + bias[n],
 * a: [K] e4m3, scale_a [ceil(K/128)], scale_b [ceil(N/128), ceil(K/128)] contiguous. */
int ayk_fp8_blockwise_gemv(const void* a, const void* b, int64_t ldb, int64_t N, int64_t K,
                           const void* scale_a, int sa_dtype,
                           const void* scale_b, int sb_dtype,
                           const void* bias, int bias_dtype,
                           void* out, int out_dtype,
                           void* workspace, size_t workspace_bytes, ayk_stream_t stream);
size_t ayk_fp8_blockwise_gemv_workspace_bytes(int64_t N, int64_t K);

/* ------------------------------------------------------------------ KV cache
 * Paged caches are [pages, page_size, heads, head_dim], flattened to `num_slots` rows of
 * `width` = heads * head_dim elements; a slot is page * page_size + offset. */

/* Replaces ayaka::cache_write_kv (kernel/triton/cache/cache_ops.py:160; oracle
 * _write_kv_reference :97 with _write_reference :40) and, with `value` == NULL,
 * ayaka::cache_scatter (cache_ops.py:65). Row t of key (and value), `src_row_stride`
 * elements apart, is written to slot slots[t] of key_cache (value_cache). An fp8 cache
 * (AYK_E4M3 / AYK_E5M2) stores round-to-nearest-even(clamp(x * inverse, +-max)); a float
 * cache stores x cast to its dtype. Negative slots are skipped; slots >= num_slots are
 * skipped too (the caller validates them, as the reference requires). */
int ayk_kv_cache_write(const void* key, const void* value, int src_dtype, int64_t num_tokens,
                       int64_t width, int64_t src_row_stride, void* key_cache, void* value_cache,
                       int cache_dtype, int64_t num_slots, const int64_t* slots,
                       float k_inverse, float v_inverse, ayk_stream_t stream);

/* Replaces ayaka::cache_gather (cache_ops.py:230; oracle _gather_reference :206).
 * dest[i] = cache[slots[i]] (repeats allowed), dequantized as float(value) * scale when
 * `dequantize`, else copied / cast to `dest_dtype`. A slot outside [0, num_slots) gives
 * a zero row. */
int ayk_kv_cache_gather(const void* cache, int cache_dtype, int64_t num_slots, int64_t width,
                        const int64_t* slots, int64_t n, void* dest, int dest_dtype, float scale,
                        int dequantize, ayk_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* AYAKA_FP8_H */
