// FP8 GEMM on gfx950 matrix cores: out[M, N] = epilogue(a[M, K] . w[N, K]^T).
//
// One kernel template serves the three W8A8 recipes of the reference
// (python/ayaka/kernel/triton/gemm/fp8_gemm.py, fp8_mxfp8_gemm.py):
//   MODE_SCALED  fp8_scaled_mm     out = acc * sa[m] * sb[n] + bias[n]
//   MODE_BLOCK   fp8_blockwise_mm  acc += (partial over 128 K) * sa[m, kb] * sb[n/128, kb]
//   MODE_MX      mxfp8_scaled_mm   per-32-K UE8M0 codes applied inside the MFMA
//
// Matrix-core mapping. The MFMA is v_mfma_scale_f32_32x32x64_f8f6f4 (e4m3 x e4m3,
// fp32 accumulate). Its "A" operand is a 32-row slab of the *weight* and its "B"
// operand a 32-row slab of the *activation*, so each lane's accumulator column is one
// activation row m and its 16 accumulator rows are weight rows n. That puts the
// per-row activation scale in one register per lane and makes the 128x128 weight
// block scale uniform over a 32-row slab, so the block rescale is one fma per
// accumulator. Within one 64-K step the hardware reads a lane's 32 operand bytes as
// two 16-byte halves, K [16h, 16h+16) and K [32+16h, 48+16h) for lane half h = lane/32,
// and applies the scale byte of lane half b to K block [32b, 32b+32). Fragments are
// read from LDS in that order, so scale block b is exactly MX group 2*step + b.
//
// Tiling. A 256-thread workgroup (4 wavefronts) owns a BN x BM output tile and
// walks K in 128-byte steps (BK = 128: one block-scale step, four MX groups). Tiles
// are staged global -> VGPR -> LDS with double buffering: the next step's 16-byte
// global loads are issued before the current step's MFMAs. LDS rows are padded to
// 144 bytes so the 32 rows a wavefront reads at one K offset fall on distinct banks.
#include "ayk_common.h"

namespace ayk {

int mx_gemv(const void* a, const uint8_t* a_scale, const void* w, int64_t ldw,
            const uint8_t* w_scale, int64_t ld_ws, int64_t N, int64_t K, const void* bias,
            int bias_dtype, void* out, int out_dtype, hipStream_t st);

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int BK = 128;
constexpr int kLdsRow = BK + 16;  // padded LDS row stride in bytes
constexpr int kScaleOne = 127;    // UE8M0 code of 1.0

enum Mode { MODE_SCALED = 0, MODE_BLOCK = 1, MODE_MX = 2 };

struct GemmArgs {
  const uint8_t* a;  // [M, K] e4m3
  int64_t lda;
  const uint8_t* w;  // [N, K] e4m3
  int64_t ldw;
  int64_t M, N, K;
  const void* sa;  // SCALED: scalar/[M]; BLOCK: [M, KB] or [KB, M]; MX: u8 [M, ld_sa]
  int sa_dtype;
  int sa_vec;      // SCALED: per-row; BLOCK: col-major flag
  int64_t ld_sa;
  const void* sb;  // SCALED: scalar/[N]; BLOCK: [NB, KB]; MX: u8 [N, ld_sb]
  int sb_dtype;
  int sb_vec;
  int64_t ld_sb;
  const void* bias;
  int bias_dtype;
  void* out;
  int out_dtype;
  int64_t ldo;
  int tiles_m;     // number of BM tiles along M
};

__device__ inline v16f mfma(const v8i& wa, const v8i& ab, const v16f& c, int sw, int sa) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wa, ab, c, 0, 0, 0, sw, 0, sa);
}

// 32 operand bytes of one lane: K [16h, 16h+16) and [32+16h, 48+16h) of the step.
__device__ inline v8i lds_frag(const uint8_t* p) {
  const uint4 lo = *reinterpret_cast<const uint4*>(p);
  const uint4 hi = *reinterpret_cast<const uint4*>(p + 32);
  v8i r;
  r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
  r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
  return r;
}

// Store four consecutive-n outputs of one activation row m.
__device__ inline void store4(const GemmArgs& g, int64_t m, int64_t n, const float* v) {
  if (m >= g.M) return;
  if (n + 3 < g.N) {
    if (g.out_dtype == AYK_BF16) {
      uint16_t* p = reinterpret_cast<uint16_t*>(g.out) + m * g.ldo + n;
      const uint32_t lo = (uint32_t)f32_to_bf16_bits(v[0]) | ((uint32_t)f32_to_bf16_bits(v[1]) << 16);
      const uint32_t hi = (uint32_t)f32_to_bf16_bits(v[2]) | ((uint32_t)f32_to_bf16_bits(v[3]) << 16);
      if ((reinterpret_cast<uintptr_t>(p) & 7) == 0) {
        *reinterpret_cast<uint2*>(p) = make_uint2(lo, hi);
        return;
      }
    } else if (g.out_dtype == AYK_F32) {
      float* p = reinterpret_cast<float*>(g.out) + m * g.ldo + n;
      if ((reinterpret_cast<uintptr_t>(p) & 15) == 0) {
        *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
        return;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (n + i < g.N) store_f32(g.out, g.out_dtype, m * g.ldo + n + i, v[i]);
  }
}

// BN: weight rows per tile, BM: activation rows per tile, WN x WM wavefront grid.
template <int MODE, int BN, int BM, int WN, int WM>
__global__ __launch_bounds__(kThreads) void fp8_gemm_kernel(GemmArgs g) {
  static_assert(WN * WM == kThreads / kWave, "4 wavefronts per workgroup");
  constexpr int TN = BN / WN, TM = BM / WM;  // wavefront tile
  constexpr int FN = TN / 32, FM = TM / 32;  // 32x32 MFMA tiles per wavefront
  static_assert(FN >= 1 && FM >= 1, "wavefront tile must be a multiple of 32x32");
  constexpr int kChunks = (BN + BM) * (BK / 16);  // 16-byte chunks per stage
  static_assert(kChunks % kThreads == 0, "chunks must divide evenly");
  constexpr int kCPT = kChunks / kThreads;

  __shared__ __attribute__((aligned(16))) uint8_t lds[2][(BN + BM) * kLdsRow];

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  const int wn = wave / WM, wm = wave % WM;
  // Tile order: consecutive workgroups walk M first within one N column of tiles, so
  // the weight slab (the larger operand) is shared by neighbours in time.
  const int tm = blockIdx.x % g.tiles_m;
  const int tn = blockIdx.x / g.tiles_m;
  const int64_t n_base = (int64_t)tn * BN;
  const int64_t m_base = (int64_t)tm * BM;
  const int nk = (int)cdiv(g.K, BK);

  // Global chunk assignment: chunk c -> tile row c / 8, 16-byte column c % 8.
  uint4 stage[kCPT];
  auto load_stage = [&](int kt) {
#pragma unroll
    for (int i = 0; i < kCPT; ++i) {
      const int c = tid + i * kThreads;
      const int row = c / (BK / 16);
      const int col = (c % (BK / 16)) * 16;
      const int64_t k = (int64_t)kt * BK + col;
      const uint8_t* src;
      bool ok;
      if (row < BN) {
        const int64_t n = n_base + row;
        ok = n < g.N && k < g.K;
        src = g.w + n * g.ldw + k;
      } else {
        const int64_t m = m_base + (row - BN);
        ok = m < g.M && k < g.K;
        src = g.a + m * g.lda + k;
      }
      stage[i] = ok ? *reinterpret_cast<const uint4*>(src) : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < kCPT; ++i) {
      const int c = tid + i * kThreads;
      const int row = c / (BK / 16);
      const int col = (c % (BK / 16)) * 16;
      *reinterpret_cast<uint4*>(&lds[buf][row * kLdsRow + col]) = stage[i];
    }
  };

  v16f acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int frag_row = lane % 32;
  const int frag_k = (lane / 32) * 16;
  const int64_t kblocks = cdiv(g.K, BK);

  load_stage(0);
  store_stage(0);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load_stage(kt + 1);

    v16f part[FN][FM];
    if constexpr (MODE == MODE_BLOCK) {
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) part[i][j][r] = 0.0f;
    }

#pragma unroll
    for (int ks = 0; ks < BK / 64; ++ks) {
      v8i wf[FN], af[FM];
      int wsc[FN], asc[FM];
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        const int row = wn * TN + i * 32 + frag_row;
        wf[i] = lds_frag(&lds[buf][row * kLdsRow + ks * 64 + frag_k]);
        wsc[i] = kScaleOne;
        if constexpr (MODE == MODE_MX) {
          const int64_t n = n_base + row;
          const int64_t grp = (int64_t)kt * 4 + ks * 2 + lane / 32;
          wsc[i] = (n < g.N && grp * 32 < g.K)
                       ? reinterpret_cast<const uint8_t*>(g.sb)[n * g.ld_sb + grp] : kScaleOne;
        }
      }
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const int row = wm * TM + j * 32 + frag_row;
        af[j] = lds_frag(&lds[buf][(BN + row) * kLdsRow + ks * 64 + frag_k]);
        asc[j] = kScaleOne;
        if constexpr (MODE == MODE_MX) {
          const int64_t m = m_base + row;
          const int64_t grp = (int64_t)kt * 4 + ks * 2 + lane / 32;
          asc[j] = (m < g.M && grp * 32 < g.K)
                       ? reinterpret_cast<const uint8_t*>(g.sa)[m * g.ld_sa + grp] : kScaleOne;
        }
      }
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) {
          if constexpr (MODE == MODE_BLOCK) part[i][j] = mfma(wf[i], af[j], part[i][j], wsc[i], asc[j]);
          else acc[i][j] = mfma(wf[i], af[j], acc[i][j], wsc[i], asc[j]);
        }
    }

    if constexpr (MODE == MODE_BLOCK) {
      // acc += partial * sa[m, kb] * sb[n / 128, kb]; one sb per 32-row weight slab.
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const int64_t m = m_base + wm * TM + j * 32 + frag_row;
        const int64_t mi = m < g.M ? m : g.M - 1;
        const float sa = load_f32(g.sa, g.sa_dtype, g.sa_vec ? (int64_t)kt * g.M + mi : mi * kblocks + kt);
#pragma unroll
        for (int i = 0; i < FN; ++i) {
          const int64_t n = n_base + wn * TN + i * 32;
          const int64_t nb = (n < g.N ? n : g.N - 1) / 128;
          const float s = sa * load_f32(g.sb, g.sb_dtype, nb * kblocks + kt);
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] = fmaf(part[i][j][r], s, acc[i][j][r]);
        }
      }
    }

    if (kt + 1 < nk) store_stage(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: scale, bias, one rounding to the output dtype.
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int64_t m = m_base + wm * TM + j * 32 + frag_row;
    float sa = 1.0f;
    if constexpr (MODE == MODE_SCALED) {
      const int64_t mi = m < g.M ? m : g.M - 1;
      sa = load_f32(g.sa, g.sa_dtype, g.sa_vec ? mi : 0);
    }
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
      for (int grp = 0; grp < 4; ++grp) {
        const int64_t n0 = n_base + wn * TN + i * 32 + grp * 8 + (lane / 32) * 4;
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t n = n0 + q;
          const int64_t ni = n < g.N ? n : g.N - 1;
          float y = acc[i][j][grp * 4 + q];
          if constexpr (MODE == MODE_SCALED) {
            y = y * sa;
            y = y * load_f32(g.sb, g.sb_dtype, g.sb_vec ? ni : 0);
          }
          if (g.bias) y += load_f32(g.bias, g.bias_dtype, ni);
          v[q] = y;
        }
        store4(g, m, n0, v);
      }
    }
  }
}

template <int MODE, int BN, int BM, int WN, int WM>
int launch_cfg(GemmArgs g, hipStream_t st, const char* op) {
  g.tiles_m = (int)cdiv(g.M, BM);
  const int64_t tiles = (int64_t)g.tiles_m * cdiv(g.N, BN);
  if (tiles > 0x7FFFFFFF) return fail(AYK_EINVAL, "%s: problem too large", op);
  hipLaunchKernelGGL((fp8_gemm_kernel<MODE, BN, BM, WN, WM>), dim3((unsigned)tiles), dim3(kThreads), 0, st, g);
  return check_launch(op);
}

template <int MODE>
int launch_gemm(const GemmArgs& g, hipStream_t st, const char* op) {
  if (g.M <= 32) return launch_cfg<MODE, 128, 32, 4, 1>(g, st, op);
  if (g.M <= 64) return launch_cfg<MODE, 128, 64, 2, 2>(g, st, op);
  return launch_cfg<MODE, 128, 128, 2, 2>(g, st, op);
}

bool is_float_dtype(int dt) { return dt == AYK_F32 || dt == AYK_F16 || dt == AYK_BF16; }

int check_common(const char* op, const void* a, int64_t lda, const void* b, int64_t ldb, int64_t M,
                 int64_t N, int64_t K, const void* bias, int bias_dtype, int out_dtype, int64_t ldo) {
  if (M < 0 || N < 0 || K < 1) return fail(AYK_EINVAL, "%s: bad shape M=%lld N=%lld K=%lld", op, (long long)M, (long long)N, (long long)K);
  if (K % 16 != 0) return fail(AYK_EINVAL, "%s: K=%lld must be a multiple of 16", op, (long long)K);
  if (lda < K || ldb < K || lda % 16 || ldb % 16) return fail(AYK_EINVAL, "%s: row strides must be >= K and multiples of 16", op);
  if (!aligned16(a) || !aligned16(b)) return fail(AYK_EINVAL, "%s: operands must be 16-byte aligned", op);
  if (!is_float_dtype(out_dtype)) return fail(AYK_EINVAL, "%s: out must be float16, bfloat16, or float32", op);
  if (bias && !is_float_dtype(bias_dtype)) return fail(AYK_EINVAL, "%s: bias must be float16, bfloat16, or float32", op);
  if (ldo < N) return fail(AYK_EINVAL, "%s: out row stride must be >= N", op);
  return AYK_OK;
}

}  // namespace
}  // namespace ayk

using namespace ayk;

extern "C" {

int ayk_fp8_scaled_mm(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t M, int64_t N,
                      int64_t K, const void* scale_a, int sa_dtype, int sa_per_row,
                      const void* scale_b, int sb_dtype, int sb_per_col, const void* bias,
                      int bias_dtype, void* out, int out_dtype, int64_t ldo, ayk_stream_t stream) {
  const char* op = "fp8_scaled_mm";
  if (int rc = check_common(op, a, lda, b, ldb, M, N, K, bias, bias_dtype, out_dtype, ldo)) return rc;
  if (!is_float_dtype(sa_dtype) || !is_float_dtype(sb_dtype)) return fail(AYK_EINVAL, "%s: scales must be float32, float16 or bfloat16", op);
  if (M == 0 || N == 0) return AYK_OK;
  if (int rc = check_device()) return rc;
  GemmArgs g{};
  g.a = static_cast<const uint8_t*>(a);
  g.lda = lda;
  g.w = static_cast<const uint8_t*>(b);
  g.ldw = ldb;
  g.M = M; g.N = N; g.K = K;
  g.sa = scale_a; g.sa_dtype = sa_dtype; g.sa_vec = sa_per_row;
  g.sb = scale_b; g.sb_dtype = sb_dtype; g.sb_vec = sb_per_col;
  g.bias = bias; g.bias_dtype = bias_dtype;
  g.out = out; g.out_dtype = out_dtype; g.ldo = ldo;
  return launch_gemm<MODE_SCALED>(g, static_cast<hipStream_t>(stream), op);
}

int ayk_fp8_blockwise_mm(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t M,
                         int64_t N, int64_t K, const void* scale_a, int sa_dtype, int sa_col_major,
                         const void* scale_b, int sb_dtype, const void* bias, int bias_dtype,
                         void* out, int out_dtype, int64_t ldo, ayk_stream_t stream) {
  const char* op = "fp8_blockwise_mm";
  if (int rc = check_common(op, a, lda, b, ldb, M, N, K, bias, bias_dtype, out_dtype, ldo)) return rc;
  if (!is_float_dtype(sa_dtype) || !is_float_dtype(sb_dtype)) return fail(AYK_EINVAL, "%s: scales must be float32, float16 or bfloat16", op);
  if (M == 0 || N == 0) return AYK_OK;
  if (int rc = check_device()) return rc;
  GemmArgs g{};
  g.a = static_cast<const uint8_t*>(a);
  g.lda = lda;
  g.w = static_cast<const uint8_t*>(b);
  g.ldw = ldb;
  g.M = M; g.N = N; g.K = K;
  g.sa = scale_a; g.sa_dtype = sa_dtype; g.sa_vec = sa_col_major;
  g.sb = scale_b; g.sb_dtype = sb_dtype;
  g.bias = bias; g.bias_dtype = bias_dtype;
  g.out = out; g.out_dtype = out_dtype; g.ldo = ldo;
  return launch_gemm<MODE_BLOCK>(g, static_cast<hipStream_t>(stream), op);
}

int ayk_mxfp8_scaled_mm(const void* a, int64_t lda, const uint8_t* a_scale, int64_t ld_as,
                        const void* w, int64_t ldw, const uint8_t* w_scale, int64_t ld_ws,
                        int64_t M, int64_t N, int64_t K, const void* bias, int bias_dtype,
                        void* out, int out_dtype, int64_t ldo, ayk_stream_t stream) {
  const char* op = "mxfp8_scaled_mm";
  if (M < 0 || N < 0 || K < 1 || K % 32) return fail(AYK_EINVAL, "%s: K=%lld must be a positive multiple of the MXFP8 group size 32", op, (long long)K);
  if (ld_as < K / 32 || ld_ws < K / 32) return fail(AYK_EINVAL, "%s: scale row strides must be >= K/32", op);
  if (M == 1) {
    if (!is_float_dtype(out_dtype)) return fail(AYK_EINVAL, "%s: out must be float16, bfloat16, or float32", op);
    if (bias && !is_float_dtype(bias_dtype)) return fail(AYK_EINVAL, "%s: bad bias dtype", op);
    if (N == 0) return AYK_OK;
    if (int rc = check_device()) return rc;
    return mx_gemv(a, a_scale, w, ldw, w_scale, ld_ws, N, K, bias, bias_dtype, out, out_dtype,
                   static_cast<hipStream_t>(stream));
  }
  if (int rc = check_common(op, a, lda, w, ldw, M, N, K, bias, bias_dtype, out_dtype, ldo)) return rc;
  if (M == 0 || N == 0) return AYK_OK;
  if (int rc = check_device()) return rc;
  GemmArgs g{};
  g.a = static_cast<const uint8_t*>(a);
  g.lda = lda;
  g.w = static_cast<const uint8_t*>(w);
  g.ldw = ldw;
  g.M = M; g.N = N; g.K = K;
  g.sa = a_scale; g.ld_sa = ld_as; g.sa_dtype = AYK_U8;
  g.sb = w_scale; g.ld_sb = ld_ws; g.sb_dtype = AYK_U8;
  g.bias = bias; g.bias_dtype = bias_dtype;
  g.out = out; g.out_dtype = out_dtype; g.ldo = ldo;
  return launch_gemm<MODE_MX>(g, static_cast<hipStream_t>(stream), op);
}

}  // extern "C"
