// W8A16 GEMM (M > 1) on gfx950: out[M, N] = x[M, K] . dequant(w[N, K])^T.
//
// Reference: python/ayaka/kernel/triton/gemm/fp8_w8a16_gemm.py:44-120. The weight
// stays e4m3 in HBM (1 byte per element) and is dequantized on the fly:
// w * scale[(n / by) * stride + k / bx] is rounded to the activation dtype (bf16 or
// fp16) -- the reference's numerics -- and fed to v_mfma_f32_32x32x16_{bf16,f16}
// with fp32 accumulation. The output is rounded once to the activation dtype.
//
// As in the W8A8 GEMM, the MFMA "A" operand is a 32-row weight slab and "B" a
// 32-row activation slab, so each lane owns one weight row n per slab and the
// per-row scale lookup happens once per 8-element K chunk. Tiles are staged through
// LDS with double buffering, 64 K elements per step.
#include "ayk_common.h"

namespace ayk {
namespace {

typedef short v8s __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int BKE = 64;                  // K elements per step
constexpr int kWRow = BKE + 16;          // weight LDS row stride (bytes)
constexpr int kXRow = BKE * 2 + 16;      // activation LDS row stride (bytes)

struct W16Args {
  const uint16_t* x;
  int64_t ldx;
  const uint8_t* w;
  int64_t ldw;
  int64_t M, N, K;
  const void* scale;
  int scale_dtype;
  int64_t srs, by, bx;
  int row_scale;  // bx >= K: one scale per weight row
  uint16_t* out;
  int64_t ldo;
  int tiles_m;
};

template <bool BF16>
__device__ inline uint16_t round16(float v) {
  if constexpr (BF16) return f32_to_bf16_bits(v);
  else return f32_to_f16_bits(v);
}

template <bool BF16>
__device__ inline v16f mfma16(const v8s& a, const v8s& b, const v16f& c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0, 0);
  }
}

template <bool BF16, int BN, int BM, int WN, int WM>
__global__ __launch_bounds__(kThreads) void w8a16_gemm_kernel(W16Args g) {
  constexpr int TN = BN / WN, TM = BM / WM;
  constexpr int FN = TN / 32, FM = TM / 32;
  static_assert(FN >= 1 && FM >= 1 && WN * WM == 4, "tile shape");
  constexpr int kWChunks = BN * (BKE / 16);      // 16-byte weight chunks per step
  constexpr int kXChunks = BM * (BKE * 2 / 16);  // 16-byte activation chunks per step
  constexpr int kWCPT = (kWChunks + kThreads - 1) / kThreads;
  constexpr int kXCPT = (kXChunks + kThreads - 1) / kThreads;

  __shared__ __attribute__((aligned(16))) uint8_t wl[2][BN * kWRow];
  __shared__ __attribute__((aligned(16))) uint8_t xl[2][BM * kXRow];

  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int wn = wave / WM, wm = wave % WM;
  const int tm = blockIdx.x % g.tiles_m, tn = blockIdx.x / g.tiles_m;
  const int64_t n_base = (int64_t)tn * BN, m_base = (int64_t)tm * BM;
  const int nk = (int)cdiv(g.K, BKE);

  uint4 ws[kWCPT], xs[kXCPT];
  auto load_stage = [&](int kt) {
#pragma unroll
    for (int i = 0; i < kWCPT; ++i) {
      const int c = tid + i * kThreads;
      if (c < kWChunks) {
        const int row = c / (BKE / 16), col = (c % (BKE / 16)) * 16;
        const int64_t n = n_base + row, k = (int64_t)kt * BKE + col;
        ws[i] = (n < g.N && k < g.K) ? *reinterpret_cast<const uint4*>(g.w + n * g.ldw + k) : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < kXCPT; ++i) {
      const int c = tid + i * kThreads;
      if (c < kXChunks) {
        const int row = c / (BKE / 8), col = (c % (BKE / 8)) * 8;  // col in elements
        const int64_t m = m_base + row, k = (int64_t)kt * BKE + col;
        xs[i] = (m < g.M && k < g.K) ? *reinterpret_cast<const uint4*>(g.x + m * g.ldx + k) : make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < kWCPT; ++i) {
      const int c = tid + i * kThreads;
      if (c < kWChunks) {
        const int row = c / (BKE / 16), col = (c % (BKE / 16)) * 16;
        *reinterpret_cast<uint4*>(&wl[buf][row * kWRow + col]) = ws[i];
      }
    }
#pragma unroll
    for (int i = 0; i < kXCPT; ++i) {
      const int c = tid + i * kThreads;
      if (c < kXChunks) {
        const int row = c / (BKE / 8), col = (c % (BKE / 8)) * 16;  // col in bytes
        *reinterpret_cast<uint4*>(&xl[buf][row * kXRow + col]) = xs[i];
      }
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
  const int frag_k = (lane / 32) * 8;  // element offset within a 16-K step
  // Per-lane weight rows and their scale-row offsets.
  int64_t srow[FN];
  float rscale[FN];
#pragma unroll
  for (int i = 0; i < FN; ++i) {
    int64_t n = n_base + wn * TN + i * 32 + frag_row;
    n = n < g.N ? n : g.N - 1;
    srow[i] = (n / g.by) * g.srs;
    rscale[i] = g.row_scale ? load_f32(g.scale, g.scale_dtype, srow[i]) : 0.0f;
  }
  const uint32_t bx = (uint32_t)g.bx;
  const bool chunk_scale = (g.bx % 8) == 0;

  load_stage(0);
  store_stage(0);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load_stage(kt + 1);
#pragma unroll
    for (int ks = 0; ks < BKE / 16; ++ks) {
      const uint32_t k0 = (uint32_t)(kt * BKE + ks * 16 + frag_k);
      v8s wf[FN], xf[FM];
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        const int row = wn * TN + i * 32 + frag_row;
        const uint2 raw = *reinterpret_cast<const uint2*>(&wl[buf][row * kWRow + ks * 16 + frag_k]);
        float f[8];
        e4m3x4_to_f32(raw.x, f);
        e4m3x4_to_f32(raw.y, f + 4);
        if (g.row_scale) {
#pragma unroll
          for (int e = 0; e < 8; ++e) f[e] *= rscale[i];
        } else if (chunk_scale) {
          const float s = load_f32(g.scale, g.scale_dtype, srow[i] + min(k0, (uint32_t)(g.K - 1)) / bx);
#pragma unroll
          for (int e = 0; e < 8; ++e) f[e] *= s;
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t k = min(k0 + (uint32_t)e, (uint32_t)(g.K - 1));  // padded tail: any valid scale
            f[e] *= load_f32(g.scale, g.scale_dtype, srow[i] + k / bx);
          }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) wf[i][e] = (short)round16<BF16>(f[e]);
      }
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const int row = wm * TM + j * 32 + frag_row;
        const uint4 raw = *reinterpret_cast<const uint4*>(&xl[buf][row * kXRow + (ks * 16 + frag_k) * 2]);
        xf[j] = __builtin_bit_cast(v8s, raw);
      }
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = mfma16<BF16>(wf[i], xf[j], acc[i][j]);
    }
    if (kt + 1 < nk) store_stage(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int64_t m = m_base + wm * TM + j * 32 + frag_row;
    if (m >= g.M) continue;
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
      for (int grp = 0; grp < 4; ++grp) {
        const int64_t n0 = n_base + wn * TN + i * 32 + grp * 8 + (lane / 32) * 4;
        uint16_t* p = g.out + m * g.ldo + n0;
        if (n0 + 3 < g.N && (reinterpret_cast<uintptr_t>(p) & 7) == 0) {
          const uint32_t lo = (uint32_t)round16<BF16>(acc[i][j][grp * 4]) | ((uint32_t)round16<BF16>(acc[i][j][grp * 4 + 1]) << 16);
          const uint32_t hi = (uint32_t)round16<BF16>(acc[i][j][grp * 4 + 2]) | ((uint32_t)round16<BF16>(acc[i][j][grp * 4 + 3]) << 16);
          *reinterpret_cast<uint2*>(p) = make_uint2(lo, hi);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (n0 + q < g.N) p[q] = round16<BF16>(acc[i][j][grp * 4 + q]);
        }
      }
    }
  }
}

template <bool BF16, int BN, int BM, int WN, int WM>
int launch_w16(W16Args g, hipStream_t st) {
  g.tiles_m = (int)cdiv(g.M, BM);
  const int64_t tiles = (int64_t)g.tiles_m * cdiv(g.N, BN);
  if (tiles > 0x7FFFFFFF) return fail(AYK_EINVAL, "fp8_weight_only_gemm: problem too large");
  hipLaunchKernelGGL((w8a16_gemm_kernel<BF16, BN, BM, WN, WM>), dim3((unsigned)tiles), dim3(kThreads), 0, st, g);
  return check_launch("fp8_weight_only_gemm");
}

template <bool BF16>
int dispatch_w16(const W16Args& g, hipStream_t st) {
  if (g.M <= 32) return launch_w16<BF16, 128, 32, 4, 1>(g, st);
  if (g.M <= 64) return launch_w16<BF16, 128, 64, 2, 2>(g, st);
  return launch_w16<BF16, 128, 128, 2, 2>(g, st);
}

}  // namespace
}  // namespace ayk

using namespace ayk;

extern "C" {

int ayk_fp8_weight_only_gemm(const void* x, int x_dtype, int64_t ldx, int64_t M, const void* w,
                             int64_t ldw, int64_t N, int64_t K, const void* scale, int scale_dtype,
                             int64_t scale_row_stride, int64_t block_size_y, int64_t block_size_x,
                             void* out, int64_t ldo, ayk_stream_t stream) {
  const char* op = "fp8_weight_only_gemm";
  if (x_dtype != AYK_BF16 && x_dtype != AYK_F16) return fail(AYK_EINVAL, "%s: input must be float16 or bfloat16", op);
  if (scale_dtype != AYK_U8 && scale_dtype != AYK_F32 && scale_dtype != AYK_BF16) {
    return fail(AYK_EINVAL, "%s: scale dtype must be e8m0 (uint8), float32 or bfloat16", op);
  }
  if (M < 0 || N < 0 || K < 1) return fail(AYK_EINVAL, "%s: bad shape", op);
  // Rows are read in 16-byte vectors up to K rounded up to 16 elements; when K is not
  // a multiple of 16 the caller zero-pads both operands to that width.
  const int64_t k16 = cdiv(K, 16) * 16;
  if (ldw % 16 || ldx % 8 || ldw < k16 || ldx < k16 || ldo < N) {
    return fail(AYK_EINVAL, "%s: row strides must cover K rounded up to 16 (weights: multiple of 16, input: of 8)", op);
  }
  if (!aligned16(x) || !aligned16(w)) return fail(AYK_EINVAL, "%s: operands must be 16-byte aligned", op);
  if (block_size_y < 1 || block_size_x < 1 || scale_row_stride < 1) return fail(AYK_EINVAL, "%s: block sizes must be positive", op);
  if (M == 0 || N == 0) return AYK_OK;
  if (int rc = check_device()) return rc;
  W16Args g{};
  g.x = static_cast<const uint16_t*>(x);
  g.ldx = ldx;
  g.w = static_cast<const uint8_t*>(w);
  g.ldw = ldw;
  g.M = M; g.N = N; g.K = K;
  g.scale = scale; g.scale_dtype = scale_dtype;
  g.srs = scale_row_stride; g.by = block_size_y; g.bx = block_size_x;
  g.row_scale = block_size_x >= K;
  g.out = static_cast<uint16_t*>(out);
  g.ldo = ldo;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return x_dtype == AYK_BF16 ? dispatch_w16<true>(g, st) : dispatch_w16<false>(g, st);
}

}  // extern "C"
