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
#include "gemm_block.h"
#include "gemm_skinny.h"
#include "gemm_tiles.h"
#include "gemm_util.h"

#include <type_traits>

namespace ayk {

int mx_gemv(const void* a, const uint8_t* a_scale, const void* w, int64_t ldw,
            const uint8_t* w_scale, int64_t ld_ws, int64_t N, int64_t K, const void* bias,
            int bias_dtype, void* out, int out_dtype, hipStream_t st);

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int BK = 128;
constexpr int kLdsRow = BK + 16;  // padded LDS row stride in bytes
constexpr int kScaleOne = 127;    // UE8M0 code of 1.0

enum Mode { MODE_SCALED = 0, MODE_BLOCK = 1, MODE_MX = 2, MODE_INT8 = 3 };
// Modes whose epilogue applies per-row / per-tensor output scales.
constexpr bool row_scaled(int mode) { return mode == MODE_SCALED || mode == MODE_INT8; }

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
  float* ws;       // split-K partials (block-scaled GEMM), ws_bytes long
  size_t ws_bytes;
  int64_t kps;     // general kernel, block mode: K per split (0: no split; blockIdx.y = split)
  // 256 x 256 pair kernel, tail split (tail_split > 1): workgroups past dp_tiles take
  // K piece (b - dp_tiles) % tail_split of tile dp_tiles + (b - dp_tiles) / tail_split.
  int dp_tiles;
  int tail_split;
  // 256 x 256 pair kernel: work items (tiles, plus tail pieces); a workgroup runs items
  // blockIdx.x, blockIdx.x + gridDim.x, ...
  int items;
  // 256 x 256 pair kernel, K split of every tile (kps > 0): with kpieces > 0 the grid is
  // one-dimensional and workgroup b takes K piece b % kpieces of tile b / kpieces;
  // 0: grid (tiles, pieces).
  int kpieces;
};

__device__ inline v16f mfma(const v8i& wa, const v8i& ab, const v16f& c, int sw, int sa) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wa, ab, c, 0, 0, 0, sw, 0, sa);
}
// The same with the scale codes taken from byte SEL of the scale registers.
template <int SEL>
__device__ inline v16f mfma_sel(const v8i& wa, const v8i& ab, const v16f& c, int sw, int sa) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wa, ab, c, 0, 0, SEL, sw, SEL, sa);
}
typedef int v16i __attribute__((ext_vector_type(16)));
typedef int v4i __attribute__((ext_vector_type(4)));
// One 64-K step of a 32x32 tile in the mode's arithmetic. INT8: two
// v_mfma_i32_32x32x32_i8 on the fragment's halves (its K order only has to match
// between the operands for a plain dot product); the int32 sums travel in the fp32
// accumulator registers bit for bit and are converted in the epilogue (acc_value).
template <int MODE>
__device__ inline v16f mma(const v8i& wa, const v8i& ab, const v16f& c, int sw, int sa) {
  if constexpr (MODE == MODE_INT8) {
    v16i acc = __builtin_bit_cast(v16i, c);
    acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_shufflevector(wa, wa, 0, 1, 2, 3), __builtin_shufflevector(ab, ab, 0, 1, 2, 3),
                                                acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_shufflevector(wa, wa, 4, 5, 6, 7), __builtin_shufflevector(ab, ab, 4, 5, 6, 7),
                                                acc, 0, 0, 0);
    return __builtin_bit_cast(v16f, acc);
  } else {
    return mfma(wa, ab, c, sw, sa);
  }
}
// Accumulator register value as a float (INT8: the exact int32 sum, converted with
// round to nearest even as torch's int32 -> float32).
template <int MODE>
__device__ inline float acc_value(float r) {
  if constexpr (MODE == MODE_INT8) return (float)__builtin_bit_cast(int, r);
  else return r;
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
__global__ __launch_bounds__(kThreads) void fp8_gemm_kernel(GemmArgs gin) {
  static_assert(WN * WM == kThreads / kWave, "4 wavefronts per workgroup");
  // Block or rowwise mode with a K split: blockIdx.y takes K range [y kps, (y + 1) kps)
  // (kps % 128 == 0) and writes its fp32 partials (rowwise: already scaled) to ws[y]
  // ([M, N]); block_split_reduce sums them, adds the bias and rounds once.
  GemmArgs g = gin;
  if constexpr (MODE == MODE_BLOCK || MODE == MODE_SCALED || MODE == MODE_MX || MODE == MODE_INT8) {
    if (gin.kps > 0) {
      const int64_t k0 = (int64_t)blockIdx.y * gin.kps, kb0 = k0 / 128, kb_total = gin.K / 128;
      g.K = gin.K - k0 < gin.kps ? gin.K - k0 : gin.kps;
      g.a = gin.a + k0;
      g.w = gin.w + k0;
      if constexpr (MODE == MODE_BLOCK) {  // K-blocked scale tables follow the K range
        g.sa = static_cast<const float*>(gin.sa) + (gin.sa_vec ? kb0 * gin.M : kb0);
        g.ld_sa = gin.sa_vec ? 0 : kb_total;
        g.sb = static_cast<const uint8_t*>(gin.sb) + kb0 * (gin.sb_dtype == AYK_F32 ? 4 : (gin.sb_dtype == AYK_U8 ? 1 : 2));
        g.ld_sb = kb_total;
      }
      if constexpr (MODE == MODE_MX) {  // UE8M0 code rows: the range's codes start k0 / 32 in
        g.sa = static_cast<const uint8_t*>(gin.sa) + k0 / 32;
        g.sb = static_cast<const uint8_t*>(gin.sb) + k0 / 32;
      }
      g.bias = nullptr;
      g.out = gin.ws + (int64_t)blockIdx.y * gin.M * gin.N;
      g.out_dtype = AYK_F32;
      g.ldo = gin.N;
    }
  }
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
          else acc[i][j] = mma<MODE>(wf[i], af[j], acc[i][j], wsc[i], asc[j]);
        }
    }

    if constexpr (MODE == MODE_BLOCK) {
      // acc += partial * sa[m, kb] * sb[n / 128, kb]; one sb per 32-row weight slab.
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const int64_t m = m_base + wm * TM + j * 32 + frag_row;
        const int64_t mi = m < g.M ? m : g.M - 1;
        const int64_t sa_ld = g.ld_sa > 0 ? g.ld_sa : kblocks, sb_ld = g.ld_sb > 0 ? g.ld_sb : kblocks;
        const float sa = load_f32(g.sa, g.sa_dtype, g.sa_vec ? (int64_t)kt * g.M + mi : mi * sa_ld + kt);
#pragma unroll
        for (int i = 0; i < FN; ++i) {
          const int64_t n = n_base + wn * TN + i * 32;
          const int64_t nb = (n < g.N ? n : g.N - 1) / 128;
          const float s = sa * load_f32(g.sb, g.sb_dtype, nb * sb_ld + kt);
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
    if constexpr (row_scaled(MODE)) {
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
          float y = acc_value<MODE>(acc[i][j][grp * 4 + q]);
          if constexpr (row_scaled(MODE)) {
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

// ---------------------------------------------------------------------------------
// Large-tile kernel (K % 64 == 0, M and N of at least one tile): a 256 x 256 output
// tile per workgroup, one 128 x 128 wavefront tile (4 x 4 MFMA tiles, 256 accumulator
// registers) on each of the four SIMDs.
//
//  * Operands move HBM/L2 -> LDS with gfx950's direct-to-LDS 16-byte buffer loads: no
//    staging registers, no VALU. One load writes 64 lanes x 16 B = 16 tile rows of one
//    64-byte K stage contiguously; the LDS layout is chosen through which 16-byte chunk
//    each lane fetches (row r holds logical chunk c at c ^ ((r >> 2) & 3)), so the 32
//    rows a fragment read touches fall on distinct bank groups.
//  * A ring of four 32 KB stages (64 K each) in four distinct LDS objects, the K loop
//    unrolled by four: loads run four steps ahead of the MFMAs. Each step waits for
//    the next step's loads and passes one barrier in the middle of its MFMAs, and reads
//    the next step's fragments while its second half executes (fragments are double
//    buffered in registers), so neither the barrier nor the fragment reads leave the
//    matrix cores idle.
//  * Workgroup b runs on XCD b % 8. Tiles are numbered so that each XCD owns a
//    contiguous range of an M-grouped order (8 M tiles per group): the ~32 tiles an
//    XCD runs at once share 8 activation and 4 weight panels through its L2; their K
//    walks start a few stages apart.
//  * Every wait on the vector-memory counter is written out with its exact count
//    (it retires in issue order); buffer windows end at the operand's last row, so
//    rows past M / N read zero and are never stored.
constexpr int kBigTile = 256;
constexpr int kBigK = 64;                         // K bytes per stage
constexpr int kBigStage = 2 * kBigTile * kBigK;   // weights + activations of one stage, bytes
constexpr int kEpilogueLds = 64 * 1024;           // epilogue staging tile (first stage object)


// Four consecutive bias values n .. n+3 (n + 3 < N, n % 4 == 0) as floats.
__device__ inline void load_bias4(const GemmArgs& g, int64_t n, float* b) {
  if (g.bias_dtype == AYK_F32) {
    const float4 v = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(g.bias) + n);
    b[0] = v.x; b[1] = v.y; b[2] = v.z; b[3] = v.w;
  } else {
    const uint2 v = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(g.bias) + n);
    const uint32_t w[2] = {v.x, v.y};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t bits = (uint16_t)(w[i / 2] >> (16 * (i % 2)));
      b[i] = g.bias_dtype == AYK_BF16 ? bf16_bits_to_f32(bits) : f16_bits_to_f32(bits);
    }
  }
}

template <int OUT>
__device__ inline void store4_typed(const GemmArgs& g, int64_t m, int64_t n, const float* v) {
  if (OUT == AYK_F32) {
    *reinterpret_cast<float4*>(reinterpret_cast<float*>(g.out) + m * g.ldo + n) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    uint16_t b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) b[i] = OUT == AYK_BF16 ? f32_to_bf16_bits(v[i]) : f32_to_f16_bits(v[i]);
    *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(g.out) + m * g.ldo + n) =
        make_uint2((uint32_t)b[0] | ((uint32_t)b[1] << 16), (uint32_t)b[2] | ((uint32_t)b[3] << 16));
  }
}

// Epilogue of the large-tile kernel, staged through LDS (free once the K loop ends).
// A lane's accumulators hold 4 consecutive n of one row m per store group, spread over
// 32 rows per instruction; writing them straight to HBM costs one cache line per lane
// pair. Instead, for each of the four 32-row MFMA slabs j, every wavefront scales,
// biases and converts its values and writes them to a [64 m][256 n] LDS staging tile
// (the two row halves come from wm = 0 / 1); then all 256 threads store that tile row by
// row with 16-byte coalesced stores. Rows past M and columns past N are not stored
// (N % 4 == 0 and a 4-aligned row stride are checked by the launcher).
template <int OUT>
struct OutBytes { static constexpr int v = OUT == AYK_F32 ? 4 : 2; };


// Output scales of one lane of the 256 x 256 kernels: the activation scale of each of
// its four m-fragment rows and the weight scales of its 64 output columns. They are
// loaded before the K loop (and before its first direct load, so the loop's exact
// vector-memory waits are unaffected) and stay in registers until the epilogue: loaded
// at the epilogue, their latency stalled every tile while the whole chip was storing.
struct BigScales {
  float sa[4];
  float sb[4][4][4];  // [n-fragment i][column group][column]
};
template <int MODE>
__device__ __attribute__((always_inline)) inline BigScales load_big_scales(const GemmArgs& g, int64_t m_tile, int64_t n_tile) {
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));  // not hoisted out of the persistent kernel's item loop
  const int lane = tid & 63, wave = tid >> 6;
  const int wn = wave >> 1, wm = wave & 1, h = lane >> 5, frow = lane & 31;
  BigScales sc;
#pragma unroll
  for (int j = 0; j < 4; ++j) sc.sa[j] = 1.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int grp = 0; grp < 4; ++grp)
#pragma unroll
      for (int q = 0; q < 4; ++q) sc.sb[i][grp][q] = 1.0f;
  if constexpr (row_scaled(MODE)) {
    const float* sa_p = reinterpret_cast<const float*>(g.sa);
    const float* sb_p = reinterpret_cast<const float*>(g.sb);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t m = m_tile + wm * 128 + j * 32 + frow;
      sc.sa[j] = sa_p[g.sa_vec ? (m < g.M ? m : 0) : 0];
    }
    if (g.sb_vec) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int grp = 0; grp < 4; ++grp) {
          const int64_t n = n_tile + wn * 128 + i * 32 + grp * 8 + h * 4;
          const float4 t = *reinterpret_cast<const float4*>(sb_p + (n < g.N ? n : 0));
          sc.sb[i][grp][0] = t.x; sc.sb[i][grp][1] = t.y; sc.sb[i][grp][2] = t.z; sc.sb[i][grp][3] = t.w;
        }
    } else {
      const float t = sb_p[0];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int grp = 0; grp < 4; ++grp)
#pragma unroll
          for (int q = 0; q < 4; ++q) sc.sb[i][grp][q] = t;
    }
  }
  return sc;
}


// `nt`: final outputs are stored nontemporally, so that they do not take the L2 that
// holds the next tiles' operand panels (Qwen2 gate_up at M = 4096: 625 -> 585 us); fp32
// partials that a reduce reads back keep plain stores.
template <int MODE, int OUT, bool BIAS>
__device__ __attribute__((always_inline)) inline void big_epilogue_impl(const GemmArgs& g, const v16f (&acc)[4][4], const BigScales& sc,
                                         int64_t m_tile, int64_t n_tile, uint8_t* stage_lds, bool nt) {
  constexpr int EB = OutBytes<OUT>::v;
  constexpr int kRowBytes = 256 * EB + 16;        // padded staging row
  constexpr int kStageRows = EB == 4 ? 32 : 64;   // rows staged at once (fits 64 KB)
  constexpr int kPasses = 64 / kStageRows;        // fp32: one pass per row half (wm)
  static_assert(kStageRows * kRowBytes <= kEpilogueLds, "staging tile must fit the first stage object");
  // Lane addresses come from an opaque copy of the thread index: in the persistent pair
  // kernel this code runs inside the item loop, and addresses hoisted out of it would
  // stay live (and spill) through every K loop.
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63, wave = tid >> 6;
  const int wn = wave >> 1, wm = wave & 1, h = lane >> 5, frow = lane & 31;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) {
      if (kPasses == 1 || wm == pass) {
        uint8_t* srow = stage_lds + ((kPasses == 1 ? wm * 32 : 0) + frow) * kRowBytes;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int grp = 0; grp < 4; ++grp) {
            const int nl = wn * 128 + i * 32 + grp * 8 + h * 4;  // column within the tile
            float bias[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if constexpr (BIAS) {
              if (n_tile + nl < g.N) load_bias4(g, n_tile + nl, bias);
            }
            float v[4];
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) {
              float y = acc_value<MODE>(acc[i][j][grp * 4 + qq]);
              if constexpr (row_scaled(MODE)) y = (y * sc.sa[j]) * sc.sb[i][grp][qq];
              v[qq] = BIAS ? y + bias[qq] : y;
            }
            if constexpr (OUT == AYK_F32) {
              *reinterpret_cast<float4*>(srow + nl * 4) = make_float4(v[0], v[1], v[2], v[3]);
            } else if constexpr (OUT == AYK_BF16) {
              *reinterpret_cast<uint2*>(srow + nl * 2) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
            } else {
              uint16_t b[4];
#pragma unroll
              for (int qq = 0; qq < 4; ++qq) b[qq] = f32_to_f16_bits(v[qq]);
              *reinterpret_cast<uint2*>(srow + nl * 2) =
                  make_uint2((uint32_t)b[0] | ((uint32_t)b[1] << 16), (uint32_t)b[2] | ((uint32_t)b[3] << 16));
            }
          }
        }
      }
      // The staging writes are visible (LDS only: the global stores of the previous pass
      // need not have completed, they read registers).
      lds_barrier();
      // Staged row r: with one pass, r < 32 is tile row j*32 + r (wm = 0) and r >= 32
      // is 128 + j*32 + (r - 32) (wm = 1); with two passes, pass*128 + j*32 + r.
      constexpr int kChunksPerRow = 256 * EB / 16;
      constexpr int kRowsPerStep = 256 / kChunksPerRow;
#pragma unroll
      for (int r0 = 0; r0 < kStageRows; r0 += kRowsPerStep) {
        const int r = r0 + tid / kChunksPerRow;
        const int c = tid % kChunksPerRow;
        const int tile_row = kPasses == 1 ? (r < 32 ? j * 32 + r : 128 + j * 32 + (r - 32)) : pass * 128 + j * 32 + r;
        const int64_t gm = m_tile + tile_row;
        const int64_t gn = n_tile + (int64_t)c * (16 / EB);
        if (gm < g.M && gn < g.N) {
          const uint4 val = *reinterpret_cast<const uint4*>(stage_lds + r * kRowBytes + c * 16);
          uint8_t* dst = reinterpret_cast<uint8_t*>(g.out) + (gm * g.ldo + gn) * EB;
          if (gn + 16 / EB <= g.N) {
            if (nt) __builtin_nontemporal_store(v4i{(int)val.x, (int)val.y, (int)val.z, (int)val.w}, reinterpret_cast<v4i*>(dst));
            else *reinterpret_cast<uint4*>(dst) = val;
          } else {  // N % 4 == 0: the first 8 bytes of the chunk are in range
            *reinterpret_cast<uint2*>(dst) = make_uint2(val.x, val.y);
          }
        }
      }
      // Every lane has read its chunks of the staging tile before it is rewritten.
      lds_barrier();
    }
  }
}

template <int MODE>
__device__ __attribute__((always_inline)) inline void big_epilogue(const GemmArgs& g, const v16f (&acc)[4][4], const BigScales& sc, int64_t m_tile,
                                    int64_t n_tile, uint8_t* stage_lds, bool nt = false) {
  if (g.bias) {
    if (g.out_dtype == AYK_BF16) big_epilogue_impl<MODE, AYK_BF16, true>(g, acc, sc, m_tile, n_tile, stage_lds, nt);
    else if (g.out_dtype == AYK_F16) big_epilogue_impl<MODE, AYK_F16, true>(g, acc, sc, m_tile, n_tile, stage_lds, nt);
    else big_epilogue_impl<MODE, AYK_F32, true>(g, acc, sc, m_tile, n_tile, stage_lds, nt);
  } else {
    if (g.out_dtype == AYK_BF16) big_epilogue_impl<MODE, AYK_BF16, false>(g, acc, sc, m_tile, n_tile, stage_lds, nt);
    else if (g.out_dtype == AYK_F16) big_epilogue_impl<MODE, AYK_F16, false>(g, acc, sc, m_tile, n_tile, stage_lds, nt);
    else big_epilogue_impl<MODE, AYK_F32, false>(g, acc, sc, m_tile, n_tile, stage_lds, nt);
  }
}

template <int MODE>
__global__ __launch_bounds__(kThreads, 1) void fp8_gemm_big_kernel(GemmArgs g) {
  static_assert(row_scaled(MODE), "per-row / per-tensor scales only");
  constexpr int FN = 4, FM = 4;                        // 32x32 MFMA tiles per wavefront (n, m)
  constexpr int kDma = kBigStage / 1024 / 4;           // direct loads per wavefront per stage (8)
  constexpr int kOps = kDma;                           // vector-memory ops per wavefront per stage
  // Four stage buffers in four distinct LDS objects, so the compiler can tell that
  // fragment reads of one stage never alias the in-flight direct loads of another. The
  // first is twice as large: after the K loop it holds the epilogue's staging tile.
  __shared__ __attribute__((aligned(1024))) uint8_t L0[kEpilogueLds];
  __shared__ __attribute__((aligned(1024))) uint8_t L1[kBigStage];
  __shared__ __attribute__((aligned(1024))) uint8_t L2[kBigStage];
  __shared__ __attribute__((aligned(1024))) uint8_t L3[kBigStage];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave_u = __builtin_amdgcn_readfirstlane(tid >> 6);  // keep descriptors in SGPRs
  const int wn = wave_u >> 1, wm = wave_u & 1;
  const int h = lane >> 5, frow = lane & 31;
  int tm, tn;
  big_tile_coords(blockIdx.x, g.tiles_m, (int)cdiv(g.N, kBigTile), tm, tn);
  const int64_t n_base = (int64_t)tn * kBigTile, m_base = (int64_t)tm * kBigTile;
  const int nk = (int)(g.K / kBigK);           // real stages
  const int nsteps = (nk + 3) & ~3;            // padded to the unroll (padding computes zeros)
  // K stagger: the tile starts its K walk at stage 2 (tm mod 8) + (tn mod 2) (mod nk).
  // The 32 tiles an XCD runs together are then a few stages apart: their requests no
  // longer arrive in lockstep, while the panel slices they share are still in the L2
  // when the later tiles reach them. Measured against no stagger and against larger
  // offsets on the config shapes: +5-15%. The accumulation order changes, not the
  // result's tolerance.
  const int stag = __builtin_amdgcn_readfirstlane((int)((unsigned)((tm & 7) * 2 + (tn & 1)) % (unsigned)nk));

  // Direct loads: wavefronts 0-1 fetch the 256 weight rows, 2-3 the 256 activation rows
  // (128 each), 64 K bytes per stage. Load jj of a wavefront fills LDS rows
  // 128 (w & 1) + 16 jj + L/4 (lane L) of its operand; lane L fetches logical chunk
  // (L & 3) ^ ((L >> 4) & 3) and the hardware writes it at physical chunk L & 3, so
  // row r holds logical chunk c at c ^ ((r >> 2) & 3). The buffer window of a wavefront
  // ends at the operand's last row: rows past M / N read zero (never stored).
  const bool w_wave = wave_u < 2;
  const int64_t ld = w_wave ? g.ldw : g.lda;
  const int ld_u = __builtin_amdgcn_readfirstlane((int)ld);
  const OperandWindow win = operand_window((w_wave ? n_base : m_base) + (wave_u & 1) * 128, w_wave ? g.N : g.M, ld);
  const __amdgpu_buffer_rsrc_t op_rsrc = uniform_rsrc((w_wave ? g.w : g.a) + win.base_offset, win.records);
  const int voff = (lane >> 2) * ld_u + (((lane & 3) ^ ((lane >> 4) & 3)) << 4);
  // Issue step s (< nsteps) into stage buffer `dst`. A padded step (s >= nk) reads at an
  // offset past every buffer window, which returns zeros: its fragments are zero and it
  // adds nothing.
  auto issue = [&](int s, uint8_t* dst) {
    int ks = (s < nk ? s : nk - 1) + stag;
    ks = __builtin_amdgcn_readfirstlane(ks >= nk ? ks - nk : ks);
    const int pad_off = __builtin_amdgcn_readfirstlane(s < nk ? 0 : 0x40000000);
#pragma unroll
    for (int jj = 0; jj < kDma; ++jj) {
      const int soff = __builtin_amdgcn_readfirstlane(jj * 16 * ld_u + ks * kBigK + pad_off);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(op_rsrc, (__attribute__((address_space(3))) void*)(dst + (wave_u * kDma + jj) * 1024),
                                               16, voff, soff, 0, 0);
    }
  };

  // Fragment reads: row r = tile_row0 + frow, whose swizzle (r >> 2) & 3 equals
  // (frow >> 2) & 3 for every fragment, so two per-lane offsets address all of them.
  const int fsw = (frow >> 2) & 3;
  const int c0 = (h ^ fsw) << 4, c1 = ((2 + h) ^ fsw) << 4;
  auto frag = [&](const uint8_t* buf, int tile_row0) -> v8i {
    const uint8_t* base = buf + (tile_row0 + frow) * kBigK;
    const uint4 lo = *reinterpret_cast<const uint4*>(base + c0);
    const uint4 hi = *reinterpret_cast<const uint4*>(base + c1);
    v8i r;
    r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
    r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
    return r;
  };
  v8i wf[2][FN], af[2][FM];  // fragments of the current and the next step
  auto read_frags = [&](int set, const uint8_t* buf) {
#pragma unroll
    for (int i = 0; i < FN; ++i) wf[set][i] = frag(buf, wn * 128 + i * 32);
#pragma unroll
    for (int j = 0; j < FM; ++j) af[set][j] = frag(buf + kBigTile * kBigK, wm * 128 + j * 32);
  };

  // Declaring an AGPR clobber makes the compiler select the AGPR form of the MFMAs,
  // so the 256 accumulators live in the accumulation registers and the 256
  // architectural VGPRs stay free for fragments and addresses.
  asm volatile("" ::: "a255");
  v16f acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  auto mfmas = [&](int set, int j0, int j1) {
#pragma unroll
    for (int j = j0; j < j1; ++j)
#pragma unroll
      for (int i = 0; i < FN; ++i) acc[i][j] = mma<MODE>(wf[set][i], af[set][j], acc[i][j], kScaleOne, kScaleOne);
  };

  constexpr int kHead = 1;  // m-fragments multiplied before the step's barrier
  // The output scales are loaded first: older than every direct load, they never
  // count against the loop's vector-memory waits.
  const BigScales scales = load_big_scales<MODE>(g, m_base, n_base);
  // Prologue: steps 0-3 in flight, step 0 visible, its fragments in set 0.
  issue(0, L0);
  issue(1, L1);
  issue(2, L2);
  issue(3, L3);
  wait_vmcnt<3 * kOps>();
  lds_barrier();
  read_frags(0, L0);

  // Step s: the MFMAs of its first m-fragment; then "step s + 1 has landed" (the
  // wavefront's own loads: steps s + 2 and s + 3 may still be in flight) and a barrier,
  // which also certifies that every wavefront has its step-s fragments in registers, so
  // step s's buffer is refilled with step s + 4; then step s + 1's fragments are read
  // while the remaining three quarters of step s's MFMAs run (a longer window than an
  // even split: +4%). Everything a wait depends on is issued in a
  // fixed order, so the counts are exact; the body has no branches.
  auto step = [&](int s, int set, uint8_t* cur, uint8_t* nxt) {
    mfmas(set, 0, kHead);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<2 * kOps>();
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue(s + 4 < nsteps ? s + 4 : nsteps - 1, cur);
    read_frags(set ^ 1, nxt);
    mfmas(set, kHead, FM);
  };
  for (int s = 0; s < nsteps; s += 4) {
    step(s, 0, L0, L1);
    step(s + 1, 1, L1, L2);
    step(s + 2, 0, L2, L3);
    step(s + 3, 1, L3, L0);
  }
  // Every issued load has landed and no wavefront still reads a stage buffer.
  wait_vmcnt<0>();
  lds_barrier();
  big_epilogue<MODE>(g, acc, scales, m_base, n_base, L0);
}

// The 256 x 256 kernel with 128-byte row loads (K % 128 == 0): a load instruction
// covers 8 rows x 128 K bytes (two 64-K steps) instead of 16 rows x 64 bytes, which
// halves the L2 requests per byte (an L2-resident probe reads 57 B/cycle per compute
// unit with the wide shape against 29 with the narrow one). Stage buffers therefore
// hold a pair of steps: two 64 KB pair buffers, the second pair's loads in flight while
// the first is multiplied. The fragment layout, the MFMA order and the epilogue are the
// narrow kernel's; the step schedule (one barrier per pair) is its own.
//
// Persistent: a workgroup runs work items blockIdx.x, blockIdx.x + gridDim.x, ... (the
// launch has at most one workgroup per CU, so item i runs on XCD i mod 8 as the tile
// order assumes). One item is a whole tile, or one K piece of a tile (the K split of a
// launch short of one round, blockIdx.y; the tail split of the last round). Across
// items the pair stream does not drain: the next item's first pair is loaded during
// the current item's last pair, and lands while the current item's epilogue runs
// (staged through the pair buffer its last pair left free); the next item's second
// pair is issued when the epilogue is done. Every item's MFMAs, loads and waits are
// those of the single-tile kernel, so a tile's result is the same bit for bit.

// Output scales and bias of one item of the persistent pair kernel, as loaded ahead of
// its epilogue: each thread fetches one column's weight scale and bias (column
// n_tile + tid) and the activation scales of its lane's four rows; the epilogue writes
// the columns' values into an LDS table that every lane reads (a lane's 64 columns in
// registers through the epilogue, 128 values with the bias, had made the kernel spill).
struct PairScales {
  float sa[4];  // activation scale of the lane's row in m-fragment j
  float sb;     // weight scale of column n_tile + tid (1 without row scales)
  float bias;   // bias of column n_tile + tid (0 without a bias)
};
template <int MODE>
__device__ __attribute__((always_inline)) inline PairScales load_pair_scales(const GemmArgs& g, int64_t m_tile, int64_t n_tile) {
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));  // not hoisted out of the item loop
  const int lane = tid & 63, wm = (tid >> 6) & 1, frow = lane & 31;
  PairScales ps;
  ps.sb = 1.0f;
  ps.bias = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) ps.sa[j] = 1.0f;
  const int64_t n = n_tile + tid;
  const int64_t nc = n < g.N ? n : g.N - 1;  // a column past N loads column N - 1 (never stored)
  if constexpr (row_scaled(MODE)) {
    const float* sa_p = reinterpret_cast<const float*>(g.sa);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t m = m_tile + wm * 128 + j * 32 + frow;
      ps.sa[j] = sa_p[g.sa_vec ? (m < g.M ? m : 0) : 0];
    }
    ps.sb = reinterpret_cast<const float*>(g.sb)[g.sb_vec ? nc : 0];
  }
  if (g.bias != nullptr) ps.bias = load_f32(g.bias, g.bias_dtype, nc);
  return ps;
}

// Epilogue of the persistent pair kernel: as big_epilogue_impl (scaled, biased and
// converted values staged through LDS, 16-byte coalesced stores), with the columns'
// scales and bias read from an LDS table, each pass's staged chunks read into
// registers before any of them is stored (so that the LDS reads pipeline), and
// nontemporal stores for final outputs (NT; fp32 partials that a reduce reads back keep
// plain stores). The staging tile and the table share the pair buffer `stage_lds`.
// An accumulator element read out of its AGPR where the epilogue uses it. The read is
// an opaque instruction, so the compiler neither copies the 256 accumulators into VGPRs
// ahead of the epilogue (they do not fit beside the rest; their spills made every pass
// wait for the previous passes' stores) nor moves them between AGPRs.
template <int MODE>
__device__ inline float acc_read(float a) {
  float v;
  asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
  return acc_value<MODE>(v);
}

// Cache policy of a nontemporal buffer store (the NT bit of gfx940+ stores).
constexpr int kNtPolicy = 2;

template <int MODE, int OUT, bool BIAS, bool NT>
__device__ __attribute__((always_inline)) inline void pair_epilogue_impl(const GemmArgs& g, v16f (&acc)[4][4], const PairScales& ps,
                                                                         int64_t m_tile, int64_t n_tile, uint8_t* stage_lds,
                                                                         float* table) {
  constexpr int EB = OutBytes<OUT>::v;
  constexpr int kRowBytes = 256 * EB + 16;        // padded staging row
  constexpr int kStageRows = EB == 4 ? 32 : 64;   // rows staged at once
  constexpr int kPasses = 64 / kStageRows;        // fp32: one pass per row half (wm)
  static_assert(kStageRows * kRowBytes <= kEpilogueLds, "staging tile must fit a pair buffer");
  constexpr bool kScaled = row_scaled(MODE);
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));  // lane addresses are not hoisted out of the item loop
  const int lane = tid & 63, wave = tid >> 6;
  const int wn = wave >> 1, wm = wave & 1, h = lane >> 5, frow = lane & 31;
  // The accumulator reads below are opaque to the compiler's hazard tracking: wait out
  // the longest MFMA-result-to-VALU-read latency (19 wait states for a 16-pass MFMA)
  // behind the kernel's last MFMA explicitly.
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  float* sb_t = table;  // its own LDS object: its reads need not wait for staging writes
  float* bias_t = table + 256;
  // The output tile as a buffer: base at (m_tile, n_tile), records up to the end of the
  // last row inside M (the launcher keeps 256 rows x ldo within 2 GB), and the columns
  // inside N.
  const int ldo_b = (int)(g.ldo * EB);
  const int64_t rows_left = g.M - m_tile < 256 ? g.M - m_tile : 256;
  const int cols_left = (int)(g.N - n_tile < 256 ? g.N - n_tile : 256);
  const bool cols_whole = cols_left == 256;
  const __amdgpu_buffer_rsrc_t out_rsrc =
      uniform_rsrc(reinterpret_cast<uint8_t*>(g.out) + (m_tile * g.ldo + n_tile) * EB, (int32_t)((rows_left - 1) * ldo_b + cols_left * EB));
  if constexpr (kScaled || BIAS) {
    if constexpr (kScaled) sb_t[tid] = ps.sb;
    if constexpr (BIAS) bias_t[tid] = ps.bias;
    lds_barrier();
  }
  constexpr int kChunksPerRow = 256 * EB / 16;
  constexpr int kRowsPerStep = 256 / kChunksPerRow;
  constexpr int kSteps = kStageRows / kRowsPerStep;
  const int c = tid % kChunksPerRow, r_base = tid / kChunksPerRow;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) {
      if (kPasses == 1 || wm == pass) {
        uint8_t* srow = stage_lds + ((kPasses == 1 ? wm * 32 : 0) + frow) * kRowBytes;
        // Column group q = 4 i + grp; its table values are read one group ahead, so that
        // their latency hides behind the previous group's arithmetic.
        auto col = [&](int q) { return wn * 128 + (q >> 2) * 32 + (q & 3) * 8 + h * 4; };
        float4 s4n = make_float4(1.0f, 1.0f, 1.0f, 1.0f), b4n = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if constexpr (kScaled) s4n = *reinterpret_cast<const float4*>(sb_t + col(0));
        if constexpr (BIAS) b4n = *reinterpret_cast<const float4*>(bias_t + col(0));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int grp = 0; grp < 4; ++grp) {
            const int q = i * 4 + grp;
            const int nl = col(q);  // column within the tile
            const float4 s4 = s4n, b4 = b4n;
            if (q + 1 < 16) {
              if constexpr (kScaled) s4n = *reinterpret_cast<const float4*>(sb_t + col(q + 1));
              if constexpr (BIAS) b4n = *reinterpret_cast<const float4*>(bias_t + col(q + 1));
            }
            const float sbv[4] = {s4.x, s4.y, s4.z, s4.w}, bv[4] = {b4.x, b4.y, b4.z, b4.w};
            float v[4];
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) {
              float y = acc_read<MODE>(acc[i][j][grp * 4 + qq]);
              if constexpr (kScaled) y = (y * ps.sa[j]) * sbv[qq];
              v[qq] = BIAS ? y + bv[qq] : y;
            }
            if constexpr (OUT == AYK_F32) {
              *reinterpret_cast<float4*>(srow + nl * 4) = make_float4(v[0], v[1], v[2], v[3]);
            } else if constexpr (OUT == AYK_BF16) {
              *reinterpret_cast<uint2*>(srow + nl * 2) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
            } else {
              // The fp32 value is rounded to fp16 on its own (torch's cast of the fp32
              // result): left free, the compiler fuses the last multiply into the
              // conversion (v_fma_mixlo_f16, one rounding), which differs at fp16 ties.
              uint16_t b[4];
#pragma unroll
              for (int qq = 0; qq < 4; ++qq) {
                asm volatile("" : "+v"(v[qq]));
                b[qq] = f32_to_f16_bits(v[qq]);
              }
              *reinterpret_cast<uint2*>(srow + nl * 2) =
                  make_uint2((uint32_t)b[0] | ((uint32_t)b[1] << 16), (uint32_t)b[2] | ((uint32_t)b[3] << 16));
            }
          }
        }
      }
      lds_barrier();  // the staging writes are visible
      // Staged row r: with one pass, r < 32 is tile row j*32 + r (wm = 0) and r >= 32
      // is 128 + j*32 + (r - 32) (wm = 1); with two passes, pass*128 + j*32 + r.
      v4i val[kSteps];
#pragma unroll
      for (int t = 0; t < kSteps; ++t)
        val[t] = *reinterpret_cast<const v4i*>(stage_lds + (t * kRowsPerStep + r_base) * kRowBytes + c * 16);
      // Stored through a buffer resource over the tile's rows: a row past M lies past
      // num_records and is dropped, offsets are 32-bit, and only the last column tile
      // checks columns. Staged row r (thread row r_base + t kRowsPerStep) is tile row
      // j*32 + r, or 128 + j*32 + (r - 32) past 32 (one pass); pass*128 + j*32 + r (two).
#pragma unroll
      for (int t = 0; t < kSteps; ++t) {
        const int r = t * kRowsPerStep + r_base;
        const int tile_row = kPasses == 1 ? (r < 32 ? j * 32 + r : 128 + j * 32 + (r - 32)) : pass * 128 + j * 32 + r;
        const int voff = tile_row * ldo_b + c * 16;
        if (cols_whole || c * (16 / EB) + 16 / EB <= cols_left) {
          __builtin_amdgcn_raw_buffer_store_b128(val[t], out_rsrc, voff, 0, NT ? kNtPolicy : 0);
        } else if (c * (16 / EB) < cols_left) {  // N % 4 == 0: the chunk's first 8 bytes
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_shufflevector(val[t], val[t], 0, 1), out_rsrc, voff, 0, 0);
        }
      }
      // Every lane has read its chunks of the staging tile before it is rewritten.
      lds_barrier();
    }
  }
}

// The pair kernel's epilogue for one item: fp32 partials (no bias, plain stores) or
// the final output in its dtype (nontemporal stores).
template <int MODE>
__device__ __attribute__((always_inline)) inline void pair_epilogue(const GemmArgs& g, bool partial, v16f (&acc)[4][4],
                                                                    const PairScales& ps, int64_t m_tile, int64_t n_tile,
                                                                    uint8_t* stage_lds, float* table) {
  if (partial) {
    pair_epilogue_impl<MODE, AYK_F32, false, false>(g, acc, ps, m_tile, n_tile, stage_lds, table);
  } else if (g.bias) {
    if (g.out_dtype == AYK_BF16) pair_epilogue_impl<MODE, AYK_BF16, true, true>(g, acc, ps, m_tile, n_tile, stage_lds, table);
    else if (g.out_dtype == AYK_F16) pair_epilogue_impl<MODE, AYK_F16, true, true>(g, acc, ps, m_tile, n_tile, stage_lds, table);
    else pair_epilogue_impl<MODE, AYK_F32, true, true>(g, acc, ps, m_tile, n_tile, stage_lds, table);
  } else {
    if (g.out_dtype == AYK_BF16) pair_epilogue_impl<MODE, AYK_BF16, false, true>(g, acc, ps, m_tile, n_tile, stage_lds, table);
    else if (g.out_dtype == AYK_F16) pair_epilogue_impl<MODE, AYK_F16, false, true>(g, acc, ps, m_tile, n_tile, stage_lds, table);
    else pair_epilogue_impl<MODE, AYK_F32, false, true>(g, acc, ps, m_tile, n_tile, stage_lds, table);
  }
}

// One work item of the pair kernel: the tile, its K range and where its result goes.
struct PairItem {
  GemmArgs g;      // operand bases and K of the item's range; out / ldo / bias of its result
  int tm, tn;
  bool partial;    // an fp32 partial (K split or tail piece): plain stores, kept in L2
};

template <int MODE>
__device__ __attribute__((always_inline)) inline PairItem pair_item(const GemmArgs& gin, int item, int piece) {
  //  * a K split of every tile (gin.kps > 0, launches short of one round): piece =
  //    blockIdx.y's K range, scaled fp32 partials to ws[piece] ([M, N]);
  //  * a tail split (gin.tail_split > 1): the last, mostly empty round of tiles is
  //    split over K across the CUs that round would leave idle; item b >= dp_tiles
  //    takes piece (b - dp_tiles) % tail_split of tile dp_tiles + (b - dp_tiles) /
  //    tail_split, a 256 x 256 scaled fp32 partial in the compact workspace
  //    [tail_split][tail tiles][256][256];
  //  * otherwise tile `item` over all of K.
  PairItem it;
  it.g = gin;
  it.partial = false;
  int tile_id = item;
  int64_t kps = gin.kps;
  bool tail = false;
  if (gin.tail_split > 1 && item >= gin.dp_tiles) {
    const int u = item - gin.dp_tiles;
    tile_id = gin.dp_tiles + u / gin.tail_split;
    piece = u % gin.tail_split;
    kps = gin.K / gin.tail_split;  // whole pairs (MX: whole 512-K chunks), by the plan
    tail = true;
  }
  big_tile_coords(tile_id, gin.tiles_m, (int)cdiv(gin.N, kBigTile), it.tm, it.tn);
  if (kps > 0) {
    GemmArgs& g = it.g;
    const int64_t k0 = (int64_t)piece * kps;  // MX: kps % 512 == 0 keeps the code rows 16-byte aligned
    g.K = gin.K - k0 < kps ? gin.K - k0 : kps;
    g.a = gin.a + k0;
    g.w = gin.w + k0;
    if constexpr (MODE == MODE_MX) {
      g.sa = static_cast<const uint8_t*>(gin.sa) + k0 / 32;
      g.sb = static_cast<const uint8_t*>(gin.sb) + k0 / 32;
    }
    g.bias = nullptr;
    g.out_dtype = AYK_F32;
    it.partial = true;
    if (tail) {
      // The epilogue addresses out + (m * ldo + n) with the tile's global (m, n): the
      // base is moved back by the tile origin so that the tile lands at its slot.
      const int tail_tiles = (int)(cdiv(gin.M, kBigTile) * cdiv(gin.N, kBigTile)) - gin.dp_tiles;
      const int64_t slot = (int64_t)piece * tail_tiles + (tile_id - gin.dp_tiles);
      g.out = gin.ws + slot * kBigTile * kBigTile - ((int64_t)it.tm * kBigTile * kBigTile + (int64_t)it.tn * kBigTile);
      g.ldo = kBigTile;
    } else {
      g.out = gin.ws + (int64_t)piece * gin.M * gin.N;
      g.ldo = gin.N;
    }
  }
  return it;
}

// What the loads of one work item need: its operand and code windows (this wavefront's
// rows), its pair count and its K stagger.
struct PairSrc {
  __amdgpu_buffer_rsrc_t op, code;
  int np, npairs, stag;
};

template <int MODE>
__global__ __launch_bounds__(kThreads, 1) void fp8_gemm_pair_kernel(GemmArgs gin) {
  static_assert(row_scaled(MODE) || MODE == MODE_MX, "per-row / per-tensor scales or MX codes");
  constexpr int FN = 4, FM = 4;        // 32x32 MFMA tiles per wavefront (n, m)
  constexpr int kPairK = 2 * kBigK;    // 128 K bytes per pair
  constexpr int kPairBytes = 2 * kBigTile * kPairK;  // 64 KB
  constexpr int kDma = kPairBytes / 1024 / 4;        // direct loads per wavefront per pair (16)
  // Two pair buffers in two distinct LDS objects (the compiler tells that reads of one
  // never alias the in-flight direct loads into the other).
  __shared__ __attribute__((aligned(1024))) uint8_t P0[kPairBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t P1[kPairBytes];
  static_assert(kPairBytes == kEpilogueLds, "a pair buffer holds the epilogue's staging tile");
  // MXFP8: the UE8M0 codes of the tile's 512 rows for a chunk of four pairs (16 bytes a
  // row), in two 8 KB halves. Chunks alternate halves along the workgroup's whole pair
  // stream (across items too), so a chunk is never loaded into the half being read.
  constexpr int kChunkBytes = 2 * kBigTile * 16;
  __shared__ __attribute__((aligned(1024))) uint8_t C[MODE == MODE_MX ? 2 * kChunkBytes : 16];
  // The epilogue's table of the tile's column scales and bias ([2][256] fp32).
  __shared__ __attribute__((aligned(16))) float T[512];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave_u = __builtin_amdgcn_readfirstlane(tid >> 6);  // keep descriptors in SGPRs
  const int wn = wave_u >> 1, wm = wave_u & 1;
  const int h = lane >> 5, frow = lane & 31;

  // Direct loads: wavefronts 0-1 fetch the 256 weight rows, 2-3 the 256 activation rows
  // (128 each). Load jj (0-15) of wavefront w reads operand rows 128 (w & 1) + 8 jj +
  // L/8 (lane L), 128 K bytes; the hardware writes lane L's 16 bytes at physical chunk
  // L & 7 of LDS row 64 w + 8 (jj & 7) + L/8 of half jj / 8 (32 KB) of the pair buffer.
  // Row r holds logical chunk c at c ^ ((r >> 1) & 7), so lane L fetches logical chunk
  // (L & 7) ^ ((4 (jj & 1) + (L >> 4)) & 7). Operand row R (0-255) of wavefront pair
  // side s (0: weight, 1: activation) is LDS row 64 (2 s + R / 128) + R % 64 of half
  // (R % 128) / 64.
  const bool w_wave = wave_u < 2;
  const int ld_u = __builtin_amdgcn_readfirstlane((int)(w_wave ? gin.ldw : gin.lda));
  const int voff_e = (lane >> 3) * ld_u + (((lane & 7) ^ ((lane >> 4) & 7)) << 4);
  const int voff_o = (lane >> 3) * ld_u + (((lane & 7) ^ ((4 + (lane >> 4)) & 7)) << 4);
  const int64_t ld_c = w_wave ? gin.ld_sb : gin.ld_sa;
  const int ldc_u = __builtin_amdgcn_readfirstlane((int)ld_c);

  using Src = PairSrc;
  auto make_src = [&](const PairItem& it) -> Src {
    const GemmArgs& g = it.g;
    const int64_t n_base = (int64_t)it.tn * kBigTile, m_base = (int64_t)it.tm * kBigTile;
    const int64_t row0 = (w_wave ? n_base : m_base) + (wave_u & 1) * 128;
    const OperandWindow win = operand_window(row0, w_wave ? g.N : g.M, w_wave ? g.ldw : g.lda);
    Src s;
    s.op = uniform_rsrc((w_wave ? g.w : g.a) + win.base_offset, win.records);
    // Code chunk loads mirror the operand loads: chunk row r (0-255 weight, 256-511
    // activation) at byte 16 r of its half. Rows past M / N read zero codes.
    const OperandWindow cwin = MODE == MODE_MX ? operand_window(row0, w_wave ? g.N : g.M, ld_c) : OperandWindow{0, 0};
    s.code = uniform_rsrc(reinterpret_cast<const uint8_t*>(w_wave ? g.sb : g.sa) + cwin.base_offset, cwin.records);
    s.np = __builtin_amdgcn_readfirstlane((int)(g.K / kPairK));  // real pairs
    s.npairs = (s.np + 1) & ~1;  // padded to the unroll (a padded pair computes zeros)
    // K stagger in pairs: (tm mod 8) + (tn mod 2) (mod np), the narrow kernel's stagger
    // of 2 (tm mod 8) + (tn mod 2) steps rounded to whole pairs.
    // MXFP8 (np % 4 == 0) staggers in whole chunks of four pairs, which is coarse: only
    // 4 ((tm mod 2) + (tn mod 2)) (mod np), the best of none, this and 4 (tm mod 8 ...).
    s.stag = __builtin_amdgcn_readfirstlane(
        MODE == MODE_MX ? 4 * (int)((unsigned)((it.tm & 1) + (it.tn & 1)) % (unsigned)(s.np / 4))
                        : (int)((unsigned)((it.tm & 7) + (it.tn & 1)) % (unsigned)s.np));
    return s;
  };
  // Issue pair p (< npairs) of `src` into pair buffer `dst`. A padded pair (p >= np)
  // reads past every buffer window, which returns zeros.
  auto issue = [&](const Src& src, int p, uint8_t* dst) {
    int kp = (p < src.np ? p : src.np - 1) + src.stag;
    kp = __builtin_amdgcn_readfirstlane(kp >= src.np ? kp - src.np : kp);
    const int pad_off = __builtin_amdgcn_readfirstlane(p < src.np ? 0 : 0x40000000);
#pragma unroll
    for (int jj = 0; jj < kDma; ++jj) {
      const int soff = __builtin_amdgcn_readfirstlane(jj * 8 * ld_u + kp * kPairK + pad_off);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          src.op, (__attribute__((address_space(3))) void*)(dst + ((jj >> 3) * (kPairBytes / 2) + (wave_u * 8 + (jj & 7)) * 1024)),
          16, (jj & 1) ? voff_o : voff_e, soff, 0, 0);
    }
  };
  // Code chunk c of `src` (pairs 4c .. 4c + 3) into half `half` of C: two 16-byte
  // direct loads of 64 rows per wavefront.
  auto issue_codes = [&](const Src& src, int c, int half) {
    if constexpr (MODE == MODE_MX) {
      int kc = c + src.stag / 4;
      kc = __builtin_amdgcn_readfirstlane(kc >= src.np / 4 ? kc - src.np / 4 : kc);
#pragma unroll
      for (int q = 0; q < 2; ++q)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            src.code, (__attribute__((address_space(3))) void*)(C + (half * kChunkBytes + (wave_u * 128 + q * 64) * 16)), 16,
            lane * ldc_u, __builtin_amdgcn_readfirstlane(q * 64 * ldc_u + kc * 16), 0, 0);
    }
  };

  // Fragment reads: a fragment's LDS row is frow plus a multiple of 32, so its swizzle
  // (row >> 1) & 7 is (frow >> 1) & 7 for all of them; step half t of the pair reads
  // logical chunks 4 t + h and 4 t + 2 + h. One 16-byte load at a single integer offset
  // from the pair buffer each (the compiler attributes an LDS access to its buffer only
  // through a short chain of address arithmetic; past it, it assumes the access may
  // alias every in-flight direct load and waits for all of them).
  const int fsw = (frow >> 1) & 7;
  const int off_t[2][2] = {{frow * kPairK + ((h ^ fsw) << 4), frow * kPairK + (((2 + h) ^ fsw) << 4)},
                           {frow * kPairK + (((4 + h) ^ fsw) << 4), frow * kPairK + (((6 + h) ^ fsw) << 4)}};
  auto frag = [&](const uint8_t* buf, int row0_bytes, int t) -> v8i {
    const v4i lo = *reinterpret_cast<const v4i*>(buf + (row0_bytes + off_t[t][0]));
    const v4i hi = *reinterpret_cast<const v4i*>(buf + (row0_bytes + off_t[t][1]));
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  };
  // Byte offset of the first row of operand rows [R, R + 32) (R % 32 == 0) of side s.
  auto rows_at = [](int s, int R) { return ((R & 127) >> 6) * (kPairBytes / 2) + (64 * (2 * s + (R >> 7)) + (R & 63)) * kPairK; };
  v8i wf[2][FN], af[2][FM];  // fragments of the current and the next step
  auto read_frags = [&](int set, const uint8_t* buf, int t) {
#pragma unroll
    for (int i = 0; i < FN; ++i) wf[set][i] = frag(buf, rows_at(0, wn * 128 + i * 32), t);
#pragma unroll
    for (int j = 0; j < FM; ++j) af[set][j] = frag(buf, rows_at(1, wm * 128 + j * 32), t);
  };

  // Declaring an AGPR clobber makes the compiler select the AGPR form of the MFMAs.
  asm volatile("" ::: "a255");
  v16f acc[FN][FM];
  // MXFP8: the codes of a fragment row for one pair are one dword (four 32-K blocks)
  // of its chunk row in C. Those of pair p + 1 are read during pair p into the second
  // set and moved to the first at the pair's end. Step half t of the pair uses block
  // 2 t + h in lane half h: the dword is shifted right by 8 h once when read, and the
  // MFMA's scale byte select takes byte 2 t.
  uint32_t wc[2][FN], ac[2][FM];
  auto read_codes = [&](int p, int set, int half) {
    if constexpr (MODE == MODE_MX) {
      const int base = half * kChunkBytes + (p & 3) * 4;
#pragma unroll
      for (int i = 0; i < FN; ++i) wc[set][i] = *reinterpret_cast<const uint32_t*>(C + (base + (wn * 128 + i * 32 + frow) * 16)) >> (8 * h);
#pragma unroll
      for (int j = 0; j < FM; ++j) ac[set][j] = *reinterpret_cast<const uint32_t*>(C + (base + (256 + wm * 128 + j * 32 + frow) * 16)) >> (8 * h);
    }
  };
  auto next_codes = [&] {
    if constexpr (MODE == MODE_MX) {
#pragma unroll
      for (int i = 0; i < FN; ++i) wc[0][i] = wc[1][i];
#pragma unroll
      for (int j = 0; j < FM; ++j) ac[0][j] = ac[1][j];
    }
  };
  auto mfmas = [&](int set, int j0, int j1) {
#pragma unroll
    for (int j = j0; j < j1; ++j)
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        if constexpr (MODE == MODE_MX) {
          // The code dwords hold blocks h, h + 2 in bytes 0, 2 (shifted by 8 h when read):
          // step half t = set takes byte 2 t through the MFMA's scale byte select.
          if (set == 0) acc[i][j] = mfma_sel<0>(wf[0][i], af[0][j], acc[i][j], (int)wc[0][i], (int)ac[0][j]);
          else acc[i][j] = mfma_sel<2>(wf[1][i], af[1][j], acc[i][j], (int)wc[0][i], (int)ac[0][j]);
        } else {
          acc[i][j] = mma<MODE>(wf[set][i], af[set][j], acc[i][j], kScaleOne, kScaleOne);
        }
      }
  };

  // Pair p in `cur`, pair p + 1 in flight into `nxt`, one barrier per pair, in two
  // halves. half0 (step 0): the 16 MFMAs of fragment set 0 interleaved one for one with
  // the reads of step 1's fragments (set 1) from `cur`. half1 (step 1): wait for pair
  // p + 1 and for this wavefront's reads, barrier (pair p + 1 is visible and nobody
  // reads `cur` any more), read the next pair's codes, issue the loads `refill` names
  // into `cur`, then the 16 MFMAs of set 1 interleaved with the direct loads and with
  // the reads of pair p + 1's step 0 fragments from `nxt`. Left to itself the scheduler
  // puts all reads after the MFMAs, and their latency then stalls the next step's first
  // MFMA. The K loop's body starts with a half1, i.e. with the wait: at its head every
  // LDS read comes after that wait, so the compiler never has to decide whether a read
  // may alias a direct load in flight from before the loop. The buffers are
  // compile-time choices (B: pair p in P0 or P1), so that every LDS access keeps its
  // object (an access the compiler cannot attribute to a buffer is assumed to alias
  // the in-flight direct loads, and it waits for all of them first).
  auto half0 = [&](auto B) __attribute__((always_inline)) {
    uint8_t* cur = decltype(B)::value == 0 ? P0 : P1;
    read_frags(1, cur, 1);
    mfmas(0, 0, FM);
#pragma unroll
    for (int i = 0; i < FN * FM; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto half1 = [&](auto B, auto&& codes_next, auto&& refill, auto&& frags_next) __attribute__((always_inline)) {
    uint8_t* cur = decltype(B)::value == 0 ? P0 : P1;
    uint8_t* nxt = decltype(B)::value == 0 ? P1 : P0;
    wait_vmcnt<0>();
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // The next pair's codes are read before any new code load is in flight (the
    // compiler cannot tell the two halves of C apart and would wait for it).
    codes_next();
    refill(cur);
    frags_next(nxt);
    mfmas(1, 0, FM);
#pragma unroll
    for (int i = 0; i < FN * FM; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one direct load
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
    }
    __builtin_amdgcn_sched_barrier(0);
    next_codes();
  };

  auto frags_step0 = [&](const uint8_t* buf) __attribute__((always_inline)) { read_frags(0, buf, 0); };
  constexpr std::integral_constant<int, 0> kBuf0{};
  constexpr std::integral_constant<int, 1> kBuf1{};
  // Piece-major K splits: workgroups are dealt to the XCDs round-robin (b % 8), so with
  // a multiple of 8 pieces every tile of one piece runs on one XCD and the piece's
  // operand slices (its K range of the weight and of the activation) are fetched into
  // that XCD's L2 once, instead of once per XCD that runs one of its tiles.
  const int piece = gin.kpieces > 0 ? (int)(blockIdx.x % (unsigned)gin.kpieces) : (int)blockIdx.y;
  int item = gin.kpieces > 0 ? (int)(blockIdx.x / (unsigned)gin.kpieces) : (int)blockIdx.x;
  Src src = make_src(pair_item<MODE>(gin, item, piece));
  int cbase = 0;  // C half of the item's code chunk 0
  // Prologue: pairs 0 and 1 in flight (pair 0's codes between them), pair 0 visible,
  // step (0, 0)'s fragments in set 0.
  issue(src, 0, P0);
  issue_codes(src, 0, 0);
  issue(src, 1, P1);
  wait_vmcnt<kDma>();
  lds_barrier();
  read_frags(0, P0, 0);
  read_codes(0, 0, 0);
  auto start_item = [&] __attribute__((always_inline)) {
    // The zero comes out of an opaque statement ordered after the previous item's
    // epilogue, so the new accumulators cannot be set up before the old ones are read
    // (both sets at once do not fit the registers).
    float zero = 0.0f;
    asm volatile("" : "+v"(zero));
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = zero;
    half0(kBuf0);  // pair 0, step 0
  };
  start_item();

  // The item loop's body starts with a half1 too (the wait), for the same reason as the
  // K loop's; an item's first half0 ends the previous iteration.
  for (;;) {
    const int npairs = src.npairs;
    // Step 1 of pairs 0 .. npairs - 3 and step 0 of pairs 1 .. npairs - 2: each half1
    // refills its buffer with pair p + 2 of this item.
    for (int p = 0; p + 2 < npairs; p += 2) {
      half1(kBuf0, [&] { read_codes(p + 1, 1, (cbase + ((p + 1) >> 2)) & 1); },
            [&](uint8_t* cur) {
              issue(src, p + 2, cur);
              if (MODE == MODE_MX && ((p + 2) & 3) == 0) issue_codes(src, (p + 2) >> 2, (cbase + ((p + 2) >> 2)) & 1);
            }, frags_step0);
      half0(kBuf1);
      half1(kBuf1, [&] { read_codes(p + 2, 1, (cbase + ((p + 2) >> 2)) & 1); },
            [&](uint8_t* cur) {
              issue(src, p + 3, cur);
              if (MODE == MODE_MX && ((p + 3) & 3) == 0) issue_codes(src, (p + 3) >> 2, (cbase + ((p + 3) >> 2)) & 1);
            }, frags_step0);
      half0(kBuf0);
    }
    // The next item (this one again when there is none: its loads then land unused).
    const int next = item + (int)gridDim.x;
    const bool more = next < gin.items;
    const Src nsrc = make_src(pair_item<MODE>(gin, more ? next : item, piece));
    const int ncbase = (cbase + npairs / 4) & 1;  // MX: npairs == np, a multiple of 4
    const PairItem it = pair_item<MODE>(gin, item, piece);
    // Pair npairs - 2, step 1: its refill is this item's output scales and bias (one and
    // a half pairs ahead of the epilogue) and the next item's pair 0 (and code chunk 0).
    PairScales scales;
    half1(kBuf0, [&] { read_codes(npairs - 1, 1, (cbase + ((npairs - 1) >> 2)) & 1); },
          [&](uint8_t* cur) {
            scales = load_pair_scales<MODE>(it.g, (int64_t)it.tm * kBigTile, (int64_t)it.tn * kBigTile);
            issue(nsrc, 0, cur);
            issue_codes(nsrc, 0, ncbase);
          }, frags_step0);
    half0(kBuf1);
    // Pair npairs - 1, step 1: no direct loads, since its buffer (P1) stages the
    // epilogue, and no fragment reads (the next item's are read after the epilogue, so
    // that they do not hold registers through it).
    half1(kBuf1, [&] { read_codes(0, 1, ncbase); }, [](uint8_t*) {}, [](const uint8_t*) {});
    // Every wavefront has passed the last pair's barrier: nobody reads P1 any more.
    pair_epilogue<MODE>(it.g, it.partial, acc, scales, (int64_t)it.tm * kBigTile, (int64_t)it.tn * kBigTile, P1, T);
    if (!more) break;
    item = next;
    src = nsrc;
    cbase = ncbase;
    issue(src, 1, P1);  // after the epilogue's last barrier: nobody reads the staging tile
    read_frags(0, P0, 0);  // pair 0 landed before the last pair's barrier
    start_item();
  }
  // Outstanding at exit: the unused reload of the last item's first pair (into a buffer
  // nobody reads) and the epilogue's stores.
  wait_vmcnt<0>();
}

// ---------------------------------------------------------------------------------
// Block-scaled kernel (fp8_blockwise_mm; K % 128 == 0, M and N >= 128): a 128 x 128
// output tile per workgroup of four wavefronts, each owning a 64 (n) x 64 (m) tile
// (2 x 2 MFMA tiles).
//
// The reference scales every 128-K partial product by sa[m, kb] * sb[n / 128, kb]
// before summing. Each wavefront keeps its partials in AGPRs (the MFMA accumulator,
// restarted from zero at each 128-K block) and the running sum in VGPRs: at the end of
// a block, one fma per element moves partial * (sa * sb) into the sum (VALU cannot read
// AGPRs, so the sum cannot live there). Larger tiles need more registers for the sums
// than a wavefront has beside its fragments. The partials of m-fragment 0 are folded
// at the end of the block's second step, those of m-fragment 1 at the start of the
// next block's first step, so the VALU work runs beside MFMAs. The loads follow the
// 256 x 256 kernel (64-K stages in a four-buffer LDS ring, direct-to-LDS, one mid-step
// barrier); each block's three scales (two sa rows per lane, one sb per wavefront: its
// 64 weight rows lie in one 128-row block) are loaded one block ahead.
constexpr int kBlkThreads = 256;
constexpr int kBlkTile = 128;
constexpr int kBlkStage = 2 * kBlkTile * kBigK;             // 16 KB
constexpr int kBlkEpilogueLds = 32 * (kBlkTile * 4 + 16);   // 32 staged rows of fp32

template <int OUT>
__device__ __attribute__((always_inline)) inline void block_epilogue(const GemmArgs& g, const float (&acc)[2][2][16], int64_t m_tile, int64_t n_tile,
                                      uint8_t* ep) {
  constexpr int EB = OutBytes<OUT>::v;
  constexpr int kRowBytes = kBlkTile * EB + 16;
  constexpr int kChunksPerRow = kBlkTile * EB / 16;
  constexpr int kRowsPerStep = kBlkThreads / kChunksPerRow;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wn = wave >> 1, wm = wave & 1, h = lane >> 5, frow = lane & 31;
#pragma unroll
  for (int wmh = 0; wmh < 2; ++wmh) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (wm == wmh) {  // the two wavefronts of this m half write its 32 rows j
        uint8_t* srow = ep + frow * kRowBytes;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
          for (int grp = 0; grp < 4; ++grp) {
            const int nl = wn * 64 + i * 32 + grp * 8 + h * 4;
            const int64_t n = n_tile + nl;
            float bias[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (g.bias && n < g.N) load_bias4(g, n, bias);
            float v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = acc[i][j][grp * 4 + q] + bias[q];
            if constexpr (OUT == AYK_F32) {
              *reinterpret_cast<float4*>(srow + nl * 4) = make_float4(v[0], v[1], v[2], v[3]);
            } else {
              uint16_t b[4];
#pragma unroll
              for (int q = 0; q < 4; ++q) b[q] = OUT == AYK_BF16 ? f32_to_bf16_bits(v[q]) : f32_to_f16_bits(v[q]);
              *reinterpret_cast<uint2*>(srow + nl * 2) =
                  make_uint2((uint32_t)b[0] | ((uint32_t)b[1] << 16), (uint32_t)b[2] | ((uint32_t)b[3] << 16));
            }
          }
        }
      }
      lds_barrier();
#pragma unroll
      for (int r0 = 0; r0 < 32; r0 += kRowsPerStep) {
        const int r = r0 + tid / kChunksPerRow, c = tid % kChunksPerRow;
        const int64_t gm = m_tile + wmh * 64 + j * 32 + r;
        const int64_t gn = n_tile + (int64_t)c * (16 / EB);
        if (gm < g.M && gn < g.N) {
          const uint4 val = *reinterpret_cast<const uint4*>(ep + r * kRowBytes + c * 16);
          uint8_t* dst = reinterpret_cast<uint8_t*>(g.out) + (gm * g.ldo + gn) * EB;
          if (gn + 16 / EB <= g.N) *reinterpret_cast<uint4*>(dst) = val;
          else *reinterpret_cast<uint2*>(dst) = make_uint2(val.x, val.y);  // N % 4 == 0
        }
      }
      lds_barrier();
    }
  }
}

// One 128 x 128 output tile (tile coordinates tm, tn) of a block-scaled GEMM, staged
// through the four LDS buffers the calling kernel declares (L0 also stages the epilogue).
__device__ __attribute__((always_inline)) inline void block_gemm_tile(const GemmArgs& g, int tm, int tn, uint8_t* L0,
                                                                      uint8_t* L1, uint8_t* L2, uint8_t* L3) {
  constexpr int FN = 2, FM = 2;
  constexpr int kWDma = 2, kADma = 2;           // direct loads per wavefront per step
  constexpr int kDma = kWDma + kADma;
  constexpr int kScaleOps = 3;                  // per block, issued one block ahead
  // Ops issued per step alternate kDma + kScaleOps (a block's first step: the refill and
  // the next block's scales) and kDma, so any two consecutive steps issue this many:
  constexpr int kAfterNext = 2 * kDma + kScaleOps;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave_u = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave_u >> 1, wm = wave_u & 1;  // 64-row n half, 64-row m half
  const int h = lane >> 5, frow = lane & 31;
  const int64_t n_base = (int64_t)tn * kBlkTile, m_base = (int64_t)tm * kBlkTile;
  const int nk = (int)(g.K / kBigK);     // even: K % 128 == 0
  const int kblocks = nk / 2;
  const int nsteps = (nk + 3) & ~3;      // the loop is unrolled by four steps (two blocks)
  // K stagger (even, so 128-K blocks stay aligned): see the 256 x 256 kernel.
  const int stag = __builtin_amdgcn_readfirstlane((int)((unsigned)(((tm & 7) + (tn & 1)) * 2) % (unsigned)nk));

  // Direct loads: wavefront w fetches weight rows [32 w, 32 w + 32) and activation rows
  // [32 w, 32 w + 32) (two loads of 16 rows each), swizzled as in the 256 x 256 kernel
  // (row r holds logical chunk c at c ^ ((r >> 2) & 3)).
  const int ldw_u = __builtin_amdgcn_readfirstlane((int)g.ldw), lda_u = __builtin_amdgcn_readfirstlane((int)g.lda);
  const OperandWindow wwin = operand_window(n_base + wave_u * 32, g.N, g.ldw);
  const OperandWindow awin = operand_window(m_base + wave_u * 32, g.M, g.lda);
  const __amdgpu_buffer_rsrc_t w_rsrc = uniform_rsrc(g.w + wwin.base_offset, wwin.records);
  const __amdgpu_buffer_rsrc_t a_rsrc = uniform_rsrc(g.a + awin.base_offset, awin.records);
  const int sw_chunk = ((lane & 3) ^ ((lane >> 4) & 3)) << 4;
  const int wvoff = (lane >> 2) * ldw_u + sw_chunk, avoff = (lane >> 2) * lda_u + sw_chunk;

  // Block scales. sa is [M, KB] row-major (element m * KB + kb) or, with sa_vec,
  // [KB, M] (kb * M + m), fp32; lane (frow, h) needs its two m rows. sb is [NB, KB] in
  // fp32 / fp16 / bf16, one value per wavefront, kept as the dword that holds it (its
  // position in the dword is wave-uniform and recomputed at use).
  // Row strides of the scale tables: ld_sa / ld_sb when set (a K range of a longer K:
  // the split-K kernel), else this problem's block count.
  const int64_t sa_ld = g.ld_sa > 0 ? g.ld_sa : kblocks, sb_ld = g.ld_sb > 0 ? g.ld_sb : kblocks;
  int64_t sa_row[FM];
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int64_t m = m_base + wm * 64 + j * 32 + frow;
    sa_row[j] = (m < g.M ? m : g.M - 1) * (g.sa_vec ? 1 : sa_ld);
  }
  const int64_t nbs = cdiv(g.N, 128);
  const int64_t nb = (n_base + wn * 64) / 128 < nbs ? (n_base + wn * 64) / 128 : nbs - 1;
  const int sb_size = g.sb_dtype == AYK_F32 ? 4 : 2;
  const int64_t sb_base = nb * sb_ld;
  // Two blocks' scales in flight (slot = block % 2). Slot 1 starts as zeros: the first
  // step folds "the previous block" from it, with zero partials: it adds 0.
  uint32_t sa_w[2][FM], sb_w[2];
  sa_w[1][0] = sa_w[1][1] = sb_w[1] = 0u;
  int kb_of[2] = {0, 0};  // the 128-K block each slot holds (uniform)

  // K stage of step s (padded steps: the last real stage; their loads read zeros).
  auto stage_of = [&](int s) {
    const int ks = (s < nk ? s : nk - 1) + stag;
    return __builtin_amdgcn_readfirstlane(ks >= nk ? ks - nk : ks);
  };
  auto issue = [&](int s, uint8_t* dst) {
    const int ks = stage_of(s);
    const int pad_off = __builtin_amdgcn_readfirstlane(s < nk ? 0 : 0x40000000);
#pragma unroll
    for (int jj = 0; jj < kWDma; ++jj) {
      const int soff = __builtin_amdgcn_readfirstlane(jj * 16 * ldw_u + ks * kBigK + pad_off);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rsrc, (__attribute__((address_space(3))) void*)(dst + (wave_u * kWDma + jj) * 1024),
                                               16, wvoff, soff, 0, 0);
    }
#pragma unroll
    for (int jj = 0; jj < kADma; ++jj) {
      const int soff = __builtin_amdgcn_readfirstlane(jj * 16 * lda_u + ks * kBigK + pad_off);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, (__attribute__((address_space(3))) void*)(dst + kBlkTile * kBigK + (wave_u * kADma + jj) * 1024),
                                               16, avoff, soff, 0, 0);
    }
  };
  // Scales of the block whose first step is s (block kb = stage / 2) into `slot`.
  auto issue_scales = [&](int s, int slot) {
    const int kb = stage_of(s) >> 1;
    kb_of[slot] = kb;
    const float* sa_p = reinterpret_cast<const float*>(g.sa);
#pragma unroll
    for (int j = 0; j < FM; ++j) sa_w[slot][j] = __float_as_uint(sa_p[g.sa_vec ? (int64_t)kb * g.M + sa_row[j] : sa_row[j] + kb]);
    const uint8_t* sbp = reinterpret_cast<const uint8_t*>(g.sb) + (sb_base + kb) * sb_size;
    sb_w[slot] = *reinterpret_cast<const uint32_t*>(sbp - (reinterpret_cast<uintptr_t>(sbp) & 3));
  };

  const int fsw = (frow >> 2) & 3;
  const int c0 = (h ^ fsw) << 4, c1 = ((2 + h) ^ fsw) << 4;
  auto frag = [&](const uint8_t* buf, int row0) -> v8i {
    const uint8_t* base = buf + (row0 + frow) * kBigK;
    const uint4 lo = *reinterpret_cast<const uint4*>(base + c0);
    const uint4 hi = *reinterpret_cast<const uint4*>(base + c1);
    v8i r;
    r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
    r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
    return r;
  };
  v8i wf[2][FN], af[2][FM];  // fragments of the current and the next step
  auto read_frags = [&](int set, const uint8_t* buf) {
#pragma unroll
    for (int i = 0; i < FN; ++i) wf[set][i] = frag(buf, wn * 64 + i * 32);
#pragma unroll
    for (int j = 0; j < FM; ++j) af[set][j] = frag(buf + kBlkTile * kBigK, wm * 64 + j * 32);
  };

  // The MFMA accumulators (the partials, 64 registers) in AGPRs; the clobber names the
  // last of them. The sums and fragments take the VGPRs.
  asm volatile("" ::: "a63");
  const v16f zero = {};
  v16f part[FN][FM];
  float acc[FN][FM][16];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      part[i][j] = zero;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    }
  // m-fragment j of a step: fresh partials at a block's first step, accumulate at its second.
  auto mfmas = [&](int set, int j, bool fresh) {
#pragma unroll
    for (int i = 0; i < FN; ++i) part[i][j] = mfma(wf[set][i], af[set][j], fresh ? zero : part[i][j], kScaleOne, kScaleOne);
  };
  const uintptr_t sb_addr0 = reinterpret_cast<uintptr_t>(g.sb) + (uintptr_t)(sb_base * sb_size);
  const bool sb_f32 = g.sb_dtype == AYK_F32, sb_bf16 = g.sb_dtype == AYK_BF16;
  // Fold m-fragment j's partials of the block in `slot` into the sums. The scale words
  // pass through an empty asm first, so nothing that reads them is hoisted to where it
  // would wait for later loads.
  auto fold = [&](int slot, int j) {
    uint32_t a = sa_w[slot][j], b = sb_w[slot];
    asm volatile("" : "+v"(a), "+v"(b));
    const uint32_t sh = (uint32_t)((sb_addr0 + (uintptr_t)kb_of[slot] * sb_size) & 3) * 8;
    const uint32_t hb = (b >> sh) & 0xFFFFu;
    const float f16v = f16_bits_to_f32((uint16_t)hb);
    const float sbv = sb_f32 ? __uint_as_float(b) : (sb_bf16 ? __uint_as_float(hb << 16) : f16v);
    const float s = __uint_as_float(a) * sbv;
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = fmaf(part[i][j][r], s, acc[i][j][r]);
  };

  // Prologue: steps 0-3 in flight and block 0's scales, in the order that keeps every
  // step's wait at kAfterNext (two steps' ops after the one waited for).
  issue(0, L0);
  issue(1, L1);
  issue_scales(0, 0);
  issue(2, L2);
  issue(3, L3);
  wait_vmcnt<kAfterNext + kDma>();  // step 0 landed
  lds_barrier();
  read_frags(0, L0);

  // Step s of block s / 2 (slot = block % 2, static under the unroll by four). A
  // block's first step folds the previous block's m-fragment 1, then refills that slot
  // with the next block's scales.
  auto step = [&](int s, int set, bool first, int slot, uint8_t* cur, uint8_t* nxt) {
    mfmas(set, 0, first);
    if (first) fold(slot ^ 1, 1);   // the previous block's m-fragment 1 (adds 0 at s == 0)
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<kAfterNext>();
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue(s + 4 < nsteps ? s + 4 : nsteps - 1, cur);
    if (first) issue_scales(s + 2 < nsteps ? s + 2 : nsteps - 2, slot ^ 1);
    read_frags(set ^ 1, nxt);
    mfmas(set, 1, first);
    if (!first) fold(slot, 0);
  };
  for (int s = 0; s < nsteps; s += 4) {
    step(s, 0, true, 0, L0, L1);
    step(s + 1, 1, false, 0, L1, L2);
    step(s + 2, 0, true, 1, L2, L3);
    step(s + 3, 1, false, 1, L3, L0);
  }
  fold(1, 1);  // the last block's m-fragment 1 (its block index is odd)
  wait_vmcnt<0>();
  lds_barrier();
  if (g.out_dtype == AYK_BF16) block_epilogue<AYK_BF16>(g, acc, m_base, n_base, L0);
  else if (g.out_dtype == AYK_F16) block_epilogue<AYK_F16>(g, acc, m_base, n_base, L0);
  else block_epilogue<AYK_F32>(g, acc, m_base, n_base, L0);
}

#define AYK_BLOCK_LDS                                                                                        \
  __shared__ __attribute__((aligned(1024))) uint8_t L0[kBlkEpilogueLds > kBlkStage ? kBlkEpilogueLds : kBlkStage]; \
  __shared__ __attribute__((aligned(1024))) uint8_t L1[kBlkStage];                                         \
  __shared__ __attribute__((aligned(1024))) uint8_t L2[kBlkStage];                                         \
  __shared__ __attribute__((aligned(1024))) uint8_t L3[kBlkStage]

__global__ __launch_bounds__(kBlkThreads, 1) void fp8_gemm_block_kernel(GemmArgs g) {
  AYK_BLOCK_LDS;
  int tm, tn;
  big_tile_coords(blockIdx.x, g.tiles_m, (int)cdiv(g.N, kBlkTile), tm, tn);
  block_gemm_tile(g, tm, tn, L0, L1, L2, L3);
}

// Split-K form for launches with too few tiles to fill the machine: blockIdx.y takes the
// K range [y kps, (y + 1) kps) (kps % 128 == 0) and writes its fp32 partial tile to
// part[y] ([M, N], row stride N); block_split_reduce sums the partials in split order,
// adds the bias and rounds once.
__global__ __launch_bounds__(kBlkThreads, 1) void fp8_gemm_block_split_kernel(GemmArgs g, int64_t kps, float* part) {
  AYK_BLOCK_LDS;
  int tm, tn;
  big_tile_coords(blockIdx.x, g.tiles_m, (int)cdiv(g.N, kBlkTile), tm, tn);
  const int64_t k0 = (int64_t)blockIdx.y * kps, kb0 = k0 / 128, kb_total = g.K / 128;
  GemmArgs s = g;
  s.K = g.K - k0 < kps ? g.K - k0 : kps;
  s.a = g.a + k0;
  s.w = g.w + k0;
  s.sa = static_cast<const float*>(g.sa) + (g.sa_vec ? kb0 * g.M : kb0);
  s.ld_sa = g.sa_vec ? 0 : kb_total;
  s.sb = static_cast<const uint8_t*>(g.sb) + kb0 * (g.sb_dtype == AYK_F32 ? 4 : 2);
  s.ld_sb = kb_total;
  s.bias = nullptr;
  s.out = part + (int64_t)blockIdx.y * g.M * g.N;
  s.out_dtype = AYK_F32;
  s.ldo = g.N;
  block_gemm_tile(s, tm, tn, L0, L1, L2, L3);
}

// Tail split of the 256 x 256 pair kernel: tile t (0 .. tail_tiles - 1) of the tail is
// tile dp_tiles + t of the XCD-aware order; its tail_split partials sit at
// part[(y tail_tiles + t) 65536 ..]. Summed in piece order, bias added, rounded once;
// four consecutive columns per thread (N % 4 == 0 on this path).
__global__ __launch_bounds__(256) void tail_split_reduce(const float* __restrict__ part, int tail_tiles, int split,
                                                         int dp_tiles, int tiles_m, int tiles_n, int64_t M, int64_t N,
                                                         const void* __restrict__ bias, int bias_dtype,
                                                         void* __restrict__ out, int out_dtype, int64_t ldo) {
  constexpr int kTileElems = kBigTile * kBigTile;
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= (int64_t)tail_tiles * kTileElems) return;
  const int t = (int)(i / kTileElems), within = (int)(i % kTileElems);
  const int r = within / kBigTile, c = within % kBigTile;
  int tm, tn;
  big_tile_coords(dp_tiles + t, tiles_m, tiles_n, tm, tn);
  const int64_t m = (int64_t)tm * kBigTile + r, n = (int64_t)tn * kBigTile + c;
  if (m >= M || n >= N) return;
  float4 v = *reinterpret_cast<const float4*>(part + i);
  // Pieces 1 .. split - 1 in order, their loads issued four at a time.
  auto piece = [&](int y) { return *reinterpret_cast<const float4*>(part + ((int64_t)y * tail_tiles + t) * kTileElems + within); };
  auto add = [&](const float4& p) { v.x += p.x; v.y += p.y; v.z += p.z; v.w += p.w; };
  int y = 1;
  for (; y + 4 <= split; y += 4) {
    const float4 a = piece(y), b = piece(y + 1), c4 = piece(y + 2), d = piece(y + 3);
    add(a); add(b); add(c4); add(d);
  }
  for (; y < split; ++y) add(piece(y));
  float o[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (bias) o[q] += load_f32(bias, bias_dtype, n + q);
    store_f32(out, out_dtype, m * ldo + n + q, o[q]);
  }
}

__global__ __launch_bounds__(256) void block_split_reduce(const float* __restrict__ part, int64_t M, int64_t N, int split,
                                                          const void* __restrict__ bias, int bias_dtype, void* __restrict__ out,
                                                          int out_dtype, int64_t ldo) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= M * N) return;
  const int64_t m = i / N, n = i - m * N;
  float v = 0.0f;
  for (int s = 0; s < split; ++s) v += part[(int64_t)s * M * N + i];
  if (bias) v += load_f32(bias, bias_dtype, n);
  store_f32(out, out_dtype, m * ldo + n, v);
}

// K split of the block-scaled large-tile GEMM (powers of two dividing K / 128, at least
// 1024 K per split). Under one round of tiles (256, one workgroup per CU): as many
// splits as still fit in that round (7168 x 18432 at M = 256: 2 splits 94 us, 4 splits
// 123 us). From one round up to kBlkSplitTarget tiles: splits until that many
// workgroups (18432 x 7168 at M = 256: 2 splits 130 us, none 139 us).
constexpr int64_t kBlkSplitTarget = 512;
int64_t block_split(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = cdiv(M, kBlkTile) * cdiv(N, kBlkTile);
  int64_t split = 1;
  if (tiles < 256) {
    while (tiles * split * 2 <= 256 && K / (split * 2) >= 1024 && (K / 128) % (split * 2) == 0) split *= 2;
    return split;
  }
  while (tiles * split < kBlkSplitTarget && K / (split * 2) >= 1024 && (K / 128) % (split * 2) == 0) split *= 2;
  return split;
}
// The same rule for the general kernel's 32- or 64-row tiles (M <= 64, K % 128 == 0).
int64_t general_split(int64_t M, int64_t N, int64_t K) {
  if (M > 64 || K % 128) return 1;
  const int64_t tiles = cdiv(M, M <= 32 ? 32 : 64) * cdiv(N, 128);
  int64_t split = 1;
  while (tiles * split < kBlkSplitTarget && K / (split * 2) >= 1024 && (K / 128) % (split * 2) == 0) split *= 2;
  return split;
}
// Rowwise / per-tensor K split for launches short of one round of bm x bn tiles (one
// round: 256 workgroups of the 256 x 256 kernel, one per CU; 512 of the general
// kernel's): as many splits as still fit in that one round, at least 1024 K each (the
// last may be shorter). Spilling into a second round doubles the time of the splits
// and multiplies the partial-sum traffic (Qwen2 down at M = 2048: 5 splits 231 us,
// 2 splits fill the round).
int64_t scaled_split(int64_t M, int64_t N, int64_t K, int bm, int bn) {
  if (K % 128) return 1;
  const int64_t round = bm == kBigTile ? 256 : kBlkSplitTarget;
  const int64_t tiles = cdiv(M, bm) * cdiv(N, bn);
  if (tiles * 2 > round) return 1;
  const int64_t want = round / tiles, most = K / 1024;
  const int64_t split = want < most ? want : most;
  if (split <= 1) return 1;
  const int64_t kps = cdiv(K / 128, split) * 128;
  return cdiv(K, kps);
}
int64_t scaled_kps(int64_t K, int64_t split) { return cdiv(K / 128, split) * 128; }
// The pair kernel's K split, launched piece-major: a planned split of 8 or more is
// rounded down to a multiple of 8, so that each piece's tiles share one XCD (its L2).
// Qwen2 down at M = 512 (28 tiles): 9 pieces over all eight XCDs fetched 2.2x the
// unique operand bytes (each XCD re-read the activation slices of every piece).
int64_t xcd_pieces(int64_t planned) { return planned >= 8 ? planned / 8 * 8 : planned; }

// Tail split of the 256 x 256 pair kernel (launches of more than one round): when the
// last round would hold at most a third of a round of tiles, those tiles are split over
// K into the largest number of pieces (at least three) that still fits in one round
// (256 workgroups), each of at least 512 K, dividing K into whole 128-K pairs (MXFP8:
// whole 512-K code chunks). The first rounds run whole tiles. A piece pays a tile's
// prologue and a 256 KB fp32 epilogue, and the partials a reduce: measured on Qwen2
// gate_up (K = 3584), M = 512 went 115 -> 105 us and M = 4096 649 -> 638 us, while a
// two-way split (M = 8192) broke even. A function of the shape only (the workspace
// query reproduces it). split = 1: no tail split.
struct TailPlan {
  int dp_tiles, split, tail_tiles;
};
TailPlan tail_plan(int64_t M, int64_t N, int64_t K, bool mx) {
  TailPlan p{0, 1, 0};
  const int64_t tiles = cdiv(M, kBigTile) * cdiv(N, kBigTile);
  const int64_t unit = mx ? 512 : 128;
  if (tiles <= 256 || tiles > 0x7FFFFFFF / 2 || K % unit) return p;
  const int64_t rem = tiles % 256;
  if (rem == 0 || rem > 256 / 3) return p;
  for (int64_t s = 256 / rem; s >= 3; --s) {
    if ((K / unit) % s == 0 && K / s >= 512) {
      p.dp_tiles = (int)(tiles - rem);
      p.split = (int)s;
      p.tail_tiles = (int)rem;
      return p;
    }
  }
  return p;
}
size_t tail_workspace(const TailPlan& p) {
  return p.split > 1 ? (size_t)p.split * (size_t)p.tail_tiles * kBigTile * kBigTile * sizeof(float) : 0;
}

size_t scaled_split_workspace(int64_t M, int64_t N, int64_t K) {
  const int bm = M <= 32 ? 32 : (M <= 64 ? 64 : 128);
  int64_t split = scaled_split(M, N, K, bm, 128);
  if (M >= 256 && N >= 256) {
    const int64_t big = scaled_split(M, N, K, kBigTile, kBigTile);
    split = big > split ? big : split;
  }
  return split > 1 ? (size_t)split * (size_t)M * (size_t)N * sizeof(float) : 0;
}
// Mirrors launch_gemm<MODE_BLOCK>: up to 64 rows the general kernel's split (any N);
// above, the 128 x 128 kernel's split when N allows that kernel (else no split).
bool block256_wanted(int64_t M, int64_t N, int64_t K);
size_t block_split_workspace(int64_t M, int64_t N, int64_t K) {
  int64_t split = M <= 64 ? general_split(M, N, K) : (N >= kBlkTile ? block_split(M, N, K) : 1);
  // The 256 x 256 kernel when it takes the launch (an upper bound: alignment may still
  // send the launch to the 128 x 128 kernel).
  if (block256_wanted(M, N, K)) {
    const int64_t s256 = block256_split(M, N, K);
    split = s256 > split ? s256 : split;
  }
  return split > 1 ? (size_t)split * (size_t)M * (size_t)N * sizeof(float) : 0;
}

// MXFP8 large-tile kernel with 128-K stages: two 64 KB LDS stages, one code dword (four
// UE8M0 codes) per fragment row and stage. The 64-K-stage kernel above would need one
// code load per row and stage, which doubles its L2 request count; until its codes
// travel in wider blocks, MXFP8 keeps this pipeline (K % 128 == 0).
constexpr int kMx128Stage = 2 * kBigTile * BK;  // 64 KB

template <int MODE>
__global__ __launch_bounds__(kThreads, 1) void fp8_gemm_mx128_kernel(GemmArgs g) {
  static_assert(MODE == MODE_MX, "MX codes only");
  constexpr int FN = 4, FM = 4;                  // 32x32 MFMA tiles per wavefront (n, m)
  constexpr int kLoads = kMx128Stage / 1024 / 4;   // direct loads per wavefront per stage
  // Two distinct LDS objects (not one array indexed by stage), so the compiler can
  // tell that reads of one stage never alias the in-flight direct loads of the other
  // and does not wait for those loads before reading.
  __shared__ __attribute__((aligned(1024))) uint8_t lds0[kMx128Stage];
  __shared__ __attribute__((aligned(1024))) uint8_t lds1[kMx128Stage];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wn = wave >> 1, wm = wave & 1;
  const int h = lane >> 5, frow = lane & 31;
  int tm, tn;
  big_tile_coords(blockIdx.x, g.tiles_m, (int)cdiv(g.N, kBigTile), tm, tn);
  const int64_t n_base = (int64_t)tn * kBigTile, m_base = (int64_t)tm * kBigTile;
  const int nk = (int)(g.K / BK);

  // Direct loads: wavefronts 0-1 fetch the 256 weight rows, 2-3 the 256 activation
  // rows (128 each), as buffer loads into LDS. Load instruction jj of a wavefront
  // fills LDS tile rows r = 8 * (16 * wave + jj) + lane/8; lane fetches logical chunk
  // (lane & 7) ^ ((r >> 1) & 7), which depends only on the lane and jj's parity. The
  // buffer resource starts at the wavefront's first row and ends at the operand's last
  // row: rows past M / N read as zero (their results are never stored), no clamping.
  // Per load: a per-lane vector offset (row, chunk) and a wave-uniform scalar offset
  // (jj's 8 rows + K step), so no 64-bit address is kept per load.
  const int q = lane >> 3, pc = lane & 7;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);  // keep the descriptor in SGPRs
  const bool w_wave = wave_u < 2;
  const int64_t ld = w_wave ? g.ldw : g.lda;
  const int64_t row0 = (w_wave ? n_base : m_base) + (wave_u & 1) * 128;
  const OperandWindow win = operand_window(row0, w_wave ? g.N : g.M, ld);
  const __amdgpu_buffer_rsrc_t op_rsrc = uniform_rsrc((w_wave ? g.w : g.a) + win.base_offset, win.records);
  const int voff[2] = {(int)(q * ld) + ((pc ^ ((q >> 1) & 7)) << 4), (int)(q * ld) + ((pc ^ ((4 + (q >> 1)) & 7)) << 4)};
  auto issue_stage = [&](int kt, uint8_t* dst) {
#pragma unroll
    for (int jj = 0; jj < kLoads; ++jj) {
      const int soff = __builtin_amdgcn_readfirstlane((int)(jj * 8 * ld) + kt * BK);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(op_rsrc, (__attribute__((address_space(3))) void*)(dst + (wave_u * kLoads + jj) * 1024),
                                               16, voff[jj & 1], soff, 0, 0);
    }
  };
  // Fragment reads. A fragment row is frow + (a multiple of 32), so its swizzle term
  // (row >> 1) & 7 == (frow >> 1) & 7 is the same for every fragment of this lane: the
  // four chunk offsets below plus compile-time row offsets address all of them.
  const int fsw = (frow >> 1) & 7;
  const int choff[4] = {(h ^ fsw) << 4, ((2 + h) ^ fsw) << 4, ((4 + h) ^ fsw) << 4, ((6 + h) ^ fsw) << 4};
  auto frag = [&](const uint8_t* buf, int tile_row0, int ks) -> v8i {
    const uint8_t* base = buf + (tile_row0 + frow) * BK;
    const uint4 lo = *reinterpret_cast<const uint4*>(base + choff[2 * ks]);
    const uint4 hi = *reinterpret_cast<const uint4*>(base + choff[2 * ks + 1]);
    v8i r;
    r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
    r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
    return r;
  };
  // MX: the four UE8M0 codes of one row for K step kt (one dword; K/32 % 4 == 0).
  uint32_t wsc[FN], asc[FM];
  // MX codes via buffer loads as well: rows past M / N read zero codes (never stored).
  const OperandWindow wcw = MODE == MODE_MX ? operand_window(n_base + (wave_u >> 1) * 128, g.N, g.ld_sb) : OperandWindow{0, 0};
  const OperandWindow acw = MODE == MODE_MX ? operand_window(m_base + (wave_u & 1) * 128, g.M, g.ld_sa) : OperandWindow{0, 0};
  const __amdgpu_buffer_rsrc_t wcode_rsrc = uniform_rsrc(reinterpret_cast<const uint8_t*>(g.sb) + wcw.base_offset, wcw.records);
  const __amdgpu_buffer_rsrc_t acode_rsrc = uniform_rsrc(reinterpret_cast<const uint8_t*>(g.sa) + acw.base_offset, acw.records);
  auto load_mx_codes = [&](int kt) {
    if constexpr (MODE == MODE_MX) {
#pragma unroll
      for (int i = 0; i < FN; ++i)
        wsc[i] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(wcode_rsrc, (int)((i * 32 + frow) * g.ld_sb), kt * 4, 0);
#pragma unroll
      for (int j = 0; j < FM; ++j)
        asc[j] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(acode_rsrc, (int)((j * 32 + frow) * g.ld_sa), kt * 4, 0);
    }
  };

  // Declaring an AGPR clobber makes the compiler select the AGPR form of the MFMAs,
  // so the 256 accumulators live in the accumulation registers and the 256
  // architectural VGPRs stay free for fragments and addresses.
  asm volatile("" ::: "a255");
  v16f acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // One K step from `cur` while the next step's loads stream into `nxt`. Fragments
  // are double-buffered: the 64-K half ks+1 is read from LDS while the 16 MFMAs of
  // half ks execute.
  //
  // The body has no branches: the next step's loads are issued unconditionally (the
  // last step re-loads itself into the buffer nobody reads again), so the whole loop
  // body is one basic block and the MFMAs cannot be moved below the barrier.
  auto stage = [&](int kt, const uint8_t* cur, uint8_t* nxt) {
    const int kn = kt + 1 < nk ? kt + 1 : kt;
    uint32_t wcur[FN], acur[FM];
#pragma unroll
    for (int i = 0; i < FN; ++i) wcur[i] = wsc[i];
#pragma unroll
    for (int j = 0; j < FM; ++j) acur[j] = asc[j];
    issue_stage(kn, nxt);
    load_mx_codes(kn);
    // Keep the next step's loads at the top of the step (the scheduler would otherwise
    // sink them next to the barrier that waits for them).
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < BK / 64; ++ks) {
      v8i af[FM], wf[FN];
#pragma unroll
      for (int j = 0; j < FM; ++j) af[j] = frag(cur, kBigTile + wm * 128 + j * 32, ks);
#pragma unroll
      for (int i = 0; i < FN; ++i) wf[i] = frag(cur, wn * 128 + i * 32, ks);
      const int shift = 8 * (ks * 2 + h);
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        const int sw = MODE == MODE_MX ? (int)((wcur[i] >> shift) & 0xFF) : kScaleOne;
#pragma unroll
        for (int j = 0; j < FM; ++j) {
          const int sa = MODE == MODE_MX ? (int)((acur[j] >> shift) & 0xFF) : kScaleOne;
          acc[i][j] = mfma(wf[i], af[j], acc[i][j], sw, sa);
        }
      }
    }
    // MFMAs touch no memory, so the compiler may sink them below the barrier, whose
    // wait for all loads would then stall on the loads just issued for the next step
    // before any MFMA of this step. Pin them above it.
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
  };

  // The loop body is the unconditional pair of steps (lds0, lds1): a conditional
  // second step would make the accumulators a phi across a branch, and the compiler
  // then copies all 256 of them between AGPRs and VGPRs every iteration. An odd step
  // count peels the first step, staged in lds1.
  const int k0 = nk & 1;
  issue_stage(0, k0 ? lds1 : lds0);
  load_mx_codes(0);
  __syncthreads();
  if (k0) stage(0, lds1, lds0);
  for (int kt = k0; kt < nk; kt += 2) {
    stage(kt, lds0, lds1);
    stage(kt + 1, lds1, lds0);
  }

  // The last step's barrier guarantees no wavefront still reads lds0 / lds1 and every
  // direct load has landed (the last issue re-loaded a step into the idle buffer).
  big_epilogue<MODE>(g, acc, BigScales{}, m_base, n_base, lds0);
}

// Compute units of the current device (cached per device): the persistent pair
// kernel launches at most this many workgroups, one per CU.
int cu_count() {
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 8) n = 256;
    cached[dev] = n & ~7;  // a multiple of 8 keeps item i on XCD i mod 8
  }
  return cached[dev];
}

// Persistent grid of the pair kernel for `items` work items.
unsigned pair_grid(int64_t items) {
  const int64_t cus = cu_count();
  return (unsigned)(items < cus ? items : cus);
}

// The pair kernel over all K, with the tail split when the plan has one (whole rounds
// of tiles, then the last round's tiles in K pieces and their fixed-order reduce).
template <int MODE>
int launch_pair_tail(GemmArgs g, int64_t tiles, hipStream_t st, const char* op) {
  const TailPlan tp = tail_plan(g.M, g.N, g.K, MODE == MODE_MX);
  g.kps = 0;
  g.dp_tiles = tp.dp_tiles;
  g.tail_split = tp.split;
  note_plan("pair tail=%d", tp.split);
  if (tp.split == 1) {
    g.items = (int)tiles;
    hipLaunchKernelGGL((fp8_gemm_pair_kernel<MODE>), dim3(pair_grid(tiles)), dim3(kThreads), 0, st, g);
    return check_launch(op);
  }
  const size_t need = tail_workspace(tp);
  if (g.ws == nullptr || g.ws_bytes < need)
    return fail(AYK_EWORKSPACE, "%s: workspace of %zu bytes required, %zu given", op, need, g.ws_bytes);
  const int64_t items = (int64_t)tp.dp_tiles + (int64_t)tp.tail_tiles * tp.split;
  g.items = (int)items;
  hipLaunchKernelGGL((fp8_gemm_pair_kernel<MODE>), dim3(pair_grid(items)), dim3(kThreads), 0, st, g);
  if (int rc = check_launch(op)) return rc;
  const int64_t threads = (int64_t)tp.tail_tiles * kBigTile * kBigTile / 4;
  hipLaunchKernelGGL(tail_split_reduce, dim3((unsigned)cdiv(threads, 256)), dim3(256), 0, st, g.ws, tp.tail_tiles,
                     tp.split, tp.dp_tiles, g.tiles_m, (int)cdiv(g.N, kBigTile), g.M, g.N, g.bias, g.bias_dtype, g.out,
                     g.out_dtype, g.ldo);
  return check_launch(op);
}

template <int MODE>
int launch_big(GemmArgs g, hipStream_t st, const char* op) {
  static_assert(MODE != MODE_BLOCK, "block scales use the general kernel");
  g.tiles_m = (int)cdiv(g.M, kBigTile);
  const int64_t tiles = (int64_t)g.tiles_m * cdiv(g.N, kBigTile);
  if (tiles > 0x7FFFFFFF) return fail(AYK_EINVAL, "%s: problem too large", op);
  if constexpr (MODE == MODE_MX) {
    if (g.K % 512 == 0 && g.ld_sa % 16 == 0 && g.ld_sb % 16 == 0 && aligned16(g.sa) && aligned16(g.sb)) {
      // K per split in whole chunks of four 128-K pairs (keeps the code rows 16-byte aligned)
      const int64_t planned = xcd_pieces(scaled_split(g.M, g.N, g.K, kBigTile, kBigTile));
      const int64_t kps = planned > 1 ? cdiv(g.K / 512, planned) * 512 : g.K;
      const int64_t split = cdiv(g.K, kps);
      g.kps = split > 1 ? kps : 0;
      if (split > 1) {
        const size_t need = (size_t)split * (size_t)g.M * (size_t)g.N * sizeof(float);
        if (g.ws == nullptr || g.ws_bytes < need)
          return fail(AYK_EWORKSPACE, "%s: workspace of %zu bytes required, %zu given", op, need, g.ws_bytes);
      }
      if (split == 1) return launch_pair_tail<MODE>(g, tiles, st, op);
      note_plan("pair split=%d", (int)split);
      g.items = (int)tiles;  // one item per workgroup, piece-major
      g.kpieces = (int)split;
      hipLaunchKernelGGL((fp8_gemm_pair_kernel<MODE>), dim3((unsigned)(tiles * split)), dim3(kThreads), 0, st, g);
      if (int rc = check_launch(op)) return rc;
      launch_split_reduce(block_split_reduce, g.ws, g.M, g.N, (int)split, g.bias, g.bias_dtype, g.out, g.out_dtype,
                          g.ldo, st);
    } else {
      note_plan("mx128");
      hipLaunchKernelGGL((fp8_gemm_mx128_kernel<MODE>), dim3((unsigned)tiles), dim3(kThreads), 0, st, g);
    }
  } else if (g.K % (2 * kBigK) == 0) {
    // INT8 never splits: a split's partial would leave the exact int32 accumulator.
    const int64_t planned = MODE == MODE_SCALED ? xcd_pieces(scaled_split(g.M, g.N, g.K, kBigTile, kBigTile)) : 1;
    g.kps = planned > 1 ? scaled_kps(g.K, planned) : 0;
    const int64_t split = planned > 1 ? cdiv(g.K, g.kps) : 1;
    if (split > 1) {
      const size_t need = (size_t)split * (size_t)g.M * (size_t)g.N * sizeof(float);
      if (g.ws == nullptr || g.ws_bytes < need)
        return fail(AYK_EWORKSPACE, "%s: workspace of %zu bytes required, %zu given", op, need, g.ws_bytes);
    }
    if (split == 1 && MODE == MODE_SCALED) return launch_pair_tail<MODE>(g, tiles, st, op);
    note_plan("pair split=%d", (int)split);
    g.items = (int)tiles;
    g.kpieces = split > 1 ? (int)split : 0;  // piece-major, one item per workgroup
    hipLaunchKernelGGL((fp8_gemm_pair_kernel<MODE>), dim3(split > 1 ? (unsigned)(tiles * split) : pair_grid(tiles)),
                       dim3(kThreads), 0, st, g);
    if (split > 1) {
      if (int rc = check_launch(op)) return rc;
      launch_split_reduce(block_split_reduce, g.ws, g.M, g.N, (int)split, g.bias, g.bias_dtype, g.out, g.out_dtype,
                          g.ldo, st);
    }
  } else {
    note_plan("big");
    hipLaunchKernelGGL((fp8_gemm_big_kernel<MODE>), dim3((unsigned)tiles), dim3(kThreads), 0, st, g);
  }
  return check_launch(op);
}

int launch_block_big(GemmArgs g, hipStream_t st, const char* op) {
  g.tiles_m = (int)cdiv(g.M, kBlkTile);
  const int64_t tiles = (int64_t)g.tiles_m * cdiv(g.N, kBlkTile);
  if (tiles > 0x7FFFFFFF) return fail(AYK_EINVAL, "%s: problem too large", op);
  const int64_t split = block_split(g.M, g.N, g.K);
  note_plan("block128 split=%d", (int)split);
  if (split == 1) {
    hipLaunchKernelGGL(fp8_gemm_block_kernel, dim3((unsigned)tiles), dim3(kBlkThreads), 0, st, g);
    return check_launch(op);
  }
  const size_t need = block_split_workspace(g.M, g.N, g.K);
  if (g.ws == nullptr || g.ws_bytes < need)
    return fail(AYK_EWORKSPACE, "%s: workspace of %zu bytes required, %zu given", op, need, g.ws_bytes);
  hipLaunchKernelGGL(fp8_gemm_block_split_kernel, dim3((unsigned)tiles, (unsigned)split), dim3(kBlkThreads), 0, st, g,
                     g.K / split, g.ws);
  if (int rc = check_launch(op)) return rc;
  launch_split_reduce(block_split_reduce, g.ws, g.M, g.N, (int)split, g.bias, g.bias_dtype, g.out, g.out_dtype,
                          g.ldo, st);
  return check_launch(op);
}

template <int MODE, int BN, int BM, int WN, int WM>
int launch_cfg(GemmArgs g, hipStream_t st, const char* op) {
  g.tiles_m = (int)cdiv(g.M, BM);
  const int64_t tiles = (int64_t)g.tiles_m * cdiv(g.N, BN);
  if (tiles > 0x7FFFFFFF) return fail(AYK_EINVAL, "%s: problem too large", op);
  const int64_t split = MODE == MODE_BLOCK ? (BM <= 64 ? general_split(g.M, g.N, g.K) : 1)
                        : (MODE == MODE_INT8 ? 1 : scaled_split(g.M, g.N, g.K, BM, BN));
  g.kps = 0;
  if (split > 1) {
    const size_t need = (size_t)split * (size_t)g.M * (size_t)g.N * sizeof(float);
    if (g.ws == nullptr || g.ws_bytes < need)
      return fail(AYK_EWORKSPACE, "%s: workspace of %zu bytes required, %zu given", op, need, g.ws_bytes);
    g.kps = MODE == MODE_BLOCK ? g.K / split : scaled_kps(g.K, split);
  }
  note_plan("general %dx%d split=%d", BM, BN, (int)split);
  hipLaunchKernelGGL((fp8_gemm_kernel<MODE, BN, BM, WN, WM>), dim3((unsigned)tiles, (unsigned)split), dim3(kThreads), 0, st, g);
  if (int rc = check_launch(op)) return rc;
  if (split > 1) {
    launch_split_reduce(block_split_reduce, g.ws, g.M, g.N, (int)split, g.bias, g.bias_dtype, g.out, g.out_dtype,
                          g.ldo, st);
    return check_launch(op);
  }
  return AYK_OK;
}

// The 256 x 256 block-scaled kernel serves launches of at least half a round (128) of
// its tiles; smaller ones keep the 128 x 128 tiles and their K split.
bool block256_wanted(int64_t M, int64_t N, int64_t K) {
  return K % 128 == 0 && M >= 256 && N >= 256 && cdiv(M, 256) * cdiv(N, 256) >= 16;
}
Block256Args block256_args(const GemmArgs& g) {
  Block256Args b{};
  b.a = g.a; b.lda = g.lda;
  b.w = g.w; b.ldw = g.ldw;
  b.M = g.M; b.N = g.N; b.K = g.K;
  b.sa = static_cast<const float*>(g.sa);
  b.ld_sa = g.sa_vec ? g.M : (g.ld_sa > 0 ? g.ld_sa : g.K / 128);
  b.sa_col_major = g.sa_vec;
  b.sb = g.sb; b.sb_dtype = g.sb_dtype;
  b.ld_sb = g.ld_sb > 0 ? g.ld_sb : cdiv(g.K, 128);
  b.bias = g.bias; b.bias_dtype = g.bias_dtype;
  b.out = g.out; b.out_dtype = g.out_dtype; b.ldo = g.ldo;
  b.ws = g.ws; b.ws_bytes = g.ws_bytes;
  return b;
}

SkinnyFp8Args skinny_args(const GemmArgs& g, int mode) {
  SkinnyFp8Args k{};
  k.mode = mode;
  k.a = g.a; k.lda = g.lda; k.w = g.w; k.ldw = g.ldw;
  k.M = g.M; k.N = g.N; k.K = g.K;
  k.sa = g.sa; k.sa_vec = g.sa_vec; k.ld_sa = g.ld_sa;
  k.sb = g.sb; k.sb_vec = g.sb_vec; k.ld_sb = g.ld_sb;
  k.bias = g.bias; k.bias_dtype = g.bias_dtype;
  k.out = g.out; k.out_dtype = g.out_dtype; k.ldo = g.ldo;
  k.ws = g.ws; k.ws_bytes = g.ws_bytes;
  if (mode == 2) {  // block-128 tables: default row strides as the block kernels
    k.ld_sa = g.ld_sa > 0 ? g.ld_sa : g.K / 128;
    k.ld_sb = g.ld_sb > 0 ? g.ld_sb : cdiv(g.K, 128);
  }
  return k;
}

template <int MODE>
int launch_gemm(const GemmArgs& g, hipStream_t st, const char* op) {
  // The large-tile kernels need K % 64 == 0 (128 for MXFP8), fp32 scales, N % 4 == 0 and 16-byte
  // aligned output rows (its epilogue stores 16-byte chunks); anything else runs the
  // general kernel.
  if constexpr (MODE != MODE_BLOCK) {
  const int64_t out_bytes = g.out_dtype == AYK_F32 ? 4 : 2;
  // (256 rows of the output, and of an fp32 partial [M, N], within 2 GB: the pair
  // kernel's epilogue addresses a tile with 32-bit offsets.)
  const bool big_ok = g.K % (MODE == MODE_MX ? BK : kBigK) == 0 && g.M >= 256 && g.N >= 256 && g.N % 4 == 0 &&
                      (g.ldo * out_bytes) % 16 == 0 && aligned16(g.out) && g.ldo < (1 << 21) && g.N < (1 << 21) &&
                      (MODE == MODE_MX || (g.sa_dtype == AYK_F32 && g.sb_dtype == AYK_F32 &&
                                           (!g.sb_vec || aligned16(g.sb)))) &&
                      (g.bias == nullptr || (reinterpret_cast<uintptr_t>(g.bias) & 15) == 0);
  if (big_ok) return launch_big<MODE>(g, st, op);
  } else {
    // The 256 x 256 block-scaled kernel from half a round of its tiles on.
    if (g.sa_dtype == AYK_F32 && block256_wanted(g.M, g.N, g.K)) {
      const Block256Args b = block256_args(g);
      if (block256_supported(b)) return block256_launch(b, st, op);
    }
    // The block-scaled 128 x 128 kernel: K % 128 == 0, fp32 activation scales, any float
    // weight-scale dtype, and the same output / bias alignment as above.
    const int64_t out_bytes = g.out_dtype == AYK_F32 ? 4 : 2;
    // 65-127 rows also take it when the K split applies (rows past M read zeros); up to
    // 64 rows the general kernel's 32- / 64-row tiles split K instead.
    const bool big_ok = g.K % 128 == 0 && (g.M >= kBlkTile || (g.M > 64 && block_split(g.M, g.N, g.K) > 1)) && g.N >= kBlkTile &&
                        g.N % 4 == 0 && g.sa_dtype == AYK_F32 &&
                        (g.ldo * out_bytes) % 16 == 0 && aligned16(g.out) &&
                        (g.bias == nullptr || (reinterpret_cast<uintptr_t>(g.bias) & 15) == 0);
    if (big_ok) return launch_block_big(g, st, op);
  }
  // Decode batches (M <= 64) with fp32 or UE8M0 scales: the weight-streaming kernel
  // (gemm_skinny.hip) where its shape and alignment rules hold.
  if constexpr (MODE == MODE_SCALED || MODE == MODE_MX || MODE == MODE_BLOCK) {
    if (g.M <= 64 && (MODE == MODE_MX || (g.sa_dtype == AYK_F32 && g.sb_dtype == AYK_F32))) {
      const SkinnyFp8Args sk = skinny_args(g, MODE == MODE_MX ? 1 : (MODE == MODE_BLOCK ? 2 : 0));
      if (skinny_fp8_supported(sk)) return skinny_fp8_launch(sk, st, op);
    }
  }
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


size_t ayk_fp8_scaled_mm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || N < 1 || K < 1) return 0;
  const size_t split = scaled_split_workspace(M, N, K);
  const size_t tail = M >= kBigTile && N >= kBigTile ? tail_workspace(tail_plan(M, N, K, false)) : 0;
  const size_t skinny = skinny_fp8_workspace(M, N, K, 0);
  return split > tail ? (split > skinny ? split : skinny) : (tail > skinny ? tail : skinny);
}

int ayk_fp8_scaled_mm(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t M, int64_t N,
                      int64_t K, const void* scale_a, int sa_dtype, int sa_per_row,
                      const void* scale_b, int sb_dtype, int sb_per_col, const void* bias,
                      int bias_dtype, void* out, int out_dtype, int64_t ldo, void* workspace,
                      size_t workspace_bytes, ayk_stream_t stream) {
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
  g.ws = static_cast<float*>(workspace); g.ws_bytes = workspace_bytes;
  return launch_gemm<MODE_SCALED>(g, static_cast<hipStream_t>(stream), op);
}

int ayk_fp8_rowwise_linear_small(const void* x, int x_dtype, int64_t ldx, int64_t M, const void* w, int64_t ldw,
                                 int64_t N, int64_t K, const float* scale_b, int sb_per_col, const void* bias,
                                 int bias_dtype, void* out, int out_dtype, int64_t ldo, ayk_stream_t stream) {
  const char* op = "fp8_rowwise_linear_small";
  if (M < 0 || N < 0 || K < 1) return fail(AYK_EINVAL, "%s: bad shape", op);
  if (!x || !w || !scale_b || !out) return fail(AYK_EINVAL, "%s: missing operand", op);
  if (!is_float_dtype(out_dtype) || (bias && !is_float_dtype(bias_dtype)) || ldo < N)
    return fail(AYK_EINVAL, "%s: bad output or bias", op);
  if (M == 0 || N == 0) return AYK_OK;
  SkinnyFp8Args g{};
  g.mode = 0;
  g.w = static_cast<const uint8_t*>(w);
  g.ldw = ldw;
  g.M = M; g.N = N; g.K = K;
  g.sa_vec = 1;
  g.sb = scale_b; g.sb_vec = sb_per_col;
  g.bias = bias; g.bias_dtype = bias_dtype;
  g.out = out; g.out_dtype = out_dtype; g.ldo = ldo;
  if (!rows_gemv_quant_supported(g, x_dtype, ldx, x))
    return fail(AYK_EINVAL, "%s: needs 2-8 rows, N * K <= 2^24, K %% 16 == 0, M * K <= 64 KiB and 16-byte aligned rows", op);
  if (int rc = check_device()) return rc;
  return rows_gemv_quant_launch(g, x, x_dtype, ldx, static_cast<hipStream_t>(stream), op);
}

size_t ayk_int8_scaled_mm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  (void)M; (void)N; (void)K;
  return 0;  // the INT8 GEMM never splits K (its int32 sums stay exact)
}

int ayk_int8_scaled_mm(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t M, int64_t N,
                       int64_t K, const float* scale_a, const float* scale_b, const void* bias,
                       int bias_dtype, void* out, int out_dtype, int64_t ldo, void* workspace, size_t workspace_bytes,
                       ayk_stream_t stream) {
  const char* op = "int8_scaled_mm";
  if (int rc = check_common(op, a, lda, b, ldb, M, N, K, bias, bias_dtype, out_dtype, ldo)) return rc;
  if ((M > 0 && scale_a == nullptr) || (N > 0 && scale_b == nullptr)) return fail(AYK_EINVAL, "%s: scale_a / scale_b are required", op);
  if (M == 0 || N == 0) return AYK_OK;
  if (int rc = check_device()) return rc;
  GemmArgs g{};
  g.a = static_cast<const uint8_t*>(a);
  g.lda = lda;
  g.w = static_cast<const uint8_t*>(b);
  g.ldw = ldb;
  g.M = M; g.N = N; g.K = K;
  g.sa = scale_a; g.sa_dtype = AYK_F32; g.sa_vec = 1;
  g.sb = scale_b; g.sb_dtype = AYK_F32; g.sb_vec = 1;
  g.bias = bias; g.bias_dtype = bias_dtype;
  g.out = out; g.out_dtype = out_dtype; g.ldo = ldo;
  g.ws = static_cast<float*>(workspace); g.ws_bytes = workspace_bytes;
  return launch_gemm<MODE_INT8>(g, static_cast<hipStream_t>(stream), op);
}

size_t ayk_fp8_blockwise_mm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || N < 1 || K < 1 || K % 128) return 0;
  const size_t split = block_split_workspace(M, N, K);
  const size_t skinny = skinny_fp8_workspace(M, N, K, 2);
  return split > skinny ? split : skinny;
}

int ayk_fp8_blockwise_mm(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t M,
                         int64_t N, int64_t K, const void* scale_a, int sa_dtype, int sa_col_major,
                         const void* scale_b, int sb_dtype, const void* bias, int bias_dtype,
                         void* out, int out_dtype, int64_t ldo, void* workspace, size_t workspace_bytes,
                         ayk_stream_t stream) {
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
  g.ws = static_cast<float*>(workspace); g.ws_bytes = workspace_bytes;
  return launch_gemm<MODE_BLOCK>(g, static_cast<hipStream_t>(stream), op);
}

// MoE grouped block-128 GEMM: expert e owns activation rows [off_e, off_e + M_e) of
// a [M_total, K] and weights b[e] = [N, K] (memory [E][N][K]); scales are fp32,
// [M_total, K/128] per row and 128-K block for the activations, [E][N/128][K/128] for
// the weights. The 256 x 256 block-128 kernel's grouped form (gemm_block.hip) takes one
// tile of one expert per workgroup; the launch is an upper bound on the tile count (no
// host synchronisation).
int ayk_fp8_grouped_blockwise_mm(const void* a, const void* b, const float* scales_a, const float* scales_a_t,
                                 const float* scales_b,
                                 const int32_t* problem_sizes, const int32_t* expert_offsets, int64_t num_experts,
                                 int64_t m_total, int64_t n, int64_t k, void* out, int out_dtype,
                                 ayk_stream_t stream) {
  const char* op = "fp8_blockwise_scaled_grouped_mm";
  if (num_experts < 0 || m_total < 0 || n < 0 || k < 0)
    return fail(AYK_EINVAL, "%s: bad shape experts=%lld M=%lld N=%lld K=%lld", op, (long long)num_experts,
                (long long)m_total, (long long)n, (long long)k);
  if (n % 128 || k % 128) return fail(AYK_EINVAL, "%s: N and K must be multiples of 128", op);
  if (out_dtype != AYK_BF16 && out_dtype != AYK_F16) return fail(AYK_EINVAL, "%s: output must be bfloat16 or half", op);
  if (num_experts > (1 << 20)) return fail(AYK_EINVAL, "%s: too many experts", op);
  if (num_experts == 0 || m_total == 0 || n == 0 || k == 0) return AYK_OK;
  if (!a || !b || !scales_a || !scales_b || !problem_sizes || !expert_offsets || !out)
    return fail(AYK_EINVAL, "%s: missing operand", op);
  if (!aligned16(a) || !aligned16(b) || !aligned16(out) || (reinterpret_cast<uintptr_t>(scales_a) & 3) ||
      (reinterpret_cast<uintptr_t>(scales_b) & 3) || (reinterpret_cast<uintptr_t>(scales_a_t) & 3))
    return fail(AYK_EINVAL, "%s: operands must be 16-byte aligned (scales 4-byte)", op);
  if (k > 0x7FFFFFFF || n * k > ((int64_t)1 << 31)) return fail(AYK_EINVAL, "%s: expert weight too large", op);
  if (int rc = check_device()) return rc;
  Grouped256Args gb{};
  gb.a = static_cast<const uint8_t*>(a);
  gb.b = static_cast<const uint8_t*>(b);
  gb.sa = scales_a;
  gb.sa_t = scales_a_t;
  gb.sb = scales_b;
  gb.out = out;
  gb.out_dtype = out_dtype;
  gb.problem_sizes = problem_sizes;
  gb.expert_offsets = expert_offsets;
  gb.num_experts = (int)num_experts;
  gb.m_total = m_total;
  gb.n = n;
  gb.k = k;
  return grouped_block256_launch(gb, static_cast<hipStream_t>(stream), op);
}

size_t ayk_mxfp8_scaled_mm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || N < 1 || K < 1) return 0;
  const size_t split = scaled_split_workspace(M, N, K);
  const size_t tail = M >= kBigTile && N >= kBigTile ? tail_workspace(tail_plan(M, N, K, true)) : 0;
  const size_t skinny = skinny_fp8_workspace(M, N, K, 1);
  return split > tail ? (split > skinny ? split : skinny) : (tail > skinny ? tail : skinny);
}

int ayk_mxfp8_scaled_mm(const void* a, int64_t lda, const uint8_t* a_scale, int64_t ld_as,
                        const void* w, int64_t ldw, const uint8_t* w_scale, int64_t ld_ws,
                        int64_t M, int64_t N, int64_t K, const void* bias, int bias_dtype,
                        void* out, int out_dtype, int64_t ldo, void* workspace, size_t workspace_bytes,
                        ayk_stream_t stream) {
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
  g.ws = static_cast<float*>(workspace); g.ws_bytes = workspace_bytes;
  return launch_gemm<MODE_MX>(g, static_cast<hipStream_t>(stream), op);
}

}  // extern "C"
