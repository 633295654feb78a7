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

#include <utility>

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

// ---------------------------------------------------------------------------------
// Decode W8A16 for 2 <= M <= 32: HBM-bound, so the design is the GEMV's (stream each
// weight byte once with 16-byte loads, fill the CUs with a K split) with the M
// activation rows multiplied on matrix cores instead of VALU FMAs.
//
// A workgroup of four wavefronts owns 128 weight rows over one K range. Its
// activation slice x[0:M, K range] (and, for block scales, the scales of its rows
// and K range) is staged once in LDS, so that inside the main loop only weight loads
// use the vector-memory counter: that counter retires in issue order, so any other
// global load issued behind the weight prefetch would have to wait for it.
//
// A wavefront owns 32 rows. Per 128-K step a lane loads four 16-byte pieces of its row
// (lane half h = lane / 32 takes bytes 32c + 16h .. +16 of row lane % 32, c = 0..3);
// D steps are in flight in a register ring. The loads are ordinary (L2-allocating):
// one instruction covers only 32 bytes of each of 32 rows, and the four instructions
// of a step complete each 128-byte line in L2, where a streaming hint would send the
// pieces to HBM separately (measured: ~1.8x slower). Each weight is dequantized (w * scale)
// and rounded to the activation dtype before the product, as the reference's W8A16
// kernel does, and feeds v_mfma_f32_32x32x16_{bf16,f16} as A, against B = the
// activation rows read from LDS in the same K order (B columns m >= M repeat row
// M - 1 and their D columns are never stored). K-split partials [split, M, N] are
// summed in a fixed order by the reduce kernel.

// s_waitcnt with only the vector-memory count constrained (gfx9 encoding: vmcnt in
// bits [3:0] and [15:14], expcnt [6:4] and lgkmcnt [11:8] left at their maxima).
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

constexpr int kSkRows = 128;          // weight rows per workgroup (32 per wavefront)
constexpr int kSkThreads = kSkRows * 2;  // 64 lanes per 32 rows
constexpr int kSkLdsBudget = 80 * 1024;  // two workgroups per CU

// LDS bytes of the staged activation slice (`pitch` elements per row): whole
// 64-vector groups, the unit of one direct-to-LDS wavefront load.
__host__ __device__ inline size_t x_lds_bytes(int64_t M, int pitch) {
  return (size_t)((M * (pitch / 8) + 63) / 64) * 64 * 16;
}

struct SkinnyArgs {
  const uint16_t* x;
  int64_t ldx;
  int64_t M;
  const uint8_t* w;
  int64_t ldw;
  int64_t N, K;
  const void* scale;
  int scale_dtype;
  int64_t srs, by, bx;
  uint16_t* out;
  int64_t ldo;
  float* part;          // [split, M, N] when gridDim.y > 1
  int64_t k_per_split;  // multiple of D * 128
  int x_pitch;          // LDS row pitch of the activation slice, elements
  int s_cols;           // LDS scale columns per row (block scales)
};

// Eight e4m3 bytes (two dwords) -> the eight products w * s rounded to 16-bit floats.
template <bool BF16>
__device__ inline v8s convert8(uint32_t lo, uint32_t hi, float s) {
  float f[8];
  e4m3x4_to_f32(lo, f);
  e4m3x4_to_f32(hi, f + 4);
  v8s r;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float v = f[e] * s;
    if constexpr (BF16) r[e] = (short)__builtin_bit_cast(uint16_t, (__bf16)v);
    else r[e] = (short)__builtin_bit_cast(uint16_t, (_Float16)v);
  }
  return r;
}

template <bool BF16, bool ROW_SCALE, int D>
__global__ __launch_bounds__(kSkThreads) void w8a16_skinny_kernel(SkinnyArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t sk_lds[];
  uint16_t* xs = reinterpret_cast<uint16_t*>(sk_lds);
  float* ss = reinterpret_cast<float*>(sk_lds + x_lds_bytes(a.M, a.x_pitch));
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, lr = lane & 31;
  const int64_t nwg = (int64_t)blockIdx.x * kSkRows;
  const int64_t n0 = nwg + wave * 32;
  const int64_t kbeg = (int64_t)blockIdx.y * a.k_per_split;
  const int64_t kend = min(a.K, kbeg + a.k_per_split);
  const int klen = (int)(kend - kbeg);

  const int64_t nrow = min(n0 + lr, a.N - 1);  // rows past N re-read row N - 1
  const uint8_t* wrow = a.w + nrow * a.ldw + h * 16;
  uint4 ring[D][4];
  auto load = [&](int d, int64_t k) {
#pragma unroll
    for (int c = 0; c < 4; ++c) ring[d][c] = *reinterpret_cast<const uint4*>(wrow + k + c * 32);
  };

  // Start-up order. The vector-memory counter retires in issue order, so a wait on any
  // load issued behind the weight ring would wait for the whole ring (and a wait the
  // compiler cannot place exactly lands inside the K loop, draining the ring on every
  // iteration). So: (1) the activation slice goes to LDS with direct-to-LDS loads;
  // (2) the scales: a per-row scale as the raw dword that holds it (converted after the
  // barrier), or the block-scale table, staged in LDS before any weight load is in
  // flight; (3) the first D weight steps; (4) one wait for "all but the ring" and a
  // workgroup barrier.
  //
  // (1) Vector p of the padded layout holds x[p / pv][kbeg + 8 * (p % pv) ..] (pv =
  // klen / 8 + 1 vectors per row, the last one padding, which - like vectors past the
  // last row - is filled from a clamped, valid address).
  {
    const int pv = a.x_pitch / 8, vpr = klen / 8;
    const int total = (int)a.M * pv;
    for (int p0 = wave * 64; p0 < total; p0 += kSkThreads) {
      const int p = min(p0 + lane, total - 1);
      const int m = p / pv, c = min(p - m * pv, vpr - 1);
      __builtin_amdgcn_global_load_lds(
          reinterpret_cast<const void*>(a.x + m * a.ldx + kbeg + c * 8),
          (__attribute__((address_space(3))) void*)(sk_lds + (size_t)__builtin_amdgcn_readfirstlane(p0) * 16), 16, 0, 0);
    }
  }
  // (2)
  RawBits row_bits{0, 0};
  if constexpr (ROW_SCALE) {
    row_bits = load_bits(a.scale, a.scale_dtype, (int64_t)((uint64_t)nrow / (uint64_t)a.by) * a.srs);
  } else {
    const int64_t c0 = kbeg / a.bx, cmax = (a.K - 1) / a.bx;
    for (int i = tid; i < kSkRows * a.s_cols; i += kSkThreads) {
      const int r = i / a.s_cols, c = i - r * a.s_cols;
      const int64_t n = min(nwg + r, a.N - 1);
      ss[i] = load_f32(a.scale, a.scale_dtype, (n / a.by) * a.srs + min(c0 + c, cmax));
    }
  }
  // (3)
#pragma unroll
  for (int d = 0; d < D; ++d) load(d, kbeg + d * 128);
  // (4)
  wait_vmcnt<4 * D>();
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wavefront's LDS writes are done
  __builtin_amdgcn_s_barrier();
  if (n0 >= a.N) return;  // whole wavefront past N (uniform; no barrier follows)

  const float row_s = ROW_SCALE ? bits_to_f32(row_bits, a.scale_dtype) : 1.0f;
  const uint16_t* xrow = xs + min(lr, (int)a.M - 1) * a.x_pitch + h * 16;
  const float* srow = ss + (wave * 32 + lr) * a.s_cols;
  const uint32_t bx = (uint32_t)a.bx;
  const uint32_t c0 = (uint32_t)(kbeg / a.bx);

  v16f acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
  auto step = [&](int d, int kl) {  // kl: K offset of the step within the slice
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int kc = kl + c * 32;
      const uint4 xa = *reinterpret_cast<const uint4*>(xrow + kc);
      const uint4 xb = *reinterpret_cast<const uint4*>(xrow + kc + 8);
      float s = row_s;
      // 16 consecutive K of a lane share one scale (bx % 32 == 0, checked on the host)
      if constexpr (!ROW_SCALE) s = srow[(uint32_t)(kbeg + kc + h * 16) / bx - c0];
      const v8s w0 = convert8<BF16>(ring[d][c].x, ring[d][c].y, s);
      const v8s w1 = convert8<BF16>(ring[d][c].z, ring[d][c].w, s);
      acc = mfma16<BF16>(w0, __builtin_bit_cast(v8s, xa), acc);
      acc = mfma16<BF16>(w1, __builtin_bit_cast(v8s, xb), acc);
    }
  };

  // klen is a multiple of D * 128: a steady loop that refills every slot it
  // consumes, then a final round without refills.
  int kl = 0;
  for (; kl + D * 128 < klen; kl += D * 128) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      step(d, kl + d * 128);
      load(d, kbeg + kl + (D + d) * 128);
    }
  }
#pragma unroll
  for (int d = 0; d < D; ++d) step(d, kl + d * 128);

  // D[n][m]: lane holds m = lr and n = n0 + 8*(r/4) + 4*h + r%4.
  if (lr >= a.M) return;
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
    const int64_t nb = n0 + grp * 8 + h * 4;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t n = nb + q;
      if (n >= a.N) continue;
      if (gridDim.y == 1) a.out[lr * a.ldo + n] = round16<BF16>(acc[grp * 4 + q]);
      else a.part[((int64_t)blockIdx.y * a.M + lr) * a.N + n] = acc[grp * 4 + q];
    }
  }
}

// Fixed-order sum over the K split, one rounding. Eight partials are loaded before
// any is added (the adds stay in split order), so the loads overlap.
template <bool BF16>
__global__ __launch_bounds__(256) void w8a16_skinny_reduce(SkinnyArgs a, int split) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t mn = a.M * a.N;
  if (i >= mn) return;
  const float* p = a.part + i;
  float v = 0.0f;
  int s = 0;
  for (; s + 8 <= split; s += 8) {
    float t[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) t[j] = p[(int64_t)(s + j) * mn];
#pragma unroll
    for (int j = 0; j < 8; ++j) v += t[j];
  }
  for (; s < split; ++s) v += p[(int64_t)s * mn];
  const int64_t m = i / a.N, n = i - m * a.N;
  a.out[m * a.ldo + n] = round16<BF16>(v);
}

// Launch plan, a function of the shapes and the scale block width only (the
// workspace query must reproduce it). Unless the rows alone give >= 768 wavefronts,
// the K split is the smallest power of two giving
// >= 1024 wavefronts (each keeps D * 4 KiB of weights in flight); more splits cost
// more partial-sum traffic than they gain (measured on Llama-3-8B shapes).
struct SkinnyPlan {
  bool ok;         // shape supported by the skinny kernel
  int depth;       // D: 128-K steps in flight
  int split;       // K split (grid.y)
  int64_t kps;     // K per split, multiple of depth * 128
  int x_pitch;     // elements
  int s_cols;      // 0 for a per-row scale
  size_t lds;      // dynamic LDS bytes
};
SkinnyPlan skinny_plan(int64_t M, int64_t N, int64_t K, int64_t bx) {
  SkinnyPlan p{};
  const bool row_scale = bx >= K;
  if (M < 1 || M > 32 || N < 1 || K < 128 || K % 128 || (!row_scale && bx % 32)) return p;
  p.depth = K % 512 == 0 ? 4 : (K % 256 == 0 ? 2 : 1);
  const int64_t unit = 128 * p.depth, units = K / unit;
  auto lds_for = [&](int64_t kps, int& pitch, int& cols) {
    pitch = (int)kps + 8;  // 16-byte pad: rows start on distinct LDS banks
    cols = row_scale ? 0 : (int)(kps / bx + 2);
    return x_lds_bytes(M, pitch) + (size_t)kSkRows * cols * 4;
  };
  const int64_t waves = cdiv(N, 32);
  int64_t split = 1;
  // A row count that already covers three quarters of the 1024 SIMDs runs unsplit: the
  // partial sums and the reduce launch cost more than the idle quarter (gate_up at M = 4:
  // 28 against 31 us).
  while (waves < 768 && waves * split < 1024 && split * 2 <= units) split *= 2;
  for (;;) {
    const int64_t kps = cdiv(units, split) * unit;
    const size_t lds = lds_for(kps, p.x_pitch, p.s_cols);
    if (lds <= (size_t)kSkLdsBudget) {
      p.kps = kps;
      p.lds = lds;
      p.split = (int)cdiv(K, kps);
      p.ok = true;
      return p;
    }
    if (split >= units) return p;
    split *= 2;
  }
}

size_t skinny_workspace(const SkinnyPlan& p, int64_t M, int64_t N) {
  return p.ok && p.split > 1 ? (size_t)p.split * (size_t)M * (size_t)N * sizeof(float) : 0;
}

template <bool BF16, bool ROW_SCALE>
void launch_skinny_kernel(const SkinnyPlan& p, const SkinnyArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)cdiv(a.N, kSkRows), (unsigned)p.split);
  const unsigned lds = (unsigned)p.lds;
  switch (p.depth) {
    case 4: hipLaunchKernelGGL((w8a16_skinny_kernel<BF16, ROW_SCALE, 4>), grid, dim3(kSkThreads), lds, st, a); break;
    case 2: hipLaunchKernelGGL((w8a16_skinny_kernel<BF16, ROW_SCALE, 2>), grid, dim3(kSkThreads), lds, st, a); break;
    default: hipLaunchKernelGGL((w8a16_skinny_kernel<BF16, ROW_SCALE, 1>), grid, dim3(kSkThreads), lds, st, a); break;
  }
}

template <bool BF16>
int launch_skinny(const SkinnyPlan& p, SkinnyArgs a, size_t ws_bytes, hipStream_t st) {
  a.k_per_split = p.kps;
  a.x_pitch = p.x_pitch;
  a.s_cols = p.s_cols;
  if (p.split > 1) {
    const size_t need = skinny_workspace(p, a.M, a.N);
    if (a.part == nullptr || ws_bytes < need) {
      return fail(AYK_EWORKSPACE, "fp8_weight_only_gemm: workspace of %zu bytes required, %zu given", need, ws_bytes);
    }
  }
  if (p.s_cols == 0) launch_skinny_kernel<BF16, true>(p, a, st);
  else launch_skinny_kernel<BF16, false>(p, a, st);
  if (int rc = check_launch("fp8_weight_only_gemm")) return rc;
  if (p.split > 1) {
    const dim3 rg((unsigned)cdiv(a.M * a.N, 256));
    hipLaunchKernelGGL((w8a16_skinny_reduce<BF16>), rg, dim3(256), 0, st, a, p.split);
    return check_launch("fp8_weight_only_gemm");
  }
  return AYK_OK;
}

// ------------------------------------------------------------ row-stream decode kernel
// Decode batches (M <= 32, K split into whole 256-K stages). A workgroup of four
// wavefronts owns R = 16 RT weight rows and streams them through LDS in stages of
// R rows x 256 K bytes, together with the stage's 256 K of every activation row
// (M rounded up to 8 rows): each direct-to-LDS load instruction moves 4 weight rows x
// 256 contiguous bytes or 2 activation rows x 512 bytes (whole 128-byte lines), the
// stages form a ring of D buffers, and one
// workgroup barrier per stage makes a stage visible and frees the oldest buffer.
// Wavefront w computes 64-K chunk w of every stage for all R rows, so its partial sums
// cover a quarter of K and meet the others' in LDS at the end.
//
// MFMA v_mfma_f32_16x16x32_{bf16,f16}, weight as operand A. Lane (r = lane % 16,
// g = lane / 16) reads 16 weight bytes of row r at K [16 g, 16 g + 16) of its chunk and
// dequantizes them (w * s rounded to the activation dtype, the reference's numerics)
// into two 8-element operands: the chunk's first MFMA sums K {16 g .. 16 g + 7}, the
// second K {16 g + 8 .. 16 g + 15}; operand B takes the same K sets of x from the
// stage (lane (m = lane % 16, g): 32 bytes of x row m at K 16 g). Weight LDS rows are 256 bytes apart, with logical 16-byte chunk c of row r stored at
// physical chunk c ^ (r % 16): the 16 rows of a fragment read fall on distinct banks.
constexpr int kRsWaves = 4;
constexpr int kRsStageK = 256;           // K bytes per stage and row
constexpr int kRsChunk = kRsStageK / kRsWaves;  // 64 K per wavefront per stage

struct RsArgs {
  const uint16_t* x;
  int64_t ldx;
  int64_t M;
  const uint8_t* w;
  int64_t ldw;
  int64_t N, K;
  const void* scale;
  int scale_dtype;
  int64_t srs, by, bx;
  uint16_t* out;
  int64_t ldo;
  float* part;          // [split, M, N] when gridDim.y > 1
  int64_t k_per_split;  // multiple of kRsStageK
};

typedef float v4f __attribute__((ext_vector_type(4)));
// One 16-byte direct-to-LDS load per lane (a device function: the builtin inside a
// lambda of a kernel template loses the kernel's host-side launch stub).
__device__ inline void dma16(const uint8_t* src, uint8_t* lds_dst) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_dst, 16, 0, 0);
}
// One 4-byte direct-to-LDS load per lane (lane i writes lds_dst + 4 i).
__device__ inline void dma4(const uint8_t* src, uint8_t* lds_dst) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_dst, 4, 0, 0);
}
__device__ inline uint32_t lds_addr(const uint8_t* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p;
}
// All LDS reads of one stage in one assembly statement that ends with
// s_waitcnt lgkmcnt(0): NB 16-byte reads into b, NS 4-byte reads into w. The compiler
// cannot relate these reads to the direct-to-LDS loads in flight into other stage
// buffers (it would otherwise wait for every one of them first), and every result
// register is final when the statement ends.
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
#define AYK_R128(o, i) "ds_read_b128 %" #o ", %" #i "\n\t"
#define AYK_R32(o, i) "ds_read_b32 %" #o ", %" #i "\n\t"
template <int NB, int NS>
__device__ inline void stage_reads(v4u (&b)[NB], uint32_t (&w)[NS], const uint32_t (&ab)[NB], const uint32_t (&as)[NS]);
template <>
__device__ inline void stage_reads<3, 1>(v4u (&b)[3], uint32_t (&w)[1], const uint32_t (&ab)[3], const uint32_t (&as)[1]) {
  asm volatile(AYK_R128(0, 4) AYK_R128(1, 5) AYK_R128(2, 6) AYK_R32(3, 7) "s_waitcnt lgkmcnt(0)"
               : "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(w[0])
               : "v"(ab[0]), "v"(ab[1]), "v"(ab[2]), "v"(as[0])
               : "memory");
}
template <>
__device__ inline void stage_reads<5, 1>(v4u (&b)[5], uint32_t (&w)[1], const uint32_t (&ab)[5], const uint32_t (&as)[1]) {
  asm volatile(AYK_R128(0, 6) AYK_R128(1, 7) AYK_R128(2, 8) AYK_R128(3, 9) AYK_R128(4, 10) AYK_R32(5, 11)
               "s_waitcnt lgkmcnt(0)"
               : "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(b[3]), "=&v"(b[4]), "=&v"(w[0])
               : "v"(ab[0]), "v"(ab[1]), "v"(ab[2]), "v"(ab[3]), "v"(ab[4]), "v"(as[0])
               : "memory");
}
template <>
__device__ inline void stage_reads<4, 2>(v4u (&b)[4], uint32_t (&w)[2], const uint32_t (&ab)[4], const uint32_t (&as)[2]) {
  asm volatile(AYK_R128(0, 6) AYK_R128(1, 7) AYK_R128(2, 8) AYK_R128(3, 9) AYK_R32(4, 10) AYK_R32(5, 11)
               "s_waitcnt lgkmcnt(0)"
               : "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(b[3]), "=&v"(w[0]), "=&v"(w[1])
               : "v"(ab[0]), "v"(ab[1]), "v"(ab[2]), "v"(ab[3]), "v"(as[0]), "v"(as[1])
               : "memory");
}
template <>
__device__ inline void stage_reads<6, 2>(v4u (&b)[6], uint32_t (&w)[2], const uint32_t (&ab)[6], const uint32_t (&as)[2]) {
  asm volatile(AYK_R128(0, 8) AYK_R128(1, 9) AYK_R128(2, 10) AYK_R128(3, 11) AYK_R128(4, 12) AYK_R128(5, 13)
               AYK_R32(6, 14) AYK_R32(7, 15) "s_waitcnt lgkmcnt(0)"
               : "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(b[3]), "=&v"(b[4]), "=&v"(b[5]), "=&v"(w[0]), "=&v"(w[1])
               : "v"(ab[0]), "v"(ab[1]), "v"(ab[2]), "v"(ab[3]), "v"(ab[4]), "v"(ab[5]), "v"(as[0]), "v"(as[1])
               : "memory");
}
template <>
__device__ inline void stage_reads<6, 4>(v4u (&b)[6], uint32_t (&w)[4], const uint32_t (&ab)[6], const uint32_t (&as)[4]) {
  asm volatile(AYK_R128(0, 10) AYK_R128(1, 11) AYK_R128(2, 12) AYK_R128(3, 13) AYK_R128(4, 14) AYK_R128(5, 15)
               AYK_R32(6, 16) AYK_R32(7, 17) AYK_R32(8, 18) AYK_R32(9, 19) "s_waitcnt lgkmcnt(0)"
               : "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(b[3]), "=&v"(b[4]), "=&v"(b[5]),
                 "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3])
               : "v"(ab[0]), "v"(ab[1]), "v"(ab[2]), "v"(ab[3]), "v"(ab[4]), "v"(ab[5]),
                 "v"(as[0]), "v"(as[1]), "v"(as[2]), "v"(as[3])
               : "memory");
}
template <>
__device__ inline void stage_reads<8, 4>(v4u (&b)[8], uint32_t (&w)[4], const uint32_t (&ab)[8], const uint32_t (&as)[4]) {
  asm volatile(AYK_R128(0, 12) AYK_R128(1, 13) AYK_R128(2, 14) AYK_R128(3, 15) AYK_R128(4, 16) AYK_R128(5, 17)
               AYK_R128(6, 18) AYK_R128(7, 19) AYK_R32(8, 20) AYK_R32(9, 21) AYK_R32(10, 22) AYK_R32(11, 23)
               "s_waitcnt lgkmcnt(0)"
               : "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(b[3]), "=&v"(b[4]), "=&v"(b[5]), "=&v"(b[6]), "=&v"(b[7]),
                 "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3])
               : "v"(ab[0]), "v"(ab[1]), "v"(ab[2]), "v"(ab[3]), "v"(ab[4]), "v"(ab[5]), "v"(ab[6]), "v"(ab[7]),
                 "v"(as[0]), "v"(as[1]), "v"(as[2]), "v"(as[3])
               : "memory");
}
#undef AYK_R128
#undef AYK_R32
template <bool BF16>
__device__ inline v4f mfma16x16(const v8s& a, const v8s& b, const v4f& c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0, 0);
  }
}

template <bool BF16, bool ROW_SCALE, int RT, int XJ>
__global__ __launch_bounds__(kRsWaves * kWave) void w8a16_rows_kernel(RsArgs a) {
  constexpr int R = 16 * RT;
  constexpr int MP = 8 * XJ;                 // activation rows staged (M rounded up to 8)
  constexpr int MT = MP > 16 ? 2 : 1;        // 16-column MFMA tiles
  constexpr int kWBytes = R * kRsStageK;     // weight part of a stage
  constexpr int kXRow = 2 * kRsStageK;       // bytes of one activation row of a stage
  constexpr int kXBytes = MP * kXRow;
  // Per-stage scale words (block scales only): entry (row, 16-K group) of the stage.
  constexpr int kSBytes = ROW_SCALE ? 0 : R * (kRsStageK / 16) * 4;
  constexpr int kStageBytes = kWBytes + kXBytes + kSBytes;
  constexpr int kDma = R / (4 * kRsWaves);   // weight load instructions per wavefront per stage
  constexpr int kSDma = ROW_SCALE ? 0 : RT;  // scale load instructions per wavefront per stage
  static_assert(R % (4 * kRsWaves) == 0, "whole load instructions per wavefront");
  constexpr int kOps = kDma + XJ + kSDma;  // vector-memory instructions per stage and wavefront
  static_assert(R * (kRsStageK / 16) == kRsWaves * kSDma * kWave || ROW_SCALE, "scale entries per stage");
  constexpr int D = 4;  // stage buffers (a deeper ring measured no faster)
  // Four distinct LDS objects for the ring, and the per-row scale words (lane i of the
  // one load writes word i).
  __shared__ __attribute__((aligned(1024))) uint8_t B0[kStageBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t B1[kStageBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t B2[kStageBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t B3[kStageBytes];
  __shared__ __attribute__((aligned(256))) uint8_t SROW[ROW_SCALE ? 4 * kWave : 4];
  auto stage_buf = [&](int d) -> uint8_t* { return d == 0 ? B0 : (d == 1 ? B1 : (d == 2 ? B2 : B3)); };
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int r16 = lane & 15, g = lane >> 4;
  const int64_t n_base = (int64_t)blockIdx.x * R;
  const int64_t kbeg = (int64_t)blockIdx.y * a.k_per_split;
  const int64_t klen = a.K - kbeg < a.k_per_split ? a.K - kbeg : a.k_per_split;
  const int ns = (int)(klen / kRsStageK);
  const int ssize = a.scale_dtype == AYK_F32 ? 4 : (a.scale_dtype == AYK_U8 ? 1 : 2);
  const uintptr_t sbase = reinterpret_cast<uintptr_t>(a.scale);
  // Scale element i is read as the aligned dword that holds it (in the same page, so
  // always readable) and shifted out after the read.
  auto scale_word = [&](int64_t i) { return reinterpret_cast<const uint8_t*>((sbase + (uintptr_t)(i * ssize)) & ~(uintptr_t)3); };
  auto scale_shift = [&](int64_t i) { return (uint32_t)((sbase + (uintptr_t)(i * ssize)) & 3) * 8; };

  // Weight DMA: load instruction j (0 .. kDma - 1) of wavefront w covers rows
  // 4 (w kDma + j) + lane / 16; lane fetches the logical chunk that lands at physical
  // chunk lane % 16 of its row.
  const uint8_t* dsrc[kDma + XJ];
  int dlds[kDma + XJ];
#pragma unroll
  for (int j = 0; j < kDma; ++j) {
    const int row = 4 * (wave * kDma + j) + (lane >> 4);
    const int64_t n = n_base + row < a.N ? n_base + row : a.N - 1;  // rows past N re-read row N - 1
    const int chunk = (lane & 15) ^ (row & 15);
    dsrc[j] = a.w + n * a.ldw + kbeg + chunk * 16;
    dlds[j] = __builtin_amdgcn_readfirstlane(4 * (wave * kDma + j) * kRsStageK);
  }
  // Activation DMA: instruction j of wavefront w covers activation rows 2 (4 j + w) and
  // 2 (4 j + w) + 1 (512 bytes each: 32 chunks of 16 bytes); logical chunk c of row m
  // sits at physical chunk c ^ 2 (m % 16), so the 16 rows of a fragment read (32
  // contiguous bytes each) fall on distinct banks. Rows past M re-read row M - 1.
#pragma unroll
  for (int j = 0; j < XJ; ++j) {
    const int row = 2 * (4 * j + wave) + (lane >> 5);
    const int64_t m = row < a.M ? row : a.M - 1;
    const int chunk = (lane & 31) ^ ((row & 15) << 1);
    dsrc[kDma + j] = reinterpret_cast<const uint8_t*>(a.x + m * a.ldx + kbeg + chunk * 8);
    dlds[kDma + j] = __builtin_amdgcn_readfirstlane(kWBytes + 2 * (4 * j + wave) * kXRow);
  }
  // Per-stage scale DMA (block scales): instruction j of wavefront w loads entries
  // e = 64 (w kSDma + j) + lane, i.e. row e / 16 and 16-K group e % 16 of the stage.
  int64_t srow_idx[kSDma > 0 ? kSDma : 1];
  int sgrp_k[kSDma > 0 ? kSDma : 1];
#pragma unroll
  for (int j = 0; j < kSDma; ++j) {
    const int e = kWave * (wave * kSDma + j) + lane;
    const int64_t n = n_base + e / 16 < a.N ? n_base + e / 16 : a.N - 1;
    srow_idx[j] = (int64_t)((uint64_t)n / (uint64_t)a.by) * a.srs;
    sgrp_k[j] = 16 * (e % 16);
  }

  // LDS read addresses (relative to the stage buffer) and scale decoding per row tile.
  uint32_t xoff[2 * MT], woff[RT], soff[RT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + r16 < a.M ? 16 * mt + r16 : (int)a.M - 1;  // columns past M repeat row M - 1
    const int c = 2 * (4 * wave + g);
    xoff[2 * mt] = kWBytes + m * kXRow + ((c ^ ((m & 15) << 1)) << 4);
    xoff[2 * mt + 1] = kWBytes + m * kXRow + (((c + 1) ^ ((m & 15) << 1)) << 4);
  }
  int64_t rowbase[RT];
  uint32_t shift[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = 16 * rt + r16;
    woff[rt] = row * kRsStageK + (((4 * wave + g) ^ (row & 15)) << 4);
    const int64_t n = n_base + row < a.N ? n_base + row : a.N - 1;
    rowbase[rt] = (int64_t)((uint64_t)n / (uint64_t)a.by) * a.srs;
    soff[rt] = ROW_SCALE ? 4 * row : kWBytes + kXBytes + 4 * (row * (kRsStageK / 16) + 4 * wave + g);
    shift[rt] = scale_shift(rowbase[rt]);
  }

  if constexpr (ROW_SCALE) {
    // One load by wavefront 0, older than every stage: the first stage's wait and
    // barrier make it visible.
    if (wave == 0) {
      const int row = lane < R ? lane : R - 1;
      const int64_t n = n_base + row < a.N ? n_base + row : a.N - 1;
      dma4(scale_word((int64_t)((uint64_t)n / (uint64_t)a.by) * a.srs), SROW);
    }
  }

  // Stage s (clamped to the last stage: the ring is always full; a clamped stage lands
  // in a buffer that no later stage reads) into ring slot d.
  auto issue = [&](int d, int s) {
    const int sc = s < ns ? s : ns - 1;
    const int64_t ks = (int64_t)sc * kRsStageK;
#pragma unroll
    for (int j = 0; j < kDma; ++j) dma16(dsrc[j] + ks, stage_buf(d) + dlds[j]);
#pragma unroll
    for (int j = 0; j < XJ; ++j) dma16(dsrc[kDma + j] + 2 * ks, stage_buf(d) + dlds[kDma + j]);
#pragma unroll
    for (int j = 0; j < kSDma; ++j) {
      const int64_t i = srow_idx[j] + (uint32_t)(kbeg + ks + sgrp_k[j]) / (uint32_t)a.bx;
      dma4(scale_word(i), stage_buf(d) + kWBytes + kXBytes + __builtin_amdgcn_readfirstlane(4 * kWave * (wave * kSDma + j)));
    }
  };

  v4f acc[RT][MT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[rt][mt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  auto compute = [&](int d, int s) {
    const uint32_t base = lds_addr(stage_buf(d));
    const uint32_t sb = ROW_SCALE ? lds_addr(SROW) : base;
    uint32_t ab[2 * MT + RT], as[RT];
#pragma unroll
    for (int i = 0; i < 2 * MT; ++i) ab[i] = base + xoff[i];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      ab[2 * MT + rt] = base + woff[rt];
      as[rt] = sb + soff[rt];
    }
    v4u v[2 * MT + RT];
    uint32_t sw[RT];
    stage_reads<2 * MT + RT, RT>(v, sw, ab, as);
    uint32_t sh[RT];
    if constexpr (ROW_SCALE) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) sh[rt] = shift[rt];
    } else {
      // 16 consecutive K of a lane share one scale (bx % 16 == 0, checked on the host)
      const int64_t kidx = (uint32_t)(kbeg + (int64_t)s * kRsStageK + 16 * (4 * wave + g)) / (uint32_t)a.bx;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) sh[rt] = scale_shift(rowbase[rt] + kidx);
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const v4u wq = v[2 * MT + rt];
      const float sc = bits_to_f32(RawBits{sw[rt], sh[rt]}, a.scale_dtype);
      const v8s lo = convert8<BF16>(wq[0], wq[1], sc);
      const v8s hi = convert8<BF16>(wq[2], wq[3], sc);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc[rt][mt] = mfma16x16<BF16>(lo, __builtin_bit_cast(v8s, v[2 * mt]), acc[rt][mt]);
        acc[rt][mt] = mfma16x16<BF16>(hi, __builtin_bit_cast(v8s, v[2 * mt + 1]), acc[rt][mt]);
      }
    }
  };

  // Ring: stages 0 .. D - 2 in flight; at stage s, wait for it (D - 2 younger stages may
  // still be in flight), barrier (stage s visible; nobody reads stage s - 1 any more),
  // refill that buffer with stage s + D - 1, compute stage s.
#pragma unroll
  for (int d = 0; d < D - 1; ++d) issue(d, d);
  for (int s0 = 0; s0 < ns; s0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int s = s0 + d;
      if (s < ns) {  // workgroup-uniform
        wait_vmcnt<(D - 2) * kOps>();
        __builtin_amdgcn_s_barrier();
        issue((d + D - 1) % D, s + D - 1);
        compute(d, s);
      }
    }
  }
  wait_vmcnt<0>();
  __syncthreads();

  // Partial sums of the four wavefronts meet in LDS (the ring is free: wavefront w
  // writes stage buffer w); wavefront w finishes tile pairs w, w + 4, ... in a fixed
  // order. D[n][m]: lane holds m = lane % 16 and n = 4 (lane / 16) + r of its 16 x 16 tile.
  static_assert(RT * MT * 4 * kWave * 4 <= kStageBytes, "a wavefront's partials fit one stage buffer");
  auto red_at = [&](int w, int slot) { return reinterpret_cast<float*>(stage_buf(w)) + (slot * kWave + lane); };
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) *red_at(wave, (rt * MT + mt) * 4 + r) = acc[rt][mt][r];
  __syncthreads();
  for (int p = wave; p < RT * MT; p += kRsWaves) {
    const int rt = p / MT, mt = p % MT;
    const int64_t m = 16 * mt + r16;
    const int64_t n0 = n_base + 16 * rt + 4 * g;
    if (m >= a.M) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = *red_at(0, p * 4 + r);
#pragma unroll
      for (int w2 = 1; w2 < kRsWaves; ++w2) v += *red_at(w2, p * 4 + r);
      const int64_t n = n0 + r;
      if (n >= a.N) continue;
      if (gridDim.y == 1) a.out[m * a.ldo + n] = round16<BF16>(v);
      else a.part[((int64_t)blockIdx.y * a.M + m) * a.N + n] = v;
    }
  }
}

template <bool BF16>
__global__ __launch_bounds__(256) void w8a16_rows_reduce(RsArgs a, int split) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t mn = a.M * a.N;
  if (i >= mn) return;
  float v = 0.0f;
  for (int s = 0; s < split; ++s) v += a.part[(int64_t)s * mn + i];
  const int64_t m = i / a.N, n = i - m * a.N;
  a.out[m * a.ldo + n] = round16<BF16>(v);
}

// Launch plan from the shapes alone (the workspace query reproduces it). R = 16 rows
// per workgroup when K is too short to split and those workgroups are one per CU (up
// to 16 activation rows: two per CU); else R = 64 for M > 16 when that still gives
// >= 384 workgroups (the activation stage is then shared by more rows), else 32. K is
// split across workgroups only while
// each split keeps >= 4096 K and there are < 512 workgroups: a split costs a second
// launch and fp32 partials, which measured slower than fewer workgroups at K = 4096
// (Llama-3-8B qkv / o / gate_up) and faster at K = 14336 (down, split 2).
struct RsPlan {
  bool ok;
  int rt, xj, split;  // xj: activation rows staged / 8
  int64_t kps;
};
RsPlan rows_plan(int64_t M, int64_t N, int64_t K, int64_t bx) {
  RsPlan p{};
  const bool row_scale = bx >= K;
  if (M < 2 || M > 32 || N < 1 || K < kRsStageK || K % kRsStageK || K >= (int64_t(1) << 31) || (!row_scale && bx % 16)) return p;
  p.xj = (int)cdiv(M, 8);
  // 16 rows per workgroup re-read the activations more often per weight byte, but the
  // extra workgroups put every CU to work: Llama-3-8B o (K = 4096) at M = 16
  // 9.5 -> 7.3 us, at M = 32 10.9 -> 8.2 us; qkv at M = 16 9.8 -> 8.4 us (at M = 32,
  // 1.5 workgroups per CU, slower); with a K split (down, K = 14336) slower.
  const int64_t rows16 = cdiv(N, 16);
  const bool narrow = K < 2 * 4096 && (rows16 <= 256 || (M <= 16 && rows16 <= 512));
  p.rt = narrow ? 1 : (M > 16 && cdiv(N, 64) >= 384 ? 4 : 2);
  const int64_t tiles = cdiv(N, 16 * p.rt);
  int64_t split = 1;
  while (tiles * split < 512 && K / (split * 2) >= 4096 && (K / kRsStageK) % (split * 2) == 0) split *= 2;
  p.kps = K / split;
  p.split = (int)split;
  p.ok = cdiv(N, 16 * p.rt) <= 0x7FFFFFFF;
  return p;
}
size_t rows_workspace(const RsPlan& p, int64_t M, int64_t N) {
  return p.ok && p.split > 1 ? (size_t)p.split * (size_t)M * (size_t)N * sizeof(float) : 0;
}

template <bool BF16, bool ROW_SCALE, int RT>
void launch_rows_rt(const RsPlan& p, const RsArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)cdiv(a.N, 16 * RT), (unsigned)p.split), block(kRsWaves * kWave);
  switch (p.xj) {
    case 1: hipLaunchKernelGGL((w8a16_rows_kernel<BF16, ROW_SCALE, RT, 1>), grid, block, 0, st, a); break;
    case 2: hipLaunchKernelGGL((w8a16_rows_kernel<BF16, ROW_SCALE, RT, 2>), grid, block, 0, st, a); break;
    case 3: hipLaunchKernelGGL((w8a16_rows_kernel<BF16, ROW_SCALE, RT, 3>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((w8a16_rows_kernel<BF16, ROW_SCALE, RT, 4>), grid, block, 0, st, a); break;
  }
}
template <bool BF16, bool ROW_SCALE>
void launch_rows_kernel(const RsPlan& p, const RsArgs& a, hipStream_t st) {
  if (p.rt == 4) launch_rows_rt<BF16, ROW_SCALE, 4>(p, a, st);
  else if (p.rt == 2) launch_rows_rt<BF16, ROW_SCALE, 2>(p, a, st);
  else launch_rows_rt<BF16, ROW_SCALE, 1>(p, a, st);
}

template <bool BF16>
int launch_rows(const RsPlan& p, RsArgs a, size_t ws_bytes, hipStream_t st) {
  note_plan("w8a16 rows rt=%d xj=%d split=%d", p.rt, p.xj, p.split);
  a.k_per_split = p.kps;
  if (p.split > 1) {
    const size_t need = rows_workspace(p, a.M, a.N);
    if (a.part == nullptr || ws_bytes < need) {
      return fail(AYK_EWORKSPACE, "fp8_weight_only_gemm: workspace of %zu bytes required, %zu given", need, ws_bytes);
    }
  }
  if (a.bx >= a.K) launch_rows_kernel<BF16, true>(p, a, st);
  else launch_rows_kernel<BF16, false>(p, a, st);
  if (int rc = check_launch("fp8_weight_only_gemm")) return rc;
  if (p.split > 1) {
    hipLaunchKernelGGL((w8a16_rows_reduce<BF16>), dim3((unsigned)cdiv(a.M * a.N, 256)), dim3(256), 0, st, a, p.split);
    return check_launch("fp8_weight_only_gemm");
  }
  return AYK_OK;
}

// ------------------------------------------------------------ stream decode kernel
// Decode batches (2 <= M <= 32). Every wavefront streams its own RW = 16 TW weight rows
// over the whole K range through a private LDS ring of D stages (16 TW rows x 256 K
// bytes, filled by direct loads of 4 rows x 256 contiguous bytes each), with no
// workgroup barrier per stage: a stage is complete for a wavefront once its own loads
// have retired. The activations are shared: the workgroup stages them into LDS in
// chunks of G stages (MP rows x 256 G elements, double-buffered), each wavefront
// loading a quarter of every chunk together with the first stage of that chunk; one
// workgroup barrier at every chunk boundary makes a chunk visible (and, G >= D - 1,
// proves the buffer it refills has been read by everyone). Activation bytes thus pass
// the vector-memory path once per workgroup, not once per wavefront.
//
// MFMA v_mfma_f32_16x16x32_{bf16,f16}, weight as operand A, in the row-stream kernel's
// K order (lane (r, g): 16 weight bytes of row r at K [16 g, 16 g + 16) of a 64-K
// window, two 8-element operands; the same K of activation row r (+ 16) as operand B).
// Logical 16-byte chunk c of an LDS row (weights or activations) sits at physical chunk
// c ^ (row % 16), so the 16 rows of a fragment read fall on distinct banks.
constexpr int kStWaves = 4;
constexpr int kStK = 256;  // K per stage

// Calls f(std::integral_constant<int, i>{}) for i = 0 .. N - 1 (an unrolled loop whose
// index is a compile-time constant in the body).
template <typename F, int... I>
__device__ inline void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ inline void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

template <int NB>
__device__ inline void window_reads(v4u (&b)[NB], const uint32_t (&ab)[NB]);
#define AYK_WR128(o, i) "ds_read_b128 %" #o ", %" #i "\n\t"
template <>
__device__ inline void window_reads<3>(v4u (&b)[3], const uint32_t (&ab)[3]) {
  asm volatile(AYK_WR128(0, 3) AYK_WR128(1, 4) AYK_WR128(2, 5) "s_waitcnt lgkmcnt(0)"
               : "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2])
               : "v"(ab[0]), "v"(ab[1]), "v"(ab[2])
               : "memory");
}
template <>
__device__ inline void window_reads<4>(v4u (&b)[4], const uint32_t (&ab)[4]) {
  asm volatile(AYK_WR128(0, 4) AYK_WR128(1, 5) AYK_WR128(2, 6) AYK_WR128(3, 7) "s_waitcnt lgkmcnt(0)"
               : "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(b[3])
               : "v"(ab[0]), "v"(ab[1]), "v"(ab[2]), "v"(ab[3])
               : "memory");
}
template <>
__device__ inline void window_reads<5>(v4u (&b)[5], const uint32_t (&ab)[5]) {
  asm volatile(AYK_WR128(0, 5) AYK_WR128(1, 6) AYK_WR128(2, 7) AYK_WR128(3, 8) AYK_WR128(4, 9) "s_waitcnt lgkmcnt(0)"
               : "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(b[3]), "=&v"(b[4])
               : "v"(ab[0]), "v"(ab[1]), "v"(ab[2]), "v"(ab[3]), "v"(ab[4])
               : "memory");
}
template <>
__device__ inline void window_reads<6>(v4u (&b)[6], const uint32_t (&ab)[6]) {
  asm volatile(AYK_WR128(0, 6) AYK_WR128(1, 7) AYK_WR128(2, 8) AYK_WR128(3, 9) AYK_WR128(4, 10) AYK_WR128(5, 11) "s_waitcnt lgkmcnt(0)"
               : "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(b[3]), "=&v"(b[4]), "=&v"(b[5])
               : "v"(ab[0]), "v"(ab[1]), "v"(ab[2]), "v"(ab[3]), "v"(ab[4]), "v"(ab[5])
               : "memory");
}
#undef AYK_WR128

// One 16-byte direct-to-LDS load per lane with the nontemporal hint: weights are read
// once, so they stream past the caches (measured 3-7% faster than the default policy).
__device__ inline void dma16_nt(const uint8_t* src, uint8_t* lds_dst) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_dst, 16, 0, 2);
}

template <bool BF16, bool ROW_SCALE, int MP, int TW, int G, int D, int KS>
__global__ __launch_bounds__(kStWaves * kWave) void w8a16_stream_kernel(RsArgs a) {
  constexpr int MT = MP > 16 ? 2 : 1;        // 16-column MFMA tiles
  constexpr int RW = 16 * TW;                // rows per wavefront
  constexpr int RG = kStWaves / KS;          // row groups per workgroup (KS K parts each)
  constexpr int R = RG * RW;                 // rows per workgroup
  constexpr int kWStage = RW * kStK;         // weight bytes of one wavefront stage
  constexpr int kWIns = kWStage / 1024;      // direct loads per wavefront stage
  constexpr int kXRow = 2 * G * kStK;        // bytes of one activation row of a chunk (one K part)
  constexpr int kXPart = MP * kXRow;         // one K part's rows of a chunk
  constexpr int kXChunk = KS * kXPart;
  constexpr int kXIns = kXChunk / (1024 * kStWaves);  // activation loads per wavefront and chunk
  constexpr int kSOps = ROW_SCALE ? 0 : 4 * TW;       // block-scale words per stage
  constexpr int kOpsW = kWIns + kSOps;
  constexpr int U = G % D == 0 ? G : (D % G == 0 ? D : G * D);  // a multiple of G and D
  static_assert(kXChunk % (1024 * kStWaves) == 0, "whole activation loads per wavefront");
  static_assert(D >= 2 && D - 1 <= G, "an activation buffer is refilled only after a barrier past its last read");
  static_assert(R <= kWStage, "the row-scale words fit one stage slot");
  // Loads issued after stage s and before its wait (stages s + 1 .. s + D - 2).
  constexpr auto wait_after = [](int u) {
    int n = 0;
    for (int t = u + 1; t <= u + D - 2; ++t) n += kOpsW + (t % G == 0 ? kXIns : 0);
    return n;
  };
  static_assert(wait_after(0) <= 63 && wait_after(G - 1) <= 63, "vmcnt range");

  __shared__ __attribute__((aligned(1024))) uint8_t wring[kStWaves * D * kWStage];
  __shared__ __attribute__((aligned(1024))) uint8_t xbuf[2 * kXChunk];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int r16 = lane & 15, g = lane >> 4;
  uint8_t* myring = wring + wave * D * kWStage;
  // With KS > 1 the wavefronts of a row group take the KS parts of the K range (sums
  // meet in LDS at the end): wavefront w is part w / RG of row group w % RG.
  const int part = wave / RG, rg = wave % RG;
  const int64_t n_wave = (int64_t)blockIdx.x * R + rg * RW;
  const int64_t kbeg = (int64_t)blockIdx.y * a.k_per_split;
  const int64_t klen = a.K - kbeg < a.k_per_split ? a.K - kbeg : a.k_per_split;
  const int64_t plen = klen / KS;            // K per part
  const int64_t kpart = kbeg + part * plen;
  const int ns = (int)(plen / kStK);  // a multiple of G (host plan)

  // Weight loads: load j of a stage covers rows 4 j .. 4 j + 3 of the wavefront, lane l
  // row 4 j + l / 16 at physical chunk l % 16; rows past N re-read row N - 1.
  const uint8_t* wsrc[kWIns];
#pragma unroll
  for (int j = 0; j < kWIns; ++j) {
    const int row = 4 * j + (lane >> 4);
    const int64_t n = n_wave + row < a.N ? n_wave + row : a.N - 1;
    wsrc[j] = a.w + n * a.ldw + kpart + 16 * ((lane & 15) ^ (row & 15));
  }
  // Activation loads: load j of wavefront w fills chunk bytes 1024 (w kXIns + j) ..:
  // K part q, row m, physical chunk p of that row; rows past M repeat row M - 1.
  const uint16_t* xsrc[kXIns];
  uint32_t xdst[kXIns];
#pragma unroll
  for (int j = 0; j < kXIns; ++j) {
    const int byte = 1024 * (wave * kXIns + j) + 16 * lane;
    const int q = byte / kXPart;
    const int m = (byte % kXPart) / kXRow;
    const int p = (byte % kXRow) / 16;
    const int64_t mm = m < a.M ? m : a.M - 1;
    xsrc[j] = a.x + mm * a.ldx + kbeg + q * plen + 8 * (p ^ (m & 15));
    xdst[j] = __builtin_amdgcn_readfirstlane(1024 * (wave * kXIns + j));
  }
  // Fragment read offsets: weights (row 16 tt + r, window chunk 4 win + g) within a stage
  // slot; activations (row m = 16 mt + r, clamped to the staged rows) within a chunk.
  uint32_t woff[TW][4];
#pragma unroll
  for (int tt = 0; tt < TW; ++tt)
#pragma unroll
    for (int win = 0; win < 4; ++win) {
      const int row = 16 * tt + r16;
      woff[tt][win] = row * kStK + 16 * ((4 * win + g) ^ (row & 15));
    }
  int64_t rowbase[TW];
#pragma unroll
  for (int tt = 0; tt < TW; ++tt) {
    const int64_t n = n_wave + 16 * tt + r16 < a.N ? n_wave + 16 * tt + r16 : a.N - 1;
    rowbase[tt] = (int64_t)((uint64_t)n / (uint64_t)a.by) * a.srs;
  }

  // Per-row scales: wavefront 0 copies the workgroup's raw scale words into its last
  // ring slot (free until the first stage's refill) ahead of everything else.
  uint32_t* srow_lds = reinterpret_cast<uint32_t*>(wring + (D - 1) * kWStage);
  constexpr int kSrowIns = ROW_SCALE ? (R + kWave - 1) / kWave : 0;
  const int ssize = a.scale_dtype == AYK_F32 ? 4 : (a.scale_dtype == AYK_U8 ? 1 : 2);
  if constexpr (ROW_SCALE) {
    if (wave == 0) {
#pragma unroll
      for (int i = 0; i < kSrowIns; ++i) {
        const int row = kWave * i + lane < R ? kWave * i + lane : R - 1;  // row of the workgroup
        const int64_t n = (int64_t)blockIdx.x * R + row < a.N ? (int64_t)blockIdx.x * R + row : a.N - 1;
        const uintptr_t p = reinterpret_cast<uintptr_t>(a.scale) + (uintptr_t)(((int64_t)((uint64_t)n / (uint64_t)a.by) * a.srs) * ssize);
        dma4(reinterpret_cast<const uint8_t*>(p & ~(uintptr_t)3), reinterpret_cast<uint8_t*>(srow_lds) + 4 * kWave * i);
      }
    }
  }

  RawBits sr[D][ROW_SCALE ? 1 : TW][ROW_SCALE ? 1 : 4];
  // Stage t (clamped to the last stage; a clamped stage only rewrites data no later
  // stage reads, or the same data) into slot t % D; the chunk's activations with the
  // chunk's first stage (XL: t % G == 0, known at compile time at every call site).
  auto issue = [&](int slot, int t, bool xl) {
    const int tc = t < ns ? t : ns - 1;
    const int64_t k = (int64_t)tc * kStK;
#pragma unroll
    for (int j = 0; j < kWIns; ++j) dma16_nt(wsrc[j] + k, myring + slot * kWStage + 1024 * j);
    if constexpr (!ROW_SCALE) {
#pragma unroll
      for (int win = 0; win < 4; ++win) {
        const int64_t kidx = (uint32_t)(kpart + k + 64 * win + 16 * g) / (uint32_t)a.bx;
#pragma unroll
        for (int tt = 0; tt < TW; ++tt) sr[slot][tt][win] = load_bits(a.scale, a.scale_dtype, rowbase[tt] + kidx);
      }
    }
    if (xl) {
      const int c = tc / G;
      uint8_t* xb = xbuf + (c & 1) * kXChunk;
#pragma unroll
      for (int j = 0; j < kXIns; ++j) dma16(reinterpret_cast<const uint8_t*>(xsrc[j] + (int64_t)c * G * kStK), xb + xdst[j]);
    }
  };

  v4f acc[TW][MT];
#pragma unroll
  for (int tt = 0; tt < TW; ++tt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[tt][mt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  float srowf[TW];
  // Stage s from slot `slot`; its activations at window base `wb` (K within the chunk)
  // of chunk buffer `xb`.
  auto compute = [&](int slot, int s, int wb) {
    const uint32_t wbase = lds_addr(myring + slot * kWStage);
    const uint32_t xbase = lds_addr(xbuf + ((s / G) & 1) * kXChunk + part * kXPart);
#pragma unroll
    for (int win = 0; win < 4; ++win) {
      constexpr int NB = TW + 2 * MT;
      uint32_t ab[NB];
      v4u v[NB];
#pragma unroll
      for (int tt = 0; tt < TW; ++tt) ab[tt] = wbase + woff[tt][win];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = 16 * mt + r16 < MP ? 16 * mt + r16 : MP - 1;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int lc = wb / 8 + 8 * win + 2 * g + h;
          ab[TW + 2 * mt + h] = xbase + m * kXRow + 16 * (lc ^ (m & 15));
        }
      }
      window_reads<NB>(v, ab);
#pragma unroll
      for (int tt = 0; tt < TW; ++tt) {
        float sc;
        if constexpr (ROW_SCALE) sc = srowf[tt];
        else sc = bits_to_f32(sr[slot][tt][win], a.scale_dtype);
        const v8s lo = convert8<BF16>(v[tt][0], v[tt][1], sc);
        const v8s hi = convert8<BF16>(v[tt][2], v[tt][3], sc);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          acc[tt][mt] = mfma16x16<BF16>(lo, __builtin_bit_cast(v8s, v[TW + 2 * mt]), acc[tt][mt]);
          acc[tt][mt] = mfma16x16<BF16>(hi, __builtin_bit_cast(v8s, v[TW + 2 * mt + 1]), acc[tt][mt]);
        }
      }
    }
  };

#pragma unroll
  for (int d = 0; d < D - 1; ++d) issue(d, d, d % G == 0);
  if constexpr (ROW_SCALE) {
    // Everything older than the ring: wavefront 0's row-scale copy.
    if (wave == 0) {
      constexpr int kRing = [] {
        int n = 0;
        for (int t = 0; t < D - 1; ++t) n += kOpsW + (t % G == 0 ? kXIns : 0);
        return n;
      }();
      wait_vmcnt<(kRing < 63 ? kRing : 63)>();
    }
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) {
      const int row = rg * RW + 16 * tt + r16;
      uint32_t word;
      asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(word) : "v"(lds_addr(reinterpret_cast<const uint8_t*>(srow_lds)) + 4 * row) : "memory");
      const uint32_t shift = (uint32_t)((reinterpret_cast<uintptr_t>(a.scale) + (uintptr_t)(rowbase[tt] * ssize)) & 3) * 8;
      srowf[tt] = bits_to_f32(RawBits{word, shift}, a.scale_dtype);
    }
  }
  // Step s: wait for stage s (its activation chunk too), at a chunk start a barrier,
  // refill slot (s - 1) % D with stage s + D - 1, compute stage s. The main loop runs
  // whole rounds of U steps with no exit inside; the remainder runs after it.
  auto step = [&](auto uc, int s) {
    constexpr int u = decltype(uc)::value;
    wait_vmcnt<wait_after(u % G)>();
    if (u % G == 0) __builtin_amdgcn_s_barrier();
    issue((u + D - 1) % D, s + D - 1, (u + D - 1) % G == 0);
    compute(u % D, s, (u % G) * kStK);
  };
  int s0 = 0;
  for (; s0 + U <= ns; s0 += U) {
    static_for<U>([&](auto uc) { step(uc, s0 + decltype(uc)::value); });
  }
  static_for<U - 1>([&](auto uc) {
    if (s0 + decltype(uc)::value < ns) step(uc, s0 + decltype(uc)::value);  // workgroup-uniform
  });
  wait_vmcnt<0>();  // no direct load may still be writing LDS when the workgroup ends

  if constexpr (KS > 1) {
    // The K parts of a row group meet in LDS (the rings are free once every wavefront
    // is past its last stage): wavefront w writes its sums at slot w, and part 0 adds
    // the parts in order.
    constexpr int kSlots = TW * MT * 4;
    static_assert(kStWaves * kSlots * kWave * 4 <= kStWaves * D * kWStage, "the sums fit the rings");
    float* red = reinterpret_cast<float*>(wring);
    __syncthreads();
#pragma unroll
    for (int tt = 0; tt < TW; ++tt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[(wave * kSlots + (tt * MT + mt) * 4 + r) * kWave + lane] = acc[tt][mt][r];
    __syncthreads();
    if (part != 0) return;
#pragma unroll
    for (int tt = 0; tt < TW; ++tt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v = 0.0f;
#pragma unroll
          for (int q = 0; q < KS; ++q) v += red[((q * RG + rg) * kSlots + (tt * MT + mt) * 4 + r) * kWave + lane];
          acc[tt][mt][r] = v;
        }
  }

  // D[n][m]: lane holds m = lane % 16 (+ 16 mt) and n = 4 (lane / 16) + r of its tile.
#pragma unroll
  for (int tt = 0; tt < TW; ++tt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int64_t m = 16 * mt + r16;
      if (m >= a.M) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t n = n_wave + 16 * tt + 4 * g + r;
        if (n >= a.N) continue;
        if (gridDim.y == 1) a.out[m * a.ldo + n] = round16<BF16>(acc[tt][mt][r]);
        else a.part[((int64_t)blockIdx.y * a.M + m) * a.N + n] = acc[tt][mt][r];
      }
    }
}

// Launch plan from the shapes alone (the workspace query reproduces it).
//  * Wide projections (N >= kStMinRows: >= 384 wavefront tiles of 64 rows), any M:
//    each wavefront owns its rows over all of K (KS = 1).
//  * Narrower projections at M <= 8: a workgroup's four wavefronts take the four K
//    quarters of 16 rows (KS = 4), so that N / 16 workgroups cover the CUs; the
//    activation chunk holds all four quarters (2 stages each).
// Narrow projections at M > 8 keep the row-stream kernel: a 16-row workgroup would read
// 2 M bytes of activations per weight byte.
constexpr int64_t kStMinRows = 24576;
struct StPlan {
  bool ok;
  int mp, tw, g, d, ks, split;
  int64_t kps;
};
StPlan stream_plan(int64_t M, int64_t N, int64_t K, int64_t bx) {
  StPlan p{};
  const bool row_scale = bx >= K;
  if (M < 2 || M > 32 || N < 1 || K % kStK || K >= (int64_t(1) << 31) || (!row_scale && bx % 16)) return p;
  p.mp = M <= 4 ? 4 : (M <= 8 ? 8 : (M <= 16 ? 16 : 32));
  p.d = 3;
  p.split = 1;
  p.kps = K;
  if (N >= kStMinRows) {
    // Up to 8 activation rows: one 16-row tile per wavefront, 32 KB of activation
    // buffers, two workgroups per CU. Above: two tiles per wavefront (the activation
    // bytes a workgroup reads are half its weight bytes at M = 32), 64 KB of activation
    // buffers, one workgroup per CU.
    p.ks = 1;
    p.tw = p.mp <= 8 ? 1 : 2;
    p.g = (p.tw == 1 ? 32 : 64) / p.mp;
    if (p.g > 8) p.g = 8;
    while (p.g > 2 && K % (kStK * p.g)) p.g /= 2;
    if (K % (kStK * p.g)) return StPlan{};
  } else if (p.mp <= 8 && N >= 512 && cdiv(N, 16) <= (p.mp == 4 ? 512 : 256)) {
    // One round of resident workgroups: 80 KB of LDS at M <= 4 (two per CU), 112 KB at
    // M <= 8 (one per CU); past it the row-stream kernel measured faster (qkv at M = 8:
    // 384 workgroups, 13.1 against 9.9 us).
    p.ks = 4;
    p.tw = 1;
    p.g = 2;
    if (K % (4 * kStK * p.g)) return StPlan{};
  } else if (p.mp == 16 && K >= 8192) {
    // 9-16 rows over a long K (Llama-3-8B down): 16-row wavefronts over whole K, 80 KB of
    // LDS (two workgroups per CU), a grid K split up to 256 workgroups (18.1 -> 16.3 us
    // at M = 16). qkv, o and every 32-row case measured faster on the row-stream kernel.
    p.ks = 1;
    p.tw = 1;
    p.g = 2;
    const int64_t wgs = cdiv(N, 16 * kStWaves);
    int64_t split = 1;
    while (wgs * split * 2 <= 256 && K % (kStK * p.g * split * 2) == 0 && K / (split * 2) >= 2048) split *= 2;
    if (K % (kStK * p.g * split)) return StPlan{};
    p.split = (int)split;
    p.kps = K / split;
  } else {
    return StPlan{};
  }
  p.ok = cdiv(N, 16 * p.tw * (kStWaves / p.ks)) <= 0x7FFFFFFF;
  return p;
}
size_t stream_workspace(const StPlan& p, int64_t M, int64_t N) {
  return p.ok && p.split > 1 ? (size_t)p.split * (size_t)M * (size_t)N * sizeof(float) : 0;
}

template <bool BF16, bool ROW_SCALE, int MP, int TW, int KS>
bool launch_stream_g(const StPlan& p, const RsArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)cdiv(a.N, 16 * TW * (kStWaves / KS)), (unsigned)p.split), block(kStWaves * kWave);
#define AYK_ST(G, D)                                                                                      \
  if (p.g == G && p.d == D) {                                                                             \
    hipLaunchKernelGGL((w8a16_stream_kernel<BF16, ROW_SCALE, MP, TW, G, D, KS>), grid, block, 0, st, a); \
    return true;                                                                                          \
  }
  // LDS: 4 D TW 4 KB of weight rings + 2 KS MP 512 G bytes of activation chunks
  if constexpr (KS == 1 && 64 / MP >= 8) { AYK_ST(8, 3) }
  if constexpr (KS == 1 && 64 / MP >= 4) { AYK_ST(4, 3) }
  AYK_ST(2, 3)
#undef AYK_ST
  return false;
}

template <bool BF16, bool ROW_SCALE>
bool launch_stream_kernel(const StPlan& p, const RsArgs& a, hipStream_t st) {
  if (p.ks == 4) {
    if (p.tw != 1) return false;
    if (p.mp == 4) return launch_stream_g<BF16, ROW_SCALE, 4, 1, 4>(p, a, st);
    if (p.mp == 8) return launch_stream_g<BF16, ROW_SCALE, 8, 1, 4>(p, a, st);
    return false;
  }
  if (p.ks != 1) return false;
  switch (p.mp * 10 + p.tw) {
    case 41: return launch_stream_g<BF16, ROW_SCALE, 4, 1, 1>(p, a, st);
    case 42: return launch_stream_g<BF16, ROW_SCALE, 4, 2, 1>(p, a, st);
    case 81: return launch_stream_g<BF16, ROW_SCALE, 8, 1, 1>(p, a, st);
    case 82: return launch_stream_g<BF16, ROW_SCALE, 8, 2, 1>(p, a, st);
    case 161: return launch_stream_g<BF16, ROW_SCALE, 16, 1, 1>(p, a, st);
    case 162: return launch_stream_g<BF16, ROW_SCALE, 16, 2, 1>(p, a, st);
    case 321: return launch_stream_g<BF16, ROW_SCALE, 32, 1, 1>(p, a, st);
    case 322: return launch_stream_g<BF16, ROW_SCALE, 32, 2, 1>(p, a, st);
    default: return false;
  }
}

template <bool BF16>
int launch_stream(const StPlan& p, RsArgs a, size_t ws_bytes, hipStream_t st) {
  note_plan("w8a16 stream mp=%d tw=%d ks=%d split=%d", p.mp, p.tw, p.ks, p.split);
  a.k_per_split = p.kps;
  if (p.split > 1) {
    const size_t need = stream_workspace(p, a.M, a.N);
    if (a.part == nullptr || ws_bytes < need) {
      return fail(AYK_EWORKSPACE, "fp8_weight_only_gemm: workspace of %zu bytes required, %zu given", need, ws_bytes);
    }
  }
  const bool launched = a.bx >= a.K ? launch_stream_kernel<BF16, true>(p, a, st) : launch_stream_kernel<BF16, false>(p, a, st);
  if (!launched) return fail(AYK_EINVAL, "fp8_weight_only_gemm: no stream kernel for this plan");
  if (int rc = check_launch("fp8_weight_only_gemm")) return rc;
  if (p.split > 1) {
    hipLaunchKernelGGL((w8a16_rows_reduce<BF16>), dim3((unsigned)cdiv(a.M * a.N, 256)), dim3(256), 0, st, a, p.split);
    return check_launch("fp8_weight_only_gemm");
  }
  return AYK_OK;
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

size_t ayk_fp8_weight_only_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t block_size_x) {
  if (M < 2) return 0;
  // An upper bound over the decode kernels (alignment decides which one runs).
  const size_t st = stream_workspace(stream_plan(M, N, K, block_size_x), M, N);
  const size_t rs = rows_workspace(rows_plan(M, N, K, block_size_x), M, N);
  const size_t sk = skinny_workspace(skinny_plan(M, N, K, block_size_x), M, N);
  return st > rs ? (st > sk ? st : sk) : (rs > sk ? rs : sk);
}

int ayk_fp8_weight_only_gemm(const void* x, int x_dtype, int64_t ldx, int64_t M, const void* w,
                             int64_t ldw, int64_t N, int64_t K, const void* scale, int scale_dtype,
                             int64_t scale_row_stride, int64_t block_size_y, int64_t block_size_x,
                             void* out, int64_t ldo, void* workspace, size_t workspace_bytes,
                             ayk_stream_t stream) {
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
  // Decode batch sizes (all three need 16-byte aligned activation rows): wide
  // projections take the stream kernel (K a multiple of 512, scale blocks of whole
  // 16 K), the others the row-stream kernel (whole 256-K stages, scale blocks of whole
  // 16 K), else the skinny streaming kernel (whole 128-K steps, scale blocks of >= 32 K).
  if (M >= 2 && ldx % 8 == 0) {
    const StPlan sp = stream_plan(M, N, K, block_size_x);
    if (sp.ok) {
      RsArgs a{};
      a.x = g.x; a.ldx = ldx; a.M = M; a.w = g.w; a.ldw = ldw; a.N = N; a.K = K;
      a.scale = scale; a.scale_dtype = scale_dtype; a.srs = scale_row_stride; a.by = block_size_y; a.bx = block_size_x;
      a.out = g.out; a.ldo = ldo; a.part = static_cast<float*>(workspace);
      return x_dtype == AYK_BF16 ? launch_stream<true>(sp, a, workspace_bytes, st)
                                 : launch_stream<false>(sp, a, workspace_bytes, st);
    }
  }
  if (M >= 2 && ldx % 8 == 0) {
    const RsPlan rp = rows_plan(M, N, K, block_size_x);
    if (rp.ok) {
      RsArgs a{};
      a.x = g.x; a.ldx = ldx; a.M = M; a.w = g.w; a.ldw = ldw; a.N = N; a.K = K;
      a.scale = scale; a.scale_dtype = scale_dtype; a.srs = scale_row_stride; a.by = block_size_y; a.bx = block_size_x;
      a.out = g.out; a.ldo = ldo; a.part = static_cast<float*>(workspace);
      return x_dtype == AYK_BF16 ? launch_rows<true>(rp, a, workspace_bytes, st)
                                 : launch_rows<false>(rp, a, workspace_bytes, st);
    }
  }
  if (M >= 2 && ldx % 8 == 0) {
    const SkinnyPlan p = skinny_plan(M, N, K, block_size_x);
    if (p.ok) {
      SkinnyArgs a{};
      a.x = g.x; a.ldx = ldx; a.M = M; a.w = g.w; a.ldw = ldw; a.N = N; a.K = K;
      a.scale = scale; a.scale_dtype = scale_dtype; a.srs = scale_row_stride; a.by = block_size_y; a.bx = block_size_x;
      a.out = g.out; a.ldo = ldo; a.part = static_cast<float*>(workspace);
      return x_dtype == AYK_BF16 ? launch_skinny<true>(p, a, workspace_bytes, st)
                                 : launch_skinny<false>(p, a, workspace_bytes, st);
    }
  }
  return x_dtype == AYK_BF16 ? dispatch_w16<true>(g, st) : dispatch_w16<false>(g, st);
}

}  // extern "C"
