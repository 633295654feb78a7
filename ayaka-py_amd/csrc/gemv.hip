// Decode GEMV (M == 1) over an [N, K] e4m3 weight, for gfx950.
//
//   out[n] = sum_k w[n, k] * x[k] * wscale(n, k) * ascale(k)  (+ bias[n])
//
// Serves three reference operators (python/ayaka/kernel/triton/gemm/fp8_gemv.py):
//   * fp8_weight_only_gemv (:323): x fp16/bf16, weight scale
//     scale[(n / by) * stride + k / bx] in UE8M0 / fp32 / bf16, no activation scale;
//   * fp8_blockwise_gemv (:433): x e4m3 with a per-128 activation scale and a
//     [N/128, K/128] weight scale, plus bias;
//   * the M == 1 MXFP8 product (fp8_mxfp8_gemm.py:163 at M == 1): x e4m3 and w e4m3,
//     each with one UE8M0 code per 32-wide K group.
//
// The kernel is HBM-bound: its cost is N * K weight bytes. Each wavefront owns R
// weight rows and walks K in 1024-byte strides (64 lanes x one 16-byte vector), so
// every weight load is a fully coalesced 128-bit load and a wave keeps U * R of them
// in flight per lane. The activation chunk a lane needs is the same for all R rows,
// so it is loaded once (L1/L2 resident) and reused R times. A K split (grid.y) is
// used only when N alone cannot fill the 256 CUs; its fp32 partials are summed by a
// second kernel in a fixed order, so results are deterministic.
#include <mutex>

#include "ayk_common.h"

namespace ayk {
namespace {

constexpr int kGemvThreads = 128;  // 2 wavefronts: small blocks schedule best for streaming
constexpr int kGemvWaves = kGemvThreads / kWave;
constexpr int kChunk = 16;                      // K elements per lane vector
constexpr int64_t kWaveK = (int64_t)kWave * kChunk;  // K elements per wave sweep

enum ActKind { ACT_BF16 = 0, ACT_F16 = 1, ACT_E4M3 = 2 };
enum WScaleKind { WS_ROW = 0, WS_CHUNK = 1 };
enum AScaleKind { AS_NONE = 0, AS_BLOCK128 = 1, AS_MX32 = 2 };

struct GemvArgs {
  const void* x;
  const uint8_t* w;
  int64_t ldw;
  int64_t N, K;
  const void* wscale;
  int wscale_dtype;
  int64_t srs;  // weight-scale row stride
  int64_t by, bx;
  const void* ascale;  // per-128 float scale or per-32 UE8M0 codes of x
  int ascale_dtype;
  const void* bias;
  int bias_dtype;
  void* out;
  int out_dtype;
  float* part;       // [split, N] partials when split > 1
  int64_t k_per_split;  // multiple of kWaveK
  int64_t pairs_per_wave;  // streaming kernel: row pairs owned by one wavefront
  int ws_is_f16;           // streaming kernel, 2-byte chunk scales: fp16 (1) or bf16 (0)
  int bx_shift;            // streaming kernel, chunk scales: log2(bx), or -1 if bx is not a power of two
};

// Load the 16 activation values of chunk `c` (elements 16c .. 16c+15) as floats.
template <int ACT>
__device__ inline void load_x_chunk(const void* x, int64_t c, float* f) {
  if constexpr (ACT == ACT_E4M3) {
    const uint4 v = reinterpret_cast<const uint4*>(x)[c];
    e4m3x4_to_f32(v.x, f);
    e4m3x4_to_f32(v.y, f + 4);
    e4m3x4_to_f32(v.z, f + 8);
    e4m3x4_to_f32(v.w, f + 12);
  } else {
    const uint4* p = reinterpret_cast<const uint4*>(x) + 2 * c;
    const uint4 a = p[0], b = p[1];
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if constexpr (ACT == ACT_BF16) {
        f[2 * i] = u2f(w[i] << 16);
        f[2 * i + 1] = u2f(w[i] & 0xFFFF0000u);
      } else {
        f[2 * i] = f16_bits_to_f32((uint16_t)(w[i] & 0xFFFFu));
        f[2 * i + 1] = f16_bits_to_f32((uint16_t)(w[i] >> 16));
      }
    }
  }
}

__device__ inline float dot16(const uint4& wv, const float* xf) {
  float wf[16];
  e4m3x4_to_f32(wv.x, wf);
  e4m3x4_to_f32(wv.y, wf + 4);
  e4m3x4_to_f32(wv.z, wf + 8);
  e4m3x4_to_f32(wv.w, wf + 12);
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s = fmaf(wf[i], xf[i], s);
  return s;
}

template <int AS>
__device__ inline float act_scale(const GemvArgs& a, int64_t k0) {
  if constexpr (AS == AS_BLOCK128) return load_f32(a.ascale, a.ascale_dtype, k0 / 128);
  else if constexpr (AS == AS_MX32) return e8m0_decode(reinterpret_cast<const uint8_t*>(a.ascale)[k0 / 32]);
  else return 1.0f;
}

// Weights are read once per call, so they are loaded non-temporally (they should
// not displace the activation vector or other live data from L2 / MALL).
typedef unsigned v4u __attribute__((ext_vector_type(4)));
__device__ inline uint4 load_stream(const uint8_t* p) {
  const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// R weight rows per wavefront; U sweeps (U * 1024 K elements) of loads issued
// before any of them is consumed, i.e. R * U 16-byte loads in flight per lane.
template <int ACT, int WS, int AS, int R, int U>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(GemvArgs a) {
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int64_t row0 = ((int64_t)blockIdx.x * kGemvWaves + wave) * R;
  const int64_t kbeg = (int64_t)blockIdx.y * a.k_per_split;
  const int64_t kend = min(a.K, kbeg + a.k_per_split);
  const uint8_t* wrow[R];
  float acc[R];
  // Scale row offsets are computed once; per-chunk column indices use 32-bit math.
  int64_t sbase[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t n = min(row0 + r, a.N - 1);  // clamp: loads stay in bounds
    wrow[r] = a.w + n * a.ldw;
    acc[r] = 0.0f;
    sbase[r] = (n / a.by) * a.srs;
  }
  float row_scale[R];
  if constexpr (WS == WS_ROW) {
#pragma unroll
    for (int r = 0; r < R; ++r) row_scale[r] = load_f32(a.wscale, a.wscale_dtype, sbase[r]);
  }
  const uint32_t bx = (uint32_t)a.bx;

  for (int64_t kb = kbeg + (int64_t)lane * kChunk; kb < kend; kb += kWaveK * U) {
    uint4 wv[U][R];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t k0 = kb + u * kWaveK;
#pragma unroll
      for (int r = 0; r < R; ++r) wv[u][r] = k0 < kend ? load_stream(wrow[r] + k0) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t k0 = kb + u * kWaveK;
      if (k0 >= kend) break;
      float xf[16];
      load_x_chunk<ACT>(a.x, k0 / kChunk, xf);
      const float sa = act_scale<AS>(a, k0);
      const uint32_t kcol = WS == WS_CHUNK ? (uint32_t)k0 / bx : 0u;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float d = dot16(wv[u][r], xf);
        if constexpr (WS == WS_ROW && AS == AS_NONE) {
          acc[r] += d;
        } else if constexpr (WS == WS_ROW) {
          acc[r] = fmaf(d, sa, acc[r]);
        } else {
          const float sw = load_f32(a.wscale, a.wscale_dtype, sbase[r] + kcol);
          acc[r] = fmaf(d, sw * sa, acc[r]);
        }
      }
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r) {
    float v = wave_sum<kWave>(acc[r]);
    if constexpr (WS == WS_ROW) v *= row_scale[r];
    const int64_t n = row0 + r;
    if (lane == 0 && n < a.N) {
      if (gridDim.y == 1) {
        if (a.bias) v += load_f32(a.bias, a.bias_dtype, n);
        store_f32(a.out, a.out_dtype, n, v);
      } else {
        a.part[(int64_t)blockIdx.y * a.N + n] = v;
      }
    }
  }
}

// Fixed-order sum over the split axis, bias, one rounding to the output dtype.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part,
                                                            int64_t N, int split,
                                                            const void* bias, int bias_dtype,
                                                            void* out, int out_dtype) {
  const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  float v = 0.0f;
  for (int s = 0; s < split; ++s) v += part[(int64_t)s * N + n];
  if (bias) v += load_f32(bias, bias_dtype, n);
  store_f32(out, out_dtype, n, v);
}

// Generic fallback (any K, stride, alignment or scale block): one wave per output
// row, element-wise byte loads, per-element scale. Correct everywhere, not fast.
template <int ACT, int AS>
__global__ __launch_bounds__(kGemvThreads) void gemv_generic_kernel(GemvArgs a) {
  const int lane = threadIdx.x % kWave;
  const int64_t n = (int64_t)blockIdx.x * kGemvWaves + threadIdx.x / kWave;
  if (n >= a.N) return;
  const uint8_t* wr = a.w + n * a.ldw;
  float acc = 0.0f;
  for (int64_t k = lane; k < a.K; k += kWave) {
    float xv;
    if constexpr (ACT == ACT_E4M3) xv = e4m3_decode(reinterpret_cast<const uint8_t*>(a.x)[k]);
    else if constexpr (ACT == ACT_BF16) xv = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(a.x)[k]);
    else xv = f16_bits_to_f32(reinterpret_cast<const uint16_t*>(a.x)[k]);
    const float sw = load_f32(a.wscale, a.wscale_dtype, (n / a.by) * a.srs + k / a.bx);
    acc = fmaf(e4m3_decode(wr[k]) * xv, sw * act_scale<AS>(a, k), acc);
  }
  acc = wave_sum<kWave>(acc);
  if (lane == 0) {
    if (a.bias) acc += load_f32(a.bias, a.bias_dtype, n);
    store_f32(a.out, a.out_dtype, n, acc);
  }
}

// ---------------------------------------------------------------------------------
// Streaming GEMV: the main path when N is large enough to fill the GPU without a K
// split. Each wavefront owns every W-th row pair (W = all wavefronts), walks its
// pairs' (pair, 1024-K sweep) items in order, and keeps kRing items of weight loads in
// flight in a register ring, across row boundaries, so the memory pipeline never
// drains between rows.
//
// The vector-memory counter retires loads in issue order, so a wavefront must never
// wait on a load issued behind the ring: it would wait for the whole ring. Hence the
// start-up order: (1) x is copied to LDS with direct-to-LDS loads; (2) each lane loads
// the raw row scale and bias of one of the wavefront's rows (read back with readlane
// and converted at that row's end); (3) the ring is issued; (4) one wait for "all but
// the ring's loads" and a workgroup barrier make x visible. Chunk scales (block-128 /
// MX / per-K-block weight scales) and activation scales travel in the ring beside
// their weights. Everything between the loads and their use is kept branch-free: a
// load issued inside a branch, or a branch between the ring's prologue and the loop,
// costs the compiler its exact wait counts, and it then waits for the whole ring.
constexpr int kStreamThreads = 256;
constexpr int kStreamWaves = kStreamThreads / kWave;
constexpr int kRing = 3;   // items in flight per wavefront (2 rows x 16 B per lane each; 3 measured best of 2-6)
constexpr int kPair = 2;   // rows per item
constexpr int kStreamLdsMax = 64 * 1024;
constexpr int kStreamRowsMax = kWave;       // rows per wavefront: one register lane each

template <int SZ>
__device__ inline uint32_t load_scale_bits(const void* p, int64_t i) {
  if constexpr (SZ == 1) return reinterpret_cast<const uint8_t*>(p)[i];
  else if constexpr (SZ == 2) return reinterpret_cast<const uint16_t*>(p)[i];
  else return reinterpret_cast<const uint32_t*>(p)[i];
}
template <int SZ>
__device__ inline float decode_scale_bits(uint32_t b, int is_f16) {
  if constexpr (SZ == 1) return e8m0_decode(b);
  else if constexpr (SZ == 2) return is_f16 ? f16_bits_to_f32((uint16_t)b) : bf16_bits_to_f32((uint16_t)b);
  else return u2f(b);
}

// LDS plan of the streaming kernel (shared by host and device).
struct StreamLds {
  int x_bytes;   // staged activation, padded to whole 1 KiB direct-load groups
  __host__ __device__ int total() const { return x_bytes; }
};
__host__ __device__ inline StreamLds stream_lds(int act, int64_t K) {
  StreamLds l;
  const int64_t xb = act == 2 ? K : 2 * K;
  l.x_bytes = (int)((xb + 1023) / 1024 * 1024);
  return l;
}

// s_waitcnt with only the vector-memory count constrained (gfx9 encoding: vmcnt in
// bits [3:0] and [15:14], expcnt [6:4] and lgkmcnt [11:8] left at their maxima).
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int ACT, int WS, int AS, int SZ>
__global__ __launch_bounds__(kStreamThreads) void gemv_stream_kernel(GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t st_lds[];
  const StreamLds L = stream_lds(ACT, a.K);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // The plan keeps N, K < 2^31: all cursors are 32-bit and wave-uniform (SGPRs).
  const int N = (int)a.N, K = (int)a.K;
  const int npairs = (N + kPair - 1) / kPair;
  const int S = (K + (int)kWaveK - 1) / (int)kWaveK;  // sweeps per row
  // Wavefront gw owns pairs gw + j * W, j < pairs_per_wave (W = all wavefronts), so
  // at any moment the wavefronts stream one compact window of the weight matrix.
  const int W = (int)gridDim.x * kStreamWaves;
  const int gw = (int)blockIdx.x * kStreamWaves + wave;
  const int ppw = (int)a.pairs_per_wave;
  const int my_pairs = gw < npairs ? min(ppw, (npairs - 1 - gw) / W + 1) : 0;
  const int n_items = my_pairs * S;
  const int lane_k = lane * kChunk;
  // K offset of the lane in the last sweep, clamped so its 16-byte load stays in the
  // row (its products are discarded when the chunk is past K).
  const int lane_k_last = min((S - 1) * (int)kWaveK + lane_k, K - kChunk) - (S - 1) * (int)kWaveK;

  // (1) x -> LDS, 64 lanes x 16 B per instruction.
  {
    const int nvec = L.x_bytes / 16;
    const int last = (ACT == ACT_E4M3 ? K : 2 * K) / 16 - 1;  // K % 16 == 0
    for (int v0 = wave * 64; v0 < nvec; v0 += kStreamThreads) {
      const int v = min(v0 + lane, last);
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint8_t*>(a.x) + (size_t)v * 16,
                                       (__attribute__((address_space(3))) void*)(st_lds + (size_t)v0 * 16), 16, 0, 0);
    }
  }
  // (2) lane l holds the raw row scale and bias of the wavefront's row l (pair l / 2,
  //     row l % 2 of it) and, for chunk scales, the offset of its scale row. Lanes past
  //     the wavefront's rows read row N - 1 (never used); a missing bias reads x[0].
  RawBits row_s_bits{0, 0}, row_b_bits;
  int64_t srow_lane;
  {
    const int n = min((gw + (lane / kPair) * W) * kPair + lane % kPair, N - 1);
    srow_lane = (int64_t)((uint32_t)n / (uint32_t)a.by) * a.srs;
    if constexpr (WS == WS_ROW) row_s_bits = load_bits(a.wscale, a.wscale_dtype, srow_lane);
    row_b_bits = a.bias ? load_bits(a.bias, a.bias_dtype, n) : load_bits(a.x, AYK_F32, 0);
  }
  auto srow_of = [&](int row) -> int64_t {  // row: wave-uniform index < 64
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)srow_lane, row);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(srow_lane >> 32), row);
    return (int64_t)(((uint64_t)hi << 32) | lo);
  };

  // (3) the ring. The issue cursor is (pair ordinal ip, sweep is) plus the uniform
  //     address of that pair's first row; it saturates at the wavefront's last item,
  //     which is re-read to keep the ring full at the end (and for a wavefront without
  //     rows, pair 0 clamped to a valid row, never consumed).
  uint4 rw[kRing][kPair];
  uint32_t rs[kRing][kPair];
  RawBits ra[kRing];  // activation scale of the lane's 16-K chunk (block-128 / MX)
  const int as_dtype = AS == AS_MX32 ? AYK_U8 : a.ascale_dtype;
  const int64_t pair_stride = (int64_t)W * kPair * a.ldw;
  int ip = 0, is = 0;
  int row0 = min(gw * kPair, N - 1);
  const uint8_t* ibase = a.w + (int64_t)row0 * a.ldw;
  int64_t r1off = row0 + 1 < N ? a.ldw : 0;
  auto issue = [&](int slot) {
    const int lk = is * (int)kWaveK + (is == S - 1 ? lane_k_last : lane_k);
    rw[slot][0] = load_stream(ibase + lk);
    rw[slot][1] = load_stream(ibase + r1off + lk);
    if constexpr (WS == WS_CHUNK) {
      const int kq = a.bx_shift >= 0 ? lk >> a.bx_shift : (int)((uint32_t)lk / (uint32_t)a.bx);
#pragma unroll
      for (int r = 0; r < kPair; ++r) rs[slot][r] = load_scale_bits<SZ>(a.wscale, srow_of(ip * kPair + r) + kq);
    }
    if constexpr (AS != AS_NONE) ra[slot] = load_bits(a.ascale, as_dtype, lk >> (AS == AS_MX32 ? 5 : 7));
    // Advance, saturating at the last item.
    const bool more = ip < my_pairs - 1 || is < S - 1;
    const bool wrap = is == S - 1;
    if (more) {
      if (wrap) {
        is = 0;
        ++ip;
        row0 += W * kPair;
        ibase += pair_stride;
        r1off = row0 + 1 < N ? a.ldw : 0;
      } else {
        ++is;
      }
    }
  };
  // Issued unconditionally (no branch), so the compiler's wait counts stay exact.
  constexpr int kRingLoads = kRing * (kPair * (WS == WS_CHUNK ? 2 : 1) + (AS != AS_NONE ? 1 : 0));
#pragma unroll
  for (int d = 0; d < kRing; ++d) issue(d);

  // (4) everything but the ring has landed (x in LDS); barrier.
  wait_vmcnt<kRingLoads>();
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  if (n_items == 0) return;
  // Row l's scale / bias, converted at its row end (converting here, between the ring
  // prologue and the loop, makes the compiler copy ring registers, which waits).
  auto lane_value = [&](RawBits rb, int row, int dtype) {
    const RawBits r{(uint32_t)__builtin_amdgcn_readlane((int)rb.word, row), (uint32_t)__builtin_amdgcn_readlane((int)rb.shift, row)};
    return bits_to_f32(r, dtype);
  };

  float acc[kPair] = {0.0f, 0.0f};
  int cp = 0, cs = 0;  // consume cursor
  auto consume = [&](int slot) {
    // Opaque from here on: otherwise the compiler hoists work on the prologue's ring
    // values into the loop preheader, where it must wait for the whole ring.
    if constexpr (WS == WS_CHUNK) {
#pragma unroll
      for (int r = 0; r < kPair; ++r) asm volatile("" : "+v"(rs[slot][r]));
    }
    if constexpr (AS != AS_NONE) asm volatile("" : "+v"(ra[slot].word), "+v"(ra[slot].shift));
    const int k0 = cs * (int)kWaveK + lane_k;
    const bool valid = k0 < K;
    const int kx = valid ? k0 : 0;
    // Products in packed 16-bit form: every e4m3 value is exact in bf16 and fp16, and
    // a product of two of them is exact in fp32; v_dot2 sums two products into fp32.
    uint32_t xp[8];  // x[kx .. kx+15] as 8 pairs (bf16 pairs for e4m3 x)
    if constexpr (ACT == ACT_E4M3) {
      const uint4 v = *reinterpret_cast<const uint4*>(st_lds + kx);
      const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xp[2 * i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w4[i], 1.0f, false));
        xp[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w4[i], 1.0f, true));
      }
    } else {
      const uint4* p = reinterpret_cast<const uint4*>(st_lds + 2 * kx);
      const uint4 lo = p[0], hi = p[1];
      xp[0] = lo.x; xp[1] = lo.y; xp[2] = lo.z; xp[3] = lo.w;
      xp[4] = hi.x; xp[5] = hi.y; xp[6] = hi.z; xp[7] = hi.w;
    }
    float sa = 1.0f;
    if constexpr (AS == AS_MX32) sa = e8m0_decode((ra[slot].word >> ra[slot].shift) & 0xFFu);
    else if constexpr (AS == AS_BLOCK128) sa = bits_to_f32(ra[slot], as_dtype);
#pragma unroll
    for (int r = 0; r < kPair; ++r) {
      const uint32_t w4[4] = {rw[slot][r].x, rw[slot][r].y, rw[slot][r].z, rw[slot][r].w};
      constexpr bool kDirect = WS == WS_ROW && AS == AS_NONE;  // accumulate in the dot chain
      float d = kDirect ? acc[r] : 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (ACT == ACT_F16) {
          typedef _Float16 h2 __attribute__((ext_vector_type(2)));
          const h2 w0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w4[i], 1.0f, false);
          const h2 w1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w4[i], 1.0f, true);
          d = __builtin_amdgcn_fdot2(w0, __builtin_bit_cast(h2, xp[2 * i]), d, false);
          d = __builtin_amdgcn_fdot2(w1, __builtin_bit_cast(h2, xp[2 * i + 1]), d, false);
        } else {
          typedef __bf16 b2 __attribute__((ext_vector_type(2)));
          const b2 w0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w4[i], 1.0f, false);
          const b2 w1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w4[i], 1.0f, true);
          d = __builtin_amdgcn_fdot2_f32_bf16(w0, __builtin_bit_cast(b2, xp[2 * i]), d, false);
          d = __builtin_amdgcn_fdot2_f32_bf16(w1, __builtin_bit_cast(b2, xp[2 * i + 1]), d, false);
        }
      }
      if constexpr (kDirect) acc[r] = valid ? d : acc[r];
      else if constexpr (WS == WS_CHUNK) acc[r] = valid ? fmaf(d, decode_scale_bits<SZ>(rs[slot][r], a.ws_is_f16) * sa, acc[r]) : acc[r];
      else acc[r] = valid ? fmaf(d, sa, acc[r]) : acc[r];
    }
    if (++cs == S) {  // end of a row pair: reduce, scale, bias, store
#pragma unroll
      for (int r = 0; r < kPair; ++r) {
        float v = wave_sum_dpp(acc[r]);
        acc[r] = 0.0f;
        const int n = (gw + cp * W) * kPair + r;
        const int src = cp * kPair + r;  // wave-uniform lane index
        if constexpr (WS == WS_ROW) v *= lane_value(row_s_bits, src, a.wscale_dtype);
        if (a.bias) v += lane_value(row_b_bits, src, a.bias_dtype);
        if (lane == 0 && n < N) store_f32(a.out, a.out_dtype, n, v);
      }
      cs = 0;
      ++cp;
    }
  };

  int it = 0;
  for (; it + kRing <= n_items; it += kRing) {
#pragma unroll
    for (int d = 0; d < kRing; ++d) {
      consume(d);
      issue(d);
    }
  }
#pragma unroll
  for (int d = 0; d < kRing; ++d) {
    if (it + d < n_items) consume(d);
  }
}

constexpr int kRows = 2;    // weight rows per wavefront
constexpr int kUnroll = 4;  // K sweeps in flight per wavefront

// Split plan from shapes only (graph-capture safe): the smallest power-of-two K
// split that gives >= 4096 wavefronts (16 per CU), never splitting below one sweep.
struct SplitPlan {
  int split;
  int64_t k_per_split;
};
SplitPlan gemv_split_plan(int64_t N, int64_t K) {
  const int64_t waves = cdiv(N, kRows);
  const int64_t sweeps = cdiv(K, kWaveK);
  int split = 1;
  while (waves * split < 4096 && split * 2 <= sweeps && split < 64) split *= 2;
  const int64_t kps = cdiv(sweeps, split) * kWaveK;
  split = (int)cdiv(K, kps);
  return {split, kps};
}

template <int ACT, int WS, int AS>
void launch_gemv_fast(GemvArgs& a, int split, hipStream_t st) {
  const dim3 grid((unsigned)cdiv(a.N, (int64_t)kGemvWaves * kRows), (unsigned)split);
  hipLaunchKernelGGL((gemv_kernel<ACT, WS, AS, kRows, kUnroll>), grid, dim3(kGemvThreads), 0, st, a);
}

// Streaming plan: used when N alone yields >= 2048 wavefronts of one row pair each
// and the staged tables fit in LDS. Each wavefront then owns ceil(pairs / 2048) pairs
// (one below 4096 pairs), four wavefronts per workgroup.
constexpr int64_t kStreamWavesTarget = 2048;
bool stream_plan(int act, int as, int64_t N, int64_t K, int64_t& ppw, int& lds) {
  const int64_t npairs = cdiv(N, kPair);
  if (npairs < kStreamWavesTarget) return false;
  // Short rows below twice the target: every wavefront takes one pair (up to 4095
  // wavefronts). Such a projection is ramp-bound, and more wavefronts put more bytes in
  // flight (Llama-3-8B qkv, 3072 pairs of K = 4096: 7.0 -> 6.85 us against 1536
  // wavefronts of two pairs). Long rows keep two pairs per wavefront (DSv3 down,
  // 3584 pairs of K = 18432: 23.5 us, against 25.4 with one).
  ppw = npairs < 2 * kStreamWavesTarget && K <= 4096 ? 1 : cdiv(npairs, kStreamWavesTarget);
  (void)as;
  lds = stream_lds(act, K).total();
  return lds <= kStreamLdsMax && ppw * kPair <= kStreamRowsMax && N < INT32_MAX && K < INT32_MAX;
}

template <int ACT, int WS, int AS, int SZ>
void launch_stream(GemvArgs& a, int lds, hipStream_t st) {
  a.bx_shift = -1;
  for (int sh = 0; sh < 31; ++sh) {
    if ((int64_t)1 << sh == a.bx) a.bx_shift = sh;
  }
  const int64_t waves = cdiv(cdiv(a.N, kPair), a.pairs_per_wave);
  const dim3 grid((unsigned)cdiv(waves, kStreamWaves));
  hipLaunchKernelGGL((gemv_stream_kernel<ACT, WS, AS, SZ>), grid, dim3(kStreamThreads), (unsigned)lds, st, a);
}

template <int ACT, int AS>
void dispatch_stream(GemvArgs& a, bool row_scale, int lds, hipStream_t st) {
  if (row_scale) return launch_stream<ACT, WS_ROW, AS, 4>(a, lds, st);
  a.ws_is_f16 = a.wscale_dtype == AYK_F16;
  switch (a.wscale_dtype) {
    case AYK_U8: return launch_stream<ACT, WS_CHUNK, AS, 1>(a, lds, st);
    case AYK_F32: return launch_stream<ACT, WS_CHUNK, AS, 4>(a, lds, st);
    default: return launch_stream<ACT, WS_CHUNK, AS, 2>(a, lds, st);
  }
}

template <int ACT, int AS>
int run_gemv(GemvArgs a, bool row_scale, size_t ws_bytes, const char* op, hipStream_t st) {
  const bool fast = aligned16(a.w) && aligned16(a.x) && a.ldw % 16 == 0 && a.K % kChunk == 0 &&
                    (row_scale || a.bx % kChunk == 0);
  if (!fast) {
    const dim3 grid((unsigned)cdiv(a.N, kGemvWaves));
    hipLaunchKernelGGL((gemv_generic_kernel<ACT, AS>), grid, dim3(kGemvThreads), 0, st, a);
    return check_launch(op);
  }
  int lds = 0;
  if (stream_plan(ACT, AS, a.N, a.K, a.pairs_per_wave, lds)) {
    dispatch_stream<ACT, AS>(a, row_scale, lds, st);
    return check_launch(op);
  }
  const SplitPlan plan = gemv_split_plan(a.N, a.K);
  a.k_per_split = plan.k_per_split;
  if (plan.split > 1) {
    const size_t need = (size_t)plan.split * (size_t)a.N * sizeof(float);
    if (a.part == nullptr || ws_bytes < need) {
      return fail(AYK_EWORKSPACE, "%s: workspace of %zu bytes required, %zu given", op, need, ws_bytes);
    }
  }
  if (row_scale) launch_gemv_fast<ACT, WS_ROW, AS>(a, plan.split, st);
  else launch_gemv_fast<ACT, WS_CHUNK, AS>(a, plan.split, st);
  if (int rc = check_launch(op)) return rc;
  if (plan.split > 1) {
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)cdiv(a.N, 256)), dim3(256), 0, st,
                       a.part, a.N, plan.split, a.bias, a.bias_dtype, a.out, a.out_dtype);
    return check_launch(op);
  }
  return AYK_OK;
}

size_t gemv_workspace(int act, int as, int64_t N, int64_t K) {
  if (N <= 0 || K <= 0) return 0;
  int64_t ppw;
  int lds;
  if (K % kChunk == 0 && stream_plan(act, as, N, K, ppw, lds)) return 0;
  const SplitPlan plan = gemv_split_plan(N, K);
  return plan.split > 1 ? (size_t)plan.split * (size_t)N * sizeof(float) : 0;
}

bool is_float_dtype(int dt) { return dt == AYK_F32 || dt == AYK_F16 || dt == AYK_BF16; }

}  // namespace

// Used by the MXFP8 GEMM entry point for M == 1.
int mx_gemv(const void* a, const uint8_t* a_scale, const void* w, int64_t ldw,
            const uint8_t* w_scale, int64_t ld_ws, int64_t N, int64_t K, const void* bias,
            int bias_dtype, void* out, int out_dtype, hipStream_t st) {
  GemvArgs g{};
  g.x = a;
  g.w = static_cast<const uint8_t*>(w);
  g.ldw = ldw;
  g.N = N;
  g.K = K;
  g.wscale = w_scale;
  g.wscale_dtype = AYK_U8;
  g.srs = ld_ws;
  g.by = 1;
  g.bx = 32;
  g.ascale = a_scale;
  g.ascale_dtype = AYK_U8;
  g.bias = bias;
  g.bias_dtype = bias_dtype;
  g.out = out;
  g.out_dtype = out_dtype;
  g.part = nullptr;
  // No workspace is available here: force a single K split.
  const bool fast = aligned16(g.w) && aligned16(g.x) && ldw % 16 == 0 && K % kChunk == 0;
  if (!fast) {
    hipLaunchKernelGGL((gemv_generic_kernel<ACT_E4M3, AS_MX32>), dim3((unsigned)cdiv(N, kGemvWaves)),
                       dim3(kGemvThreads), 0, st, g);
    return check_launch("mxfp8_scaled_mm(M=1)");
  }
  int lds = 0;
  if (stream_plan(ACT_E4M3, AS_MX32, N, K, g.pairs_per_wave, lds)) {
    launch_stream<ACT_E4M3, WS_CHUNK, AS_MX32, 1>(g, lds, st);
    return check_launch("mxfp8_scaled_mm(M=1)");
  }
  g.k_per_split = cdiv(K, kWaveK) * kWaveK;
  launch_gemv_fast<ACT_E4M3, WS_CHUNK, AS_MX32>(g, 1, st);
  return check_launch("mxfp8_scaled_mm(M=1)");
}

// ---------------------------------------------------------------- allocation-free form
// A file-scope device array replaces the caller's workspace for callers that cannot
// allocate. The split plan bounds the partials: the split doubles only while
// waves * split < 4096 with waves = ceil(N / 2), so split * N < 16384 and the partials
// stay below 64 KiB for every shape. Each GPU holds its own copy of the array; its
// address is looked up once per device (hipGetSymbolAddress) and only that address is
// handed to kernels. Every split writes all N of its partials before the reduce reads
// them, so nothing needs clearing between calls.
constexpr size_t kScratchBytes = 64 * 1024;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch_ptr[kMaxDevices] = {};

int scratch_of_current_device(float** out) {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return fail(AYK_EARCH, "no HIP device is available");
  if (device < 0 || device >= kMaxDevices) return fail(AYK_EARCH, "device index %d out of range", device);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[device] == nullptr) {
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || p == nullptr) {
      return fail(AYK_ELAUNCH, "static scratch of device %d unavailable: %s", device, hipGetErrorString(err));
    }
    g_scratch_ptr[device] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[device];
  return AYK_OK;
}

}  // namespace ayk

using namespace ayk;

extern "C" {

int ayk_fp8_weight_only_gemv_static(const void* x, int x_dtype, const void* w, int64_t ldw, int64_t N,
                                    int64_t K, const void* scale, int scale_dtype,
                                    int64_t scale_row_stride, int64_t block_size_y,
                                    int64_t block_size_x, void* out, ayk_stream_t stream) {
  const char* op = "fp8_weight_only_gemv_static";
  if (N > 0 && K > 0) {
    const size_t need = gemv_workspace(ACT_BF16, AS_NONE, N, K);
    if (need > kScratchBytes) {
      return fail(AYK_EWORKSPACE, "%s: N=%lld K=%lld needs %zu bytes of partials, above the static scratch of %zu",
                  op, (long long)N, (long long)K, need, kScratchBytes);
    }
  }
  if (N <= 0 || K <= 0) {  // the allocating entry point reports the argument error
    return ayk_fp8_weight_only_gemv(x, x_dtype, w, ldw, N, K, scale, scale_dtype, scale_row_stride, block_size_y,
                                    block_size_x, out, nullptr, 0, stream);
  }
  float* ws = nullptr;
  if (int rc = scratch_of_current_device(&ws)) return rc;
  return ayk_fp8_weight_only_gemv(x, x_dtype, w, ldw, N, K, scale, scale_dtype, scale_row_stride, block_size_y,
                                  block_size_x, out, ws, kScratchBytes, stream);
}

size_t ayk_fp8_weight_only_gemv_static_max_bytes(void) { return kScratchBytes; }

size_t ayk_fp8_weight_only_gemv_workspace_bytes(int64_t N, int64_t K) { return gemv_workspace(ACT_BF16, AS_NONE, N, K); }
size_t ayk_fp8_blockwise_gemv_workspace_bytes(int64_t N, int64_t K) { return gemv_workspace(ACT_E4M3, AS_BLOCK128, N, K); }

int ayk_fp8_weight_only_gemv(const void* x, int x_dtype, const void* w, int64_t ldw, int64_t N,
                             int64_t K, const void* scale, int scale_dtype,
                             int64_t scale_row_stride, int64_t block_size_y,
                             int64_t block_size_x, void* out, void* workspace,
                             size_t workspace_bytes, ayk_stream_t stream) {
  const char* op = "fp8_weight_only_gemv";
  if (x_dtype != AYK_BF16 && x_dtype != AYK_F16) return fail(AYK_EINVAL, "%s: input must be float16 or bfloat16", op);
  if (scale_dtype != AYK_U8 && scale_dtype != AYK_F32 && scale_dtype != AYK_BF16) {
    return fail(AYK_EINVAL, "%s: scale dtype must be e8m0 (uint8), float32 or bfloat16", op);
  }
  if (N < 0 || K < 1 || ldw < K) return fail(AYK_EINVAL, "%s: bad shape N=%lld K=%lld ldw=%lld", op, (long long)N, (long long)K, (long long)ldw);
  if (block_size_y < 1 || block_size_x < 1) return fail(AYK_EINVAL, "%s: block sizes must be positive", op);
  if (scale_row_stride < 1) return fail(AYK_EINVAL, "%s: scale_row_stride must be positive", op);
  if (N == 0) return AYK_OK;
  if (int rc = check_device()) return rc;
  GemvArgs g{};
  g.x = x;
  g.w = static_cast<const uint8_t*>(w);
  g.ldw = ldw;
  g.N = N;
  g.K = K;
  g.wscale = scale;
  g.wscale_dtype = scale_dtype;
  g.srs = scale_row_stride;
  g.by = block_size_y;
  g.bx = block_size_x;
  g.ascale = nullptr;
  g.ascale_dtype = AYK_F32;
  g.bias = nullptr;
  g.bias_dtype = AYK_F32;
  g.out = out;
  g.out_dtype = x_dtype;
  g.part = static_cast<float*>(workspace);
  const bool row_scale = block_size_x >= K;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (x_dtype == AYK_BF16) return run_gemv<ACT_BF16, AS_NONE>(g, row_scale, workspace_bytes, op, st);
  return run_gemv<ACT_F16, AS_NONE>(g, row_scale, workspace_bytes, op, st);
}

int ayk_fp8_blockwise_gemv(const void* a, const void* b, int64_t ldb, int64_t N, int64_t K,
                           const void* scale_a, int sa_dtype, const void* scale_b, int sb_dtype,
                           const void* bias, int bias_dtype, void* out, int out_dtype,
                           void* workspace, size_t workspace_bytes, ayk_stream_t stream) {
  const char* op = "fp8_blockwise_gemv";
  if (!is_float_dtype(sa_dtype) || !is_float_dtype(sb_dtype)) return fail(AYK_EINVAL, "%s: scales must be float32, float16 or bfloat16", op);
  if (!is_float_dtype(out_dtype)) return fail(AYK_EINVAL, "%s: out must be float16, bfloat16, or float32", op);
  if (bias && !is_float_dtype(bias_dtype)) return fail(AYK_EINVAL, "%s: bad bias dtype", op);
  if (N < 0 || K < 1 || ldb < K) return fail(AYK_EINVAL, "%s: bad shape N=%lld K=%lld", op, (long long)N, (long long)K);
  if (N == 0) return AYK_OK;
  if (int rc = check_device()) return rc;
  GemvArgs g{};
  g.x = a;
  g.w = static_cast<const uint8_t*>(b);
  g.ldw = ldb;
  g.N = N;
  g.K = K;
  g.wscale = scale_b;
  g.wscale_dtype = sb_dtype;
  g.srs = cdiv(K, 128);
  g.by = 128;
  g.bx = 128;
  g.ascale = scale_a;
  g.ascale_dtype = sa_dtype;
  g.bias = bias;
  g.bias_dtype = bias_dtype;
  g.out = out;
  g.out_dtype = out_dtype;
  g.part = static_cast<float*>(workspace);
  return run_gemv<ACT_E4M3, AS_BLOCK128>(g, false, workspace_bytes, op, static_cast<hipStream_t>(stream));
}

}  // extern "C"
