// FP8 x FP8 GEMM for decode batches, M <= 64 (fp8_scaled_mm rowwise / per-tensor,
// mxfp8_scaled_mm and fp8_blockwise_mm), gfx950.
//
//   out[m, n] = sum_k a[m, k] w[n, k] * sa[m] * sb[n] (+ bias[n])          (fp32 scales)
//   out[m, n] = sum_k a[m, k] 2^ea[m, k/32] w[n, k] 2^ew[n, k/32] (+ bias)   (UE8M0 codes)
//   out[m, n] = sum_kb sa[m, kb] sb[n/128, kb] sum_{k in kb} a[m, k] w[n, k] (+ bias)  (block-128)
//
// (python/ayaka/kernel/triton/gemm/fp8_gemm.py:127-204, 246, fp8_mxfp8_gemm.py:163;
// oracle reference/gemm.py:17-92.) At these batch sizes the weight bytes bound the
// work, so the kernel is a weight stream, the structure of the W8A16 decode stream
// kernel: every wavefront streams its own 32 FN weight rows through a private LDS ring
// of 3 stages, one 128-K "pair" per stage, filled by direct-to-LDS loads of 8 rows x
// 128 contiguous bytes (nontemporal: read once), with no workgroup barrier per stage.
// The activation rows are shared: the workgroup stages them into double-buffered LDS
// chunks of G pairs, each wavefront loading its share with the chunk's first stage,
// one barrier per chunk. With KS > 1 the KS wavefronts of a row group take the KS
// parts of the K range and their sums meet in LDS at the end.
//
// MFMA v_mfma_scale_f32_32x32x64_f8f6f4 in the 256 x 256 pair kernel's arrangement:
// the weight is operand A (a 32-row tile), the activations operand B (32 rows); for
// step t of a pair, lane (r = lane % 32, h = lane / 32) holds K [64 t + 16 h, + 16) and
// [64 t + 32 + 16 h, + 16) of its row, which puts the hardware's 32-K scale block b at
// memory K [64 t + 32 b, + 32), i.e. MX group 2 t + b: lane half h passes byte 2 t + h
// of its row's code dword for the pair. LDS row r holds logical 16-byte chunk c at
// physical chunk c ^ ((r >> 1) & 7), so the 32 rows of a fragment read fall on distinct
// banks. fp32 scales (and the bias) are applied in the epilogue; MX codes enter the
// MFMA (the MX UE8M0 decode of the reference, code 0 as 2^-127, is the MFMA's); block-128
// scales fold each 128-K stage's partial sums.
#include "gemm_skinny.h"

#include <utility>

#include "ayk_common.h"
#include "gemm_util.h"
#include "quant_math.h"

namespace ayk {
namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kPairK = 128;  // K bytes per stage
constexpr int kDepth = 3;    // stages in a wavefront's ring
constexpr int kCodeOne = 127;

// Scale modes: fp32 per-row / per-tensor scales in the epilogue, UE8M0 codes inside the
// MFMA, or block-128 fp32 scales folded after every 128-K stage.
constexpr int kSmScaled = 0, kSmMx = 1, kSmBlock = 2;
// Scale loads per stage (64 dwords each, through LDS): MX, one code dword per weight and
// activation row; block-128, one activation scale per row plus the wavefront's weight
// scale (its rows lie in one 128-row block).
constexpr int scale_ins(int sm, int fn, int fm) {
  return sm == kSmMx ? (fn + fm + 1) / 2 : (sm == kSmBlock ? (32 * fm + 64) / 64 : 0);
}

template <typename F, int... I>
__device__ inline void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ inline void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

__device__ inline uint32_t lds_u32(const uint8_t* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p;
}
__device__ inline void dma16_nt(const uint8_t* src, uint8_t* lds_dst) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_dst, 16, 0, 2);
}
__device__ inline void dma16(const uint8_t* src, uint8_t* lds_dst) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_dst, 16, 0, 0);
}

// All LDS reads of one step in one assembly statement ending with lgkmcnt(0): the
// compiler cannot relate them to the direct loads in flight into other buffers (it would
// otherwise wait for all of them first), and every result is final when it ends.
template <int NB>
__device__ inline void step_reads(v4u (&b)[NB], const uint32_t (&ab)[NB]);
#define AYK_SR(o, i) "ds_read_b128 %" #o ", %" #i "\n\t"
template <>
__device__ inline void step_reads<4>(v4u (&b)[4], const uint32_t (&ab)[4]) {
  asm volatile(AYK_SR(0, 4) AYK_SR(1, 5) AYK_SR(2, 6) AYK_SR(3, 7) "s_waitcnt lgkmcnt(0)"
               : "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(b[3])
               : "v"(ab[0]), "v"(ab[1]), "v"(ab[2]), "v"(ab[3])
               : "memory");
}
template <>
__device__ inline void step_reads<6>(v4u (&b)[6], const uint32_t (&ab)[6]) {
  asm volatile(AYK_SR(0, 6) AYK_SR(1, 7) AYK_SR(2, 8) AYK_SR(3, 9) AYK_SR(4, 10) AYK_SR(5, 11) "s_waitcnt lgkmcnt(0)"
               : "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(b[3]), "=&v"(b[4]), "=&v"(b[5])
               : "v"(ab[0]), "v"(ab[1]), "v"(ab[2]), "v"(ab[3]), "v"(ab[4]), "v"(ab[5])
               : "memory");
}
template <>
__device__ inline void step_reads<8>(v4u (&b)[8], const uint32_t (&ab)[8]) {
  asm volatile(AYK_SR(0, 8) AYK_SR(1, 9) AYK_SR(2, 10) AYK_SR(3, 11) AYK_SR(4, 12) AYK_SR(5, 13) AYK_SR(6, 14)
               AYK_SR(7, 15) "s_waitcnt lgkmcnt(0)"
               : "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(b[3]), "=&v"(b[4]), "=&v"(b[5]), "=&v"(b[6]), "=&v"(b[7])
               : "v"(ab[0]), "v"(ab[1]), "v"(ab[2]), "v"(ab[3]), "v"(ab[4]), "v"(ab[5]), "v"(ab[6]), "v"(ab[7])
               : "memory");
}
#undef AYK_SR

// The code dwords of a stage (one per fragment row), likewise in one statement.
template <int NC>
__device__ inline void code_reads(uint32_t (&c)[NC], const uint32_t (&ac)[NC]);
template <>
__device__ inline void code_reads<2>(uint32_t (&c)[2], const uint32_t (&ac)[2]) {
  asm volatile("ds_read_b32 %0, %2\n\tds_read_b32 %1, %3\n\ts_waitcnt lgkmcnt(0)"
               : "=&v"(c[0]), "=&v"(c[1])
               : "v"(ac[0]), "v"(ac[1])
               : "memory");
}
template <>
__device__ inline void code_reads<3>(uint32_t (&c)[3], const uint32_t (&ac)[3]) {
  asm volatile("ds_read_b32 %0, %3\n\tds_read_b32 %1, %4\n\tds_read_b32 %2, %5\n\ts_waitcnt lgkmcnt(0)"
               : "=&v"(c[0]), "=&v"(c[1]), "=&v"(c[2])
               : "v"(ac[0]), "v"(ac[1]), "v"(ac[2])
               : "memory");
}
template <>
__device__ inline void code_reads<4>(uint32_t (&c)[4], const uint32_t (&ac)[4]) {
  asm volatile(
      "ds_read_b32 %0, %4\n\tds_read_b32 %1, %5\n\tds_read_b32 %2, %6\n\tds_read_b32 %3, %7\n\ts_waitcnt lgkmcnt(0)"
      : "=&v"(c[0]), "=&v"(c[1]), "=&v"(c[2]), "=&v"(c[3])
      : "v"(ac[0]), "v"(ac[1]), "v"(ac[2]), "v"(ac[3])
      : "memory");
}

struct KArgs {
  SkinnyFp8Args g;
  int64_t kps;  // K per grid-y split
};

// Epilogue: scales (fp32 mode), bias, output type, or the grid-y partials.
// acc[i][j][4 grp + qq] = D[n = n_wave + 32 i + 8 grp + 4 h + qq][m = 32 j + frow].
template <int SM, int FN, int FM>
__device__ inline void store_tiles(const KArgs& ka, const v16f (&acc)[FN][FM], int64_t n_wave, int frow, int h) {
  const SkinnyFp8Args& g = ka.g;
  const bool split = gridDim.y > 1;
  const float* sa = static_cast<const float*>(g.sa);
  const float* sb = static_cast<const float*>(g.sb);
  const int eb = g.out_dtype == AYK_F32 ? 4 : 2;
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int64_t m = 32 * j + frow;
    if (m >= g.M) continue;
    const float sam = SM == kSmScaled ? sa[g.sa_vec ? m : 0] : 1.0f;
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int grp = 0; grp < 4; ++grp) {
        const int64_t n0 = n_wave + 32 * i + 8 * grp + 4 * h;
        float v[4];
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const int64_t n = n0 + qq < g.N ? n0 + qq : g.N - 1;
          float y = acc[i][j][4 * grp + qq];
          if constexpr (SM == kSmScaled) y = (y * sam) * sb[g.sb_vec ? n : 0];
          if (!split && g.bias) y += load_f32(g.bias, g.bias_dtype, n);
          v[qq] = y;
        }
        if (split) {
          float* pr = ka.g.ws + ((int64_t)blockIdx.y * g.M + m) * g.N;
#pragma unroll
          for (int qq = 0; qq < 4; ++qq)
            if (n0 + qq < g.N) pr[n0 + qq] = v[qq];
        } else if (n0 + 3 < g.N && eb == 2 &&
                   (reinterpret_cast<uintptr_t>(static_cast<uint16_t*>(g.out) + m * g.ldo + n0) & 7) == 0) {
          uint32_t pk[2];
#pragma unroll
          for (int qq = 0; qq < 2; ++qq) {
            if (g.out_dtype == AYK_BF16) pk[qq] = pack_bf16x2(v[2 * qq], v[2 * qq + 1]);
            else pk[qq] = (uint32_t)f32_to_f16_bits(v[2 * qq]) | ((uint32_t)f32_to_f16_bits(v[2 * qq + 1]) << 16);
          }
          *reinterpret_cast<uint2*>(static_cast<uint16_t*>(g.out) + m * g.ldo + n0) = make_uint2(pk[0], pk[1]);
        } else {
#pragma unroll
          for (int qq = 0; qq < 4; ++qq)
            if (n0 + qq < g.N) store_f32(g.out, g.out_dtype, m * g.ldo + n0 + qq, v[qq]);
        }
      }
  }
}

// FN 32-row weight tiles per wavefront, FM 32-row activation tiles (M <= 32 FM), KS K
// parts per row group, G pairs per activation chunk, CH stages per scale load (1: one
// 4-byte scale per row and stage; 4: one 16-byte load per row covers four stages,
// double-buffered per wavefront, for 16-byte aligned scale rows).
template <int SM, int FN, int FM, int KS, int G, int CH>
__global__ __launch_bounds__(kWaves * kWave, FN == 1 && KS == 1 ? 2 : 1) void fp8_skinny_kernel(KArgs ka) {
  const SkinnyFp8Args& g = ka.g;
  constexpr bool MX = SM == kSmMx, BLK = SM == kSmBlock;
  constexpr int D = kDepth;
  constexpr int RW = 32 * FN;                // weight rows per wavefront
  constexpr int RG = kWaves / KS;            // row groups per workgroup
  constexpr int R = RG * RW;                 // weight rows per workgroup
  constexpr int MP = 32 * FM;                // activation rows staged
  constexpr int kWStage = RW * kPairK;       // bytes of a wavefront stage
  constexpr int kWIns = kWStage / 1024;      // direct loads per wavefront stage
  constexpr int kXRow = kPairK * G;          // bytes of one activation row of a chunk part
  constexpr int kXPart = MP * kXRow;
  constexpr int kXChunk = KS * kXPart;
  constexpr int kXIns = kXChunk / (1024 * kWaves);  // activation loads per wavefront and chunk
  constexpr int kCodeIns = scale_ins(SM, FN, FM);  // scale loads per stage (CH = 1) or per CH stages
  static_assert(CH == 1 || (CH == 4 && D - 1 <= CH), "a scale buffer is refilled after its last stage");
  constexpr int lcm2 = G % D == 0 ? G : (D % G == 0 ? D : G * D);
  constexpr int U = lcm2 % CH == 0 ? lcm2 : (CH % lcm2 == 0 ? CH : lcm2 * CH);  // a multiple of G, D and CH
  static_assert(kXChunk % (1024 * kWaves) == 0, "whole activation loads per wavefront");
  static_assert(D - 1 <= G, "an activation buffer is refilled only after a barrier past its last read");
  constexpr auto wait_after = [](int u) {  // loads issued after stage s, before its wait
    int n = 0;
    for (int t = u + 1; t <= u + D - 2; ++t) n += kWIns + (t % CH == 0 ? kCodeIns : 0) + (t % G == 0 ? kXIns : 0);
    return n;
  };
  static_assert(wait_after(0) <= 63 && wait_after(G - 1) <= 63, "vmcnt range");

  __shared__ __attribute__((aligned(1024))) uint8_t wring[kWaves * D * kWStage];
  __shared__ __attribute__((aligned(1024))) uint8_t xbuf[2 * kXChunk];
  constexpr int kCodeSlots = CH == 1 ? D : 2;  // scale buffers per wavefront
  __shared__ __attribute__((aligned(16))) uint32_t cring[kCodeIns ? kWaves * kCodeSlots * kCodeIns * kWave * CH : 1];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int frow = lane & 31, h = lane >> 5;
  uint8_t* myring = wring + wave * D * kWStage;
  const int part = wave / RG, rg = wave % RG;
  const int64_t n_wave = (int64_t)blockIdx.x * R + rg * RW;
  const int64_t kbeg = (int64_t)blockIdx.y * ka.kps;
  const int64_t klen = g.K - kbeg < ka.kps ? g.K - kbeg : ka.kps;
  const int64_t plen = klen / KS;  // whole chunks of G pairs (host plan)
  const int64_t kpart = kbeg + part * plen;
  const int ns = (int)(plen / kPairK);

  // Weight loads: load j of a stage covers rows 8 j .. 8 j + 7 of the wavefront, lane L
  // row 8 j + L / 8 at physical chunk L % 8; rows past N re-read row N - 1.
  const uint8_t* wsrc[kWIns];
#pragma unroll
  for (int j = 0; j < kWIns; ++j) {
    const int row = 8 * j + (lane >> 3);
    const int64_t n = n_wave + row < g.N ? n_wave + row : g.N - 1;
    wsrc[j] = g.w + n * g.ldw + kpart + 16 * ((lane & 7) ^ ((row >> 1) & 7));
  }
  // Activation loads: load j of wavefront w fills chunk bytes 1024 (w kXIns + j) ..:
  // K part q, row m, pair segment sg and physical chunk p of that row; rows past M
  // repeat row M - 1.
  const uint8_t* xsrc[kXIns];
  uint32_t xdst[kXIns];
#pragma unroll
  for (int j = 0; j < kXIns; ++j) {
    const int byte = 1024 * (wave * kXIns + j) + 16 * lane;
    const int q = byte / kXPart;
    const int m = (byte % kXPart) / kXRow;
    const int within = byte % kXRow;
    const int sg = within / kPairK, p = (within % kPairK) / 16;
    const int64_t mm = m < g.M ? m : g.M - 1;
    xsrc[j] = g.a + mm * g.lda + kbeg + q * plen + sg * kPairK + 16 * (p ^ ((m >> 1) & 7));
    xdst[j] = __builtin_amdgcn_readfirstlane(1024 * (wave * kXIns + j));
  }
  // Scale dwords of a stage, through LDS like the operands (a register load would be
  // waited for with every direct load before it). Entry e = 64 j + lane of load j, at
  // csrc[j] + stage cstep[j]:
  //   MX: weight row e of the wavefront for e < 32 FN, then activation row e - 32 FN;
  //   block-128: activation row e for e < 32 FM, then the wavefront's weight scale.
  // Entries past the last repeat it; rows past N or M repeat the last row.
  const uint8_t* csrc[kCodeIns ? kCodeIns : 1];
  uint32_t cstep[kCodeIns ? kCodeIns : 1];
  uint32_t* mycodes = cring + wave * kCodeSlots * kCodeIns * kWave * CH;
  if constexpr (MX) {
#pragma unroll
    for (int j = 0; j < kCodeIns; ++j) {
      int e = kWave * j + lane;
      e = e < 32 * (FN + FM) ? e : 32 * (FN + FM) - 1;
      if (e < 32 * FN) {
        const int64_t n = n_wave + e < g.N ? n_wave + e : g.N - 1;
        csrc[j] = static_cast<const uint8_t*>(g.sb) + n * g.ld_sb + kpart / 32;
      } else {
        const int64_t m = e - 32 * FN < g.M ? e - 32 * FN : g.M - 1;
        csrc[j] = static_cast<const uint8_t*>(g.sa) + m * g.ld_sa + kpart / 32;
      }
      cstep[j] = kPairK / 32;
    }
  }
  if constexpr (BLK) {
    const int64_t kb0 = kpart / kPairK;
    const int64_t nb = (n_wave < g.N ? n_wave : g.N - 1) / 128;
#pragma unroll
    for (int j = 0; j < kCodeIns; ++j) {
      int e = kWave * j + lane;
      e = e < 32 * FM + 1 ? e : 32 * FM;
      if (e < 32 * FM) {
        const int64_t m = e < g.M ? e : g.M - 1;
        csrc[j] = reinterpret_cast<const uint8_t*>(static_cast<const float*>(g.sa) +
                                                   (g.sa_vec ? kb0 * g.M + m : m * g.ld_sa + kb0));
        cstep[j] = g.sa_vec ? 4 * (uint32_t)g.M : 4;
      } else {
        csrc[j] = reinterpret_cast<const uint8_t*>(static_cast<const float*>(g.sb) + nb * g.ld_sb + kb0);
        cstep[j] = 4;
      }
    }
  }

  // Stage t (clamped to the last; a clamped stage only rewrites data no later stage
  // reads, or the same data) into slot t % D; the chunk's activations with its first
  // stage (xl: t % G == 0) and, with CH = 4, the scales of stages t .. t + 3 with stage t
  // (sl: t % 4 == 0), both known at compile time at every call site.
  auto issue = [&](int slot, int t, bool xl, bool sl) {
    const int tc = t < ns ? t : ns - 1;
    const int64_t k = (int64_t)tc * kPairK;
#pragma unroll
    for (int j = 0; j < kWIns; ++j) dma16_nt(wsrc[j] + k, myring + slot * kWStage + 1024 * j);
    if constexpr (kCodeIns > 0 && CH == 1) {
#pragma unroll
      for (int j = 0; j < kCodeIns; ++j)
        __builtin_amdgcn_global_load_lds(csrc[j] + (int64_t)tc * cstep[j],
                                         (__attribute__((address_space(3))) void*)(mycodes + (slot * kCodeIns + j) * kWave),
                                         4, 0, 0);
    }
    if constexpr (kCodeIns > 0 && CH == 4) {
      if (sl) {
        const int c = tc / CH;
#pragma unroll
        for (int j = 0; j < kCodeIns; ++j)
          dma16(csrc[j] + (int64_t)c * CH * cstep[j],
                reinterpret_cast<uint8_t*>(mycodes + ((c & 1) * kCodeIns + j) * kWave * CH));
      }
    }
    if (xl) {
      const int c = tc / G;
      uint8_t* xb = xbuf + (c & 1) * kXChunk;
#pragma unroll
      for (int j = 0; j < kXIns; ++j) dma16(xsrc[j] + (int64_t)c * kXRow, xb + xdst[j]);
    }
  };

  v16f acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  const int fsw = (frow >> 1) & 7;
  auto compute = [&](int slot, int s) {
    const uint32_t wbase = lds_u32(myring + slot * kWStage);
    const uint32_t xbase = lds_u32(xbuf + ((s / G) & 1) * kXChunk + part * kXPart) + (uint32_t)((s % G) * kPairK);
    uint32_t wc[FN], xc[FM];
    float bsc[FM];  // block-128: sa[m, kb] sb[n / 128, kb] of this lane's row of tile j
    // Scale entry e of this stage: buffer base + e (4 CH) + 4 (s mod CH).
    const uint32_t cb = CH == 1 ? lds_u32(reinterpret_cast<const uint8_t*>(mycodes + slot * kCodeIns * kWave))
                                : lds_u32(reinterpret_cast<const uint8_t*>(mycodes + ((s / CH) & 1) * kCodeIns * kWave * CH)) +
                                      4 * (s % CH);
    if constexpr (BLK) {
      uint32_t ca[FM + 1], cv[FM + 1];
#pragma unroll
      for (int j = 0; j < FM; ++j) ca[j] = cb + 4 * CH * (32 * j + frow);
      ca[FM] = cb + 4 * CH * 32 * FM;
      code_reads<FM + 1>(cv, ca);
#pragma unroll
      for (int j = 0; j < FM; ++j) bsc[j] = __builtin_bit_cast(float, cv[j]) * __builtin_bit_cast(float, cv[FM]);
    }
    v16f part[BLK ? FN : 1][BLK ? FM : 1];
    if constexpr (MX) {
      uint32_t ca[FN + FM];
#pragma unroll
      for (int i = 0; i < FN + FM; ++i) ca[i] = cb + 4 * CH * (32 * i + frow);
      uint32_t cv[FN + FM];
      code_reads<FN + FM>(cv, ca);
#pragma unroll
      for (int i = 0; i < FN; ++i) wc[i] = cv[i];
#pragma unroll
      for (int j = 0; j < FM; ++j) xc[j] = cv[FN + j];
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      constexpr int NB = 2 * (FN + FM);
      uint32_t ab[NB];
      v4u v[NB];
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        const uint32_t row = wbase + (32 * i + frow) * kPairK;
        ab[2 * i] = row + (((4 * t + h) ^ fsw) << 4);
        ab[2 * i + 1] = row + (((4 * t + 2 + h) ^ fsw) << 4);
      }
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const uint32_t row = xbase + (32 * j + frow) * kXRow;
        ab[2 * FN + 2 * j] = row + (((4 * t + h) ^ fsw) << 4);
        ab[2 * FN + 2 * j + 1] = row + (((4 * t + 2 + h) ^ fsw) << 4);
      }
      step_reads<NB>(v, ab);
      const int sh = 8 * (2 * t + h);
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        const v8i wf = __builtin_shufflevector(__builtin_bit_cast(v4i, v[2 * i]), __builtin_bit_cast(v4i, v[2 * i + 1]), 0, 1, 2, 3, 4, 5, 6, 7);
        const int cw = MX ? (int)(wc[i] >> sh) : kCodeOne;
#pragma unroll
        for (int j = 0; j < FM; ++j) {
          const v8i xf = __builtin_shufflevector(__builtin_bit_cast(v4i, v[2 * FN + 2 * j]),
                                                 __builtin_bit_cast(v4i, v[2 * FN + 2 * j + 1]), 0, 1, 2, 3, 4, 5, 6, 7);
          const int cx = MX ? (int)(xc[j] >> sh) : kCodeOne;
          if constexpr (BLK) {
            const v16f c = t == 0 ? v16f{} : part[i][j];
            part[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf, xf, c, 0, 0, 0, cw, 0, cx);
          } else {
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf, xf, acc[i][j], 0, 0, 0, cw, 0, cx);
          }
        }
      }
    }
    if constexpr (BLK) {  // fold the 128-K block: one fma per accumulator
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] = __builtin_fmaf(part[i][j][r], bsc[j], acc[i][j][r]);
    }
  };

#pragma unroll
  for (int d = 0; d < D - 1; ++d) issue(d, d, d % G == 0, d % CH == 0);
  // Step s: wait for stage s (its activation chunk too), at a chunk start a barrier,
  // refill slot (s - 1) % D with stage s + D - 1, compute stage s. The main loop runs
  // whole rounds of U steps with no exit inside; the remainder runs after it.
  auto step = [&](auto uc, int s) {
    constexpr int u = decltype(uc)::value;
    wait_vmcnt<wait_after(u % G)>();
    if (u % G == 0) __builtin_amdgcn_s_barrier();
    issue((u + D - 1) % D, s + D - 1, (u + D - 1) % G == 0, (u + D - 1) % CH == 0);
    compute(u % D, s);
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
    // The K parts of a row group meet in LDS in part order (the rings are free once
    // every wavefront is past its last stage).
    constexpr int kSlots = FN * FM * 16;
    static_assert(kWaves * kSlots * kWave * 4 <= kWaves * D * kWStage, "the sums fit the rings");
    float* red = reinterpret_cast<float*>(wring);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) red[(wave * kSlots + (i * FM + j) * 16 + r) * kWave + lane] = acc[i][j][r];
    __syncthreads();
    if (part != 0) return;
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float v = 0.0f;
#pragma unroll
          for (int qq = 0; qq < KS; ++qq) v += red[((qq * RG + rg) * kSlots + (i * FM + j) * 16 + r) * kWave + lane];
          acc[i][j][r] = v;
        }
  }

  store_tiles<SM, FN, FM>(ka, acc, n_wave, frow, h);
}

// Fixed-order sum of the grid-y partials, bias, one rounding.
__global__ __launch_bounds__(256) void skinny_reduce(const float* __restrict__ part, int64_t M, int64_t N, int split,
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

// Launch plan from the shape alone (the workspace query reproduces it), in three tiers
// (below), from a sweep over (FN, KS, G, split) on the decode shapes: two resident
// workgroups of 32-row wavefronts beat one of 64-row wavefronts or of K parts wherever
// the grid reaches half the chip (DeepSeek-V3 block-128 at M = 32, up and down: 42.7 ->
// 37.9 us and 37.7 -> 31.6 us against the previous plan).
struct SkPlan {
  bool ok;
  int fn, fm, ks, g, split;
  int64_t kps;
};
constexpr int64_t skinny_lds(int fn, int fm, int ks, int g, int sm, int ch = 1) {
  return (int64_t)kWaves * kDepth * 4096 * fn + 2LL * ks * 32 * fm * kPairK * g +
         (int64_t)kWaves * (ch == 1 ? kDepth : 2) * scale_ins(sm, fn, fm) * kWave * 4 * ch;
}
SkPlan skinny_plan(int64_t M, int64_t N, int64_t K, int sm) {
  SkPlan p{};
  if (M < 1 || M > 64 || N < 1 || K % 256 || K >= ((int64_t)1 << 31)) return p;
  p.fm = M <= 32 ? 1 : 2;
  // 1. 64 rows per wavefront (256 a workgroup) where that alone gives >= 192 workgroups.
  if (cdiv(N, 256) >= 192 && skinny_lds(2, p.fm, 1, 2, sm) <= 160 * 1024) {
    p.fn = 2;
    p.ks = 1;
    p.g = p.fm == 1 && K % (4 * kPairK) == 0 ? 4 : 2;
    p.split = 1;
    p.kps = K;
    p.ok = true;
    return p;
  }
  // 2. 32 rows per wavefront, whole K per wavefront, 2-pair chunks: <= 80 KB of LDS, two
  // workgroups per CU; a grid K split up to 256 workgroups (>= 2048 K each), taken when
  // it reaches >= 128 workgroups.
  {
    const int64_t w1 = cdiv(N, 128);
    int64_t split = 1;
    while (w1 * split * 2 <= 256 && K % (2 * kPairK * split * 2) == 0 && K / (split * 2) >= 2048) split *= 2;
    if (w1 * split >= 128) {
      p.fn = 1;
      p.ks = 1;
      p.g = 2;
      p.split = (int)split;
      p.kps = K / split;
      p.ok = w1 <= 0x7FFFFFFF;
      return p;
    }
  }
  // 3. Narrow projections: K parts inside the workgroup. The first of (FN, KS) = (1, 1),
  // (2, 4), (1, 2), (1, 4) giving >= 192 workgroups (R >= 32 FM, K a multiple of KS
  // 2-pair chunks, LDS within 160 KB), else the last admissible, then a grid K split up
  // to 256 workgroups.
  const int cand[4][2] = {{1, 1}, {2, 4}, {1, 2}, {1, 4}};
  int pick = -1;
  for (int c = 0; c < 4; ++c) {
    const int fn = cand[c][0], ks = cand[c][1];
    const int r = 32 * fn * (kWaves / ks);
    if (r < 32 * p.fm || K % (ks * kPairK * 2) || skinny_lds(fn, p.fm, ks, 2, sm) > 160 * 1024) continue;
    pick = c;
    if (cdiv(N, r) >= 192) break;
  }
  if (pick < 0) return p;
  p.fn = cand[pick][0];
  p.ks = cand[pick][1];
  p.g = 2;
  const int64_t wgs = cdiv(N, 32 * p.fn * (kWaves / p.ks));
  const int64_t gran = (int64_t)p.ks * kPairK * p.g;  // K of one chunk over all parts
  int64_t split = 1;
  while (wgs * split * 2 <= 256 && K % (gran * split * 2) == 0 && K / (split * 2) >= 2048) split *= 2;
  p.split = (int)split;
  p.kps = K / split;
  p.ok = wgs <= 0x7FFFFFFF;
  return p;
}

template <int SM, int FN, int FM, int KS, int CH>
bool launch_gc(const SkPlan& p, const KArgs& ka, hipStream_t st) {
  const dim3 grid((unsigned)cdiv(ka.g.N, 32 * FN * (kWaves / KS)), (unsigned)p.split), block(kWaves * kWave);
  if constexpr (skinny_lds(FN, FM, KS, 2, SM, CH) <= 160 * 1024) {
    if (p.g == 2) {
      hipLaunchKernelGGL((fp8_skinny_kernel<SM, FN, FM, KS, 2, CH>), grid, block, 0, st, ka);
      return true;
    }
  }
  if constexpr (KS * FM == 1 && skinny_lds(FN, FM, KS, 4, SM, CH) <= 160 * 1024) {
    if (p.g == 4) {
      hipLaunchKernelGGL((fp8_skinny_kernel<SM, FN, FM, KS, 4, CH>), grid, block, 0, st, ka);
      return true;
    }
  }
  return false;
}
template <int SM, int FN, int FM, int KS>
bool launch_g(const SkPlan& p, const KArgs& ka, hipStream_t st, int ch) {
  if (ch == 4) return launch_gc<SM, FN, FM, KS, 4>(p, ka, st);
  return launch_gc<SM, FN, FM, KS, 1>(p, ka, st);
}

template <int SM>
bool launch_sm(const SkPlan& p, const KArgs& ka, hipStream_t st, int ch) {
  const int key = p.fn * 100 + p.fm * 10 + p.ks;
  switch (key) {
    case 211: return launch_g<SM, 2, 1, 1>(p, ka, st, ch);
    case 221: return launch_g<SM, 2, 2, 1>(p, ka, st, ch);
    case 111: return launch_g<SM, 1, 1, 1>(p, ka, st, ch);
    case 121: return launch_g<SM, 1, 2, 1>(p, ka, st, ch);
    case 214: return launch_g<SM, 2, 1, 4>(p, ka, st, ch);
    case 112: return launch_g<SM, 1, 1, 2>(p, ka, st, ch);
    case 122: return launch_g<SM, 1, 2, 2>(p, ka, st, ch);
    case 114: return launch_g<SM, 1, 1, 4>(p, ka, st, ch);
    default: return false;
  }
}

// Stages per scale load: 4 (one 16-byte load per scale row) when every row of scales is
// 16-byte aligned at each part's first stage and a part's stages come in whole fours, and
// the extra LDS keeps the plan's workgroups per CU; else 1. Block-128 needs row-major
// activation scales (a row's blocks contiguous).
int scale_chunk(const SkinnyFp8Args& g, const SkPlan& p) {
  if (g.mode == kSmScaled) return 1;
  const int64_t plen = p.kps / p.ks;
  if (plen % (4 * kPairK) || (reinterpret_cast<uintptr_t>(g.sa) & 15) || (reinterpret_cast<uintptr_t>(g.sb) & 15)) return 1;
  if (g.mode == kSmMx && (g.ld_sa % 16 || g.ld_sb % 16)) return 1;
  if (g.mode == kSmBlock && (g.sa_vec || g.ld_sa % 4 || g.ld_sb % 4)) return 1;
  const int64_t l1 = skinny_lds(p.fn, p.fm, p.ks, p.g, g.mode, 1), l4 = skinny_lds(p.fn, p.fm, p.ks, p.g, g.mode, 4);
  if (l4 > 160 * 1024 || (l1 <= 80 * 1024 && l4 > 80 * 1024)) return 1;
  return 4;
}

// Small decode batches of the fp32-scaled (rowwise / per-tensor) GEMM: 2 to 8 rows
// against a weight of at most 2^24 bytes, where the MFMA decode-batch kernel's fixed
// cost (its LDS ring, 32-row fragments and at least 32 weight rows per wavefront) is
// most of its time. A GEMV-shaped kernel instead: the workgroup stages the activation
// rows (M x K bytes) in LDS, each wavefront owns two weight rows and walks K in
// 1024-byte sweeps (one 16-byte vector per lane and row), and each lane keeps 2 x MR
// fp32 sums of exact fp8 products (VALU fmas), reduced across the wavefront at the
// end. out = (sum * sa[m]) * sb[n] + bias[n], rounded once, as the MFMA kernels.
// Measured against the MFMA kernel: Cfg1's 3072 x 1024 at M = 8 7.2 -> 5.7 us,
// 4096 x 2048 at M = 8 9.2 -> 7.9 us, 4096 x 4096 at M = 2 11.0 -> 5.9 us.
constexpr int kRgThreads = 256;
constexpr int kRgRows = 2 * (kRgThreads / kWave);  // weight rows per workgroup
// QUANT: the activation arrives in bf16 / fp16 / fp32 (T, at x with row stride ldx in
// elements) and the workgroup quantizes it per token itself, with the per-token
// quantizer's arithmetic (quant_math.h: magnitude-bit amax, clamp_min(1e-10) / 448,
// Markstein quotient or IEEE division for non-finite rows), into the same e4m3 bytes
// and fp32 scales that per_token_quant_fp8 writes; the product is then the one the
// unfused pair of launches computes, bit for bit.
template <int MR, bool QUANT, typename T>
__global__ __launch_bounds__(kRgThreads) void fp8_rows_gemv_kernel(SkinnyFp8Args g, const void* x, int64_t ldx) {
  extern __shared__ __attribute__((aligned(16))) uint8_t xs[];  // [M][K] e4m3
  __shared__ float sas[QUANT ? MR : 1];                       // per-token scales (QUANT)
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int K = (int)g.K, M = (int)g.M;
  if constexpr (QUANT) {
    // Wavefront w quantizes rows w and w + 4. The loads of both rows are issued before
    // any reduction, and the first kHeld vectors per lane of each row stay in registers
    // for the quantizing pass (a second read only past kHeld * 64 vectors), so the
    // prologue is one memory round trip rather than two per row.
    constexpr int V = Vec16<T>::N;
    constexpr int kWaves = kRgThreads / kWave;
    constexpr int kRowsPerWave = (MR + kWaves - 1) / kWaves;
    constexpr int kHeld = 4;
    const int nvec = K / V;
    uint4 held[kRowsPerWave][kHeld];
#pragma unroll
    for (int rr = 0; rr < kRowsPerWave; ++rr) {
      const int m = wave + kWaves * rr;
      const uint4* xr = reinterpret_cast<const uint4*>(static_cast<const typename T::storage*>(x) + (int64_t)(m < M ? m : 0) * ldx);
#pragma unroll
      for (int h = 0; h < kHeld; ++h) {
        const int v = lane + kWave * h;
        held[rr][h] = m < M && v < nvec ? xr[v] : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int rr = 0; rr < kRowsPerWave; ++rr) {
      const int m = wave + kWaves * rr;
      if (m >= M) continue;  // wavefront-uniform
      const uint4* xr = reinterpret_cast<const uint4*>(static_cast<const typename T::storage*>(x) + (int64_t)m * ldx);
      uint32_t bits = 0;
#pragma unroll
      for (int h = 0; h < kHeld; ++h) bits = absbits_max<T>(held[rr][h], bits);  // zeros past the row add nothing
      for (int v = lane + kWave * kHeld; v < nvec; v += kWave) bits = absbits_max<T>(xr[v], bits);
      bits = wave_max_u32<kWave>(absbits_f32<T>(bits));
      const float sc = floor_amax(u2f(bits)) / kE4M3Max;
      if (lane == 0) sas[m] = sc;
      float f[V];
      if (bits < kInfBits) {  // wavefront-uniform
        const float r = 1.0f / sc;
#pragma unroll
        for (int h = 0; h < kHeld; ++h) {
          const int v = lane + kWave * h;
          if (v < nvec) {
            unpack16<T>(held[rr][h], f);
            store_quant_finite<V>(xs + m * K + v * V, f, sc, r);
          }
        }
        for (int v = lane + kWave * kHeld; v < nvec; v += kWave) {
          unpack16<T>(xr[v], f);
          store_quant_finite<V>(xs + m * K + v * V, f, sc, r);
        }
      } else {
        const Divisor dv = make_divisor(sc);
#pragma unroll
        for (int h = 0; h < kHeld; ++h) {
          const int v = lane + kWave * h;
          if (v < nvec) {
            unpack16<T>(held[rr][h], f);
            store_quant<V>(xs + m * K + v * V, f, dv);
          }
        }
        for (int v = lane + kWave * kHeld; v < nvec; v += kWave) {
          unpack16<T>(xr[v], f);
          store_quant<V>(xs + m * K + v * V, f, dv);
        }
      }
    }
  } else {
    // Stage the activation rows (rows past M are never read).
    for (int i = tid; i < M * (K / 16); i += kRgThreads) {
      const int m = i / (K / 16), c = i - m * (K / 16);
      reinterpret_cast<uint4*>(xs)[i] = *reinterpret_cast<const uint4*>(g.a + (int64_t)m * g.lda + 16 * c);
    }
  }
  const int64_t n0 = (int64_t)blockIdx.x * kRgRows + 2 * wave;
  const int64_t r0 = n0 < g.N ? n0 : g.N - 1, r1 = n0 + 1 < g.N ? n0 + 1 : g.N - 1;  // rows past N re-read N - 1
  const uint8_t* w0 = g.w + r0 * g.ldw;
  const uint8_t* w1 = g.w + r1 * g.ldw;
  __syncthreads();
  float acc[2][MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[0][m] = acc[1][m] = 0.0f;
  for (int k = 16 * lane; k < K; k += 16 * kWave) {
    const uint4 a0 = *reinterpret_cast<const uint4*>(w0 + k), a1 = *reinterpret_cast<const uint4*>(w1 + k);
    float f0[16], f1[16];
    e4m3x4_to_f32(a0.x, f0); e4m3x4_to_f32(a0.y, f0 + 4); e4m3x4_to_f32(a0.z, f0 + 8); e4m3x4_to_f32(a0.w, f0 + 12);
    e4m3x4_to_f32(a1.x, f1); e4m3x4_to_f32(a1.y, f1 + 4); e4m3x4_to_f32(a1.z, f1 + 8); e4m3x4_to_f32(a1.w, f1 + 12);
    // All MR activation chunks first, then 2 MR independent fma chains per element.
    float fx[MR][16];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const uint4 xv = m < M ? *reinterpret_cast<const uint4*>(xs + m * K + k) : make_uint4(0, 0, 0, 0);
      e4m3x4_to_f32(xv.x, fx[m]); e4m3x4_to_f32(xv.y, fx[m] + 4); e4m3x4_to_f32(xv.z, fx[m] + 8); e4m3x4_to_f32(xv.w, fx[m] + 12);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        acc[0][m] = fmaf(f0[i], fx[m][i], acc[0][m]);
        acc[1][m] = fmaf(f1[i], fx[m][i], acc[1][m]);
      }
  }
  // Wavefront sums (butterfly: every lane ends with the totals).
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int d = 32; d >= 1; d >>= 1) acc[r][m] += __shfl_xor(acc[r][m], d, kWave);
  // Lane 2 m + r stores (row n0 + r, activation row m): every lane picks its total with
  // selects, then one scale / bias load and one store per lane, all lanes at once.
  const int r = lane & 1, m = lane >> 1;
  float total = 0.0f;
#pragma unroll
  for (int mm = 0; mm < MR; ++mm) total = m == mm ? (r ? acc[1][mm] : acc[0][mm]) : total;
  const int64_t n = n0 + r;
  if (m < M && n < g.N) {
    const float* sa = static_cast<const float*>(g.sa);
    const float* sb = static_cast<const float*>(g.sb);
    const float sam = QUANT ? sas[m] : sa[g.sa_vec ? m : 0];
    float y = (total * sam) * sb[g.sb_vec ? n : 0];
    if (g.bias) y += load_f32(g.bias, g.bias_dtype, n);
    store_f32(g.out, g.out_dtype, (int64_t)m * g.ldo + n, y);
  }
}

bool rows_gemv_wanted(const SkinnyFp8Args& g) {
  return g.mode == kSmScaled && g.M >= 2 && g.M <= 8 && g.N * g.K <= ((int64_t)1 << 24) && g.K % 16 == 0 &&
         g.M * g.K <= 64 * 1024 && g.lda % 16 == 0 && g.ldw % 16 == 0 && aligned16(g.a) && aligned16(g.w);
}
int launch_rows_gemv(const SkinnyFp8Args& g, hipStream_t st, const char* op) {
  note_plan("rows_gemv");
  const dim3 grid((unsigned)cdiv(g.N, kRgRows)), block(kRgThreads);
  const unsigned lds = (unsigned)(g.M * g.K);
  if (g.M <= 2) hipLaunchKernelGGL((fp8_rows_gemv_kernel<2, false, BF16T>), grid, block, lds, st, g, nullptr, 0);
  else if (g.M <= 4) hipLaunchKernelGGL((fp8_rows_gemv_kernel<4, false, BF16T>), grid, block, lds, st, g, nullptr, 0);
  else hipLaunchKernelGGL((fp8_rows_gemv_kernel<8, false, BF16T>), grid, block, lds, st, g, nullptr, 0);
  return check_launch(op);
}
template <typename T>
void launch_rows_gemv_quant(const SkinnyFp8Args& g, const void* x, int64_t ldx, hipStream_t st) {
  const dim3 grid((unsigned)cdiv(g.N, kRgRows)), block(kRgThreads);
  const unsigned lds = (unsigned)(g.M * g.K);
  if (g.M <= 2) hipLaunchKernelGGL((fp8_rows_gemv_kernel<2, true, T>), grid, block, lds, st, g, x, ldx);
  else if (g.M <= 4) hipLaunchKernelGGL((fp8_rows_gemv_kernel<4, true, T>), grid, block, lds, st, g, x, ldx);
  else hipLaunchKernelGGL((fp8_rows_gemv_kernel<8, true, T>), grid, block, lds, st, g, x, ldx);
}

}  // namespace

bool skinny_fp8_supported(const SkinnyFp8Args& g) {
  const bool out_ok = g.out_dtype == AYK_F32 || g.out_dtype == AYK_BF16 || g.out_dtype == AYK_F16;
  // The GEMV-shaped kernel has rules of its own (any K % 16 == 0), so that the unfused
  // quantizer + GEMM pair takes the same kernel as the fused small-batch linear.
  if (rows_gemv_wanted(g)) return out_ok;
  const SkPlan p = skinny_plan(g.M, g.N, g.K, g.mode);
  if (!p.ok) return false;
  if (g.lda % 16 || g.ldw % 16 || !aligned16(g.a) || !aligned16(g.w)) return false;
  if (g.mode == kSmMx) {
    // code dwords of one 128-K pair are 4-byte aligned loads
    if ((reinterpret_cast<uintptr_t>(g.sa) & 3) || (reinterpret_cast<uintptr_t>(g.sb) & 3) || g.ld_sa % 4 || g.ld_sb % 4)
      return false;
  }
  if (g.mode == kSmBlock) {
    if ((reinterpret_cast<uintptr_t>(g.sa) & 3) || (reinterpret_cast<uintptr_t>(g.sb) & 3) || g.ld_sb < g.K / 128 ||
        (!g.sa_vec && g.ld_sa < g.K / 128))
      return false;
  }
  return out_ok;
}

size_t skinny_fp8_workspace(int64_t M, int64_t N, int64_t K, int mode) {
  const SkPlan p = skinny_plan(M, N, K, mode);
  return p.ok && p.split > 1 ? (size_t)p.split * (size_t)M * (size_t)N * sizeof(float) : 0;
}

int skinny_fp8_launch(const SkinnyFp8Args& g, hipStream_t st, const char* op) {
  if (rows_gemv_wanted(g)) return launch_rows_gemv(g, st, op);
  const SkPlan p = skinny_plan(g.M, g.N, g.K, g.mode);
  if (!p.ok) return fail(AYK_EINVAL, "%s: no decode-batch plan for this shape", op);
  if (p.split > 1) {
    const size_t need = (size_t)p.split * (size_t)g.M * (size_t)g.N * sizeof(float);
    if (g.ws == nullptr || g.ws_bytes < need)
      return fail(AYK_EWORKSPACE, "%s: workspace of %zu bytes required, %zu given", op, need, g.ws_bytes);
  }
  KArgs ka{g, p.kps};
  const int ch = scale_chunk(g, p);
  note_plan("skinny fn=%d fm=%d ks=%d g=%d ch=%d split=%d", p.fn, p.fm, p.ks, p.g, ch, (int)p.split);
  const bool launched = g.mode == kSmMx      ? launch_sm<kSmMx>(p, ka, st, ch)
                        : g.mode == kSmBlock ? launch_sm<kSmBlock>(p, ka, st, ch)
                                             : launch_sm<kSmScaled>(p, ka, st, ch);
  if (!launched) return fail(AYK_EINVAL, "%s: no decode-batch kernel for this plan", op);
  if (int rc = check_launch(op)) return rc;
  if (p.split > 1) {
    launch_split_reduce(skinny_reduce, g.ws, g.M, g.N, p.split, g.bias, g.bias_dtype, g.out, g.out_dtype, g.ldo, st);
    return check_launch(op);
  }
  return AYK_OK;
}

bool rows_gemv_quant_supported(const SkinnyFp8Args& g, int x_dtype, int64_t ldx, const void* x) {
  const int64_t es = x_dtype == AYK_F32 ? 4 : 2;
  SkinnyFp8Args q = g;
  q.mode = kSmScaled;
  q.a = static_cast<const uint8_t*>(x);  // alignment of the activation rows, as for e4m3 rows
  q.lda = ldx * es;
  return (x_dtype == AYK_BF16 || x_dtype == AYK_F16 || x_dtype == AYK_F32) && ldx >= g.K && rows_gemv_wanted(q);
}

int rows_gemv_quant_launch(const SkinnyFp8Args& g, const void* x, int x_dtype, int64_t ldx, hipStream_t st,
                           const char* op) {
  if (!rows_gemv_quant_supported(g, x_dtype, ldx, x))
    return fail(AYK_EINVAL, "%s: needs 2-8 rows, N * K <= 2^24, K %% 16 == 0, M * K <= 64 KiB, 16-byte aligned rows", op);
  note_plan("rows_gemv quant");
  if (x_dtype == AYK_BF16) launch_rows_gemv_quant<BF16T>(g, x, ldx, st);
  else if (x_dtype == AYK_F16) launch_rows_gemv_quant<F16T>(g, x, ldx, st);
  else launch_rows_gemv_quant<F32T>(g, x, ldx, st);
  return check_launch(op);
}

}  // namespace ayk
