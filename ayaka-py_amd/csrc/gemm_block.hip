// Block-scaled fp8 GEMM (fp8_blockwise_mm) on 256 x 256 tiles, gfx950.
//
//   out[m, n] = sum_kb (a[m, kb] . w[n, kb]) * sa[m, kb] * sb[n / 128, kb]  (+ bias[n])
//
// with 128-wide K blocks kb (python/ayaka/kernel/triton/gemm/fp8_gemm.py:127-204;
// oracle reference/gemm.py:40-70).
//
// Rescaling without a per-block fold. Each block's scale c = sa[m, kb] * sb[nb, kb] is
// split into a power of two and a mantissa, c = mu * 2^E with mu in [1, 2). The power of
// two goes into the scaled MFMA's E8M0 activation-scale operand (one code per lane, i.e.
// per activation row m), which multiplies the block's products by exactly 2^E. The
// accumulator U holds the running sum in units of the current block's mantissa:
//   U_kb = U_{kb-1} * (mu_{kb-1} / mu_kb) + 2^E_kb * P_kb,   out = U_last * mu_last,
// so a block costs one multiply per accumulator (the ratio) instead of a fold of a
// separate partial (a read and an fma), and the accumulators stay within a factor of two
// of the true sum. A zero or subnormal c is passed as code 0 (2^-127: such a block adds
// below 1e-38 of its products) with mu unchanged; an infinite or NaN c as code 0xFF,
// which the MFMA turns into NaN.
//
// Tiling. 512 threads = 8 wavefronts, two per SIMD, so one wavefront's rescale (VALU)
// runs beside the other's MFMAs. Wavefront (wn, wm) owns weight rows [128 wn, +128) --
// inside one 128-row scale block -- and activation rows [64 wm, +64) (wave_role: the two
// wavefronts of a SIMD own activation rows in different halves of the tile, so that a
// wavefront whose rows all lie past M skips its MFMAs without idling a SIMD): 4 x 2 MFMA tiles of
// 32 x 32, 128 fp32 accumulators in VGPRs (this file is compiled with the VGPR form of
// the MFMAs). One 128-K block is one "pair" of 64-K MFMA steps; operands move HBM/L2 ->
// LDS with direct-to-LDS 16-byte loads covering 8 rows x 128 bytes each, into two 64 KB
// pair buffers (the next pair lands while the current one is multiplied). Wavefronts
// 0-3 load the 256 weight rows, 4-7 the 256 activation rows. LDS row r holds logical
// 16-byte chunk c at physical chunk c ^ ((r >> 1) & 7), so the 32 rows of a fragment
// read fall on distinct banks.
#include "gemm_block.h"

#include "ayk_common.h"
#include "gemm_tiles.h"
#include "gemm_util.h"

namespace ayk {
namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kThreads = 512;
constexpr int kTile = 256;
constexpr int kPairK = 128;                      // K bytes per pair buffer: one scale block
constexpr int kPairBytes = 2 * kTile * kPairK;   // 64 KB: 256 weight rows, then 256 activation rows
constexpr int kDma = kPairBytes / 1024 / 8;      // direct loads per wavefront per pair (8)
constexpr int FN = 4, FM = 2;                    // MFMA tiles per wavefront (n, m)
constexpr int kCodeOne = 127;                    // UE8M0 code of 1.0
constexpr int kRegion = 16 * 1024;               // a wavefront's epilogue staging region

// Wavefront w -> (wn, wm). Wavefronts w and w + 4 share a SIMD; they get wm and wm + 2.
__device__ inline void wave_role(int w, int& wn, int& wm) {
  wn = (w >> 1) & 1;
  wm = (w & 1) | ((w >> 2) << 1);
}

__device__ inline v16f mfma_scaled(const v8i& w, const v8i& a, const v16f& c, int code_a) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w, a, c, 0, 0, 0, kCodeOne, 0, code_a);
}

// Block scale c -> (E8M0 code of its power of two, its mantissa); mu keeps the previous
// mantissa for a zero, subnormal or non-finite c (see the file comment).
__device__ inline int split_scale(float c, float mu_prev, float& mu) {
  const uint32_t b = __float_as_uint(c);
  const uint32_t e = (b >> 23) & 0xFFu;
  const uint32_t normal = (e - 1u < 254u) ? 0xFFFFFFFFu : 0u;  // a v_cmp + v_cndmask, no branch
  mu = __uint_as_float((((b & 0x807FFFFFu) | 0x3F800000u) & normal) | (__float_as_uint(mu_prev) & ~normal));
  const uint32_t special = e == 0 ? 0u : 0xFFu;
  return (int)((e & normal) | (special & ~normal));
}

template <int OUT>
struct OutBytes { static constexpr int v = OUT == AYK_F32 ? 4 : 2; };

// Epilogue: out = U * mu (+ bias), one rounding. Each wavefront stages its 128 (n) x 32
// (m) slab of m-fragment j in a private 16 KB LDS region (16-byte chunks XOR-swizzled by
// row), then stores it row by row with coalesced 16-byte stores. No workgroup barrier:
// the region belongs to the wavefront.
template <int OUT, bool BIAS>
__device__ __attribute__((always_inline)) inline void block256_epilogue(const Block256Args& g, const v16f (&U)[FN][FM],
                                                                        const float (&mu)[FM], int64_t m_tile,
                                                                        int64_t n_tile, uint8_t* region) {
  constexpr int EB = OutBytes<OUT>::v;
  constexpr int kRowBytes = 128 * EB;
  constexpr int kChunks = kRowBytes / 16;           // 16 (bf16 / fp16) or 32 (fp32)
  constexpr int kRowsPerStore = 64 / kChunks;       // rows one store instruction covers
  static_assert(32 * kRowBytes <= kRegion, "staging slab must fit the region");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int wn, wm;
  wave_role(wave, wn, wm);
  const int h = lane >> 5, frow = lane & 31;
  const int64_t n_w = n_tile + wn * 128;
#pragma unroll
  for (int j = 0; j < FM; ++j) {
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
      for (int grp = 0; grp < 4; ++grp) {
        const int nl = 32 * i + 8 * grp + 4 * h;  // column within the wavefront's 128
        float bias[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (BIAS) {
          const int64_t n = n_w + nl;
          if (n < g.N) {
            if (g.bias_dtype == AYK_F32) {
              const float4 t = *reinterpret_cast<const float4*>(static_cast<const float*>(g.bias) + n);
              bias[0] = t.x; bias[1] = t.y; bias[2] = t.z; bias[3] = t.w;
            } else {
              const uint2 t = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(g.bias) + n);
              const uint32_t wds[2] = {t.x, t.y};
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const uint16_t bits = (uint16_t)(wds[q / 2] >> (16 * (q % 2)));
                bias[q] = g.bias_dtype == AYK_BF16 ? bf16_bits_to_f32(bits) : f16_bits_to_f32(bits);
              }
            }
          }
        }
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = U[i][j][4 * grp + q] * mu[j] + bias[q];
        const int byte = nl * EB;
        const int chunk = (byte >> 4) ^ (frow & (kChunks - 1) & 15);
        uint8_t* dst = region + frow * kRowBytes + chunk * 16 + (byte & 15);
        if constexpr (OUT == AYK_F32) {
          *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
        } else if constexpr (OUT == AYK_BF16) {
          *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
        } else {
          *reinterpret_cast<uint2*>(dst) =
              make_uint2((uint32_t)f32_to_f16_bits(v[0]) | ((uint32_t)f32_to_f16_bits(v[1]) << 16),
                         (uint32_t)f32_to_f16_bits(v[2]) | ((uint32_t)f32_to_f16_bits(v[3]) << 16));
        }
      }
    }
    // The wavefront's own staging writes are complete before it reads them back (and the
    // compiler may not move LDS accesses across this point).
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int r0 = 0; r0 < 32; r0 += kRowsPerStore) {
      const int rr = r0 + lane / kChunks, cc = lane % kChunks;
      const int64_t gm = m_tile + wm * 64 + j * 32 + rr;
      const int64_t gn = n_w + (int64_t)cc * (16 / EB);
      const uint4 val = *reinterpret_cast<const uint4*>(region + rr * kRowBytes + ((cc ^ (rr & (kChunks - 1) & 15)) * 16));
      if (gm < g.M && gn < g.N) {
        uint8_t* out = static_cast<uint8_t*>(g.out) + (gm * g.ldo + gn) * EB;
        if (gn + 16 / EB <= g.N) {
          if (g.nt_stores) __builtin_nontemporal_store(v4i{(int)val.x, (int)val.y, (int)val.z, (int)val.w}, reinterpret_cast<v4i*>(out));
          else *reinterpret_cast<uint4*>(out) = val;
        } else {  // the row's last columns, element by element (an expert's N need not be a multiple of 4)
          const uint32_t vw[4] = {val.x, val.y, val.z, val.w};
          const int64_t left = g.N - gn;
#pragma unroll
          for (int c = 0; c < 16 / EB - 1; ++c) {
            if (c < left) {
              if constexpr (EB == 4) reinterpret_cast<uint32_t*>(out)[c] = vw[c];
              else reinterpret_cast<uint16_t*>(out)[c] = (uint16_t)(vw[c / 2] >> (16 * (c % 2)));
            }
          }
        }
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
}

template <int OUT>
__device__ __attribute__((always_inline)) inline void block256_epilogue_out(const Block256Args& g, const v16f (&U)[FN][FM],
                                                                            const float (&mu)[FM], int64_t m_tile,
                                                                            int64_t n_tile, uint8_t* region) {
  if (g.bias) block256_epilogue<OUT, true>(g, U, mu, m_tile, n_tile, region);
  else block256_epilogue<OUT, false>(g, U, mu, m_tile, n_tile, region);
}

// One 256 x 256 output tile (tm, tn) over the K range [k0, k0 + klen) (whole 128-K
// blocks), written to g.out; P0 / P1 are the workgroup's two pair buffers.
__device__ __attribute__((always_inline)) inline void block256_tile(const Block256Args& g, int tm, int tn, int64_t k0,
                                                                    int64_t klen, uint8_t* P0, uint8_t* P1) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave_u = __builtin_amdgcn_readfirstlane(tid >> 6);
  int wn, wm;
  wave_role(wave_u, wn, wm);
  const int h = lane >> 5, frow = lane & 31;
  const int64_t n_base = (int64_t)tn * kTile, m_base = (int64_t)tm * kTile;
  // Activation rows past M (an expert's or the tile tail's): a wavefront with none of
  // its 64 rows below M skips its MFMAs and its epilogue (wave-uniform).
  const bool rows_live = m_base + 64 * wm < g.M;
  const int np = (int)(klen / kPairK);   // K blocks of this range (>= 1)
  const int npairs = (np + 1) & ~1;      // the loop runs pairs two at a time
  const int kb0 = (int)(k0 / kPairK);
  // K stagger: tile (tm, tn) starts at block (tm mod 8) + (tn mod 2), so the tiles an XCD
  // runs together do not request the same K slices in lockstep.
  const int stag = __builtin_amdgcn_readfirstlane((int)((unsigned)((tm & 7) + (tn & 1)) % (unsigned)np));
  auto block_of = [&](int p) {  // local block of loop pair p (< np)
    const int b = p + stag;
    return __builtin_amdgcn_readfirstlane(b >= np ? b - np : b);
  };

  // Direct loads: wavefront w < 4 fetches weight rows [64 w, 64 w + 64), w >= 4 activation
  // rows [64 (w - 4), +64). Load jj covers rows 8 jj + L / 8 (lane L), 128 K bytes, written
  // as LDS rows 256 (w / 4) + 64 (w % 4) + 8 jj + L / 8; lane L fetches logical chunk
  // (L & 7) ^ ((4 (jj & 1) + (L >> 4)) & 7) so that it lands at physical chunk L & 7.
  const int side = wave_u >> 2;
  const int64_t ld = side == 0 ? g.ldw : g.lda;
  const int ld_u = __builtin_amdgcn_readfirstlane((int)ld);
  const OperandWindow win = operand_window((side == 0 ? n_base : m_base) + 64 * (wave_u & 3), side == 0 ? g.N : g.M, ld);
  const __amdgpu_buffer_rsrc_t rsrc = uniform_rsrc((side == 0 ? g.w : g.a) + win.base_offset + k0, win.records);
  const int voff_e = (lane >> 3) * ld_u + (((lane & 7) ^ ((lane >> 4) & 7)) << 4);
  const int voff_o = (lane >> 3) * ld_u + (((lane & 7) ^ ((4 + (lane >> 4)) & 7)) << 4);
  // A wavefront whose 64 rows all lie past M (activations) or N (weights) loads nothing:
  // its LDS rows feed only MFMAs whose results are never stored (a wavefront with no
  // live activation row skips its MFMAs; a weight row past N makes an output column
  // past N). MoE tiles with at most 128 expert rows thus issue a quarter fewer loads.
  const bool loads_live = (side == 0 ? n_base : m_base) + 64 * (wave_u & 3) < (side == 0 ? g.N : g.M);
  auto issue = [&](int p, uint8_t* dst) {
    if (!loads_live) return;
    const int kb = block_of(p);
#pragma unroll
    for (int jj = 0; jj < kDma; ++jj) {
      const int soff = __builtin_amdgcn_readfirstlane(jj * 8 * ld_u + kb * kPairK);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)(dst + (wave_u * kDma + jj) * 1024),
                                               16, (jj & 1) ? voff_o : voff_e, soff, 0, 0);
    }
  };

  // Scales of a block: this lane's two activation rows, and the wavefront's weight block
  // row (its 128 weight rows share one). They are fetched as raw dwords through buffer
  // descriptors (32-bit offsets, no waits at the load) and decoded in `prepare`, after
  // the pair's vector-memory wait.
  const int64_t nbs = cdiv(g.N, 128);
  const int64_t nb = (n_base + wn * 128) / 128 < nbs ? (n_base + wn * 128) / 128 : nbs - 1;
  const int sb_size = g.sb_dtype == AYK_F32 ? 4 : 2;
  const int64_t sa_elems = g.sa_col_major ? (cdiv(g.K, 128) - 1) * g.ld_sa + g.M : g.M * g.ld_sa;
  const __amdgpu_buffer_rsrc_t sa_rsrc = uniform_rsrc(g.sa, (int32_t)(sa_elems * 4 < 0x7FFFFFFF ? sa_elems * 4 : 0x7FFFFFFF));
  // sb through a descriptor on its 4-byte-aligned span: a 16-bit scale is read as the
  // aligned dword that holds it, which never leaves that span.
  const uintptr_t sb_addr = reinterpret_cast<uintptr_t>(g.sb);
  const int sb_lead = (int)(sb_addr & 3);
  const int64_t sb_span = (sb_lead + nbs * g.ld_sb * sb_size + 3) & ~(int64_t)3;
  const __amdgpu_buffer_rsrc_t sb_rsrc =
      uniform_rsrc(reinterpret_cast<const void*>(sb_addr - sb_lead), (int32_t)(sb_span < 0x7FFFFFFF ? sb_span : 0x7FFFFFFC));
  const int sb_row_byte = sb_lead + (int)(nb * g.ld_sb * sb_size);
  uint32_t sa_off[FM];  // byte offsets of this lane's rows at block 0
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int64_t m = m_base + wm * 64 + j * 32 + frow;
    const int64_t mi = m < g.M ? m : g.M - 1;
    sa_off[j] = (uint32_t)((g.sa_col_major ? mi : mi * g.ld_sa) * 4);
  }
  const uint32_t sa_kstride = (uint32_t)((g.sa_col_major ? g.ld_sa : 1) * 4);
  struct Scales {
    uint32_t sa[FM];
    uint32_t sb;   // the dword holding sb[nb, kb]
    uint32_t sh;   // bit position of sb in it (fp16 / bf16)
  };
  auto load_scales = [&](int p) {
    const int kb = kb0 + block_of(p);
    Scales s;
#pragma unroll
    for (int j = 0; j < FM; ++j)
      s.sa[j] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(sa_rsrc, (int)(sa_off[j] + (uint32_t)kb * sa_kstride), 0, 0);
    const int sb_byte = __builtin_amdgcn_readfirstlane(sb_row_byte + kb * sb_size);
    s.sb = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(sb_rsrc, 0, sb_byte & ~3, 0);
    s.sh = (uint32_t)(sb_byte & 3) * 8;
    return s;
  };
  const bool sb_f32 = g.sb_dtype == AYK_F32, sb_bf16 = g.sb_dtype == AYK_BF16;
  float mu[FM] = {1.0f, 1.0f}, ratio[FM] = {1.0f, 1.0f};
  int code[FM] = {kCodeOne, kCodeOne};
  auto prepare = [&](Scales s) {
    asm volatile("" : "+v"(s.sb));
    const uint32_t half = (s.sb >> s.sh) & 0xFFFFu;
    const float sbv = sb_f32 ? __uint_as_float(s.sb) : (sb_bf16 ? __uint_as_float(half << 16) : f16_bits_to_f32((uint16_t)half));
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      asm volatile("" : "+v"(s.sa[j]));
      float m_new;
      code[j] = split_scale(__uint_as_float(s.sa[j]) * sbv, mu[j], m_new);
      ratio[j] = mu[j] / m_new;
      mu[j] = m_new;
    }
  };

  // Fragment reads (the 256 x 256 rowwise kernel's scheme): LDS row of weight row R is R,
  // of activation row R is 256 + R; step t reads logical chunks 4 t + h and 4 t + 2 + h.
  const int fsw = (frow >> 1) & 7;
  const int off_t[2][2] = {{frow * kPairK + ((h ^ fsw) << 4), frow * kPairK + (((2 + h) ^ fsw) << 4)},
                           {frow * kPairK + (((4 + h) ^ fsw) << 4), frow * kPairK + (((6 + h) ^ fsw) << 4)}};
  auto frag = [&](const uint8_t* buf, int row0, int t) -> v8i {
    const v4i lo = *reinterpret_cast<const v4i*>(buf + (row0 * kPairK + off_t[t][0]));
    const v4i hi = *reinterpret_cast<const v4i*>(buf + (row0 * kPairK + off_t[t][1]));
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  };
  v8i wf[2][FN], af[2][FM];
  auto read_frags = [&](int set, const uint8_t* buf, int t) {
#pragma unroll
    for (int i = 0; i < FN; ++i) wf[set][i] = frag(buf, wn * 128 + i * 32, t);
#pragma unroll
    for (int j = 0; j < FM; ++j) af[set][j] = frag(buf, 256 + wm * 64 + j * 32, t);
  };

  v16f U[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) U[i][j][r] = 0.0f;

  // Prologue: pair 0 (and pair 1) in flight with their scales; pair 0 visible.
  Scales s_next = load_scales(0);
  issue(0, P0);
  wait_vmcnt<0>();
  lds_barrier();
  prepare(s_next);
  if (np > 1) {
    s_next = load_scales(1);
    issue(1, P1);
  }
  read_frags(0, P0, 0);

  // Pair p in `cur` (visible, step-0 fragments in set 0, rescale of block p prepared);
  // pair p + 1 in flight into `nxt` with its scales in s_next.
  // A pair runs in two phases around its barrier, eight MFMAs each, so that the LDS reads
  // and the rescale multiplies spread over MFMAs of the same wavefront:
  //  * before the barrier: step 0's MFMAs; beside them, step 1's fragment reads and the
  //    m-fragment 1 rescale into this block's units (one MFMA, then 16 multiplies);
  //  * after it (pair p + 1 has landed, `cur` is free): step 1's MFMAs; beside them the
  //    next pair's step-0 fragment reads and the m-fragment 0 rescale into block p + 1's
  //    units (behind that m-fragment's last MFMA of this block).
  // U is zero before the first block, so its rescale is moot.
  constexpr int kSchedMfma = 0x008, kSchedValu = 0x002, kSchedDsRead = 0x100;
  auto pair = [&](int p, uint8_t* cur, uint8_t* nxt) {
    const bool live = p < np && rows_live;  // wave-uniform
    if (live) {
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        U[i][0] = mfma_scaled(wf[0][i], af[0][0], U[i][0], code[0]);
#pragma unroll
        for (int r = 0; r < 16; ++r) U[i][1][r] *= ratio[1];
      }
#pragma unroll
      for (int i = 0; i < FN; ++i) U[i][1] = mfma_scaled(wf[0][i], af[0][1], U[i][1], code[1]);
      read_frags(1, cur, 1);
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedValu, 16, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
      }
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
      }
    }
    const int code1 = code[1], code0 = code[0];
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<0>();  // pair p + 1 and its scales have landed
    lds_barrier();    // ... for every wavefront, and no wavefront reads `cur` any more
    __builtin_amdgcn_sched_barrier(0);
    const bool more = p + 1 < np;
    if (more) {
      prepare(s_next);
      if (p + 2 < np) {
        s_next = load_scales(p + 2);
        issue(p + 2, cur);
      }
    }
    const float ratio0 = more ? ratio[0] : 1.0f;  // after the last block the units stay
    if (live) {
#pragma unroll
      for (int i = 0; i < FN; ++i) U[i][0] = mfma_scaled(wf[1][i], af[1][0], U[i][0], code0);
      read_frags(0, nxt, 0);  // after the last pair: stale data, never used
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        U[i][1] = mfma_scaled(wf[1][i], af[1][1], U[i][1], code1);
#pragma unroll
        for (int r = 0; r < 16; ++r) U[i][0][r] *= ratio0;
      }
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
      }
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedValu, 16, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
      }
    }
  };
  for (int p = 0; p < npairs; p += 2) {
    pair(p, P0, P1);
    pair(p + 1, P1, P0);
  }
  wait_vmcnt<0>();
  lds_barrier();  // no wavefront still reads a pair buffer: they become staging regions

  uint8_t* region = (wave_u < 4 ? P0 : P1) + (wave_u & 3) * kRegion;
  if (!rows_live) return;
  if (g.out_dtype == AYK_BF16) block256_epilogue_out<AYK_BF16>(g, U, mu, m_base, n_base, region);
  else if (g.out_dtype == AYK_F16) block256_epilogue_out<AYK_F16>(g, U, mu, m_base, n_base, region);
  else block256_epilogue_out<AYK_F32>(g, U, mu, m_base, n_base, region);
}

// blockIdx.x: tile (XCD-aware order); blockIdx.y: K split (kps > 0: K range
// [y kps, (y + 1) kps), fp32 partial to ws[y], no bias).
__global__ __launch_bounds__(kThreads, 1) void fp8_block256_kernel(Block256Args gin, int tiles_m, int64_t kps) {
  __shared__ __attribute__((aligned(1024))) uint8_t P0[kPairBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t P1[kPairBytes];
  Block256Args g = gin;
  g.nt_stores = 1;
  int64_t k0 = 0, klen = gin.K;
  if (kps > 0) {
    k0 = (int64_t)blockIdx.y * kps;
    klen = gin.K - k0 < kps ? gin.K - k0 : kps;
    g.bias = nullptr;
    g.out = gin.ws + (int64_t)blockIdx.y * gin.M * gin.N;
    g.out_dtype = AYK_F32;
    g.ldo = gin.N;
    g.nt_stores = 0;  // partials are read back by the reduce: keep them in L2
  }
  int tm, tn;
  big_tile_coords(blockIdx.x, tiles_m, (int)cdiv(g.N, kTile), tm, tn);
  block256_tile(g, tm, tn, k0, klen, P0, P1);
}

// Expert e's problem, clamped to what the operands hold (rows past M_total, N_e > n,
// K_e > k, K in whole 128-K blocks as the reference's K // 128), so device-side
// metadata can never address outside the tensors.
struct Expert256 {
  int64_t off, m, n, k;
};
__device__ inline Expert256 expert256(const Grouped256Args& ga, int e) {
  Expert256 p;
  const int64_t off = ga.expert_offsets[e];
  p.off = off < 0 ? 0 : (off > ga.m_total ? ga.m_total : off);
  const int64_t m = ga.problem_sizes[3 * e], n = ga.problem_sizes[3 * e + 1], k = ga.problem_sizes[3 * e + 2];
  p.m = m < 0 ? 0 : (m > ga.m_total - p.off ? ga.m_total - p.off : m);
  p.n = n < 0 ? 0 : (n > ga.n ? ga.n : n);
  p.k = k < 0 ? 0 : ((k > ga.k ? ga.k : k) / kPairK) * kPairK;
  return p;
}
__device__ inline int64_t expert256_tiles(const Expert256& p) { return cdiv(p.m, kTile) * cdiv(p.n, kTile); }

// Grouped (MoE) form: workgroup b takes logical tile pid of the concatenation of every
// expert's tiles (row tiles first within a column tile). Workgroup b runs on XCD b % 8;
// pid maps the 16 logical tiles 16 x .. 16 x + 15 to workgroups 8 apart (one XCD,
// dispatched together), so an expert's column tiles share its activation rows in that
// XCD's L2 while each reads its own weight panel once. The grid is an upper bound (a
// multiple of 128); workgroups past the real tile count leave at once.
__global__ __launch_bounds__(kThreads, 1) void fp8_grouped_block256_kernel(Grouped256Args ga) {
  __shared__ __attribute__((aligned(1024))) uint8_t P0[kPairBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t P1[kPairBytes];
  const int lane = threadIdx.x & 63;
  const int E = ga.num_experts, per = (E + 63) / 64;
  const int64_t b = blockIdx.x;
  const int64_t pid = (b & ~(int64_t)127) + 16 * (b & 7) + ((b >> 3) & 15);
  // Locate the expert: lane l sums the tiles of experts [l per, l per + per), a wave
  // scan makes prefixes, the first lane whose inclusive prefix passes pid owns it.
  int64_t mine = 0;
  for (int i = 0; i < per; ++i) {
    const int e = lane * per + i;
    if (e < E) mine += expert256_tiles(expert256(ga, e));
  }
  int64_t incl = mine;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int64_t v = __shfl_up(incl, d, 64);
    if (lane >= d) incl += v;
  }
  const uint64_t owners = __ballot(incl > pid);
  if (owners == 0) return;  // past the real tile count (uniform: the ballot is)
  const int owner = __ffsll((unsigned long long)owners) - 1;
  int64_t start = __shfl(incl - mine, owner, 64);
  int e = owner * per;
  Expert256 p = expert256(ga, e);
  for (int64_t t = expert256_tiles(p); pid >= start + t; t = expert256_tiles(p)) {
    start += t;
    p = expert256(ga, ++e);
  }
  // Everything below is wavefront-uniform: keep it in scalar registers.
  auto uni64 = [](int64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)v >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
  };
  e = __builtin_amdgcn_readfirstlane(e);
  p.off = uni64(p.off);
  p.m = uni64(p.m);
  p.n = uni64(p.n);
  p.k = uni64(p.k);
  const int64_t local = uni64(pid - start);
  const int64_t tiles_m = cdiv(p.m, kTile);
  const int tm = __builtin_amdgcn_readfirstlane((int)(local % tiles_m));
  const int tn = __builtin_amdgcn_readfirstlane((int)(local / tiles_m));
  const int eb = ga.out_dtype == AYK_F32 ? 4 : 2;
  if (p.k == 0) {  // no whole 128-K block: the sum is empty, the tile is zeros
    for (int idx = threadIdx.x; idx < kTile * kTile; idx += kThreads) {
      const int64_t gm = (int64_t)tm * kTile + idx / kTile, gn = (int64_t)tn * kTile + idx % kTile;
      if (gm < p.m && gn < p.n) store_f32(ga.out, ga.out_dtype, (p.off + gm) * ga.n + gn, 0.0f);
    }
    return;
  }
  const int64_t kb_total = ga.k / kPairK;
  Block256Args g{};
  g.nt_stores = 1;
  g.a = ga.a + p.off * ga.k;
  g.lda = ga.k;
  g.w = ga.b + (int64_t)e * ga.n * ga.k;
  g.ldw = ga.k;
  g.M = p.m;
  g.N = p.n;
  g.K = p.k;
  // The reference's pointer tables: expert e's scales start at row off_e of sa and at
  // block row e (n / 128) of sb, both with row stride K_e / 128. An expert over the
  // whole K reads the transposed copy instead when there is one (the same values: row
  // off_e + r, block kb), from column off_e with K-block stride m_total.
  if (ga.sa_t != nullptr && p.k == ga.k) {
    g.sa = ga.sa_t + p.off;
    g.ld_sa = ga.m_total;
    g.sa_col_major = 1;
  } else {
    g.sa = ga.sa + p.off * kb_total;
    g.ld_sa = p.k / kPairK;
    g.sa_col_major = 0;
  }
  g.sb = ga.sb + (int64_t)e * (ga.n / kPairK) * kb_total;
  g.sb_dtype = AYK_F32;
  g.ld_sb = p.k / kPairK;
  g.bias = nullptr;
  g.out = static_cast<uint8_t*>(ga.out) + p.off * ga.n * eb;
  g.out_dtype = ga.out_dtype;
  g.ldo = ga.n;
  block256_tile(g, tm, tn, 0, p.k, P0, P1);
}

// Fixed-order sum of the K-split partials, bias, one rounding.
__global__ __launch_bounds__(256) void block256_reduce(const float* __restrict__ part, int64_t M, int64_t N, int split,
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

}  // namespace

bool block256_supported(const Block256Args& g) {
  const int64_t out_bytes = g.out_dtype == AYK_F32 ? 4 : 2;
  return g.K % kPairK == 0 && g.K < ((int64_t)1 << 30) && g.M >= kTile && g.N >= kTile && g.N % 4 == 0 &&
         (g.ldo * out_bytes) % 16 == 0 && aligned16(g.out) && aligned16(g.a) && aligned16(g.w) &&
         g.lda % 16 == 0 && g.ldw % 16 == 0 && 64 * g.lda < ((int64_t)1 << 31) && 64 * g.ldw < ((int64_t)1 << 31) &&
         (g.bias == nullptr || aligned16(g.bias)) && (g.sb_dtype == AYK_F32 || g.sb_dtype == AYK_BF16 || g.sb_dtype == AYK_F16);
}

// Under half a round of tiles (256 workgroups, one per CU): as many K pieces as fit in
// that round, each at least 1024 K and a whole number of 128-K blocks (the last one may
// be shorter). Returns the number of pieces; block256_kps gives their K.
int64_t block256_kps(int64_t K, int64_t split) { return cdiv(K / kPairK, split) * kPairK; }
int64_t block256_split(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = cdiv(M, kTile) * cdiv(N, kTile);
  if (tiles * 2 > 256) return 1;
  const int64_t want = 256 / tiles, most = K / 1024;
  const int64_t split = want < most ? want : most;
  if (split <= 1) return 1;
  return cdiv(K, block256_kps(K, split));
}

int block256_launch(const Block256Args& g, hipStream_t st, const char* op) {
  const int tiles_m = (int)cdiv(g.M, kTile);
  const int64_t tiles = (int64_t)tiles_m * cdiv(g.N, kTile);
  if (tiles > 0x7FFFFFFF) return fail(AYK_EINVAL, "%s: problem too large", op);
  const int64_t split = block256_split(g.M, g.N, g.K);
  note_plan("block256 split=%d", (int)split);
  if (split == 1) {
    hipLaunchKernelGGL(fp8_block256_kernel, dim3((unsigned)tiles), dim3(kThreads), 0, st, g, tiles_m, (int64_t)0);
    return check_launch(op);
  }
  const size_t need = (size_t)split * (size_t)g.M * (size_t)g.N * sizeof(float);
  if (g.ws == nullptr || g.ws_bytes < need)
    return fail(AYK_EWORKSPACE, "%s: workspace of %zu bytes required, %zu given", op, need, g.ws_bytes);
  hipLaunchKernelGGL(fp8_block256_kernel, dim3((unsigned)tiles, (unsigned)split), dim3(kThreads), 0, st, g, tiles_m,
                     block256_kps(g.K, split));
  if (int rc = check_launch(op)) return rc;
  launch_split_reduce(block256_reduce, g.ws, g.M, g.N, (int)split, g.bias, g.bias_dtype, g.out, g.out_dtype, g.ldo, st);
  return check_launch(op);
}

int grouped_block256_launch(const Grouped256Args& ga, hipStream_t st, const char* op) {
  // Upper bound on the tiles: every expert adds at most one partial 256-row tile.
  const int64_t bound = cdiv((cdiv(ga.m_total, kTile) + ga.num_experts) * cdiv(ga.n, kTile), 128) * 128;
  if (bound > 0x7FFFFFFF) return fail(AYK_EINVAL, "%s: problem too large", op);
  note_plan("grouped_block256");
  hipLaunchKernelGGL(fp8_grouped_block256_kernel, dim3((unsigned)bound), dim3(kThreads), 0, st, ga);
  return check_launch(op);
}

}  // namespace ayk
