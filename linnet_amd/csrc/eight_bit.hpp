// The 8-bit x 8-bit tiled MFMA product (mm8_kernel) and the software FP8 E4M3
// encoder, shared by eight_bit.hip (row-scaled int8 / FP8 products, per-token
// rounding) and fp8_block.hip (block-scaled FP8 product, per-group rounding).
// The two files instantiate different forms of the kernel and are compiled
// with different MFMA register forms (AGPR accumulators here, VGPR ones for the
// block-scaled form, which keeps a partial tile beside the accumulated one).
#pragma once

#include <type_traits>

#include "common.hpp"

namespace lnq {

// f32 (|v| <= 448) -> FP8 E4M3 bits, round to nearest even (software, exact).
__host__ __device__ inline uint32_t f32_to_e4m3(float v) {
  const uint32_t bits = __builtin_bit_cast(uint32_t, v);
  const uint32_t sign = (bits >> 24) & 0x80u;
  const uint32_t mag = bits & 0x7fffffffu;
  uint32_t code;
  if (mag >= 0x3c800000u) {  // |v| >= 2^-6: normal
    const uint32_t r = mag + 0x7ffffu + ((mag >> 20) & 1u);
    code = (((r >> 23) - 120u) << 3) | ((r >> 20) & 7u);
  } else {  // subnormal: multiples of 2^-9 (exact scaling by 512, then rint)
    code = static_cast<uint32_t>(rintf(__builtin_bit_cast(float, mag) * 512.0f));
  }
  if (code > 0x7eu) code = 0x7eu;
  return code | sign;
}

// ======================================================================= mm8
// 8-bit x 8-bit products on gfx950 MFMA: FP8 E4M3 rows times FP8 weights
// (v_mfma_scale_f32_32x32x64_f8f6f4 with unit E8M0 scales, f32 sums) or int8
// rows times int8 weights (v_mfma_i32_32x32x32_i8, exact int32 sums); the
// per-row and per-column scales are applied in f32 at the end.
//
// Tiles: 256 rows by BN = 256 or 128 columns per workgroup of 8 waves, two
// per SIMD (the other wave of a SIMD covers the issue stalls of a wave's
// loads); a wave owns 128 x 64 (BN = 256) or 64 x 64 (BN = 128) outputs as
// MFMA 32x32 tiles. 128 input bytes per step, moved HBM/L2 -> LDS without
// registers (buffer_load ... lds) one step ahead into two stages per operand,
// rows of 128 bytes with 16-byte columns XOR-swizzled by bits 1..3 of the row.
// A step's kk sub-steps are scheduling regions of one MFMA per slot
// (sched_barrier), each slot carrying its share of the next kk's operand
// reads; the one barrier per step sits before the last kk, whose MFMAs run
// while the next step's first operands are read.
//
// Block-scaled FP8 (BLK): the weight has a scale per 128 x 128 block
// (scale [N/128, K/128]) and the rows one per 128 inputs (x_scale [K/128, rows],
// column-major with stride xs_stride), so a step (128 inputs, one block column)
// sums into a partial tile P, which is added to the tile scaled by
// x_scale[m, step] * scale[n / 128, step] once the step's MFMAs are done: the
// block-wise product `torch._scaled_mm` computes for the reference. 128-column
// tiles only (a wave's 64 columns lie in one weight block).
namespace mm8 {
constexpr int BM = 256;
constexpr int BK = 128;  // bytes (= elements) per step
constexpr int THREADS = 512;
constexpr int GROUP_M = 4;
constexpr int XCDS = 8;

template <int BN>
struct Cfg;
template <>
struct Cfg<256> {
  static constexpr int WAVES_N = 4;  // waves of 128 x 64, 2 x 4
  static constexpr int FA = 4;
  static constexpr int FB = 2;
};
template <>
struct Cfg<128> {
  static constexpr int WAVES_N = 2;  // waves of 64 x 64, 4 x 2
  static constexpr int FA = 2;
  static constexpr int FB = 2;
};
}  // namespace mm8

// Byte offset of 16-byte column c16 of row `row` in a swizzled stage (rows of
// 128 bytes; rows 2i and 2i+1 share a 256-byte bank line, so the XOR key is
// bits 1..3 of the row).
__device__ inline int swz8(int row, int c16) { return row * mm8::BK + ((c16 ^ ((row >> 1) & 7)) << 4); }

__device__ inline void mm8_tile_of(int b, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  const int per_xcd = (total + mm8::XCDS - 1) / mm8::XCDS;
  const int xcd = b % mm8::XCDS;
  const int local = b / mm8::XCDS;
  int logical = xcd * per_xcd + local;
  if (total % mm8::XCDS != 0) {
    const int full = total - (per_xcd - 1) * mm8::XCDS;
    logical = xcd < full ? xcd * per_xcd + local : full * per_xcd + (xcd - full) * (per_xcd - 1) + local;
  }
  const int per_group = mm8::GROUP_M * tiles_n;
  const int first_m = (logical / per_group) * mm8::GROUP_M;
  const int rows = min(tiles_m - first_m, mm8::GROUP_M);
  tm = first_m + (logical % per_group) % rows;
  tn = (logical % per_group) / rows;
}

typedef int i32x16 __attribute__((ext_vector_type(16)));

template <int DT, int FP8, int BN, bool BLK = false>
__global__ __launch_bounds__(mm8::THREADS, 1) void mm8_kernel(
    const uint8_t* __restrict__ qx, const uint8_t* __restrict__ weight,
    const float* __restrict__ x_scale, const float* __restrict__ scale,
    uint16_t* __restrict__ y, int M, int N, int K, int xs_stride) {
  using namespace mm8;
  static_assert(!BLK || (FP8 && BN == 128), "block scales: FP8, 128-column tiles");
  using E = Elem<DT>;
  constexpr int FA = Cfg<BN>::FA, FB = Cfg<BN>::FB, WAVES_N = Cfg<BN>::WAVES_N;
  constexpr int NMF = FA * FB;           // MFMA slots of one kk
  constexpr int KPM = FP8 ? 64 : 32;     // inputs per MFMA
  constexpr int KK = BK / KPM;           // kk sub-steps per step
  constexpr int CPL = KPM / 32;          // 16-byte columns of an operand per lane
  constexpr int BLOADS = BN / 64;        // weight loads of a wave per step
  using Op = typename std::conditional<FP8, i32x8, i32x4>::type;
  using Acc = typename std::conditional<FP8, f32x16, i32x16>::type;
  // Stages per operand: three (loads two steps ahead) where they fit in LDS.
  constexpr int S = BN == 256 ? 2 : 3;
  constexpr int LPW = 4 + BLOADS;  // loads of a wave per step
  __shared__ __attribute__((aligned(16))) uint8_t A0[BM * BK];
  __shared__ __attribute__((aligned(16))) uint8_t A1[BM * BK];
  __shared__ __attribute__((aligned(16))) uint8_t A2[S > 2 ? BM * BK : 16];
  __shared__ __attribute__((aligned(16))) uint8_t B0[BN * BK];
  __shared__ __attribute__((aligned(16))) uint8_t B1[BN * BK];
  __shared__ __attribute__((aligned(16))) uint8_t B2[S > 2 ? BN * BK : 16];
  if constexpr (!BLK) LNQ_MFMA_IN_AGPRS();

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WAVES_N;
  const int wn = wave % WAVES_N;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  mm8_tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  if (tm >= tiles_m || tn >= tiles_n) return;
  const int m0 = tm * BM, n0 = tn * BN;
  const int steps = K / BK;

  // Rows past M (N) read zeros through the descriptors' range checks; a step
  // past the end reads through a 0-byte descriptor.
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(qx, static_cast<uint32_t>(static_cast<size_t>(M) * K));
  const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(weight, static_cast<uint32_t>(static_cast<size_t>(N) * K));
  const __amdgpu_buffer_rsrc_t rnull = buffer_rsrc(weight, 0);

  // Load i of wave w writes stage rows 64 i + 8 w .. + 7 (1 KB; lane l at byte
  // 16 l: row 64 i + 8 w + l / 8, stored column l % 8 holding source column
  // (l % 8) ^ key(row), key = (row >> 1) & 7, the same for every i).
  const int lrow8 = 8 * wave + (lane >> 3);
  const int lcol = (lane & 7) ^ ((lrow8 >> 1) & 7);
  const int aoff_g = (m0 + lrow8) * K + lcol * 16;
  const int boff_g = (n0 + lrow8) * K + lcol * 16;
  const int lds_w = wave * 1024;
  auto load_a = [&](uint8_t* dst, __amdgpu_buffer_rsrc_t r, int k0, int i) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)(dst + lds_w + i * 64 * BK), 16, aoff_g, k0 + i * 64 * K, 0, 0);
  };
  auto load_b = [&](uint8_t* dst, __amdgpu_buffer_rsrc_t r, int k0, int i) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)(dst + lds_w + i * 64 * BK), 16, boff_g, k0 + i * 64 * K, 0, 0);
  };

  Acc acc[FA][FB];
#pragma unroll
  for (int a = 0; a < FA; ++a)
#pragma unroll
    for (int b = 0; b < FB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0;
  // Block scales: the step's partial tile, the rows' scales of the step (lane
  // row m = l % 32 of fragment a; rows past M read row M - 1; loaded as the step
  // starts, they land with its operands), and the weight block row of this
  // wave's columns.
  Acc part[BLK ? FA : 1][BLK ? FB : 1];
  float sx[BLK ? FA : 1];
  int xs_row[BLK ? FA : 1];
  const int kblocks = K / BK;
  const float* wscale = scale + static_cast<size_t>((n0 + wn * FB * 32) / 128) * kblocks;
  if constexpr (BLK) {
#pragma unroll
    for (int a = 0; a < FA; ++a) xs_row[a] = min(m0 + wm * FA * 32 + a * 32 + (lane & 31), M - 1);
  }

  const int lrow = lane & 31;
  const int lk = lane >> 5;
  // Operand byte offsets within a stage per (kk, column j of the lane): the
  // fragments of one kk are 32 rows (4096 bytes) apart with the same key.
  uint32_t aoff[KK][CPL], boff[KK][CPL];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk)
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c16 = kk * 2 * CPL + lk * CPL + j;
      const uint32_t col = static_cast<uint32_t>((c16 ^ ((lrow >> 1) & 7)) << 4);
      aoff[kk][j] = static_cast<uint32_t>((wm * FA * 32 + lrow) * BK) + col;
      boff[kk][j] = static_cast<uint32_t>((wn * FB * 32 + lrow) * BK) + col;
    }
  auto rd = [&](const uint8_t* stage, uint32_t off, int frag) -> u32x4 {
    return *reinterpret_cast<const u32x4*>(stage + off + frag * 4096);
  };
  auto set_op = [](Op& o, int j, u32x4 v) {
    if constexpr (FP8) {
      o[4 * j + 0] = (int)v.x;
      o[4 * j + 1] = (int)v.y;
      o[4 * j + 2] = (int)v.z;
      o[4 * j + 3] = (int)v.w;
    } else {
      o = __builtin_bit_cast(i32x4, v);
    }
  };
  auto mma = [](const Op& a, const Op& b, Acc c) -> Acc {
    if constexpr (FP8)
      return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0x7f7f7f7f, 0, 0x7f7f7f7f);
    else
      return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  };
  // Operand fragments: set 0 holds even kk, set 1 odd kk.
  Op af[2][FA], bf[2][FB];
  constexpr int READS = (FA + FB) * CPL;
  // Read number r of a kk: fragment r / CPL (A first, then B), column r % CPL.
  auto read_one = [&](int set, const uint8_t* as, const uint8_t* bs, int kk, int r) {
    const int f = r / CPL, j = r % CPL;
    if (f < FA) set_op(af[set][f], j, rd(as, aoff[kk][j], f));
    else set_op(bf[set][f - FA], j, rd(bs, boff[kk][j], f - FA));
  };

  // One kk on operand set `cur`: NMF MFMA slots; the slots read the next kk's
  // operands (set cur ^ 1) from (as, bs) at nkk, READS spread over the NMF
  // slots, and issue vm(slot).
  auto region = [&](int cur, const uint8_t* as, const uint8_t* bs, int nkk, auto&& vm, bool first) {
#pragma unroll
    for (int s = 0; s < NMF; ++s) {
      if constexpr (BLK) {
        const Acc zero{};
        part[s / FB][s % FB] = mma(bf[cur][s % FB], af[cur][s / FB], first ? zero : part[s / FB][s % FB]);
      } else {
        acc[s / FB][s % FB] = mma(bf[cur][s % FB], af[cur][s / FB], acc[s / FB][s % FB]);
      }
#pragma unroll
      for (int r = s * READS / NMF; r < (s + 1) * READS / NMF; ++r) read_one(cur ^ 1, as, bs, nkk, r);
      vm(s);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Step ks on stage (ac, bc): the loads of step ks + S - 1 go into (al, bl)
  // over the first kk (that stage was last read before the previous barrier).
  // After kk = KK - 2, this wave's loads of step ks + 1 have landed (at most
  // the (S - 2) * LPW loads issued after them remain) and its reads are done
  // (lgkmcnt(0)); past the barrier every wave's are, and the last kk's MFMAs
  // run while the next step's kk = 0 operands are read from (an, bn).
  auto step = [&](int ks, const uint8_t* ac, const uint8_t* bc, const uint8_t* an, const uint8_t* bn, uint8_t* al,
                  uint8_t* bl) {
    const bool in = ks + S - 1 < steps;
    const __amdgpu_buffer_rsrc_t qa = in ? ra : rnull, qb = in ? rb : rnull;
    const int k0 = in ? (ks + S - 1) * BK : 0;
    auto vm = [&](int kk, int s) {
      if (kk != 0) return;
      for (int i = 0; i < LPW; ++i)
        if (s == (i * NMF) / LPW) {
          if (i < 4) load_a(al, qa, k0, i);
          else load_b(bl, qb, k0, i - 4);
        }
    };
    if constexpr (BLK) {
#pragma unroll
      for (int a = 0; a < FA; ++a) {
        sx[a] = x_scale[static_cast<size_t>(ks) * xs_stride + xs_row[a]];
      }
    }
#pragma unroll
    for (int kk = 0; kk + 1 < KK; ++kk)
      region(kk & 1, ac, bc, kk + 1, [&](int s) { vm(kk, s); }, kk == 0);
    if constexpr (S == 2) __asm__ volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)" ::: "memory");
    else __asm__ volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)" ::"n"((S - 2) * LPW) : "memory");
    __builtin_amdgcn_s_barrier();
    region((KK - 1) & 1, an, bn, 0, [&](int) {}, KK == 1);
    if constexpr (BLK) {
      const float sw = wscale[ks];
#pragma unroll
      for (int a = 0; a < FA; ++a) {
        const float f = sx[a] * sw;
#pragma unroll
        for (int b = 0; b < FB; ++b)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[a][b][r] = fmaf(part[a][b][r], f, acc[a][b][r]);
      }
      // The next step's first MFMAs overwrite the partial tile: keep them after
      // the fold (overlapped, they would need a second partial tile).
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Prologue: steps 0 .. S - 2 requested; step 0 waited for.
#pragma unroll
  for (int j = 0; j < S - 1; ++j) {
    uint8_t* a = j == 0 ? A0 : A1;
    uint8_t* b = j == 0 ? B0 : B1;
    const bool in = j < steps;
#pragma unroll
    for (int i = 0; i < 4; ++i) load_a(a, in ? ra : rnull, in ? j * BK : 0, i);
#pragma unroll
    for (int i = 0; i < BLOADS; ++i) load_b(b, in ? rb : rnull, in ? j * BK : 0, i);
  }
  if constexpr (S == 2) __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"((S - 2) * LPW) : "memory");
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int r = 0; r < READS; ++r) read_one(0, A0, B0, 0, r);

  // Step j on stage j % S.
  int ks = 0;
  if constexpr (S == 2) {
    for (; ks + 2 <= steps; ks += 2) {
      step(ks, A0, B0, A1, B1, A1, B1);
      step(ks + 1, A1, B1, A0, B0, A0, B0);
    }
    if (ks < steps) step(ks, A0, B0, A1, B1, A1, B1);
  } else {
    for (; ks + 3 <= steps; ks += 3) {
      step(ks, A0, B0, A1, B1, A2, B2);
      step(ks + 1, A1, B1, A2, B2, A0, B0);
      step(ks + 2, A2, B2, A0, B0, A1, B1);
    }
    if (ks < steps) step(ks, A0, B0, A1, B1, A2, B2);
    if (ks + 1 < steps) step(ks + 1, A1, B1, A2, B2, A0, B0);
  }
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Epilogue. The MFMAs compute the transposed tile (the weight as the A
  // operand): lane l, register r holds row m = l % 32 and output feature
  // 8 (r / 4) + 4 (l / 32) + r % 4 of its 32x32 tile; registers 4q..4q+3 are
  // four consecutive features of one row of y, stored as 8 bytes when N % 4 == 0.
  const bool vec_out = (N & 3) == 0;
#pragma unroll
  for (int a = 0; a < FA; ++a) {
    const int m = m0 + wm * FA * 32 + a * 32 + (lane & 31);
    if (m >= M) continue;
    const float xs = BLK ? 1.0f : x_scale[m];
    uint16_t* yrow = y + static_cast<size_t>(m) * N;
#pragma unroll
    for (int b = 0; b < FB; ++b) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int n = n0 + wn * FB * 32 + b * 32 + 8 * q4 + 4 * (lane >> 5);
        uint16_t out[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float ws = BLK ? 1.0f : (n + i < N ? scale[n + i] : 0.f);
          out[i] = E::from_f32(static_cast<float>(acc[a][b][4 * q4 + i]) * xs * ws);
        }
        if (vec_out && n + 3 < N) {
          *reinterpret_cast<u32x2*>(yrow + n) =
              u32x2{static_cast<uint32_t>(out[0]) | (static_cast<uint32_t>(out[1]) << 16),
                    static_cast<uint32_t>(out[2]) | (static_cast<uint32_t>(out[3]) << 16)};
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (n + i < N) yrow[n + i] = out[i];
        }
      }
    }
  }
}

}  // namespace lnq
