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
  // (l % 8) ^ key(row), key = (row >> 1) & 7, the same for every i). Each
  // load's row offset is in its lane offset and only the step's k offset in
  // the uniform one, so rows past M are out of range whether or not the
  // uniform offset is range-checked.
  const int lrow8 = 8 * wave + (lane >> 3);
  const int lcol = (lane & 7) ^ ((lrow8 >> 1) & 7);
  const int aoff_g = (m0 + lrow8) * K + lcol * 16;
  const int boff_g = (n0 + lrow8) * K + lcol * 16;
  const int lds_w = wave * 1024;
  auto load_a = [&](uint8_t* dst, __amdgpu_buffer_rsrc_t r, int k0, int i) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)(dst + lds_w + i * 64 * BK), 16, aoff_g + i * 64 * K, k0, 0, 0);
  };
  auto load_b = [&](uint8_t* dst, __amdgpu_buffer_rsrc_t r, int k0, int i) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)(dst + lds_w + i * 64 * BK), 16, boff_g + i * 64 * K, k0, 0, 0);
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

// ------------------------------------------ weight-streaming 256 x 128 form
// mm8w_kernel: mm8_kernel<.., 128>'s tiles, waves and MFMA schedule, for the
// shapes that stream the weight (few row tiles: config 4 at 256 rows). There a
// tile keeps two steps of its 16 KB weight step in flight, too few for HBM's
// latency, and more stages of x beside them do not fit. So the operands get
// stages of their own -- SX of x (32 KB each) and SW of weights (16 KB each),
// loaded SX - 1 and SW - 1 steps ahead -- and their loads go to waves of their
// own: waves 0..3 load x (8 loads of 1 KB a step), waves 4..7 the weights (4).
// Loads retire in order per wave, so a wave waiting for its x of step s + 1
// waits for no weight loads, and one waiting for its weights of s + 1 leaves
// those of s + 2 .. s + SW - 1 in flight. Each role runs a K loop of its own
// (the same steps and barriers), so no step branches on the role. Config 4 at
// 256 rows (us): (SX, SW) = (3, 4) 70.5, (3, 3) 72.9, (2, 4) 74.0, (2, 5)
// 75.4, (2, 6) 75.5; the 128-column tile kernel 73.2. The same MFMAs in the
// same k order as mm8_kernel: the same bits.
namespace mm8w {
constexpr int BM = 256, BN = 128, BK = 128, THREADS = 512;
constexpr int XL = 8;  // x loads of an x wave a step (32 KB over 4 waves)
constexpr int WL = 4;  // weight loads of a weight wave a step (16 KB over 4 waves)
}  // namespace mm8w

template <int DT, int FP8, int SX, int SW>
__global__ __launch_bounds__(mm8w::THREADS, 1) void mm8w_kernel(
    const uint8_t* __restrict__ qx, const uint8_t* __restrict__ weight,
    const float* __restrict__ x_scale, const float* __restrict__ scale,
    uint16_t* __restrict__ y, int M, int N, int K) {
  using namespace mm8w;
  static_assert(SX >= 2 && SX <= 3 && SW >= 2 && SW <= 6 && SX * BM * BK + SW * BN * BK <= 160 * 1024, "LDS");
  using E = Elem<DT>;
  constexpr int FA = 2, FB = 2, WAVES_N = 2;  // waves of 64 x 64, 4 x 2
  constexpr int NMF = FA * FB;
  constexpr int KPM = FP8 ? 64 : 32;
  constexpr int KK = BK / KPM;
  constexpr int CPL = KPM / 32;
  using Op = typename std::conditional<FP8, i32x8, i32x4>::type;
  using Acc = typename std::conditional<FP8, f32x16, i32x16>::type;
  // A stage array of its own each (the compiler tracks LDS-bound loads per
  // array); unused stages are never declared, so the used ones may fill all
  // 160 KB.
  __shared__ __attribute__((aligned(16))) uint8_t A0[BM * BK];
  __shared__ __attribute__((aligned(16))) uint8_t A1[BM * BK];
  __shared__ __attribute__((aligned(16))) uint8_t B0[BN * BK];
  __shared__ __attribute__((aligned(16))) uint8_t B1[BN * BK];
  uint8_t *A2 = A0, *B2 = B0, *B3 = B0, *B4 = B0, *B5 = B0;
  if constexpr (SX > 2) {
    __shared__ __attribute__((aligned(16))) uint8_t a2[BM * BK];
    A2 = a2;
  }
  if constexpr (SW > 2) {
    __shared__ __attribute__((aligned(16))) uint8_t b2[BN * BK];
    B2 = b2;
  }
  if constexpr (SW > 3) {
    __shared__ __attribute__((aligned(16))) uint8_t b3[BN * BK];
    B3 = b3;
  }
  if constexpr (SW > 4) {
    __shared__ __attribute__((aligned(16))) uint8_t b4[BN * BK];
    B4 = b4;
  }
  if constexpr (SW > 5) {
    __shared__ __attribute__((aligned(16))) uint8_t b5[BN * BK];
    B5 = b5;
  }
  LNQ_MFMA_IN_AGPRS();

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool xw = wave < 4;  // this wave's loads: x (waves 0..3) or weights (4..7)
  const int lw = wave & 3;
  const int wm = wave / WAVES_N;
  const int wn = wave % WAVES_N;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  mm8_tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  if (tm >= tiles_m || tn >= tiles_n) return;
  const int m0 = tm * BM, n0 = tn * BN;
  const int steps = K / BK;

  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(qx, static_cast<uint32_t>(static_cast<size_t>(M) * K));
  const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(weight, static_cast<uint32_t>(static_cast<size_t>(N) * K));
  const __amdgpu_buffer_rsrc_t rnull = buffer_rsrc(weight, 0);

  // Load i of loading wave lw writes stage rows 32 i + 8 lw .. + 7 (1 KB; lane
  // l: row 32 i + 8 lw + l / 8, stored column l % 8 holding source column
  // (l % 8) ^ key(row), key = (row >> 1) & 7, the same for every i).
  const int lrow8 = 8 * lw + (lane >> 3);
  const int lcol = (lane & 7) ^ ((lrow8 >> 1) & 7);
  const int off_x = (m0 + lrow8) * K + lcol * 16, off_w = (n0 + lrow8) * K + lcol * 16;
  const int lds_w = lw * 1024;
  // Load i (x wave: 0..XL-1, weight wave: 0..WL-1) into stage `dst` through
  // descriptor r at step offset k0.
  auto load_x = [&](uint8_t* dst, __amdgpu_buffer_rsrc_t r, int k0, int i) __attribute__((always_inline)) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)(dst + lds_w + i * 32 * BK), 16, off_x + i * 32 * K, k0, 0, 0);
  };
  auto load_w = [&](uint8_t* dst, __amdgpu_buffer_rsrc_t r, int k0, int i) __attribute__((always_inline)) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)(dst + lds_w + i * 32 * BK), 16, off_w + i * 32 * K, k0, 0, 0);
  };

  Acc acc[FA][FB];
#pragma unroll
  for (int a = 0; a < FA; ++a)
#pragma unroll
    for (int b = 0; b < FB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0;

  const int lrow = lane & 31;
  const int lk = lane >> 5;
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
  auto rd = [&](const uint8_t* stage, uint32_t off, int frag) __attribute__((always_inline)) -> u32x4 {
    return *reinterpret_cast<const u32x4*>(stage + off + frag * 4096);
  };
  auto set_op = [](Op& o, int j, u32x4 v) __attribute__((always_inline)) {
    if constexpr (FP8) {
      o[4 * j + 0] = (int)v.x;
      o[4 * j + 1] = (int)v.y;
      o[4 * j + 2] = (int)v.z;
      o[4 * j + 3] = (int)v.w;
    } else {
      o = __builtin_bit_cast(i32x4, v);
    }
  };
  auto mma = [](const Op& a, const Op& b, Acc c) __attribute__((always_inline)) -> Acc {
    if constexpr (FP8)
      return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0x7f7f7f7f, 0, 0x7f7f7f7f);
    else
      return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  };
  Op af[2][FA], bf[2][FB];
  constexpr int READS = (FA + FB) * CPL;
  auto read_one = [&](int set, const uint8_t* as, const uint8_t* bs, int kk, int r) __attribute__((always_inline)) {
    const int f = r / CPL, j = r % CPL;
    if (f < FA) set_op(af[set][f], j, rd(as, aoff[kk][j], f));
    else set_op(bf[set][f - FA], j, rd(bs, boff[kk][j], f - FA));
  };
  auto region = [&](int cur, const uint8_t* as, const uint8_t* bs, int nkk, auto&& vm) __attribute__((always_inline)) {
#pragma unroll
    for (int sl = 0; sl < NMF; ++sl) {
      acc[sl / FB][sl % FB] = mma(bf[cur][sl % FB], af[cur][sl / FB], acc[sl / FB][sl % FB]);
#pragma unroll
      for (int r = sl * READS / NMF; r < (sl + 1) * READS / NMF; ++r) read_one(cur ^ 1, as, bs, nkk, r);
      vm(sl);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Step s on stages (ac, bc), the next step's on (an, bn); this wave's loads
  // over the first kk: x of step s + SX - 1 into al (an x wave, X) or weights
  // of step s + SW - 1 into bl -- stages last read before the previous barrier.
  // Then this wave's loads of step s + 1 have landed (x waves leave the SX - 2
  // later steps' in flight, weight waves the SW - 2 later steps'), the barrier,
  // and the last kk reads the next step's first operands.
  auto step = [&](auto XW, int s, const uint8_t* ac, const uint8_t* bc, const uint8_t* an, const uint8_t* bn,
                  uint8_t* al, uint8_t* bl) __attribute__((always_inline)) {
    constexpr bool X = decltype(XW)::value;
    const int jl = s + (X ? SX : SW) - 1;
    const __amdgpu_buffer_rsrc_t q = jl < steps ? (X ? ra : rb) : rnull;
    const int k0 = jl < steps ? jl * BK : 0;
    auto vm = [&](int kk, int sl) __attribute__((always_inline)) {
      if (kk != 0) return;
      if constexpr (X) {
#pragma unroll
        for (int i = 0; i < XL; ++i)
          if (sl == (i * NMF) / XL) load_x(al, q, k0, i);
      } else {
#pragma unroll
        for (int i = 0; i < WL; ++i)
          if (sl == (i * NMF) / WL) load_w(bl, q, k0, i);
      }
    };
#pragma unroll
    for (int kk = 0; kk + 1 < KK; ++kk) region(kk & 1, ac, bc, kk + 1, [&](int sl) __attribute__((always_inline)) { vm(kk, sl); });
    if constexpr (X) __asm__ volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)" ::"n"((SX - 2) * XL) : "memory");
    else __asm__ volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)" ::"n"((SW - 2) * WL) : "memory");
    __builtin_amdgcn_s_barrier();
    region((KK - 1) & 1, an, bn, 0, [&](int) __attribute__((always_inline)) {});
  };

  // The whole K loop for one role (x waves, X, or weight waves): the same
  // steps and barriers for both, the role fixed at compile time so a step
  // holds no branch. Prologue: x of steps 0 .. SX - 2 or weights of steps
  // 0 .. SW - 2 requested, step 0 waited for, its first operands read.
  uint8_t* const As[3] = {A0, A1, A2};
  uint8_t* const Bs[6] = {B0, B1, B2, B3, B4, B5};
  auto run = [&](auto XW) __attribute__((always_inline)) {
    constexpr bool X = decltype(XW)::value;
    if constexpr (X) {
#pragma unroll
      for (int j = 0; j < SX - 1; ++j) {
        const __amdgpu_buffer_rsrc_t q = j < steps ? ra : rnull;
        const int k0 = j < steps ? j * BK : 0;
#pragma unroll
        for (int i = 0; i < XL; ++i) load_x(As[j], q, k0, i);
      }
      __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"((SX - 2) * XL) : "memory");
    } else {
#pragma unroll
      for (int j = 0; j < SW - 1; ++j) {
        const __amdgpu_buffer_rsrc_t q = j < steps ? rb : rnull;
        const int k0 = j < steps ? j * BK : 0;
#pragma unroll
        for (int i = 0; i < WL; ++i) load_w(Bs[j], q, k0, i);
      }
      __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"((SW - 2) * WL) : "memory");
    }
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int r = 0; r < READS; ++r) read_one(0, A0, B0, 0, r);

    // Step s on stages (A s % SX, B s % SW); they cycle every L = lcm(SX, SW).
    constexpr int L = SX == 2 ? (SW % 2 == 0 ? SW : 2 * SW) : (SW % 3 == 0 ? SW : 3 * SW);
#define LNQ_MM8W_STEP(S_, J_)                                                                                 \
  step(XW, S_, As[(J_) % SX], Bs[(J_) % SW], As[((J_) + 1) % SX], Bs[((J_) + 1) % SW], As[((J_) + SX - 1) % SX], \
       Bs[((J_) + SW - 1) % SW])
    int ks = 0;
    for (; ks + L <= steps; ks += L) {
#pragma unroll
      for (int j = 0; j < L; ++j) LNQ_MM8W_STEP(ks + j, j);
    }
#pragma unroll
    for (int j = 0; j + 1 < L; ++j)
      if (ks + j < steps) LNQ_MM8W_STEP(ks + j, j);
#undef LNQ_MM8W_STEP
  };
  if (xw) run(std::true_type{});
  else run(std::false_type{});
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Epilogue (mm8_kernel's).
  const bool vec_out = (N & 3) == 0;
#pragma unroll
  for (int a = 0; a < FA; ++a) {
    const int m = m0 + wm * FA * 32 + a * 32 + (lane & 31);
    if (m >= M) continue;
    const float xs = x_scale[m];
    uint16_t* yrow = y + static_cast<size_t>(m) * N;
#pragma unroll
    for (int b = 0; b < FB; ++b) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int n = n0 + wn * FB * 32 + b * 32 + 8 * q4 + 4 * (lane >> 5);
        uint16_t out[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float ws = n + i < N ? scale[n + i] : 0.f;
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

// ------------------------------------------------- persistent 256 x 256 form
// mm8p_kernel: one workgroup per CU walks its tiles (tile b, b + G, b + 2G, ..
// of the grid's XCD-grouped order, G workgroups), and the k-steps of all its
// tiles form one stream: the loads of step g + 2 -- the next tile's near a
// tile's end -- are issued while step g multiplies.
//
// 4 waves, one per SIMD, each owning 128 x 128 outputs (4 x 4 MFMA 32x32
// tiles, 256 accumulator registers): per MFMA a wave reads half the operand
// bytes of mm8_kernel's 128 x 64 waves. 128 input bytes a step in two stages
// of 64 KB (rows of 128 bytes, A rows 0..255 then B rows), filled by
// buffer_load ... lds, 8 rows x 128 bytes an instruction so that every L2
// request is a whole line (64-byte steps split each line in two requests and
// doubled the L2 traffic); 16-byte columns XOR-swizzled by bits 1..3 of the
// row (swz8). Per step, a region per kk: MFMAs on kk's operands while kk + 1's
// are read. One barrier, before the last kk: past it every wave's loads of
// step g + 1 have landed and no wave reads step g's stage again, so the last
// region reads step g + 1's first operands and issues step g + 2's loads into
// step g's stage -- a whole step ahead of their use. At a tile's end the wave
// folds the row and column scales into its tile and stores it; the next
// tile's first MFMAs start from C = 0.
namespace mm8p {
constexpr int BM = 256, BN = 256, BK = 128, NW = 4, THREADS = 64 * NW;
constexpr int FA = 4, FB = 4;                    // 32-row / 32-column fragments of a wave
constexpr int STAGE = (BM + BN) * BK;            // bytes of a stage
constexpr int LPW = (BM + BN) * BK / 1024 / NW;  // 1 KB loads of a wave a step
static_assert(LPW == 16, "a wave's loads a step");
}  // namespace mm8p

template <int DT, int FP8>
__global__ __launch_bounds__(mm8p::THREADS, 1) void mm8p_kernel(
    const uint8_t* __restrict__ qx, const uint8_t* __restrict__ weight,
    const float* __restrict__ x_scale, const float* __restrict__ scale,
    uint16_t* __restrict__ y, int M, int N, int K) {
  using namespace mm8p;
  using E = Elem<DT>;
  constexpr int KPM = FP8 ? 64 : 32;  // inputs per MFMA
  constexpr int KK = BK / KPM;        // MFMAs of a fragment pair a step (2 or 4)
  constexpr int CPL = KPM / 32;       // 16-byte columns of a lane's operand
  using Op = typename std::conditional<FP8, i32x8, i32x4>::type;
  using Acc = typename std::conditional<FP8, f32x16, i32x16>::type;
  // One array per stage: the compiler then waits, before reading a stage, for
  // that stage's loads only.
  __shared__ __attribute__((aligned(16))) uint8_t L0[STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t L1[STAGE];
  LNQ_MFMA_IN_AGPRS();

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = N / BN;
  const int total = tiles_m * tiles_n;
  const int G = gridDim.x;
  const int b0 = blockIdx.x;
  if (b0 >= total) return;
  const int mine = (total - 1 - b0) / G + 1;  // tiles b0, b0 + G, ..
  const int steps = K / BK;                   // even (K % 256 == 0)
  const int nsteps = mine * steps;

  // Rows past M read zeros through the range check: a load's whole row offset
  // is in its lane offset (VGPR), only the step's k offset in the uniform one,
  // so a row past M is out of range whether or not the uniform offset is
  // range-checked. Steps past the stream read through a 0-byte descriptor (no
  // traffic, the same count of loads).
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(qx, static_cast<uint32_t>(static_cast<size_t>(M) * K));
  const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(weight, static_cast<uint32_t>(static_cast<size_t>(N) * K));
  const __amdgpu_buffer_rsrc_t rnull = buffer_rsrc(weight, 0);

  // Load i (0..15) of wave w fills stage rows 8 (4 i + w) .. + 7 (i < 8: A rows
  // 32 i + 8 w + l / 8 of the tile; else B rows 32 (i - 8) + 8 w + l / 8): lane
  // l at byte 16 l of the 1 KB, stored column l % 8 holding source column
  // (l % 8) ^ key(row), key = (row >> 1) & 7, the same for every i.
  const int lr = 8 * wave + (lane >> 3);
  const int lane_off = lr * K + 16 * ((lane & 7) ^ ((lr >> 1) & 7));
  // The lane offsets of tile r's rows (r past this workgroup's tiles: any
  // offsets, their loads go through the 0-byte descriptor).
  uint32_t voff[LPW];
  auto tile_offsets = [&](int r) {
    int tm, tn;
    mm8_tile_of(b0 + r * G, tiles_m, tiles_n, tm, tn);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      voff[i] = static_cast<uint32_t>((tm * BM + 32 * i) * K + lane_off);
      voff[8 + i] = static_cast<uint32_t>((tn * BN + 32 * i) * K + lane_off);
    }
  };
  // Load i of k-step ks (tile offsets in voff) into stage st.
  auto load_one = [&](uint8_t* st, bool in, int ks, int i) {
    const __amdgpu_buffer_rsrc_t q = in ? (i < 8 ? ra : rb) : rnull;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(q, (lds_ptr)(st + (4 * i + wave) * 1024), 16, voff[i],
                                              in ? ks * BK : 0, 0, 0);
  };

  // Each tile's first step starts its accumulators with C = 0 (no clearing:
  // a zeroed register would make the compiler keep the accumulators in VGPRs).
  Acc acc[FA][FB];

  // Operand offsets within a stage per (kk, column j): fragments of one operand
  // are 32 rows (4096 bytes) apart with the same swizzle key.
  const int lrow = lane & 31, lk = lane >> 5;
  uint32_t aoff[KK][CPL], boff[KK][CPL];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk)
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c16 = kk * 2 * CPL + lk * CPL + j;
      aoff[kk][j] = static_cast<uint32_t>(swz8(wm * 128 + lrow, c16));
      boff[kk][j] = static_cast<uint32_t>(swz8(BM + wn * 128 + lrow, c16));
    }
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
  // Operand registers: set 0 holds even kk, set 1 odd kk (KK is even).
  Op af[2][FA], bf[2][FB];
  constexpr int READS = (FA + FB) * CPL;  // 16-byte reads of one kk's operands
  constexpr int NMF = FA * FB;            // MFMAs of one kk
  auto read_one = [&](int set, const uint8_t* st, int kk, int r) {
    const int f = r / CPL, j = r % CPL;
    if (f < FA)
      set_op(af[set][f], j, *reinterpret_cast<const u32x4*>(st + aoff[kk][j] + f * 4096));
    else
      set_op(bf[set][f - FA], j, *reinterpret_cast<const u32x4*>(st + boff[kk][j] + (f - FA) * 4096));
  };

  // The epilogue of a tile (m0, n0): lane l, register r of fragment (a, b) holds
  // row m = m0 + 128 wm + 32 a + l % 32 and column n0 + 128 wn + 32 b + 8 (r / 4)
  // + 4 (l / 32) + r % 4 (the weight is the MFMA's A operand).
  auto epilogue = [&](int m0, int n0) {
    float xs[FA];
#pragma unroll
    for (int a = 0; a < FA; ++a) xs[a] = x_scale[min(m0 + wm * 128 + a * 32 + lrow, M - 1)];
#pragma unroll
    for (int b = 0; b < FB; ++b) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int n = n0 + wn * 128 + b * 32 + 8 * q4 + 4 * lk;
        const f32x4 ws = *reinterpret_cast<const f32x4*>(scale + n);
#pragma unroll
        for (int a = 0; a < FA; ++a) {
          const int m = m0 + wm * 128 + a * 32 + lrow;
          uint32_t o[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = E::from_f32(static_cast<float>(acc[a][b][4 * q4 + i]) * xs[a] * ws[i]);
          if (m < M)
            *reinterpret_cast<u32x2*>(y + static_cast<size_t>(m) * N + n) = u32x2{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
        }
      }
      // One column fragment at a time: the next tile's operands are live here.
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // One kk of step g on stage `cur` (operand set kk & 1): NMF MFMA slots, the
  // slots reading kk + 1's operands from `cur`, or, in the last kk, step g +
  // 1's first operands from `nxt` and issuing step g + 2's loads (k-step ks2,
  // `ld2` whether inside the stream) into `cur`, one a slot.
  auto region = [&](int kk, auto first_tag, const uint8_t* cur, const uint8_t* nxt, bool ld2, int ks2) {
    constexpr bool FIRST = decltype(first_tag)::value;  // a tile's first step
    const int set = kk & 1;
    const bool last = kk == KK - 1;
#pragma unroll
    for (int s = 0; s < NMF; ++s) {
      const int a = s / FB, b = s % FB;
      if (FIRST && kk == 0) acc[a][b] = mma(bf[set][b], af[set][a], Acc{});
      else acc[a][b] = mma(bf[set][b], af[set][a], acc[a][b]);
#pragma unroll
      for (int r = s * READS / NMF; r < (s + 1) * READS / NMF; ++r) {
        if (last) read_one(set ^ 1, nxt, 0, r);
        else read_one(set ^ 1, cur, kk + 1, r);
      }
      if (last) {
#pragma unroll
        for (int i = s * LPW / NMF; i < (s + 1) * LPW / NMF; ++i) load_one(const_cast<uint8_t*>(cur), ld2, ks2, i);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Step g on stage `cur` (step g + 1 on `nxt`): regions kk = 0 .. KK - 2; this
  // wave's loads of step g + 1 landed (nothing is issued after them before this
  // point but the previous epilogue's stores) and its reads done; barrier; the
  // last region.
  auto step = [&](auto first_tag, const uint8_t* cur, const uint8_t* nxt, bool ld2, int ks2) {
#pragma unroll
    for (int kk = 0; kk + 1 < KK; ++kk) region(kk, first_tag, cur, nxt, false, 0);
    wait_vm<0>();
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    region(KK - 1, first_tag, cur, nxt, ld2, ks2);
  };

  // Prologue: steps 0 and 1 (of tile 0: a tile has at least two steps)
  // requested; step 0 landed (this wave's, then every wave's); its kk = 0
  // operands read.
  tile_offsets(0);
#pragma unroll
  for (int i = 0; i < LPW; ++i) load_one(L0, true, 0, i);
#pragma unroll
  for (int i = 0; i < LPW; ++i) load_one(L1, true, 1, i);
  wait_vm<LPW>();
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int r = 0; r < READS; ++r) read_one(0, L0, 0, r);

  // Pairs of steps (K % 256 == 0: a tile is whole pairs) g, g + 1 of tile r at
  // k-step ks on stages L0, L1: they issue steps g + 2, g + 3, the next pair's
  // (tile r, or r + 1 after a tile's last pair), with no branch inside the
  // pair: the compiler would otherwise move the MFMAs across the blocks it
  // split the pair into. A tile's first pair is its own copy (accumulators
  // started at zero).
  using T = std::integral_constant<bool, true>;
  using F = std::integral_constant<bool, false>;
  auto pair = [&](int g, int r, int ks, auto first_tag) {
    const bool ends = ks + 2 == steps;
    const int ks_n = ends ? 0 : ks + 2;
    tile_offsets(r + (ends ? 1 : 0));
    step(first_tag, L0, L1, g + 2 < nsteps, ks_n);
    step(F{}, L1, L0, g + 3 < nsteps, ks_n + 1);
  };
  int g = 0;
  for (int r = 0; r < mine; ++r) {
    pair(g, r, 0, T{});
    g += 2;
    for (int ks = 2; ks < steps; ks += 2, g += 2) pair(g, r, ks, F{});
    int tm, tn;
    mm8_tile_of(b0 + r * G, tiles_m, tiles_n, tm, tn);
    epilogue(tm * BM, tn * BN);
  }
  // Loads of the steps past the stream (0-byte reads) may be in flight.
  wait_vm<0>();
}

}  // namespace lnq
