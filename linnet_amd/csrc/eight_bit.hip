// 8-bit weights (std.quant::Int8Linear / Int8GroupLinear / Fp8Linear / Fp8BlockLinear)
// on gfx950:
//   - w8_skinny:  weight-only product for few rows (gemv8 / w8a16), weights
//                 widened in registers and multiplied on MFMA, x unrounded;
//   - dequant8:   the weight widened and scaled, rounded to the output dtype;
//   - rows8:      dynamic per-token FP8 / int8 rounding of activations;
//   - mm8:        int8 x int8 (int32 sums) or FP8 x FP8 (f32 sums) tiled MFMA GEMM
//                 with the row-scale epilogue (the kernel template: eight_bit.hpp;
//                 its block-scaled FP8 form: fp8_block.hip);
//   - int8_quantize: symmetric group-wise int8 rounding, bit-exact with numpy.
#include "eight_bit.hpp"

namespace lnq {

// ------------------------------------------------------------------ helpers

// 4 FP8 E4M3 bytes -> 4 f32 (exact) via the hardware conversion.
__device__ inline void fp8x4_to_f32(uint32_t w, float (&f)[4]) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), false);
  const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), true);
  f[0] = lo.x;
  f[1] = lo.y;
  f[2] = hi.x;
  f[3] = hi.y;
}

// Two f32 values that are exact in the 16-bit type, packed (low = a). For bf16
// the top halves are the value (low halves are zero for these small-mantissa
// values); f16 converts.
template <int DT>
__device__ inline uint32_t pack_exact2(float a, float b) {
  if constexpr (DT == LNQ_BF16) {
    return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, b), __builtin_bit_cast(uint32_t, a),
                                 0x07060302u);
  } else {
    return static_cast<uint32_t>(f32_to_f16_bits(a)) | (static_cast<uint32_t>(f32_to_f16_bits(b)) << 16);
  }
}

// 4 weight bytes as 4 values of the 16-bit type (two dwords, element order).
// int8: the byte plus 128 (0..255, exact in bf16 / f16), undone by the
// epilogue's -128 * sum(x); FP8: the value itself (the hardware conversion,
// two values an instruction).
template <int DT, int FP8>
__device__ inline void widen4(uint32_t w, uint32_t& d0, uint32_t& d1) {
  if constexpr (FP8) {
    // Two E4M3 bytes to two 16-bit values in one instruction (exact: E4M3's 3
    // mantissa bits and 2^-9 .. 448 fit both bf16 and f16).
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    if constexpr (DT == LNQ_BF16) {
      d0 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
      d1 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true));
    } else {
      d0 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false));
      d1 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true));
    }
    return;
  }
  float f[4];
  {
    const uint32_t u = w ^ 0x80808080u;
    f[0] = static_cast<float>(u & 0xffu);
    f[1] = static_cast<float>((u >> 8) & 0xffu);
    f[2] = static_cast<float>((u >> 16) & 0xffu);
    f[3] = static_cast<float>(u >> 24);
  }
  d0 = pack_exact2<DT>(f[0], f[1]);
  d1 = pack_exact2<DT>(f[2], f[3]);
}

// =================================================================== skinny
// One workgroup (4 waves) owns 16 output features and 16*MT rows of x; the
// waves split K into contiguous quarters, reduced through LDS. A chunk is 64
// inputs: lane (col, j) reads 16 bytes of row n0 + col at byte 64c + 16j and
// feeds MFMA t (t = 0, 1) elements 8t..8t+7 of them. A group (of `group`
// inputs, or the whole row when the scale is per row) closes with
//   acc += s * (C - offset * Cx),  Cx = sum of x over the group (B = ones).
// ONE (one row of x, MT = 1): x is staged in LDS once (dynamic shared memory
// of K 16-bit values) and the ring holds only weight bytes, 16 chunks deep.
template <int DT, int FP8, int MT, bool ONE = false>
__global__ __launch_bounds__(256) void w8_skinny_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ weight,
    const float* __restrict__ scale, uint16_t* __restrict__ y, int M, int N, int K, int G,
    int row_block, int scale_cols) {
  using E = Elem<DT>;
  constexpr float offset = FP8 ? 0.0f : 128.0f;
  static_assert(!ONE || MT == 1, "the one-row form has one x tile");
  __shared__ f32x4 red[4][MT][64];
  extern __shared__ __attribute__((aligned(16))) uint16_t xl[];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int j = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int m0 = blockIdx.y * 16 * MT;
  const int nrow = min(n0 + col, N - 1);
  const int chunks = K >> 6;
  const int per_wave = (chunks + 3) >> 2;
  const int cb = min(chunks, wave * per_wave);
  const int ce = min(chunks, cb + per_wave);
  const int chunks_per_group = G >> 6;

  const uint8_t* wrow = weight + static_cast<size_t>(nrow) * K;
  const float* srow = scale + static_cast<size_t>(nrow / row_block) * scale_cols;

  const uint16_t* xrow[MT];
  bool mok[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = m0 + 16 * mt + col;
    mok[mt] = m < M;
    xrow[mt] = x + static_cast<size_t>(mok[mt] ? m : 0) * K;
  }
  u32x4 ones;
  ones.x = ones.y = ones.z = ones.w = E::ONE2;

  f32x4 acc[MT], C[MT], Cx[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    C[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    Cx[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // A ring of D chunks in flight per wave: the weight bytes (streamed once,
  // non-temporal) and the x values they meet, requested D chunks ahead so the
  // wave keeps D loads of each in flight instead of waiting on every chunk.
  constexpr int D = ONE ? 16 : MT == 1 ? 8 : MT == 2 ? 4 : 2;
  u32x4 rw[D];
  u32x4 rx[ONE ? 1 : D][MT][2];
  auto fetch = [&](int slot, int c) {
    rw[slot] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + 64 * c + 16 * j));
    if constexpr (!ONE) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < 2; ++t)
          rx[slot][mt][t] = *reinterpret_cast<const u32x4*>(xrow[mt] + 64 * c + 16 * j + 8 * t);
    }
  };
#pragma unroll
  for (int i = 0; i < D; ++i)
    if (cb + i < ce) fetch(i, cb + i);
  if constexpr (ONE) {
    // Staged while the first D weight chunks are in flight.
    for (int i = 8 * threadIdx.x; i < K; i += 8 * 256)
      *reinterpret_cast<u32x4*>(&xl[i]) = *reinterpret_cast<const u32x4*>(&x[i]);
    __syncthreads();
  }
  for (int c0 = cb; c0 < ce; c0 += D) {
#pragma unroll
    for (int i = 0; i < D; ++i) {
      const int c = c0 + i;
      if (c >= ce) break;
      const u32x4 w = rw[i];
      u32x4 xa[MT][2];
      if constexpr (ONE) {
        // Every lane takes row 0: the 15 copies of it land in output rows
        // past M, which are not stored.
#pragma unroll
        for (int t = 0; t < 2; ++t) xa[0][t] = *reinterpret_cast<const u32x4*>(&xl[64 * c + 16 * j + 8 * t]);
      } else {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int t = 0; t < 2; ++t) xa[mt][t] = mok[mt] ? rx[i][mt][t] : u32x4{0u, 0u, 0u, 0u};
      }
      if (c + D < ce) fetch(i, c + D);
      const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        uint32_t b0, b1, b2, b3;
        widen4<DT, FP8>(words[2 * t], b0, b1);
        widen4<DT, FP8>(words[2 * t + 1], b2, b3);
        const u32x4 b = {b0, b1, b2, b3};
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          C[mt] = mfma16x16x32<DT>(xa[mt][t], b, C[mt]);
          if constexpr (!FP8) Cx[mt] = mfma16x16x32<DT>(xa[mt][t], ones, Cx[mt]);
        }
      }
      const bool closes = ((c + 1) % chunks_per_group == 0) || (c + 1 == ce);
      if (closes) {
        const float s = srow[c / chunks_per_group];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float d = FP8 ? C[mt][r] : fmaf(-offset, Cx[mt][r], C[mt][r]);
            acc[mt][r] = fmaf(s, d, acc[mt][r]);
          }
          C[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
          Cx[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
  }

#pragma unroll
  for (int mt = 0; mt < MT; ++mt) red[wave][mt][lane] = acc[mt];
  __syncthreads();
  const int olane = threadIdx.x & 63;
  const int r = threadIdx.x >> 6;
  const int n = n0 + (olane & 15);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = m0 + 16 * mt + 4 * (olane >> 4) + r;
    const float v = red[0][mt][olane][r] + red[1][mt][olane][r] + red[2][mt][olane][r] +
                    red[3][mt][olane][r];
    if (m < M && n < N) y[static_cast<size_t>(m) * N + n] = E::from_f32(v);
  }
}

// =================================================================== one row
// One row of x (a decoding step), groups a multiple of 128 inputs, K % 512 == 0.
// The skinny kernel's workgroups (16 output features, 4 waves each a quarter of
// K, x staged in LDS) with wider reads: a wave instruction reads 8 rows x 128
// contiguous bytes (lane: row l % 8, 16-byte piece l / 8) instead of 16 rows x 64
// bytes, which streams faster (a 235 MB pure read in this workgroup shape: 34-35
// against 39 us). Lane l then holds, for B column c = l % 16, piece 2 (l / 16) +
// c / 8 of row c % 8: columns 0-7 carry the even pieces and 8-15 the odd ones
// of the same 8 rows, so A row 0 takes x at the even pieces and A row 1 at the
// odd ones, and row r's sum is C[0][r] + C[1][8 + r]. Two loads (rows 0-7 and
// 8-15) per 128 inputs, each two MFMA 16x16x32 (bytes 0-7 and 8-15 of a piece).
//
// NW waves split K; D loads in flight per wave. K = 4096 runs
// w8_row_slices_kernel below instead.
template <int DT, int FP8, int NW = 4, int D = 16>
__global__ __launch_bounds__(64 * NW) void w8_row_kernel(const uint16_t* __restrict__ x,
                                                         const uint8_t* __restrict__ weight,
                                                         const float* __restrict__ scale,
                                                         uint16_t* __restrict__ y, int N, int K, int G,
                                                         int row_block, int scale_cols) {
  using E = Elem<DT>;
  constexpr float offset = FP8 ? 0.0f : 128.0f;
  constexpr int THREADS = 64 * NW;
  __shared__ float red[NW][16];
  extern __shared__ __attribute__((aligned(16))) uint16_t xl[];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int j = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int steps = K >> 7;  // 128 inputs a step
  const int per_wave = steps / NW;
  const int sb = wave * per_wave, se = sb + per_wave;
  const int steps_per_group = G >> 7;

  // Load rows: half h reads rows n0 + 8h + l % 8 (clamped: rows past N are not stored).
  const uint8_t* wrow[2];
  const float* srow[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    wrow[h] = weight + static_cast<size_t>(min(n0 + 8 * h + (lane & 7), N - 1)) * K + 16 * (lane >> 3);
    // The scale of this lane's B column (row n0 + 8h + col % 8).
    const int srow_n = min(n0 + 8 * h + (col & 7), N - 1);
    srow[h] = scale + static_cast<size_t>(srow_n / row_block) * scale_cols;
  }
  u32x4 ones;
  ones.x = ones.y = ones.z = ones.w = E::ONE2;
  f32x4 acc[2], C[2], Cx;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    acc[h] = f32x4{0.f, 0.f, 0.f, 0.f};
    C[h] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  Cx = f32x4{0.f, 0.f, 0.f, 0.f};

  u32x4 rw[D];
  auto fetch = [&](int slot, int step) {
    rw[slot] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[slot & 1] + 128 * step));
  };
  // x and the scales of the wave's first group into registers first, then the
  // ring's weight loads, and only then x into LDS: a store of x right after its
  // load would hold every weight load back by x's round trip. (Loads retire in
  // issue order, so x and the scales land ahead of the weights.)
  constexpr int XR = 8192 / (8 * THREADS);  // x chunks a thread loads (K <= 8192 from registers)
  u32x4 xr[XR];
#pragma unroll
  for (int r = 0; r < XR; ++r) {
    const int i = 8 * (threadIdx.x + THREADS * r);
    xr[r] = i < K ? *reinterpret_cast<const u32x4*>(&x[i]) : u32x4{0u, 0u, 0u, 0u};
  }
  const int g_first = sb / steps_per_group;
  float s_first[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) s_first[h] = srow[h][g_first];
  __asm__ volatile("" ::: "memory");
  // (Unconditional: a wave with fewer than D / 2 steps re-reads its last one,
  // unused, so that the number of loads in flight is known where x is stored.)
#pragma unroll
  for (int i = 0; i < D; ++i) fetch(i, min(sb + (i >> 1), se - 1));
  __asm__ volatile("" ::: "memory");
#pragma unroll
  for (int r = 0; r < XR; ++r) {
    const int i = 8 * (threadIdx.x + THREADS * r);
    if (i < K) *reinterpret_cast<u32x4*>(&xl[i]) = xr[r];
  }
  for (int i = 8 * (threadIdx.x + THREADS * XR); i < K; i += 8 * THREADS)
    *reinterpret_cast<u32x4*>(&xl[i]) = *reinterpret_cast<const u32x4*>(&x[i]);
  __syncthreads();
  // A row m (lane m = l % 16): x at piece 2 j + (m & 1); rows 2..15 repeat rows
  // 0 / 1 and their outputs are not used.
  const int apiece = 2 * j + (col & 1);
  for (int s0 = sb; s0 < se; s0 += D / 2) {
#pragma unroll
    for (int i = 0; i < D / 2; ++i) {
      const int step = s0 + i;
      if (step >= se) break;
      u32x4 xa[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) xa[t] = *reinterpret_cast<const u32x4*>(&xl[128 * step + 16 * apiece + 8 * t]);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const u32x4 w = rw[2 * i + h];
        if (step + D / 2 < se) fetch(2 * i + h, step + D / 2);
        const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          uint32_t b0, b1, b2, b3;
          widen4<DT, FP8>(words[2 * t], b0, b1);
          widen4<DT, FP8>(words[2 * t + 1], b2, b3);
          C[h] = mfma16x16x32<DT>(xa[t], u32x4{b0, b1, b2, b3}, C[h]);
        }
      }
      if constexpr (!FP8) {
#pragma unroll
        for (int t = 0; t < 2; ++t) Cx = mfma16x16x32<DT>(xa[t], ones, Cx);
      }
      // A group closes at its last step or where this wave's quarter of K ends.
      if ((step + 1) % steps_per_group == 0 || step + 1 == se) {
        const int g = step / steps_per_group;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float sc = s_first[h];
          if (g != g_first) {
            // (The asm keeps this load in its branch: loaded speculatively, the
            // wait for it would add a round trip to every group's end.)
            __asm__ volatile("" ::: "memory");
            sc = srow[h][g];
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float d = FP8 ? C[h][r] : fmaf(-offset, Cx[r], C[h][r]);
            acc[h][r] = fmaf(sc, d, acc[h][r]);
          }
          C[h] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        Cx = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
  }
  // Lane col (j = 0) holds A row 0 in register 0 and row 1 in register 1: row
  // col % 8 of half h is C[0][col % 8] + C[1][8 + col % 8].
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float mine = col < 8 ? acc[h][0] : acc[h][1];
    const float v = mine + __shfl_xor(mine, 8, 64);
    if (j == 0 && col < 8) red[wave][8 * h + col] = v;
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    const int n = n0 + threadIdx.x;
    float v = red[0][threadIdx.x];
#pragma unroll
    for (int w = 1; w < NW; ++w) v += red[w][threadIdx.x];
    if (n < N) y[n] = E::from_f32(v);
  }
}

// One row of x at K = 4096 (config 1's int8 4096 x 4096 GEMV): the workgroups
// and loads of w8_row_kernel (16 output features, lane l reading row l % 8,
// piece l / 8 of a 128-input step), with K split over 16 waves of 2 steps, so
// every load of a CU is in flight at once and each wave multiplies as soon as
// its own loads land. Each wave loads just the 256 inputs of x its steps use,
// straight into its MFMA A-operand registers (32 bytes of x a lane a step,
// issued before the weights): no LDS stage of x and no workgroup barrier ahead of
// the products (6.2 -> 5.6 us for config 1). The sums are w8_row_kernel's, in
// the same order (the same bits).
template <int DT, int FP8>
__global__ __launch_bounds__(1024) void w8_row_slices_kernel(const uint16_t* __restrict__ x,
                                                             const uint8_t* __restrict__ weight,
                                                             const float* __restrict__ scale,
                                                             uint16_t* __restrict__ y, int N, int G, int row_block,
                                                             int scale_cols) {
  using E = Elem<DT>;
  constexpr float offset = FP8 ? 0.0f : 128.0f;
  constexpr int K = 4096;
  constexpr int NW = 16;
  constexpr int PW = K / 128 / NW;  // steps a wave
  __shared__ float red[NW][16];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int j = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int sb = wave * PW;
  const int steps_per_group = G >> 7;

  const uint8_t* wrow[2];
  const float* srow[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    wrow[h] = weight + static_cast<size_t>(min(n0 + 8 * h + (lane & 7), N - 1)) * K + 16 * (lane >> 3);
    const int srow_n = min(n0 + 8 * h + (col & 7), N - 1);
    srow[h] = scale + static_cast<size_t>(srow_n / row_block) * scale_cols;
  }
  u32x4 ones;
  ones.x = ones.y = ones.z = ones.w = E::ONE2;
  f32x4 acc[2], C[2], Cx;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    acc[h] = f32x4{0.f, 0.f, 0.f, 0.f};
    C[h] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  Cx = f32x4{0.f, 0.f, 0.f, 0.f};

  // A row m (lane m = l % 16) takes x at piece 2 j + (m & 1) of each step; rows
  // 2..15 repeat rows 0 / 1 and their outputs are not used.
  const int apiece = 2 * j + (col & 1);
  u32x4 xa[PW][2];
#pragma unroll
  for (int i = 0; i < PW; ++i)
#pragma unroll
    for (int t = 0; t < 2; ++t) xa[i][t] = *reinterpret_cast<const u32x4*>(&x[128 * (sb + i) + 16 * apiece + 8 * t]);
  const int g_first = sb / steps_per_group;
  float s_first[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) s_first[h] = srow[h][g_first];
  __asm__ volatile("" ::: "memory");
  u32x4 rw[2 * PW];
#pragma unroll
  for (int i = 0; i < 2 * PW; ++i)
    rw[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[i & 1] + 128 * (sb + (i >> 1))));

#pragma unroll
  for (int i = 0; i < PW; ++i) {
    const int step = sb + i;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const u32x4 w = rw[2 * i + h];
      const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        uint32_t b0, b1, b2, b3;
        widen4<DT, FP8>(words[2 * t], b0, b1);
        widen4<DT, FP8>(words[2 * t + 1], b2, b3);
        C[h] = mfma16x16x32<DT>(xa[i][t], u32x4{b0, b1, b2, b3}, C[h]);
      }
    }
    if constexpr (!FP8) {
#pragma unroll
      for (int t = 0; t < 2; ++t) Cx = mfma16x16x32<DT>(xa[i][t], ones, Cx);
    }
    // A group closes at its last step or where this wave's steps end.
    if ((step + 1) % steps_per_group == 0 || i + 1 == PW) {
      const int g = step / steps_per_group;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float sc = s_first[h];
        if (g != g_first) {
          // (The asm keeps this load in its branch, as in w8_row_kernel.)
          __asm__ volatile("" ::: "memory");
          sc = srow[h][g];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float d = FP8 ? C[h][r] : fmaf(-offset, Cx[r], C[h][r]);
          acc[h][r] = fmaf(sc, d, acc[h][r]);
        }
        C[h] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      Cx = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  // Row col % 8 of half h is C[0][col % 8] + C[1][8 + col % 8] (w8_row_kernel).
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float mine = col < 8 ? acc[h][0] : acc[h][1];
    const float v = mine + __shfl_xor(mine, 8, 64);
    if (j == 0 && col < 8) red[wave][8 * h + col] = v;
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    const int n = n0 + threadIdx.x;
    float v = red[0][threadIdx.x];
#pragma unroll
    for (int w = 1; w < NW; ++w) v += red[w][threadIdx.x];
    if (n < N) y[n] = E::from_f32(v);
  }
}

// ================================================================== dequant8
// 16 weight bytes per thread: out = widen(w) * scale in f32, rounded once.
template <int DT, int FP8>
__global__ __launch_bounds__(256) void dequant8_kernel(const uint8_t* __restrict__ weight,
                                                       const float* __restrict__ scale,
                                                       typename Elem<DT>::storage* __restrict__ out,
                                                       int64_t units, int K, int G, int row_block,
                                                       int scale_cols) {
  using E = Elem<DT>;
  const int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (u >= units) return;
  const int64_t per_row = K >> 4;
  const int64_t n = u / per_row;
  const int k0 = static_cast<int>(u - n * per_row) << 4;
  const float* srow = scale + (G == 0 ? n : (n / row_block) * scale_cols);
  const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(weight + (u << 4)));
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
  typename E::storage* dst = out + n * K + k0;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    float f[4];
    if constexpr (FP8) {
      fp8x4_to_f32(words[d], f);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        f[i] = static_cast<float>(static_cast<int8_t>((words[d] >> (8 * i)) & 0xffu));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = k0 + 4 * d + i;
      const float s = G == 0 ? srow[0] : srow[k / G];
      dst[4 * d + i] = E::from_f32(f[i] * s);
    }
  }
}

// ===================================================================== rows8
// One workgroup per row. scale = max(max|x|, 1e-12) / (448 | 127) in f32;
// q = x / scale (IEEE divide) then FP8 E4M3 round-to-nearest-even of
// clamp(q, +-448), or int8 clamp(trunc(q +- 0.5), +-127) with the add in f32.

template <int DT, int FP8>
__global__ __launch_bounds__(256) void rows8_kernel(const typename Elem<DT>::storage* __restrict__ x,
                                                    uint8_t* __restrict__ q,
                                                    float* __restrict__ x_scale, int K) {
  using E = Elem<DT>;
  __shared__ float partial[4];
  const int64_t row = blockIdx.x;
  const typename E::storage* src = x + row * K;
  float top = 0.0f;
  for (int i = threadIdx.x; i < K; i += 256) top = fmaxf(top, fabsf(E::to_f32(src[i])));
  top = wave_max(top);
  if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = top;
  __syncthreads();
  top = fmaxf(fmaxf(partial[0], partial[1]), fmaxf(partial[2], partial[3]));
  const float largest = FP8 ? 448.0f : 127.0f;
  const float s = fmaxf(top, 1e-12f) / largest;
  uint8_t* dst = q + row * K;
  for (int i = threadIdx.x; i < K; i += 256) {
    const float v = E::to_f32(src[i]) / s;
    if constexpr (FP8) {
      dst[i] = static_cast<uint8_t>(f32_to_e4m3(fminf(fmaxf(v, -448.0f), 448.0f)));
    } else {
      const float h = v >= 0.0f ? __fadd_rn(v, 0.5f) : __fsub_rn(v, 0.5f);
      dst[i] = static_cast<uint8_t>(static_cast<int8_t>(fminf(fmaxf(truncf(h), -127.0f), 127.0f)));
    }
  }
  if (threadIdx.x == 0) x_scale[row] = s;
}

// The same per row with 16-byte loads and VEC-byte stores (K % VEC == 0 and
// 16-byte aligned rows). R > 0: each thread keeps its R vectors of the row in
// registers between the pass for max|x| and the pass that quantizes (rows of
// up to R * VEC * 256 elements); R == 0: the second pass reads the row again.
// Same arithmetic as rows8_kernel.
template <int DT, int FP8, int R>
__global__ __launch_bounds__(256) void rows8_vec_kernel(const typename Elem<DT>::storage* __restrict__ x,
                                                        uint8_t* __restrict__ q, float* __restrict__ x_scale, int K) {
  using E = Elem<DT>;
  constexpr int VEC = 16 / static_cast<int>(sizeof(typename E::storage));  // elements per 16 bytes
  __shared__ float partial[4];
  const int64_t row = blockIdx.x;
  const typename E::storage* src = x + row * K;
  // (f32 rows load as a float vector: this toolchain folds __builtin_bit_cast
  // of an ext_vector element to element 0.)
  auto load = [&](int i, float (&v)[VEC]) {
    if constexpr (VEC == 8) {
      const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + i));
      const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[2 * j] = E::to_f32(static_cast<uint16_t>(d[j] & 0xffffu));
        v[2 * j + 1] = E::to_f32(static_cast<uint16_t>(d[j] >> 16));
      }
    } else {
      const f32x4 w = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(src + i));
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = w[j];
    }
  };
  uint8_t* dst = q + row * K;
  auto put = [&](int i, const float (&v)[VEC], float s) {
    uint32_t b[VEC / 4];
#pragma unroll
    for (int j = 0; j < VEC / 4; ++j) b[j] = 0;
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const float t = v[j] / s;
      uint32_t code;
      if constexpr (FP8) {
        code = f32_to_e4m3(fminf(fmaxf(t, -448.0f), 448.0f));
      } else {
        const float h = t >= 0.0f ? __fadd_rn(t, 0.5f) : __fsub_rn(t, 0.5f);
        code = static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int8_t>(fminf(fmaxf(truncf(h), -127.0f), 127.0f))));
      }
      b[j / 4] |= code << (8 * (j % 4));
    }
    if constexpr (VEC == 8) {
      *reinterpret_cast<u32x2*>(dst + i) = u32x2{b[0], b[1]};
    } else {
      *reinterpret_cast<uint32_t*>(dst + i) = b[0];
    }
  };
  auto scale_of = [&](float top) {
    top = wave_max(top);
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = top;
    __syncthreads();
    top = fmaxf(fmaxf(partial[0], partial[1]), fmaxf(partial[2], partial[3]));
    const float largest = FP8 ? 448.0f : 127.0f;
    return fmaxf(top, 1e-12f) / largest;
  };
  float top = 0.0f;
  float s;
  if constexpr (R > 0) {
    float v[R > 0 ? R : 1][VEC];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = VEC * (static_cast<int>(threadIdx.x) + 256 * r);
      if (i < K) {
        load(i, v[r]);
      } else {
#pragma unroll
        for (int j = 0; j < VEC; ++j) v[r][j] = 0.0f;
      }
#pragma unroll
      for (int j = 0; j < VEC; ++j) top = fmaxf(top, fabsf(v[r][j]));
    }
    s = scale_of(top);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = VEC * (static_cast<int>(threadIdx.x) + 256 * r);
      if (i < K) put(i, v[r], s);
    }
  } else {
    for (int i = VEC * threadIdx.x; i < K; i += VEC * 256) {
      float v[VEC];
      load(i, v);
#pragma unroll
      for (int j = 0; j < VEC; ++j) top = fmaxf(top, fabsf(v[j]));
    }
    s = scale_of(top);
    for (int i = VEC * threadIdx.x; i < K; i += VEC * 256) {
      float v[VEC];
      load(i, v);
      put(i, v, s);
    }
  }
  if (threadIdx.x == 0) x_scale[row] = s;
}

// ============================================================= int8 quantize
// One wave per group, numpy's f32 order of operations (linnet/quant.py:112-120).
__device__ inline float round_storage(float v, int dtype) {
  if (dtype == LNQ_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  if (dtype == LNQ_F16) return static_cast<float>(static_cast<_Float16>(v));
  return v;
}

__global__ __launch_bounds__(256) void int8_quantize_kernel(const float* __restrict__ w,
                                                            int8_t* __restrict__ q,
                                                            float* __restrict__ scale,
                                                            int64_t total_groups, int G,
                                                            int dtype) {
  const int lane = threadIdx.x & 63;
  const int64_t grp = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (grp >= total_groups) return;
  const float* p = w + grp * G;
  float top = 0.0f;
  for (int i = lane; i < G; i += 64) top = fmaxf(top, fabsf(p[i]));
  top = wave_max(top);
  float s = top / 127.0f;
  if (!(s > 0.0f)) s = 1.0f;
  s = round_storage(s, dtype);
  int8_t* dst = q + grp * G;
  for (int i = lane; i < G; i += 64)
    dst[i] = static_cast<int8_t>(fminf(fmaxf(rintf(p[i] / s), -127.0f), 127.0f));
  if (lane == 0) scale[grp] = s;
}

// ================================================================ launchers

template <int DT, int FP8>
static void launch_w8_skinny(const void* x, const uint8_t* w, const float* s, void* y, int M,
                             int N, int K, int G, int rb, int cols, hipStream_t stream) {
  const auto* xs = static_cast<const uint16_t*>(x);
  auto* ys = static_cast<uint16_t*>(y);
  if (M == 1 && K == 4096 && G % 128 == 0)
    hipLaunchKernelGGL((w8_row_slices_kernel<DT, FP8>), dim3((N + 15) / 16), dim3(1024), 0, stream, xs, w, s, ys, N, G,
                       rb, cols);
  else if (M == 1 && K <= 32768 && K % 512 == 0 && G % 128 == 0)
    hipLaunchKernelGGL((w8_row_kernel<DT, FP8>), dim3((N + 15) / 16), dim3(256), K * 2, stream, xs, w, s, ys, N, K, G,
                       rb, cols);
  else if (M == 1 && K <= 32768)
    hipLaunchKernelGGL((w8_skinny_kernel<DT, FP8, 1, true>), dim3((N + 15) / 16, 1), dim3(256), K * 2, stream,
                       xs, w, s, ys, M, N, K, G, rb, cols);
  else if (M <= 16)
    hipLaunchKernelGGL((w8_skinny_kernel<DT, FP8, 1>), dim3((N + 15) / 16, 1), dim3(256), 0, stream,
                       xs, w, s, ys, M, N, K, G, rb, cols);
  else if (M <= 32)
    hipLaunchKernelGGL((w8_skinny_kernel<DT, FP8, 2>), dim3((N + 15) / 16, 1), dim3(256), 0, stream,
                       xs, w, s, ys, M, N, K, G, rb, cols);
  else
    hipLaunchKernelGGL((w8_skinny_kernel<DT, FP8, 4>), dim3((N + 15) / 16, (M + 63) / 64), dim3(256),
                       0, stream, xs, w, s, ys, M, N, K, G, rb, cols);
}

}  // namespace lnq

using namespace lnq;

extern "C" {

LNQ_API LnqStatus lnq_int8_quantize(const float* weight, int8_t* q, float* scale,
                                    int64_t out_features, int64_t in_features, int64_t group,
                                    int32_t scale_dtype, void* stream) {
  LNQ_REQUIRE(scale_dtype == LNQ_BF16 || scale_dtype == LNQ_F16 || scale_dtype == LNQ_F32,
              "lnq_int8_quantize: scales are stored as bf16, f16 or f32, not dtype %d", scale_dtype);
  LNQ_REQUIRE(out_features >= 0 && in_features >= 0, "lnq_int8_quantize: bad shape");
  LNQ_REQUIRE(group > 0 && (in_features == 0 || in_features % group == 0) && group <= INT32_MAX,
              "lnq_int8_quantize: groups of %lld must divide the %lld inputs", (long long)group,
              (long long)in_features);
  const int64_t total = out_features * (in_features / group);
  if (total == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(weight && q && scale, "lnq_int8_quantize: null pointer");
  hipLaunchKernelGGL(int8_quantize_kernel, dim3(static_cast<unsigned>((total + 3) / 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), weight, q, scale, total,
                     static_cast<int>(group), scale_dtype);
  return launched("int8_quantize");
}

static const char* check_scales(int64_t N, int64_t K, int64_t group, int64_t row_block) {
  if (group < 0 || row_block <= 0) return "group must be >= 0 and row_block > 0";
  if (group > 0 && (K % group != 0 || N % row_block != 0)) return "scale blocks must tile the weight";
  return nullptr;
}

LNQ_API LnqStatus lnq_w8a16(const void* x, const uint8_t* weight, const float* scale, void* y,
                            int64_t rows, int64_t out_features, int64_t in_features, int32_t fp8,
                            int64_t group, int64_t row_block, int32_t dtype, void* stream) {
  LNQ_REQUIRE(dtype == LNQ_BF16 || dtype == LNQ_F16, "lnq_w8a16: x is bf16 or f16, not dtype %d", dtype);
  LNQ_REQUIRE(rows >= 0 && out_features > 0 && in_features > 0 && in_features % 128 == 0,
              "lnq_w8a16: bad shape rows=%lld out=%lld in=%lld (in %% 128 == 0)", (long long)rows,
              (long long)out_features, (long long)in_features);
  const char* bad = check_scales(out_features, in_features, group, row_block);
  LNQ_REQUIRE(bad == nullptr, "lnq_w8a16: %s", bad ? bad : "");
  LNQ_REQUIRE(group == 0 || group % 64 == 0,
              "lnq_w8a16: the fused kernel takes scales per row or per 64k inputs, not %lld",
              (long long)group);
  LNQ_REQUIRE(rows <= INT32_MAX && out_features <= INT32_MAX && in_features <= INT32_MAX,
              "lnq_w8a16: sizes exceed 2^31");
  LNQ_REQUIRE(x && weight && scale && y, "lnq_w8a16: null pointer");
  LNQ_REQUIRE(aligned(x, 16) && aligned(weight, 16), "lnq_w8a16: x and weight must be 16-byte aligned");
  if (rows == 0) {
    clear_error();
    return LNQ_OK;
  }
  const int M = (int)rows, N = (int)out_features, K = (int)in_features;
  const int G = group == 0 ? K : (int)group;
  const int rb = group == 0 ? 1 : (int)row_block;
  const int cols = group == 0 ? 1 : (int)(in_features / group);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == LNQ_BF16) {
    if (fp8) launch_w8_skinny<LNQ_BF16, 1>(x, weight, scale, y, M, N, K, G, rb, cols, s);
    else launch_w8_skinny<LNQ_BF16, 0>(x, weight, scale, y, M, N, K, G, rb, cols, s);
  } else {
    if (fp8) launch_w8_skinny<LNQ_F16, 1>(x, weight, scale, y, M, N, K, G, rb, cols, s);
    else launch_w8_skinny<LNQ_F16, 0>(x, weight, scale, y, M, N, K, G, rb, cols, s);
  }
  return launched("w8_skinny");
}

LNQ_API LnqStatus lnq_dequantize8(const uint8_t* weight, const float* scale, void* out,
                                  int64_t out_features, int64_t in_features, int32_t fp8,
                                  int64_t group, int64_t row_block, int32_t dtype, void* stream) {
  LNQ_REQUIRE(dtype == LNQ_BF16 || dtype == LNQ_F16 || dtype == LNQ_F32,
              "lnq_dequantize8: output dtype %d is not bf16, f16 or f32", dtype);
  LNQ_REQUIRE(out_features >= 0 && in_features >= 0 && in_features % 16 == 0,
              "lnq_dequantize8: bad shape (in %% 16 == 0)");
  const char* bad = check_scales(out_features, in_features, group, row_block);
  LNQ_REQUIRE(bad == nullptr, "lnq_dequantize8: %s", bad ? bad : "");
  LNQ_REQUIRE(in_features <= INT32_MAX, "lnq_dequantize8: in_features exceeds 2^31");
  if (out_features == 0 || in_features == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(weight && scale && out, "lnq_dequantize8: null pointer");
  LNQ_REQUIRE(aligned(weight, 16), "lnq_dequantize8: weight must be 16-byte aligned");
  const int64_t units = out_features * (in_features / 16);
  const dim3 grid(static_cast<unsigned>((units + 255) / 256));
  const int K = (int)in_features, G = (int)group, rb = (int)row_block;
  const int cols = group == 0 ? 1 : (int)(in_features / group);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define LNQ_DQ8(DT, F)                                                                                  \
  hipLaunchKernelGGL((dequant8_kernel<DT, F>), grid, dim3(256), 0, s, weight, scale,                   \
                     static_cast<typename Elem<DT>::storage*>(out), units, K, G, rb, cols)
  if (dtype == LNQ_BF16) { if (fp8) LNQ_DQ8(LNQ_BF16, 1); else LNQ_DQ8(LNQ_BF16, 0); }
  else if (dtype == LNQ_F16) { if (fp8) LNQ_DQ8(LNQ_F16, 1); else LNQ_DQ8(LNQ_F16, 0); }
  else { if (fp8) LNQ_DQ8(LNQ_F32, 1); else LNQ_DQ8(LNQ_F32, 0); }
#undef LNQ_DQ8
  return launched("dequant8");
}

LNQ_API LnqStatus lnq_rows8(const void* x, uint8_t* q, float* x_scale, int64_t rows,
                            int64_t in_features, int32_t fp8, int32_t dtype, void* stream) {
  LNQ_REQUIRE(dtype == LNQ_BF16 || dtype == LNQ_F16 || dtype == LNQ_F32,
              "lnq_rows8: x dtype %d is not bf16, f16 or f32", dtype);
  LNQ_REQUIRE(rows >= 0 && in_features >= 0 && in_features <= INT32_MAX && rows <= INT32_MAX,
              "lnq_rows8: bad shape");
  if (rows == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(x && q && x_scale, "lnq_rows8: null pointer");
  const dim3 grid(static_cast<unsigned>(rows));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int K = (int)in_features;
  const int esize = dtype == LNQ_F32 ? 4 : 2;
  const bool vec = (K % (16 / esize)) == 0 && aligned(x, 16) && aligned(q, 8) && (static_cast<size_t>(K) * esize) % 16 == 0;
  // Vectors of 16 bytes a thread holds: the row in registers up to 8 of them.
  const int per_thread = vec ? (K / (16 / esize) + 255) / 256 : 0;
  const int keep = per_thread <= 2 ? 2 : per_thread <= 4 ? 4 : per_thread <= 8 ? 8 : 0;
#define LNQ_R8V(DT, F, R) \
  hipLaunchKernelGGL((rows8_vec_kernel<DT, F, R>), grid, dim3(256), 0, s, static_cast<const typename Elem<DT>::storage*>(x), q, x_scale, K)
#define LNQ_R8(DT, F)                                                                              \
  if (vec) {                                                                                       \
    if (keep == 2) LNQ_R8V(DT, F, 2);                                                              \
    else if (keep == 4) LNQ_R8V(DT, F, 4);                                                         \
    else if (keep == 8) LNQ_R8V(DT, F, 8);                                                         \
    else LNQ_R8V(DT, F, 0);                                                                        \
  } else                                                                                           \
    hipLaunchKernelGGL((rows8_kernel<DT, F>), grid, dim3(256), 0, s,                              \
                       static_cast<const typename Elem<DT>::storage*>(x), q, x_scale, K)
  if (dtype == LNQ_BF16) { if (fp8) { LNQ_R8(LNQ_BF16, 1); } else { LNQ_R8(LNQ_BF16, 0); } }
  else if (dtype == LNQ_F16) { if (fp8) { LNQ_R8(LNQ_F16, 1); } else { LNQ_R8(LNQ_F16, 0); } }
  else { if (fp8) { LNQ_R8(LNQ_F32, 1); } else { LNQ_R8(LNQ_F32, 0); } }
#undef LNQ_R8
#undef LNQ_R8V
  return launched("rows8");
}


// The kernel of an 8-bit product: 256-column tiles read half the bytes per
// FLOP of 128-column ones, but only pay while they still give every compute
// unit a tile; there, FP8 takes the persistent form where it applies (config 4
// at 4096 rows: 2468 against 2173 TFLOP/s for the 256-column tiles; int8 stays
// on the tiles: 2231 against 2177). Below that, 128-column tiles; FP8 past 128
// rows in the weight-streaming form (config 4 at 256 rows: 70.5 against 73.2
// us for the 128-column tile kernel; at 16 or 64 rows it is slower, and int8
// gains nothing at 256).
static int mm8_kernel_for(int M, int N, int K, bool fp8) {
  const long tiles256 = static_cast<long>((M + mm8::BM - 1) / mm8::BM) * ((N + 255) / 256);
  if (tiles256 < compute_units()) return fp8 && M > 128 ? LNQ_MM8_STREAM : 128;
  return fp8 && N % 256 == 0 && K % 256 == 0 ? LNQ_MM8_PERSISTENT : 256;
}

LNQ_API LnqStatus lnq_mm8_tiles(const uint8_t* qx, const uint8_t* weight, const float* x_scale,
                                const float* scale, void* y, int64_t rows, int64_t out_features,
                                int64_t in_features, int32_t fp8, int32_t dtype, int32_t tile_n,
                                void* stream) {
  LNQ_REQUIRE(dtype == LNQ_BF16 || dtype == LNQ_F16, "lnq_mm8: output is bf16 or f16, not dtype %d", dtype);
  LNQ_REQUIRE(rows >= 0 && out_features > 0 && in_features > 0 && in_features % 128 == 0,
              "lnq_mm8: bad shape rows=%lld out=%lld in=%lld (in %% 128 == 0)", (long long)rows,
              (long long)out_features, (long long)in_features);
  LNQ_REQUIRE(rows <= INT32_MAX && out_features <= INT32_MAX && in_features <= INT32_MAX,
              "lnq_mm8: sizes exceed 2^31");
  LNQ_REQUIRE(tile_n == 0 || tile_n == LNQ_MM8_PERSISTENT || tile_n == LNQ_MM8_STREAM || tile_n == 128 ||
                  tile_n == 256,
              "lnq_mm8: tile_n is 0, 1 (persistent), 2 (streaming), 128 or 256, not %d", tile_n);
  LNQ_REQUIRE(tile_n != LNQ_MM8_PERSISTENT || (out_features % 256 == 0 && in_features % 256 == 0),
              "lnq_mm8: the persistent form takes out %% 256 == 0 and in %% 256 == 0, got out=%lld in=%lld",
              (long long)out_features, (long long)in_features);
  LNQ_REQUIRE(qx && weight && x_scale && scale && y, "lnq_mm8: null pointer");
  LNQ_REQUIRE(aligned(qx, 16) && aligned(weight, 16), "lnq_mm8: operands must be 16-byte aligned");
  if (rows == 0) {
    clear_error();
    return LNQ_OK;
  }
  const int M = (int)rows, N = (int)out_features, K = (int)in_features;
  LNQ_REQUIRE(static_cast<size_t>(M) * K < (1ull << 31) && static_cast<size_t>(N) * K < (1ull << 31),
              "lnq_mm8: operands exceed the 2 GiB buffer range");
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto* ys = static_cast<uint16_t*>(y);
  const int bn = tile_n == 0 ? mm8_kernel_for(M, N, K, fp8 != 0) : tile_n;
  if (bn == LNQ_MM8_PERSISTENT) {
    const int tiles = ((M + mm8p::BM - 1) / mm8p::BM) * (N / mm8p::BN);
    const dim3 grid(tiles < compute_units() ? tiles : compute_units());
#define LNQ_MM8P(DT, F) \
  hipLaunchKernelGGL((mm8p_kernel<DT, F>), grid, dim3(mm8p::THREADS), 0, s, qx, weight, x_scale, scale, ys, M, N, K)
    if (dtype == LNQ_BF16) { if (fp8) { LNQ_MM8P(LNQ_BF16, 1); } else { LNQ_MM8P(LNQ_BF16, 0); } }
    else { if (fp8) { LNQ_MM8P(LNQ_F16, 1); } else { LNQ_MM8P(LNQ_F16, 0); } }
#undef LNQ_MM8P
    return launched("mm8p");
  }
  if (bn == LNQ_MM8_STREAM) {
    const dim3 grid(((M + mm8w::BM - 1) / mm8w::BM) * ((N + mm8w::BN - 1) / mm8w::BN));
#define LNQ_MM8W(DT, F)                                                                                        \
  hipLaunchKernelGGL((mm8w_kernel<DT, F, 3, 4>), grid, dim3(mm8w::THREADS), 0, s, qx, weight, x_scale, scale, \
                     ys, M, N, K)
    if (dtype == LNQ_BF16) { if (fp8) { LNQ_MM8W(LNQ_BF16, 1); } else { LNQ_MM8W(LNQ_BF16, 0); } }
    else { if (fp8) { LNQ_MM8W(LNQ_F16, 1); } else { LNQ_MM8W(LNQ_F16, 0); } }
#undef LNQ_MM8W
    return launched("mm8w");
  }
  const bool wide = bn == 256;
  const int tiles = ((M + mm8::BM - 1) / mm8::BM) * ((N + bn - 1) / bn);
#define LNQ_MM8(DT, F, BN)                                                                          \
  hipLaunchKernelGGL((mm8_kernel<DT, F, BN>), dim3(tiles), dim3(mm8::THREADS), 0, s, qx, weight,   \
                     x_scale, scale, ys, M, N, K, 0)
#define LNQ_MM8_BN(DT, F) \
  if (wide) LNQ_MM8(DT, F, 256); else LNQ_MM8(DT, F, 128)
  if (dtype == LNQ_BF16) { if (fp8) { LNQ_MM8_BN(LNQ_BF16, 1); } else { LNQ_MM8_BN(LNQ_BF16, 0); } }
  else { if (fp8) { LNQ_MM8_BN(LNQ_F16, 1); } else { LNQ_MM8_BN(LNQ_F16, 0); } }
#undef LNQ_MM8_BN
#undef LNQ_MM8
  return launched("mm8");
}

LNQ_API LnqStatus lnq_mm8(const uint8_t* qx, const uint8_t* weight, const float* x_scale,
                          const float* scale, void* y, int64_t rows, int64_t out_features,
                          int64_t in_features, int32_t fp8, int32_t dtype, void* stream) {
  return lnq_mm8_tiles(qx, weight, x_scale, scale, y, rows, out_features, in_features, fp8, dtype, 0, stream);
}

LNQ_API LnqStatus lnq_mm8_plan(int64_t rows, int64_t out_features, int64_t in_features, int32_t fp8,
                               int32_t* tile_n) {
  LNQ_REQUIRE(tile_n != nullptr, "lnq_mm8_plan: null pointer");
  LNQ_REQUIRE(rows >= 0 && rows <= INT32_MAX && out_features > 0 && out_features <= INT32_MAX &&
                  in_features > 0 && in_features % 128 == 0,
              "lnq_mm8_plan: bad shape rows=%lld out=%lld in=%lld", (long long)rows, (long long)out_features,
              (long long)in_features);
  *tile_n = mm8_kernel_for(static_cast<int>(rows), static_cast<int>(out_features), static_cast<int>(in_features),
                           fp8 != 0);
  clear_error();
  return LNQ_OK;
}

}  // extern "C"
