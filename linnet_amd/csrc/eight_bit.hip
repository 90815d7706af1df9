// 8-bit weights (std.quant::Int8Linear / Int8GroupLinear / Fp8Linear / Fp8BlockLinear)
// on gfx950:
//   - w8_skinny:  weight-only product for few rows (gemv8 / w8a16), weights
//                 widened in registers and multiplied on MFMA, x unrounded;
//   - dequant8:   the weight widened and scaled, rounded to the output dtype;
//   - rows8:      dynamic per-token FP8 / int8 rounding of activations;
//   - mm8:        int8 x int8 (int32 sums) or FP8 x FP8 (f32 sums) tiled MFMA GEMM
//                 with the row-scale epilogue;
//   - int8_quantize: symmetric group-wise int8 rounding, bit-exact with numpy.
#include "common.hpp"

#include <type_traits>

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
// epilogue's -128 * sum(x); FP8: the value itself.
template <int DT, int FP8>
__device__ inline void widen4(uint32_t w, uint32_t& d0, uint32_t& d1) {
  float f[4];
  if constexpr (FP8) {
    fp8x4_to_f32(w, f);
  } else {
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
// 16-byte aligned rows): a pass for max|x|, then a pass that quantizes from a
// second read of the row (an L2 hit). Same arithmetic as rows8_kernel.
template <int DT, int FP8>
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
  float top = 0.0f;
  for (int i = VEC * threadIdx.x; i < K; i += VEC * 256) {
    float v[VEC];
    load(i, v);
#pragma unroll
    for (int j = 0; j < VEC; ++j) top = fmaxf(top, fabsf(v[j]));
  }
  top = wave_max(top);
  if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = top;
  __syncthreads();
  top = fmaxf(fmaxf(partial[0], partial[1]), fmaxf(partial[2], partial[3]));
  const float largest = FP8 ? 448.0f : 127.0f;
  const float s = fmaxf(top, 1e-12f) / largest;
  uint8_t* dst = q + row * K;
  for (int i = VEC * threadIdx.x; i < K; i += VEC * 256) {
    float v[VEC];
    load(i, v);
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
  }
  if (threadIdx.x == 0) x_scale[row] = s;
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

template <int DT, int FP8, int BN>
__global__ __launch_bounds__(mm8::THREADS, 1) void mm8_kernel(
    const uint8_t* __restrict__ qx, const uint8_t* __restrict__ weight,
    const float* __restrict__ x_scale, const float* __restrict__ scale,
    uint16_t* __restrict__ y, int M, int N, int K) {
  using namespace mm8;
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
  LNQ_MFMA_IN_AGPRS();

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
  auto region = [&](int cur, const uint8_t* as, const uint8_t* bs, int nkk, auto&& vm) {
#pragma unroll
    for (int s = 0; s < NMF; ++s) {
      acc[s / FB][s % FB] = mma(bf[cur][s % FB], af[cur][s / FB], acc[s / FB][s % FB]);
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
#pragma unroll
    for (int kk = 0; kk + 1 < KK; ++kk)
      region(kk & 1, ac, bc, kk + 1, [&](int s) { vm(kk, s); });
    if constexpr (S == 2) __asm__ volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)" ::: "memory");
    else __asm__ volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)" ::"n"((S - 2) * LPW) : "memory");
    __builtin_amdgcn_s_barrier();
    region((KK - 1) & 1, an, bn, 0, [&](int) {});
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
  if (M == 1 && K <= 32768)
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
#define LNQ_R8(DT, F)                                                                              \
  if (vec)                                                                                         \
    hipLaunchKernelGGL((rows8_vec_kernel<DT, F>), grid, dim3(256), 0, s,                          \
                       static_cast<const typename Elem<DT>::storage*>(x), q, x_scale, K);          \
  else                                                                                             \
    hipLaunchKernelGGL((rows8_kernel<DT, F>), grid, dim3(256), 0, s,                              \
                       static_cast<const typename Elem<DT>::storage*>(x), q, x_scale, K)
  if (dtype == LNQ_BF16) { if (fp8) { LNQ_R8(LNQ_BF16, 1); } else { LNQ_R8(LNQ_BF16, 0); } }
  else if (dtype == LNQ_F16) { if (fp8) { LNQ_R8(LNQ_F16, 1); } else { LNQ_R8(LNQ_F16, 0); } }
  else { if (fp8) { LNQ_R8(LNQ_F32, 1); } else { LNQ_R8(LNQ_F32, 0); } }
#undef LNQ_R8
  return launched("rows8");
}

LNQ_API LnqStatus lnq_mm8(const uint8_t* qx, const uint8_t* weight, const float* x_scale,
                          const float* scale, void* y, int64_t rows, int64_t out_features,
                          int64_t in_features, int32_t fp8, int32_t dtype, void* stream) {
  LNQ_REQUIRE(dtype == LNQ_BF16 || dtype == LNQ_F16, "lnq_mm8: output is bf16 or f16, not dtype %d", dtype);
  LNQ_REQUIRE(rows >= 0 && out_features > 0 && in_features > 0 && in_features % 128 == 0,
              "lnq_mm8: bad shape rows=%lld out=%lld in=%lld (in %% 128 == 0)", (long long)rows,
              (long long)out_features, (long long)in_features);
  LNQ_REQUIRE(rows <= INT32_MAX && out_features <= INT32_MAX && in_features <= INT32_MAX,
              "lnq_mm8: sizes exceed 2^31");
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
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) cus = v;
  }
  // 256-column tiles read half the bytes per FLOP of 128-column ones, but only
  // pay while they still give every compute unit a tile.
  const long tiles256 = static_cast<long>((M + mm8::BM - 1) / mm8::BM) * ((N + 255) / 256);
  const bool wide = tiles256 >= cus;
  const int bn = wide ? 256 : 128;
  const int tiles = ((M + mm8::BM - 1) / mm8::BM) * ((N + bn - 1) / bn);
#define LNQ_MM8(DT, F, BN)                                                                          \
  hipLaunchKernelGGL((mm8_kernel<DT, F, BN>), dim3(tiles), dim3(mm8::THREADS), 0, s, qx, weight,   \
                     x_scale, scale, ys, M, N, K)
#define LNQ_MM8_BN(DT, F) \
  if (wide) LNQ_MM8(DT, F, 256); else LNQ_MM8(DT, F, 128)
  if (dtype == LNQ_BF16) { if (fp8) { LNQ_MM8_BN(LNQ_BF16, 1); } else { LNQ_MM8_BN(LNQ_BF16, 0); } }
  else { if (fp8) { LNQ_MM8_BN(LNQ_F16, 1); } else { LNQ_MM8_BN(LNQ_F16, 0); } }
#undef LNQ_MM8_BN
#undef LNQ_MM8
  return launched("mm8");
}

}  // extern "C"
