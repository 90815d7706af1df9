// NF4 linear layers (std.quant::Nf4Linear, stdlib/quant.linnet:177-215): QLoRA's
// 4-bit NormalFloat codes, two a byte with the first input in the low nibble,
// weight [Out, In / 2] bytes and one f32 scale (the block's absmax) for each
// `block` consecutive inputs of a row, absmax [Out, In / block]:
//     weight[o, i] = nf4(q[o, i]) * absmax[o, i / block].
//
// Three kernels:
// - nf4_dequant_kernel: the weight in T, the f32 product of the code's value and
//   the scale rounded once (`dequantize_nf4`, quant.linnet:180-187), bit for bit.
// - nf4_gemv_kernel: y = x W^T (+ bias) for up to 8 rows of x, the weight read
//   once from HBM as it is stored. NF4's values are no affine function of the
//   code, so the widening is a table lookup done in registers: the 16 values'
//   16-bit patterns (bf16 or f16, x's type) are held as two 16-byte planes (low
//   bytes, high bytes) in 8 SGPRs, and v_perm_b32 selects four codes' bytes from
//   a plane at once (two perms over the 8-entry halves, v_bfi_b32 on the code's
//   bit 3, itself spread to a byte mask by a v_perm_b32). Each pair of values meets a pair of x in one v_dot2_f32_{bf16,f16};
//   a block's sum is scaled by its absmax and added in f32. The values are
//   rounded to x's type once (as the reference's body rounds the scaled weight
//   to T before its product), so the result is within T's rounding of the
//   exact product, not bit-identical to it.
// - nf4_repack_kernel: a bitsandbytes 4-bit layer as Nf4Linear holds it (the
//   reference's `_bnb_nf4`, python/linnet/src/linnet/quant.py:414-466): bytes
//   with their nibbles swapped (bitsandbytes keeps the first code of a pair in
//   the high nibble) and, for double quantization, each block's absmax decoded
//   from its 8-bit code, nested_map[code] * nested_absmax[i / nested_block] +
//   offset, in f32 with two roundings as the reference computes it.
//
// GEMV layout: one workgroup of 256 lanes per ROWS consecutive output rows. The
// inputs are cut in units of 16 (8 bytes of codes a row); lane t owns units
// t, t + 256, ... (SLOTS of them), so its x stays in registers across the rows,
// a wave's weight loads read 512 consecutive bytes of a row, and a row's 8 KB
// (In = 16384) or less is spread over the whole workgroup. Each lane's partial
// sums (ROWS x rows of x) go through LDS, [output][lane] with the lanes
// contiguous, and 256 / (ROWS * MR) lanes add each output's 256 partial sums in
// a fixed order.
#include "common.hpp"

namespace lnq {

namespace nf4 {
// The 16 values by code, as bitsandbytes' NF4 map stores them (the reference's
// NF4 table, quant.py:374-394, and std.dtypes::nf4).
constexpr float VALUES[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.2461123019456863f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f,
};
constexpr int UNIT = 16;       // inputs of a lane's unit
constexpr int THREADS = 256;   // lanes of a GEMV workgroup
constexpr int MAX_SLOTS = 8;   // In <= 16 * 256 * 8 = 32768 for the GEMV
constexpr int MAX_ROWS_X = 8;  // rows of x a GEMV launch takes (In <= 8192; 4 past that)
}  // namespace nf4

__constant__ float kNf4Values[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.2461123019456863f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f,
};

// The values' 16-bit patterns in x's type as byte planes: byte c of lo[] (c = 4
// * dword + byte) is the low byte of value c, hi[] the high bytes.
struct Nf4Planes {
  uint32_t lo[4];
  uint32_t hi[4];
};

// ---------------------------------------------------------------- dequantize
// Thread i widens UNIT_BYTES bytes (2 * UNIT_BYTES inputs) of the weight,
// bytes [UNIT_BYTES * i, ...) of the [Out, In / 2] array.
template <int DT, int UNIT_BYTES>
__global__ __launch_bounds__(256) void nf4_dequant_kernel(const uint8_t* __restrict__ codes,
                                                          const float* __restrict__ absmax,
                                                          typename Elem<DT>::storage* __restrict__ out,
                                                          int64_t units, int64_t row_bytes, int block,
                                                          int blocks_per_row) {
  using E = Elem<DT>;
  __shared__ float table[16];
  if (threadIdx.x < 16) table[threadIdx.x] = kNf4Values[threadIdx.x];
  __syncthreads();
  const int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (u >= units) return;
  const int64_t byte0 = u * UNIT_BYTES;
  const int64_t row = byte0 / row_bytes;
  const int64_t col_byte = byte0 - row * row_bytes;
  const float* scales = absmax + row * blocks_per_row;
  uint8_t b[UNIT_BYTES];
  if constexpr (UNIT_BYTES == 8) {
    const u32x2 v = *reinterpret_cast<const u32x2*>(codes + byte0);
#pragma unroll
    for (int j = 0; j < 8; ++j) b[j] = static_cast<uint8_t>((j < 4 ? v.x : v.y) >> (8 * (j & 3)));
  } else {
    b[0] = codes[byte0];
  }
  typename E::storage w[2 * UNIT_BYTES];
#pragma unroll
  for (int j = 0; j < UNIT_BYTES; ++j) {
    // The two inputs of a byte lie in one block (block is even).
    const int k = static_cast<int>(2 * (col_byte + j));
    const float s = scales[k / block];
    w[2 * j] = E::from_f32(table[b[j] & 15] * s);
    w[2 * j + 1] = E::from_f32(table[b[j] >> 4] * s);
  }
  typename E::storage* dst = out + 2 * byte0;
#pragma unroll
  for (int j = 0; j < 2 * UNIT_BYTES; ++j) dst[j] = w[j];
}

// ---------------------------------------------------------------------- GEMV
// Values of the eight codes of w (nibble j is input j of the 8) as four pairs
// of 16-bit patterns, the first of each pair in the low half: v[0] = (0, 2),
// v[1] = (4, 6), v[2] = (1, 3), v[3] = (5, 7). For the four codes of one nibble
// position (low nibbles, then high), v_perm_b32 looks up their low and high
// bytes in the 8-entry halves of the planes (selector = code & 7), and v_bfi_b32
// keeps the upper half's bytes where the code's bit 3 is set. That mask comes
// from one more v_perm_b32: its selectors 8..11 replicate bit 15, 31, 47 or 63
// of the 8-byte source, and shifts of w put bit 3 of the four codes there
// (selector dword 0x090B080A: byte 0 <- bit 47, 1 <- 15, 2 <- 63, 3 <- 31).
__device__ inline void nf4_lookup8(uint32_t w, const Nf4Planes& p, uint32_t v[4]) {
  const uint32_t upper_lo = __builtin_amdgcn_perm(w << 12, w << 4, 0x090B080Au);  // bits 3, 11, 19, 27
  const uint32_t upper_hi = __builtin_amdgcn_perm(w << 8, w, 0x090B080Au);        // bits 7, 15, 23, 31
  const uint32_t sel[2] = {w & 0x07070707u, (w >> 4) & 0x07070707u};
  const uint32_t upper[2] = {upper_lo, upper_hi};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t lo = (upper[h] & __builtin_amdgcn_perm(p.lo[3], p.lo[2], sel[h])) |
                        (~upper[h] & __builtin_amdgcn_perm(p.lo[1], p.lo[0], sel[h]));
    const uint32_t hi = (upper[h] & __builtin_amdgcn_perm(p.hi[3], p.hi[2], sel[h])) |
                        (~upper[h] & __builtin_amdgcn_perm(p.hi[1], p.hi[0], sel[h]));
    v[2 * h] = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
    v[2 * h + 1] = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
  }
}

template <int DT>
__device__ inline float nf4_dot2(uint32_t w, uint32_t x, float c) {
  if constexpr (DT == LNQ_BF16) {
    typedef __bf16 v2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, w), __builtin_bit_cast(v2, x), c, false);
  } else {
    typedef _Float16 v2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, w), __builtin_bit_cast(v2, x), c, false);
  }
}

// Output rows a GEMV workgroup takes: 8 at one unit slot (In <= 4096), about 16
// units of codes in flight a lane past it, and 4..32 partial sums a lane
// (ROWS * MR) for the reduction's lane groups. 4096 -> 14336 at one row of x:
// 8 rows 11.6 us, 16 rows 12.0, 32 rows 12.9; at 14336 -> 4096, 2 rows of x, 16
// units in flight 13.4 us against 15.8 with 8.
constexpr int nf4_rows(int mr, int slots) {
  int r = slots == 1 ? 8 : 16 / slots;
  if (r > 32 / mr) r = 32 / mr;
  if (r < 4 / mr) r = 4 / mr;
  return r < 1 ? 1 : r;
}

template <int DT, int MR, int SLOTS>
__global__ __launch_bounds__(nf4::THREADS) void nf4_gemv_kernel(const uint16_t* __restrict__ x, int64_t x_stride,
                                                                int rows, const uint8_t* __restrict__ codes,
                                                                const float* __restrict__ absmax,
                                                                const uint16_t* __restrict__ bias,
                                                                uint16_t* __restrict__ y, int64_t y_stride,
                                                                int out_features, int in_features, int block,
                                                                Nf4Planes planes) {
  using E = Elem<DT>;
  constexpr int ROWS = nf4_rows(MR, SLOTS);
  constexpr int OUTS = ROWS * MR;
  constexpr int PAD = nf4::THREADS + 16;
  __shared__ float red[OUTS * PAD];
  const int t = threadIdx.x;
  const int n0 = blockIdx.x * ROWS;
  const int units = in_features / nf4::UNIT;
  const int row_bytes = in_features / 2;
  const int blocks_per_row = in_features / block;
  // Range-checked descriptors: x's rows past `rows`, units past In and weight
  // rows past Out read zeros.
  const __amdgpu_buffer_rsrc_t rx =
      buffer_rsrc(x, static_cast<uint32_t>(((rows - 1) * x_stride + in_features) * 2));
  const __amdgpu_buffer_rsrc_t rq = buffer_rsrc(codes, static_cast<uint32_t>(int64_t{out_features} * row_bytes));
  const __amdgpu_buffer_rsrc_t ra =
      buffer_rsrc(absmax, static_cast<uint32_t>(int64_t{out_features} * blocks_per_row * 4));
  constexpr uint32_t OUTSIDE = 0x80000000u;

  // x of this lane's units, as pairs (k, k + 2) in the order the lookups give the
  // weights: per 8 inputs (k0 k2) (k4 k6) (k1 k3) (k5 k7).
  uint32_t xv[MR][SLOTS][8];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
      const int g = t + nf4::THREADS * s;
      const uint32_t off = m < rows && g < units ? static_cast<uint32_t>((m * x_stride + g * nf4::UNIT) * 2) : OUTSIDE;
      const u32x4 d0 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
      const u32x4 d1 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 16, 0));
      const u32x4 h[2] = {d0, d1};
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        xv[m][s][4 * e + 0] = __builtin_amdgcn_perm(h[e].y, h[e].x, 0x05040100u);
        xv[m][s][4 * e + 1] = __builtin_amdgcn_perm(h[e].w, h[e].z, 0x05040100u);
        xv[m][s][4 * e + 2] = __builtin_amdgcn_perm(h[e].y, h[e].x, 0x07060302u);
        xv[m][s][4 * e + 3] = __builtin_amdgcn_perm(h[e].w, h[e].z, 0x07060302u);
      }
    }
  // Scales, then the codes: every load of the wave is issued before any is used
  // (the scheduling barrier below keeps the compiler from trading loads in
  // flight for registers).
  int blk[SLOTS];
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) blk[s] = ((t + nf4::THREADS * s) * nf4::UNIT) / block;
  float sc[ROWS][SLOTS];
  u32x2 q[ROWS][SLOTS];
#pragma unroll
  for (int i = 0; i < ROWS; ++i)
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
      const int g = t + nf4::THREADS * s;
      const int n = n0 + i;
      const bool in = n < out_features && g < units;
      const uint32_t aoff = in ? static_cast<uint32_t>((n * blocks_per_row + blk[s]) * 4) : OUTSIDE;
      sc[i][s] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ra, aoff, 0, 0));
    }
#pragma unroll
  for (int i = 0; i < ROWS; ++i)
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
      const int g = t + nf4::THREADS * s;
      const int n = n0 + i;
      const bool in = n < out_features && g < units;
      const uint32_t qoff = in ? static_cast<uint32_t>(n * row_bytes + g * 8) : OUTSIDE;
      // Plain (temporal) loads: 11.0 us against 11.6 with the non-temporal hint at
      // 4096 -> 14336, one row (the int4 GEMV's LDS-DMA weight loads measure the
      // other way round).
      q[i][s] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rq, qoff, 0, 0));
    }
  __builtin_amdgcn_sched_barrier(0);

  float acc[ROWS][MR];
#pragma unroll
  for (int i = 0; i < ROWS; ++i) {
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[i][m] = 0.0f;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
      uint32_t wv[8];
#pragma unroll
      for (int e = 0; e < 2; ++e) nf4_lookup8(e == 0 ? q[i][s].x : q[i][s].y, planes, wv + 4 * e);
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        float part = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) part = nf4_dot2<DT>(wv[j], xv[m][s][j], part);
        acc[i][m] += part * sc[i][s];
      }
    }
  }

  // Partial sums [output][lane]; S lanes add an output's 256 values.
#pragma unroll
  for (int i = 0; i < ROWS; ++i)
#pragma unroll
    for (int m = 0; m < MR; ++m) red[(i * MR + m) * PAD + t] = acc[i][m];
  __syncthreads();
  constexpr int S = nf4::THREADS / OUTS;  // 8..64, within a wave
  const int o = t / S, j = t % S;
  float v = 0.0f;
#pragma unroll
  for (int r = 0; r < nf4::THREADS / S; ++r) v += red[o * PAD + j + S * r];
#pragma unroll
  for (int off = S / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  const int i = o / MR, m = o % MR;
  const int n = n0 + i;
  if (j == 0 && n < out_features && m < rows) {
    if (bias) v += E::to_f32(bias[n]);
    y[m * y_stride + n] = E::from_f32(v);
  }
}

// -------------------------------------------------------------------- repack
// Thread i swaps the nibbles of bytes [4i, 4i + 4) and decodes scale i.
__global__ __launch_bounds__(256) void nf4_repack_kernel(const uint8_t* __restrict__ packed, uint8_t* __restrict__ swapped,
                                                         int64_t bytes, const void* __restrict__ absmax_in,
                                                         const float* __restrict__ nested_absmax,
                                                         const float* __restrict__ nested_map, int64_t nested_block,
                                                         float offset, float* __restrict__ absmax, int64_t scales) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (4 * i + 3 < bytes) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(packed + 4 * i);
    *reinterpret_cast<uint32_t*>(swapped + 4 * i) = ((w >> 4) & 0x0f0f0f0fu) | ((w << 4) & 0xf0f0f0f0u);
  } else {
    for (int64_t b = 4 * i; b < bytes; ++b) {
      const uint32_t w = packed[b];
      swapped[b] = static_cast<uint8_t>((w >> 4) | ((w << 4) & 0xf0u));
    }
  }
  if (i < scales) {
    if (nested_map) {
      const uint8_t code = static_cast<const uint8_t*>(absmax_in)[i];
      absmax[i] = __fadd_rn(__fmul_rn(nested_map[code], nested_absmax[i / nested_block]), offset);
    } else {
      absmax[i] = static_cast<const float*>(absmax_in)[i];
    }
  }
}

namespace {

uint32_t bf16_pattern(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;  // round to nearest even (finite values)
}

Nf4Planes planes_for(int dtype) {
  Nf4Planes p{};
  for (int c = 0; c < 16; ++c) {
    const uint32_t bits = dtype == LNQ_BF16 ? bf16_pattern(nf4::VALUES[c])
                                            : __builtin_bit_cast(uint16_t, static_cast<_Float16>(nf4::VALUES[c]));
    p.lo[c / 4] |= (bits & 0xffu) << (8 * (c % 4));
    p.hi[c / 4] |= (bits >> 8) << (8 * (c % 4));
  }
  return p;
}

}  // namespace

}  // namespace lnq

using namespace lnq;

extern "C" {

LNQ_API LnqStatus lnq_nf4_dequant(const uint8_t* codes, const float* absmax, void* out, int64_t out_features,
                                  int64_t in_features, int64_t block, int32_t dtype, void* stream) {
  LNQ_REQUIRE(dtype == LNQ_BF16 || dtype == LNQ_F16 || dtype == LNQ_F32,
              "lnq_nf4_dequant: the weight is bf16, f16 or f32, not dtype %d", dtype);
  LNQ_REQUIRE(out_features >= 0 && in_features >= 0, "lnq_nf4_dequant: negative size");
  LNQ_REQUIRE(block > 0 && block % 2 == 0 && in_features % block == 0,
              "lnq_nf4_dequant: %lld inputs do not make blocks of %lld (an even block)",
              static_cast<long long>(in_features), static_cast<long long>(block));
  if (out_features == 0 || in_features == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(codes && absmax && out, "lnq_nf4_dequant: null pointer");
  const int64_t row_bytes = in_features / 2;
  const int64_t bytes = out_features * row_bytes;
  // 8 bytes a thread when a row's bytes split that way and the buffers allow it.
  const bool wide = row_bytes % 8 == 0 && aligned(codes, 8) && aligned(out, 16);
  const int64_t units = wide ? bytes / 8 : bytes;
  const int64_t grid = (units + 255) / 256;
  LNQ_REQUIRE(grid <= INT32_MAX && in_features / block <= INT32_MAX && block <= INT32_MAX,
              "lnq_nf4_dequant: too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int b = static_cast<int>(block), bpr = static_cast<int>(in_features / block);
#define LNQ_NF4_DQ(DT, U)                                                                                     \
  hipLaunchKernelGGL((nf4_dequant_kernel<DT, U>), dim3(static_cast<unsigned>(grid)), dim3(256), 0, s, codes, \
                     absmax, static_cast<typename Elem<DT>::storage*>(out), units, row_bytes, b, bpr)
#define LNQ_NF4_DQ_U(DT) \
  if (wide) {            \
    LNQ_NF4_DQ(DT, 8);   \
  } else {               \
    LNQ_NF4_DQ(DT, 1);   \
  }
  if (dtype == LNQ_BF16) {
    LNQ_NF4_DQ_U(LNQ_BF16)
  } else if (dtype == LNQ_F16) {
    LNQ_NF4_DQ_U(LNQ_F16)
  } else {
    LNQ_NF4_DQ_U(LNQ_F32)
  }
#undef LNQ_NF4_DQ_U
#undef LNQ_NF4_DQ
  return launched("nf4_dequant");
}

LNQ_API LnqStatus lnq_nf4_linear(const void* x, int64_t x_stride, int64_t rows, const uint8_t* codes,
                                 const float* absmax, const void* bias, void* y, int64_t y_stride,
                                 int64_t out_features, int64_t in_features, int64_t block, int32_t dtype,
                                 void* stream) {
  LNQ_REQUIRE(dtype == LNQ_BF16 || dtype == LNQ_F16, "lnq_nf4_linear: x is bf16 or f16, not dtype %d", dtype);
  LNQ_REQUIRE(rows >= 0 && out_features >= 0 && in_features >= 0, "lnq_nf4_linear: negative size");
  LNQ_REQUIRE(block > 0 && block % nf4::UNIT == 0 && in_features % block == 0,
              "lnq_nf4_linear: %lld inputs in blocks of %lld (the product takes blocks of a multiple of 16)",
              static_cast<long long>(in_features), static_cast<long long>(block));
  LNQ_REQUIRE(in_features <= nf4::UNIT * nf4::THREADS * nf4::MAX_SLOTS,
              "lnq_nf4_linear: in %lld is past the product's %d", static_cast<long long>(in_features),
              nf4::UNIT * nf4::THREADS * nf4::MAX_SLOTS);
  LNQ_REQUIRE(out_features * (in_features / 2) < (int64_t{1} << 31) && out_features <= INT32_MAX,
              "lnq_nf4_linear: a weight past 2 GiB");
  if (rows == 0 || out_features == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(in_features > 0, "lnq_nf4_linear: in_features is 0");
  LNQ_REQUIRE(x && codes && absmax && y, "lnq_nf4_linear: null pointer");
  LNQ_REQUIRE(x_stride >= in_features && y_stride >= out_features,
              "lnq_nf4_linear: row strides shorter than a row");
  LNQ_REQUIRE(aligned(x, 16) && x_stride % 8 == 0 && aligned(codes, 8),
              "lnq_nf4_linear: x (with its row stride) must be 16-byte aligned and the codes 8-byte aligned");
  const int units = static_cast<int>(in_features / nf4::UNIT);
  const int need = (units + nf4::THREADS - 1) / nf4::THREADS;
  const int slots = need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : 8;
  const Nf4Planes planes = planes_for(dtype);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int O = static_cast<int>(out_features), K = static_cast<int>(in_features), B = static_cast<int>(block);
  // Up to 8 rows of x a launch (4 past In = 8192); more rows take more launches
  // over the same weight.
  // x's registers grow with rows x slots: 8 rows a pass up to 2 slots, else 4.
  const int per_pass = slots <= 2 ? nf4::MAX_ROWS_X : 4;
  for (int64_t r0 = 0; r0 < rows; r0 += per_pass) {
    const int part = static_cast<int>(rows - r0 < per_pass ? rows - r0 : per_pass);
    const int mr = part == 1 ? 1 : part == 2 ? 2 : part <= 4 ? 4 : 8;
    LNQ_REQUIRE((part - 1) * x_stride + in_features < (int64_t{1} << 30), "lnq_nf4_linear: x past 1 GiB");
    const auto* xs = static_cast<const uint16_t*>(x) + r0 * x_stride;
    auto* ys = static_cast<uint16_t*>(y) + r0 * y_stride;
    const auto* bs = static_cast<const uint16_t*>(bias);
#define LNQ_NF4_GO(DT, M, SL)                                                                                     \
  do {                                                                                                            \
    constexpr int R = nf4_rows(M, SL);                                                                            \
    hipLaunchKernelGGL((nf4_gemv_kernel<DT, M, SL>), dim3(static_cast<unsigned>((O + R - 1) / R)),             \
                       dim3(nf4::THREADS), 0, s, xs, x_stride, part, codes, absmax, bs, ys, y_stride, O, K, B,  \
                       planes);                                                                                   \
  } while (0)
#define LNQ_NF4_SL(DT, M)             \
  switch (slots) {                    \
    case 1: LNQ_NF4_GO(DT, M, 1); break; \
    case 2: LNQ_NF4_GO(DT, M, 2); break; \
    case 4: LNQ_NF4_GO(DT, M, 4); break; \
    default: LNQ_NF4_GO(DT, M, 8); break; \
  }
#define LNQ_NF4_SL8(DT)                 \
  switch (slots) {                      \
    case 1: LNQ_NF4_GO(DT, 8, 1); break; \
    default: LNQ_NF4_GO(DT, 8, 2); break; \
  }
#define LNQ_NF4_MR(DT)                  \
  switch (mr) {                         \
    case 1: LNQ_NF4_SL(DT, 1); break;   \
    case 2: LNQ_NF4_SL(DT, 2); break;   \
    case 4: LNQ_NF4_SL(DT, 4); break;   \
    default: LNQ_NF4_SL8(DT); break;    \
  }
    if (dtype == LNQ_BF16) {
      LNQ_NF4_MR(LNQ_BF16)
    } else {
      LNQ_NF4_MR(LNQ_F16)
    }
#undef LNQ_NF4_MR
#undef LNQ_NF4_SL8
#undef LNQ_NF4_SL
#undef LNQ_NF4_GO
    const LnqStatus st = launched("nf4_gemv");
    if (st != LNQ_OK) return st;
  }
  return LNQ_OK;
}

LNQ_API LnqStatus lnq_nf4_repack(const uint8_t* packed, const void* absmax_in, const float* nested_absmax,
                                 const float* nested_map, int64_t nested_block, float offset, uint8_t* codes,
                                 float* absmax, int64_t out_features, int64_t in_features, int64_t block,
                                 void* stream) {
  LNQ_REQUIRE(out_features >= 0 && in_features >= 0, "lnq_nf4_repack: negative size");
  LNQ_REQUIRE(block > 0 && block % 2 == 0 && in_features % block == 0,
              "lnq_nf4_repack: %lld inputs do not make blocks of %lld", static_cast<long long>(in_features),
              static_cast<long long>(block));
  LNQ_REQUIRE((nested_map == nullptr) == (nested_absmax == nullptr),
              "lnq_nf4_repack: double quantization takes both nested_absmax and nested_map");
  LNQ_REQUIRE(nested_map == nullptr || nested_block > 0, "lnq_nf4_repack: nested_block must be positive");
  const int64_t bytes = out_features * (in_features / 2);
  const int64_t scales = out_features * (in_features / block);
  if (bytes == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(packed && absmax_in && codes && absmax, "lnq_nf4_repack: null pointer");
  LNQ_REQUIRE(aligned(packed, 4) && aligned(codes, 4), "lnq_nf4_repack: packed and codes must be 4-byte aligned");
  const int64_t threads = (bytes + 3) / 4 > scales ? (bytes + 3) / 4 : scales;
  const int64_t grid = (threads + 255) / 256;
  LNQ_REQUIRE(grid <= INT32_MAX, "lnq_nf4_repack: too large");
  hipLaunchKernelGGL(nf4_repack_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), packed, codes, bytes, absmax_in, nested_absmax, nested_map,
                     nested_block, offset, absmax, scales);
  return launched("nf4_repack");
}

}  // extern "C"
