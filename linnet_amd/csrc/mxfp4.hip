// MXFP4 mixture-of-experts products for a decoding step (std.quant::mxfp4_experts,
// the reference's `mxfp4_experts` Triton kernel, python/linnet/src/linnet/torch/
// kernels.py:94-209): y[r, k, o] = sum_i x[r, k, i] * W[experts[r, k], o, i], the
// weights MXFP4 as gpt-oss checkpoints store them -- blocks [E, Out, G, 16] bytes
// (32 FP4 E2M1 values a block, element 2j in the low nibble of byte j) and scales
// [E, Out, G] E8M0 bytes (2^(s - 127)) -- read once, as they are.
//
// gfx950 converts a byte of two E2M1 values to two bf16 / f16 values in one
// instruction (v_cvt_scalef32_pk_{bf16,f16}_fp4, exact: E2M1 needs two significant
// bits), which then meet the matching pair of x in one v_dot2_f32_{bf16,f16}; a
// block's sum times its scale (v_ldexp_f32, exact) is added to the row's sum in
// f32, as the reference applies the scale after the block's products.
//
// Layout of the work: one workgroup per (row, chosen slot) pair and 16 output
// rows of its expert, 4 waves of 4 rows. Lane l owns blocks l, l + 64, ... of
// every row it visits, so its 32 inputs of x per block stay in registers across
// the rows and a wave's weight loads read 64 consecutive blocks (1 KB) of a row.
// All of a wave's loads are issued before any is used, x and the scales first
// (buffer loads: rows past Out, blocks past G and the rows of an out-of-range
// expert read zeros through the range check). A row's sum is the lanes' partial
// sums added across the wave (fixed order).
#include "common.hpp"

namespace lnq {

namespace mx {
constexpr int WAVES = 4;
constexpr int MAX_SLOTS = 4;  // blocks of a lane per row: G <= 256 (In <= 8192)
// Output rows of a wave (gpt-oss's 2880 -> 5760 at one token: 11.3 us with 4,
// 11.9 with 2, 12.4 with 8; 32 tokens: 55, 63, 55 us).
constexpr int ROWS = 4;
}  // namespace mx

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// sum over byte j of w (two E2M1 codes, elements 2j and 2j + 1) of the codes'
// values times x's pair j (packed 16-bit values, element order), plus c.
template <int DT>
__device__ inline float fp4_dot_byte(uint32_t w, int j, uint32_t xpair, float c) {
  if constexpr (DT == LNQ_BF16) {
    bf16x2_t v;
    switch (j) {
      case 0: v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 0); break;
      case 1: v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 1); break;
      case 2: v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 2); break;
      default: v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 3); break;
    }
    return __builtin_amdgcn_fdot2_f32_bf16(v, __builtin_bit_cast(bf16x2_t, xpair), c, false);
  } else {
    f16x2_t v;
    switch (j) {
      case 0: v = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 0); break;
      case 1: v = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 1); break;
      case 2: v = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 2); break;
      default: v = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 3); break;
    }
    return __builtin_amdgcn_fdot2(v, __builtin_bit_cast(f16x2_t, xpair), c, false);
  }
}

template <int DT, int SLOTS>
__global__ __launch_bounds__(64 * mx::WAVES) void mxfp4_experts_kernel(
    const uint16_t* __restrict__ x, int64_t x_row_stride, int64_t x_slot_stride, int chosen,
    const uint8_t* __restrict__ blocks, const uint8_t* __restrict__ scales,
    const int64_t* __restrict__ experts, int num_experts, uint16_t* __restrict__ y, int out_features,
    int groups) {
  using E = Elem<DT>;
  const int pair = blockIdx.x;
  const int r = pair / chosen, k = pair % chosen;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  constexpr int ROWS = mx::ROWS;
  const int o0 = (blockIdx.y * mx::WAVES + wave) * ROWS;
  const int64_t expert = experts[pair];
  // An expert index outside 0 .. E-1 reads nothing (a 0-byte range) and gives
  // zero rows; rows past Out and blocks past G read zeros through the range.
  const bool valid = expert >= 0 && expert < num_experts;
  const size_t expert_blocks = static_cast<size_t>(out_features) * groups;
  const size_t e0 = valid ? static_cast<size_t>(expert) * expert_blocks : 0;
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(blocks + e0 * 16, valid ? static_cast<uint32_t>(expert_blocks * 16) : 0);
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(scales + e0, valid ? static_cast<uint32_t>(expert_blocks) : 0);
  const uint16_t* xp = x + r * x_row_stride + k * x_slot_stride;

  // x of this lane's blocks first (32 values, 16 dwords in element order, a
  // block), then the scales, then the weights: the memory pipeline serves a CU's
  // loads in the order they arrive, so the small loads issued first land first
  // and the multiply starts as soon as the weights do (one round trip in all).
  u32x4 xv[SLOTS][4];
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) {
    const int g = lane + 64 * s;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      xv[s][q] = g < groups ? *reinterpret_cast<const u32x4*>(xp + g * 32 + 8 * q) : u32x4{0u, 0u, 0u, 0u};
  }
  // Blocks of rows past Out, or past G within a row, land outside the range.
  uint32_t blk[ROWS][SLOTS];
  int sc[ROWS][SLOTS];
#pragma unroll
  for (int i = 0; i < ROWS; ++i)
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
      const int g = lane + 64 * s;
      const int o = o0 + i;
      blk[i][s] = o < out_features && g < groups ? static_cast<uint32_t>(o * groups + g) : 0xffffffffu >> 4;
      sc[i][s] = __builtin_amdgcn_raw_buffer_load_b8(rs, blk[i][s], 0, 0);
    }
  u32x4 w[ROWS][SLOTS];
#pragma unroll
  for (int i = 0; i < ROWS; ++i)
#pragma unroll
    for (int s = 0; s < SLOTS; ++s)
      w[i][s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, blk[i][s] * 16, 0, 2 /* non-temporal */));

  float acc[ROWS];
#pragma unroll
  for (int i = 0; i < ROWS; ++i) {
    acc[i] = 0.0f;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
      float part = 0.0f;
#pragma unroll
      for (int d = 0; d < 4; ++d)
#pragma unroll
        for (int j = 0; j < 4; ++j) part = fp4_dot_byte<DT>(w[i][s][d], j, xv[s][d][j], part);
      acc[i] += ldexpf(part, sc[i][s] - 127);
    }
  }
#pragma unroll
  for (int i = 0; i < ROWS; ++i) {
    const float v = wave_sum(acc[i]);
    const int o = o0 + i;
    if (lane == 0 && o < out_features) y[static_cast<size_t>(pair) * out_features + o] = E::from_f32(v);
  }
}

}  // namespace lnq

using namespace lnq;

extern "C" {

LNQ_API LnqStatus lnq_mxfp4_experts(const void* x, int64_t x_row_stride, int64_t x_slot_stride,
                                    const uint8_t* blocks, const uint8_t* scales, const int64_t* experts,
                                    void* y, int64_t rows, int64_t chosen, int64_t num_experts,
                                    int64_t out_features, int64_t in_features, int32_t dtype, void* stream) {
  LNQ_REQUIRE(dtype == LNQ_BF16 || dtype == LNQ_F16, "lnq_mxfp4_experts: x is bf16 or f16, not dtype %d", dtype);
  LNQ_REQUIRE(rows >= 0 && chosen >= 0 && num_experts > 0 && out_features >= 0 && in_features >= 0,
              "lnq_mxfp4_experts: negative size");
  LNQ_REQUIRE(in_features % 32 == 0 && in_features <= 32 * 64 * mx::MAX_SLOTS,
              "lnq_mxfp4_experts: in %lld is not a multiple of 32 up to %d", static_cast<long long>(in_features),
              32 * 64 * mx::MAX_SLOTS);
  LNQ_REQUIRE(rows * chosen <= INT32_MAX && out_features * (in_features / 32) * 16 < (int64_t{1} << 32) - 16,
              "lnq_mxfp4_experts: too large (one expert's blocks past 4 GiB)");
  if (rows == 0 || chosen == 0 || out_features == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE((x || in_features == 0) && blocks && scales && experts && y, "lnq_mxfp4_experts: null pointer");
  LNQ_REQUIRE(aligned(x, 16) && aligned(blocks, 16) && x_row_stride % 8 == 0 && x_slot_stride % 8 == 0,
              "lnq_mxfp4_experts: x (with its row and slot strides) and blocks must be 16-byte aligned");
  const int groups = static_cast<int>(in_features / 32);
  const int slots = (groups + 63) / 64;
  const int per_wg = mx::WAVES * mx::ROWS;
  const dim3 grid(static_cast<unsigned>(rows * chosen), static_cast<unsigned>((out_features + per_wg - 1) / per_wg));
  LNQ_REQUIRE(grid.y <= 65535, "lnq_mxfp4_experts: too many output features");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* xs = static_cast<const uint16_t*>(x);
  auto* ys = static_cast<uint16_t*>(y);
  const int C = static_cast<int>(chosen), NE = static_cast<int>(num_experts), O = static_cast<int>(out_features);
#define LNQ_MX(DT, S)                                                                                                 \
  hipLaunchKernelGGL((mxfp4_experts_kernel<DT, S>), grid, dim3(64 * mx::WAVES), 0, s, xs, x_row_stride, x_slot_stride, \
                     C, blocks, scales, experts, NE, ys, O, groups)
#define LNQ_MX_S(DT)                 \
  switch (slots) {                   \
    case 0:                          \
    case 1: LNQ_MX(DT, 1); break;    \
    case 2: LNQ_MX(DT, 2); break;    \
    case 3: LNQ_MX(DT, 3); break;    \
    default: LNQ_MX(DT, 4); break;   \
  }
  if (dtype == LNQ_BF16) {
    LNQ_MX_S(LNQ_BF16);
  } else {
    LNQ_MX_S(LNQ_F16);
  }
#undef LNQ_MX_S
#undef LNQ_MX
  return launched("mxfp4_experts");
}

}  // extern "C"
