// Block-scaled FP8 (std.quant::Fp8BlockLinear, 128 x 128 weight blocks) with
// FP8 activations on gfx950:
//   - groups8: each 128 inputs of each row rounded to FP8 E4M3 with a scale of
//     their own (the reference's `fp8_groups`, torch/kernels.py:757-802);
//   - mm8_kernel<..., BLK = true>: the block-wise product `torch._scaled_mm`
//     computes for the reference (torch/quantized.py:159-166), a partial tile per
//     128-input step folded into the accumulated one with both scales.
// Compiled with VGPR-form MFMA accumulators (the partial and the accumulated
// tile, 2 x 64 registers a lane, fit beside the operands only without the
// AGPR / VGPR split).
#include "eight_bit.hpp"

namespace lnq {

// ================================================================ fp8 groups
// Each 128 inputs of each row rounded to FP8 E4M3 with a scale of their own:
// scale = max(max|x|, 1e-12) / 448 over the group (f32, IEEE divide), q = E4M3
// round-to-nearest-even of clamp(x / scale, +-448); rows rows .. padded - 1 are
// zeros with a scale of 1. One wave a group (two inputs a lane), four groups a
// workgroup; scales column-major, x_scale[g * padded + row].
template <int DT>
__global__ __launch_bounds__(256) void groups8_kernel(const typename Elem<DT>::storage* __restrict__ x,
                                                      uint8_t* __restrict__ q, float* __restrict__ x_scale,
                                                      int rows, int padded, int K) {
  using E = Elem<DT>;
  const int row = blockIdx.x;
  const int g = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (g >= K / 128) return;  // the whole wave
  const int k = g * 128 + 2 * lane;
  float v0 = 0.0f, v1 = 0.0f;
  if (row < rows) {
    const typename E::storage* src = x + static_cast<size_t>(row) * K + k;
    v0 = E::to_f32(src[0]);
    v1 = E::to_f32(src[1]);
  }
  const float top = wave_max(fmaxf(fabsf(v0), fabsf(v1)));
  const float sc = row < rows ? fmaxf(top, 1e-12f) / 448.0f : 1.0f;
  const uint32_t c0 = f32_to_e4m3(fminf(fmaxf(v0 / sc, -448.0f), 448.0f));
  const uint32_t c1 = f32_to_e4m3(fminf(fmaxf(v1 / sc, -448.0f), 448.0f));
  *reinterpret_cast<uint16_t*>(q + static_cast<size_t>(row) * K + k) = static_cast<uint16_t>(c0 | (c1 << 8));
  if (lane == 0) x_scale[static_cast<size_t>(g) * padded + row] = sc;
}

}  // namespace lnq

using namespace lnq;

extern "C" {

LNQ_API LnqStatus lnq_fp8_groups(const void* x, uint8_t* q, float* x_scale, int64_t rows, int64_t padded,
                                 int64_t in_features, int64_t group, int32_t dtype, void* stream) {
  LNQ_REQUIRE(dtype == LNQ_BF16 || dtype == LNQ_F16 || dtype == LNQ_F32,
              "lnq_fp8_groups: x dtype %d is not bf16, f16 or f32", dtype);
  LNQ_REQUIRE(group == 128, "lnq_fp8_groups: groups of 128 inputs, not %lld", static_cast<long long>(group));
  LNQ_REQUIRE(rows >= 0 && padded >= rows && in_features >= 0 && in_features % 128 == 0,
              "lnq_fp8_groups: bad shape rows=%lld padded=%lld in=%lld (in %% 128 == 0, padded >= rows)",
              static_cast<long long>(rows), static_cast<long long>(padded), static_cast<long long>(in_features));
  LNQ_REQUIRE(padded <= 65535 * 64 && padded * in_features < (int64_t{1} << 31), "lnq_fp8_groups: too large");
  if (padded == 0 || in_features == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE((x || rows == 0) && q && x_scale, "lnq_fp8_groups: null pointer");
  LNQ_REQUIRE(aligned(q, 2), "lnq_fp8_groups: q is not 2-byte aligned");
  const dim3 grid(static_cast<unsigned>(padded), static_cast<unsigned>((in_features / 128 + 3) / 4));
  LNQ_REQUIRE(grid.y <= 65535, "lnq_fp8_groups: in too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int R = static_cast<int>(rows), P = static_cast<int>(padded), K = static_cast<int>(in_features);
#define LNQ_G8(DT)                                                                                                 \
  hipLaunchKernelGGL((groups8_kernel<DT>), grid, dim3(256), 0, s, static_cast<const typename Elem<DT>::storage*>(x), \
                     q, x_scale, R, P, K)
  if (dtype == LNQ_BF16) LNQ_G8(LNQ_BF16);
  else if (dtype == LNQ_F16) LNQ_G8(LNQ_F16);
  else LNQ_G8(LNQ_F32);
#undef LNQ_G8
  return launched("fp8_groups");
}

LNQ_API LnqStatus lnq_mm8_block(const uint8_t* qx, const uint8_t* weight, const float* x_scale, int64_t xs_stride,
                                const float* scale, void* y, int64_t rows, int64_t out_features, int64_t in_features,
                                int32_t dtype, void* stream) {
  LNQ_REQUIRE(dtype == LNQ_BF16 || dtype == LNQ_F16, "lnq_mm8_block: output is bf16 or f16, not dtype %d", dtype);
  LNQ_REQUIRE(rows >= 0 && out_features > 0 && in_features > 0 && in_features % 128 == 0 && out_features % 128 == 0,
              "lnq_mm8_block: bad shape rows=%lld out=%lld in=%lld (in, out %% 128 == 0)", static_cast<long long>(rows),
              static_cast<long long>(out_features), static_cast<long long>(in_features));
  LNQ_REQUIRE(xs_stride >= rows, "lnq_mm8_block: x_scale stride %lld < rows %lld", static_cast<long long>(xs_stride),
              static_cast<long long>(rows));
  LNQ_REQUIRE(rows <= INT32_MAX && out_features <= INT32_MAX && in_features <= INT32_MAX && xs_stride <= INT32_MAX,
              "lnq_mm8_block: sizes exceed 2^31");
  if (rows == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(qx && weight && x_scale && scale && y, "lnq_mm8_block: null pointer");
  LNQ_REQUIRE(aligned(qx, 16) && aligned(weight, 16), "lnq_mm8_block: operands must be 16-byte aligned");
  const int M = static_cast<int>(rows), N = static_cast<int>(out_features), K = static_cast<int>(in_features);
  LNQ_REQUIRE(static_cast<size_t>(M) * K < (1ull << 31) && static_cast<size_t>(N) * K < (1ull << 31),
              "lnq_mm8_block: operands exceed the 2 GiB buffer range");
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto* ys = static_cast<uint16_t*>(y);
  const int tiles = ((M + mm8::BM - 1) / mm8::BM) * (N / 128);
  if (dtype == LNQ_BF16)
    hipLaunchKernelGGL((mm8_kernel<LNQ_BF16, 1, 128, true>), dim3(tiles), dim3(mm8::THREADS), 0, s, qx, weight,
                       x_scale, scale, ys, M, N, K, static_cast<int>(xs_stride));
  else
    hipLaunchKernelGGL((mm8_kernel<LNQ_F16, 1, 128, true>), dim3(tiles), dim3(mm8::THREADS), 0, s, qx, weight,
                       x_scale, scale, ys, M, N, K, static_cast<int>(xs_stride));
  return launched("mm8_block");
}

}  // extern "C"
