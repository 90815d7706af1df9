// The prefill-shape int4 dequant-GEMM on gfx950 MFMA.
//
// y[M, N] = x[M, K] @ W^T with W[n, k] = (q - z) * s dequantized to the
// activation dtype exactly as the reference rounds it (f32 product, one
// rounding), so that every MFMA product is x * bf16(W) as in the reference's
// dequant + BLAS path (src/backend/torch_source.cpp:1561-1566).
//
// Tiles: 256 x 128 outputs per workgroup of 4 waves (2 x 2), each wave a
// 128 x 64 block of 4 x 2 MFMA 32x32x16 tiles; 64 inputs per step, double
// buffered in LDS (2 x (32 KB of x + 16 KB of W)). Each step every thread
// moves 8 x 16 bytes of x and dequantizes 16 packed bytes (32 weights) of W
// into LDS; rows of 64 elements are stored with their 16-byte columns
// XOR-swizzled by (row & 7), so the MFMA operand reads hit distinct banks.
//
// Workgroups are numbered so that each XCD (workgroup b runs on XCD b % 8)
// owns a contiguous run of tiles, ordered in groups of 4 row tiles: the
// tiles resident on one XCD share x and W tiles in its L2.
#include "common.hpp"

namespace lnq {

namespace gemm {
constexpr int BM = 256;
constexpr int BN = 128;
constexpr int BK = 64;
constexpr int THREADS = 256;
constexpr int GROUP_M = 4;
constexpr int XCDS = 8;
}  // namespace gemm

template <int DT>
__device__ inline f32x16 mfma32x32x16(u32x4 a, u32x4 b, f32x16 c);

template <>
__device__ inline f32x16 mfma32x32x16<LNQ_BF16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

template <>
__device__ inline f32x16 mfma32x32x16<LNQ_F16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Two f32 values rounded to the 16-bit type and packed (low = a).
template <int DT>
__device__ inline uint32_t pack2(float a, float b) {
  return static_cast<uint32_t>(Elem<DT>::from_f32(a)) |
         (static_cast<uint32_t>(Elem<DT>::from_f32(b)) << 16);
}

// Element offset of 16-byte column c16 of row `row` in a swizzled 64-wide tile.
__device__ inline int swz(int row, int c16) { return row * gemm::BK + ((c16 ^ (row & 7)) << 3); }

// Workgroup -> (row tile, column tile): XCD-contiguous, then grouped by GROUP_M rows.
__device__ inline void tile_of(int b, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  const int per_xcd = (total + gemm::XCDS - 1) / gemm::XCDS;
  const int xcd = b % gemm::XCDS;
  const int local = b / gemm::XCDS;
  int logical = xcd * per_xcd + local;
  // The last XCDs may own fewer tiles when total % 8 != 0: the excess
  // logical ids fold back onto the tail workgroups' slots.
  const int full = total - (per_xcd - 1) * gemm::XCDS;  // XCDs owning per_xcd tiles
  if (total % gemm::XCDS != 0) {
    logical = xcd < full ? xcd * per_xcd + local : full * per_xcd + (xcd - full) * (per_xcd - 1) + local;
  }
  const int per_group = gemm::GROUP_M * tiles_n;
  const int first_m = (logical / per_group) * gemm::GROUP_M;
  const int rows = min(tiles_m - first_m, gemm::GROUP_M);
  tm = first_m + (logical % per_group) % rows;
  tn = (logical % per_group) / rows;
}

template <int DT>
__global__ __launch_bounds__(gemm::THREADS, 1) void int4_tiled_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ packed,
    const uint16_t* __restrict__ scale, const uint8_t* __restrict__ zero,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int M, int N, int K, int G) {
  using namespace gemm;
  using E = Elem<DT>;
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * BK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * BK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;  // 0..1: 128-row half
  const int wn = wave & 1;   // 0..1: 64-column half
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  if (tm >= tiles_m || tn >= tiles_n) return;
  const int m0 = tm * BM;
  const int n0 = tn * BN;
  const int groups = K / G;
  const int steps = K / BK;

  // x tile loads: 8 x 16 bytes per thread; chunk id = tid + 256 i -> row id/8, column id%8.
  const uint16_t* xsrc[8];
  int adst[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int id = tid + THREADS * i;
    const int row = id >> 3;
    const int c16 = id & 7;
    const int m = min(m0 + row, M - 1);
    xsrc[i] = x + static_cast<size_t>(m) * K + c16 * 8;
    adst[i] = swz(row, c16);
  }
  // W tile: thread -> row n0 + tid/2, 32 weights (16 bytes) at k offset 32*(tid%2).
  const int brow = tid >> 1;
  const int bhalf = tid & 1;
  const int nsrc = min(n0 + brow, N - 1);
  const uint8_t* wsrc = packed + static_cast<size_t>(nsrc) * (K >> 1) + bhalf * 16;
  const uint16_t* ssrc = scale + static_cast<size_t>(nsrc) * groups;
  const uint8_t* zsrc = zero + static_cast<size_t>(nsrc) * groups;

  u32x4 areg[8];
  u32x4 wreg;
  float sreg, zsreg;

  auto load_step = [&](int ks) {
    const int k0 = ks * BK;
#pragma unroll
    for (int i = 0; i < 8; ++i) areg[i] = *reinterpret_cast<const u32x4*>(xsrc[i] + k0);
    wreg = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wsrc + (k0 >> 1)));
    const int g = (k0 + 32 * bhalf) / G;
    sreg = E::to_f32(ssrc[g]);
    zsreg = static_cast<float>(zsrc[g]) * sreg;  // exact: 4-bit times a 16-bit float
  };

  auto store_step = [&](int stage) {
#pragma unroll
    for (int i = 0; i < 8; ++i) *reinterpret_cast<u32x4*>(&As[stage][adst[i]]) = areg[i];
    // 32 weights, element order; (q - z) * s = fma(q, s, -z*s) is exact in f32.
    const uint32_t words[4] = {wreg.x, wreg.y, wreg.z, wreg.w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t lo = words[d] & 0x0f0f0f0fu;
      const uint32_t hi = (words[d] >> 4) & 0x0f0f0f0fu;
      float v[8];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        v[2 * b] = fmaf(static_cast<float>((lo >> (8 * b)) & 0xffu), sreg, -zsreg);
        v[2 * b + 1] = fmaf(static_cast<float>((hi >> (8 * b)) & 0xffu), sreg, -zsreg);
      }
      u32x4 o;
      o.x = pack2<DT>(v[0], v[1]);
      o.y = pack2<DT>(v[2], v[3]);
      o.z = pack2<DT>(v[4], v[5]);
      o.w = pack2<DT>(v[6], v[7]);
      *reinterpret_cast<u32x4*>(&Bs[stage][swz(brow, 4 * bhalf + d)]) = o;
    }
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

  load_step(0);
  store_step(0);
  __syncthreads();

  const int lrow = lane & 31;
  const int lk = lane >> 5;  // which 8 of an MFMA's 16 inputs
  for (int ks = 0; ks < steps; ++ks) {
    const int stage = ks & 1;
    if (ks + 1 < steps) load_step(ks + 1);
    const uint16_t* as = As[stage];
    const uint16_t* bs = Bs[stage];
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int c16 = 2 * kk + lk;
      u32x4 af[4], bf[2];
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int row = wm * 128 + a * 32 + lrow;
        af[a] = *reinterpret_cast<const u32x4*>(&as[swz(row, c16)]);
      }
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const int row = wn * 64 + b * 32 + lrow;
        bf[b] = *reinterpret_cast<const u32x4*>(&bs[swz(row, c16)]);
      }
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = mfma32x32x16<DT>(af[a], bf[b], acc[a][b]);
    }
    if (ks + 1 < steps) store_step(stage ^ 1);
    __syncthreads();
  }

  // Epilogue. MFMA 32x32 output: lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4,
  // column l%32.
#pragma unroll
  for (int a = 0; a < 4; ++a) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int n = n0 + wn * 64 + b * 32 + (lane & 31);
      if (n >= N) continue;
      const float bv = bias != nullptr ? E::to_f32(bias[n]) : 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * 128 + a * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m < M) {
          uint16_t out = E::from_f32(acc[a][b][r]);
          if (bias != nullptr) out = E::from_f32(E::to_f32(out) + bv);
          y[static_cast<size_t>(m) * N + n] = out;
        }
      }
    }
  }
}

bool int4_tiled_supports(int M, int N, int K, int G, int dtype) {
  return (dtype == LNQ_BF16 || dtype == LNQ_F16) && M > 0 && N > 0 && K % gemm::BK == 0 &&
         K >= gemm::BK && G % 32 == 0 && K % G == 0;
}

LnqStatus launch_int4_tiled(const void* x, const uint8_t* packed, const void* scale,
                            const uint8_t* zero, const void* bias, void* y, int M, int N, int K,
                            int G, int dtype, hipStream_t stream) {
  const int tiles = ((M + gemm::BM - 1) / gemm::BM) * ((N + gemm::BN - 1) / gemm::BN);
  const dim3 grid(tiles), block(gemm::THREADS);
  const auto* xs = static_cast<const uint16_t*>(x);
  const auto* ss = static_cast<const uint16_t*>(scale);
  const auto* bs = static_cast<const uint16_t*>(bias);
  auto* ys = static_cast<uint16_t*>(y);
  if (dtype == LNQ_BF16)
    hipLaunchKernelGGL((int4_tiled_kernel<LNQ_BF16>), grid, block, 0, stream, xs, packed, ss, zero,
                       bs, ys, M, N, K, G);
  else
    hipLaunchKernelGGL((int4_tiled_kernel<LNQ_F16>), grid, block, 0, stream, xs, packed, ss, zero,
                       bs, ys, M, N, K, G);
  return launched("int4_tiled");
}

}  // namespace lnq
