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

// Two exact f32 products rounded to the 16-bit type and packed (low = a): one
// hardware conversion (round to nearest even) for the pair.
template <int DT>
__device__ inline uint32_t pack2(float a, float b) {
  if constexpr (DT == LNQ_BF16) return pack_bf16x2(a, b);
  else return pack_f16x2(a, b);
}

// Element offset of 16-byte column c16 of row `row` in a swizzled 64-wide tile
// (rows of 128 bytes). The 16-byte columns are XOR-swizzled by bits 1..3 of the
// row: an MFMA operand read takes 16 consecutive rows at one column, and rows
// 2i and 2i+1 share a 256-byte bank line in opposite halves, so the XOR must
// separate row pairs, not single rows.
__device__ inline int swz(int row, int c16) { return row * gemm::BK + ((c16 ^ ((row >> 1) & 7)) << 3); }

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
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int M, int N, int K, int G,
    int gshift) {
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

  // Operands through buffer descriptors: 32-bit lane offsets, the step's offset
  // in an SGPR, no per-lane 64-bit address arithmetic.
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(x, static_cast<uint32_t>(static_cast<size_t>(M) * K * 2));
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(packed, static_cast<uint32_t>(static_cast<size_t>(N) * (K >> 1)));
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(scale, static_cast<uint32_t>(N * groups * 2));
  const __amdgpu_buffer_rsrc_t rz = buffer_rsrc(zero, static_cast<uint32_t>(N * groups));

  // x tile loads: 8 x 16 bytes per thread; chunk tid + 256 i -> row tid/8 + 32 i,
  // column tid%8. Rows 32 i apart differ by a uniform offset (an SGPR), and
  // by 32 * 64 elements in LDS, where the swizzle (bits 1..3 of the row) is the
  // same. Rows past M (and of W past N) read zeros through the range check.
  const int xrow = tid >> 3;
  const int xc16 = tid & 7;
  const int xoff = (m0 + xrow) * K * 2 + xc16 * 16;
  const int adst = swz(xrow, xc16);
  // W tile: thread -> row n0 + tid/2, 32 weights (16 bytes) at k offset 32*(tid%2).
  const int brow = tid >> 1;
  const int bhalf = tid & 1;
  const int nsrc = n0 + brow;
  const int woff = nsrc * (K >> 1) + bhalf * 16;
  const int soff = nsrc * groups * 2;
  const int zoff = nsrc * groups;

  // What one step brings from HBM/L2 to registers: 8 x 16 bytes of x, 16 bytes
  // of packed weights, the step's scale (16-bit) and zero point (converted when used).
  struct Stage {
    u32x4 a[8];
    u32x4 w;
    uint32_t s, z;
  };
  // The scale, zero point and weights are requested before x, so that the
  // dequantization waits only for them (loads retire in order). A step past the
  // end reads through a 0-byte descriptor: zeros, no traffic.
  const __amdgpu_buffer_rsrc_t rnull = buffer_rsrc(packed, 0);
  auto load_step = [&](int ks, Stage& st) {
    const bool in = ks < steps;
    const int k0 = in ? ks * BK : 0;
    const int g = gshift >= 0 ? (k0 + 32 * bhalf) >> gshift : (k0 + 32 * bhalf) / G;
    st.s = static_cast<uint16_t>(__builtin_amdgcn_raw_buffer_load_b16(in ? rs : rnull, soff + 2 * g, 0, 0));
    st.z = __builtin_amdgcn_raw_buffer_load_b8(in ? rz : rnull, zoff + g, 0, 0);
    st.w = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(in ? rw : rnull, woff, k0 >> 1, 0));
#pragma unroll
    for (int i = 0; i < 8; ++i)
      st.a[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(in ? rx : rnull, xoff, 2 * k0 + i * 64 * K, 0));
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

  // Dequantize packed dword d of this thread's 32 weights (elements 8d..8d+7)
  // and store them as one 16-byte column of the W tile.
  float sreg = 0.f, zsreg = 0.f;
  auto store_w = [&](int stage, int d, const Stage& st) {
    if (d == 0) {
      sreg = E::to_f32(static_cast<uint16_t>(st.s));
      zsreg = static_cast<float>(st.z & 0xffu) * sreg;  // exact: 4-bit times a 16-bit float
    }
    const uint32_t word = d == 0 ? st.w.x : d == 1 ? st.w.y : d == 2 ? st.w.z : st.w.w;
    const uint32_t lo = opaque(word & 0x0f0f0f0fu);
    const uint32_t hi = opaque((word >> 4) & 0x0f0f0f0fu);
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
  };
  auto store_x = [&](int stage, int i0, const Stage& st) {
#pragma unroll
    for (int i = i0; i < i0 + 2; ++i) *reinterpret_cast<u32x4*>(&As[stage][adst + i * 32 * BK]) = st.a[i];
  };

  // One register stage: step ks + 1 is requested at the start of step ks and
  // written to the other LDS stage between step ks's MFMAs.
  Stage nx;
  load_step(0, nx);
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    store_w(0, d, nx);
    store_x(0, 2 * d, nx);
  }
  __syncthreads();

  const int lrow = lane & 31;
  const int lk = lane >> 5;  // which 8 of an MFMA's 16 inputs
  for (int ks = 0; ks < steps; ++ks) {
    const int stage = ks & 1;
    const bool more = ks + 1 < steps;
    load_step(ks + 1, nx);
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
      // The next step's tiles go to the other stage while these MFMAs run.
      if (more) {
        store_w(stage ^ 1, kk, nx);
        store_x(stage ^ 1, 2 * kk, nx);
      }
    }
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
  // Buffer offsets are 32-bit: x and the packed weight stay under 2 GiB.
  return (dtype == LNQ_BF16 || dtype == LNQ_F16) && M > 0 && N > 0 && K % gemm::BK == 0 &&
         K >= gemm::BK && G % 32 == 0 && K % G == 0 &&
         static_cast<size_t>(M) * K * 2 < (1ull << 31) && static_cast<size_t>(N) * (K >> 1) < (1ull << 31);
}

LnqStatus launch_int4_tiled(const void* x, const uint8_t* packed, const void* scale,
                            const uint8_t* zero, const void* bias, void* y, int M, int N, int K,
                            int G, int dtype, hipStream_t stream) {
  const int tiles = ((M + gemm::BM - 1) / gemm::BM) * ((N + gemm::BN - 1) / gemm::BN);
  const dim3 grid(tiles), block(gemm::THREADS);
  const int gshift = (G & (G - 1)) == 0 ? __builtin_ctz(static_cast<unsigned>(G)) : -1;
  const auto* xs = static_cast<const uint16_t*>(x);
  const auto* ss = static_cast<const uint16_t*>(scale);
  const auto* bs = static_cast<const uint16_t*>(bias);
  auto* ys = static_cast<uint16_t*>(y);
  if (dtype == LNQ_BF16)
    hipLaunchKernelGGL((int4_tiled_kernel<LNQ_BF16>), grid, block, 0, stream, xs, packed, ss, zero,
                       bs, ys, M, N, K, G, gshift);
  else
    hipLaunchKernelGGL((int4_tiled_kernel<LNQ_F16>), grid, block, 0, stream, xs, packed, ss, zero,
                       bs, ys, M, N, K, G, gshift);
  return launched("int4_tiled");
}

}  // namespace lnq
