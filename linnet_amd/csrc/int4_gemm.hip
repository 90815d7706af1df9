// The prefill-shape int4 dequant-GEMM on gfx950 MFMA.
//
// y[M, N] = x[M, K] @ W^T with W[n, k] = (q - z) * s dequantized to the
// activation dtype exactly as the reference rounds it (f32 product, one
// rounding), so that every MFMA product is x * bf16(W) as in the reference's
// dequant + BLAS path (src/backend/torch_source.cpp:1561-1566).
//
// Tiles: 256 x 128 outputs per workgroup of 4 waves (2 x 2), each wave a
// 128 x 64 block of 4 x 2 MFMA 32x32x16 tiles; 64 inputs per step.
//
// Pipeline, per step ks:
//   * x moves HBM/L2 -> LDS without registers (buffer_load ... lds), two steps
//     ahead, into a ring of three 32 KB stages;
//   * the packed weights (16 bytes per thread), scale and zero point of step
//     ks + 2 are requested into one of two register sets;
//   * while step ks's MFMAs run, the register set of step ks + 1 is
//     dequantized into the other of two 16 KB W stages;
//   * each wave waits for its own x loads of step ks + 1 (an explicit vmcnt
//     that leaves step ks + 2's loads in flight), then one barrier.
// The barriers are bare s_barrier with explicit waits: __syncthreads()'s fence
// would wait for every outstanding load, including the ones two steps ahead.
// Stage indices are compile-time (the loop is unrolled by 6 = lcm(3, 2)) so
// that the compiler can tell the stages' LDS accesses apart.
//
// Rows of 64 elements are stored with their 16-byte columns XOR-swizzled by
// bits 1..3 of the row, so the MFMA operand reads hit distinct banks; the x
// loads pick their source column so that the contiguous LDS writes of one
// buffer_load ... lds land in that layout.
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

// The issue order the scheduler is asked for within one kk: each of the 8
// MFMAs followed by one operand read (of the next kk) and VALU instructions of
// the dequantization, then the W tile writes, so that the matrix core is fed
// while the rest of the step's work issues beside it.
template <bool READS, int VALU, int WRITES>
__device__ inline void interleave() {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    if constexpr (READS) {
      if (i < 6) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
    }
    if constexpr (VALU > 0) __builtin_amdgcn_sched_group_barrier(0x002, VALU, 0);
  }
  if constexpr (WRITES > 0) __builtin_amdgcn_sched_group_barrier(0x200, WRITES, 0);  // DS write
}

template <int DT>
__global__ __launch_bounds__(gemm::THREADS, 1) void int4_tiled_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ packed,
    const uint16_t* __restrict__ scale, const uint8_t* __restrict__ zero,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int M, int N, int K, int G,
    int gshift) {
  using namespace gemm;
  using E = Elem<DT>;
  __shared__ __attribute__((aligned(16))) uint16_t X0[BM * BK];
  __shared__ __attribute__((aligned(16))) uint16_t X1[BM * BK];
  __shared__ __attribute__((aligned(16))) uint16_t X2[BM * BK];
  __shared__ __attribute__((aligned(16))) uint16_t W0[BN * BK];
  __shared__ __attribute__((aligned(16))) uint16_t W1[BN * BK];

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
  // in an SGPR. Rows past M (and of W past N) read zeros through the range check.
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(x, static_cast<uint32_t>(static_cast<size_t>(M) * K * 2));
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(packed, static_cast<uint32_t>(static_cast<size_t>(N) * (K >> 1)));
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(scale, static_cast<uint32_t>(N * groups * 2));
  const __amdgpu_buffer_rsrc_t rz = buffer_rsrc(zero, static_cast<uint32_t>(N * groups));
  // A step past the end reads through a 0-byte descriptor: zeros, no traffic,
  // and the same number of loads in flight as any other step.
  const __amdgpu_buffer_rsrc_t rnull = buffer_rsrc(packed, 0);

  // x: load i of wave w writes LDS rows 32 i + 8 w .. + 7 (1 KB, lane l at byte
  // 16 l: row 32 i + 8 w + l / 8, stored column l % 8). The stored column holds
  // source column (l % 8) ^ key(row); key = (row >> 1) & 7 = (4 w + l / 16) & 7
  // does not depend on i, so the 8 loads differ only by a uniform offset.
  const int xrow = 8 * wave + (lane >> 3);
  const int xcol = (lane & 7) ^ ((xrow >> 1) & 7);
  const int xoff = (m0 + xrow) * K * 2 + xcol * 16;
  const int xlds = wave * 512;  // elements
  auto load_x = [&](uint16_t* dst, int ks) {
    const bool in = ks < steps;
    const int k0 = in ? ks * BK : 0;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(in ? rx : rnull, (lds_ptr)(dst + xlds + i * 32 * BK), 16, xoff,
                                                2 * k0 + i * 64 * K, 0, 0);
  };

  // W: thread -> row n0 + tid / 2, 32 weights (16 packed bytes) at k offset 32 * (tid % 2).
  const int brow = tid >> 1;
  const int bhalf = tid & 1;
  const int nsrc = n0 + brow;
  const int woff = nsrc * (K >> 1) + bhalf * 16;
  const int soff = nsrc * groups * 2;
  const int zoff = nsrc * groups;
  struct WRegs {
    u32x4 w;
    uint32_t s, z;
  };
  auto load_w = [&](WRegs& r, int ks) {
    const bool in = ks < steps;
    const int k0 = in ? ks * BK : 0;
    const int g = gshift >= 0 ? (k0 + 32 * bhalf) >> gshift : (k0 + 32 * bhalf) / G;
    r.s = static_cast<uint16_t>(__builtin_amdgcn_raw_buffer_load_b16(in ? rs : rnull, soff + 2 * g, 0, 0));
    r.z = __builtin_amdgcn_raw_buffer_load_b8(in ? rz : rnull, zoff + g, 0, 0);
    r.w = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(in ? rw : rnull, woff, k0 >> 1, 0));
  };
  // Dequantize packed dword d (elements 8d..8d+7 of the thread's 32) into one
  // 16-byte column of the W tile: (q - z) * s = fma(q, s, -z*s), exact in f32
  // (z * s: 4 bits times a 16-bit float), then one rounding to the 16-bit type.
  float sreg = 0.f, zsreg = 0.f;
  auto store_w = [&](uint16_t* dst, int d, const WRegs& r) {
    if (d == 0) {
      sreg = E::to_f32(static_cast<uint16_t>(r.s));
      zsreg = static_cast<float>(r.z & 0xffu) * sreg;
    }
    const uint32_t word = d == 0 ? r.w.x : d == 1 ? r.w.y : d == 2 ? r.w.z : r.w.w;
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
    *reinterpret_cast<u32x4*>(&dst[swz(brow, 4 * bhalf + d)]) = o;
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

  const int lrow = lane & 31;
  const int lk = lane >> 5;  // which 8 of an MFMA's 16 inputs
  // Operand fragments: f0 holds even kk, f1 odd kk. kk + 1's are read from LDS
  // while kk's MFMAs run; step ks + 1's kk = 0 is read right after the barrier,
  // under step ks's last MFMAs.
  u32x4 af0[4], bf0[2], af1[4], bf1[2];
  auto read = [&](const uint16_t* xs, const uint16_t* ws, int kk, u32x4* a_, u32x4* b_) {
    const int c16 = 2 * kk + lk;
#pragma unroll
    for (int a = 0; a < 4; ++a) a_[a] = *reinterpret_cast<const u32x4*>(&xs[swz(wm * 128 + a * 32 + lrow, c16)]);
#pragma unroll
    for (int b = 0; b < 2; ++b) b_[b] = *reinterpret_cast<const u32x4*>(&ws[swz(wn * 64 + b * 32 + lrow, c16)]);
  };
  auto mfmas = [&](const u32x4* a_, const u32x4* b_) {
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b) acc[a][b] = mfma32x32x16<DT>(a_[a], b_[b], acc[a][b]);
  };
  // One step: MFMAs on (xc, wcur) with kk = 0 already in f0; step ks + 2
  // requested into (xn2, later); step ks + 1's weights (next) dequantized into
  // wnext, which with xn1 holds step ks + 1's operands after the barrier.
  auto step = [&](int ks, const uint16_t* xc, const uint16_t* xn1, uint16_t* xn2, const uint16_t* wcur,
                  uint16_t* wnext, const WRegs& next, WRegs& later) {
    load_w(later, ks + 2);
    load_x(xn2, ks + 2);
    read(xc, wcur, 1, af1, bf1);
    mfmas(af0, bf0);
    store_w(wnext, 0, next);
    interleave<true, 3, 1>();
    read(xc, wcur, 2, af0, bf0);
    mfmas(af1, bf1);
    store_w(wnext, 1, next);
    interleave<true, 3, 1>();
    read(xc, wcur, 3, af1, bf1);
    mfmas(af0, bf0);
    store_w(wnext, 2, next);
    store_w(wnext, 3, next);
    interleave<true, 6, 2>();
    // This wave's x loads of step ks + 1 are done once at most the 11 loads
    // issued after them (step ks + 2's 3 weight loads and 8 x loads) remain;
    // its W stores and kk = 3 reads are done at lgkmcnt(0). Past the barrier
    // every wave's are: step ks + 1's operands are in LDS, and no wave reads
    // step ks's stages again, so the next step's loads may overwrite them.
    __asm__ volatile("s_waitcnt vmcnt(11)\n\ts_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    read(xn1, wnext, 0, af0, bf0);
    mfmas(af1, bf1);
    interleave<true, 0, 0>();
    __builtin_amdgcn_sched_barrier(0);
  };

  WRegs ra, rb;
  load_w(ra, 0);
  load_x(X0, 0);
  load_w(rb, 1);
  load_x(X1, 1);
#pragma unroll
  for (int d = 0; d < 4; ++d) store_w(W0, d, ra);
  __asm__ volatile("s_waitcnt vmcnt(11)\n\ts_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  read(X0, W0, 0, af0, bf0);

  // Stages: x step j in X[j % 3], W step j in W[j % 2], registers of step j in
  // (ra, rb)[j % 2].
  int ks = 0;
  for (; ks + 6 <= steps; ks += 6) {
    step(ks, X0, X1, X2, W0, W1, rb, ra);
    step(ks + 1, X1, X2, X0, W1, W0, ra, rb);
    step(ks + 2, X2, X0, X1, W0, W1, rb, ra);
    step(ks + 3, X0, X1, X2, W1, W0, ra, rb);
    step(ks + 4, X1, X2, X0, W0, W1, rb, ra);
    step(ks + 5, X2, X0, X1, W1, W0, ra, rb);
  }
  // The last steps % 6 steps continue the same stage sequence.
  const int rest = steps - ks;
  if (rest > 0) step(ks, X0, X1, X2, W0, W1, rb, ra);
  if (rest > 1) step(ks + 1, X1, X2, X0, W1, W0, ra, rb);
  if (rest > 2) step(ks + 2, X2, X0, X1, W0, W1, rb, ra);
  if (rest > 3) step(ks + 3, X0, X1, X2, W1, W0, ra, rb);
  if (rest > 4) step(ks + 4, X1, X2, X0, W0, W1, rb, ra);
  // Loads of the two steps past the end (zeros through rnull) may be in flight.
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");

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
