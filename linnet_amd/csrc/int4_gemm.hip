// The prefill-shape int4 dequant-GEMM on gfx950 MFMA.
//
// y[M, N] = x[M, K] @ W^T with W[n, k] = (q - z) * s dequantized to the
// activation dtype exactly as the reference rounds it (f32 product, one
// rounding), so that every MFMA product is x * bf16(W) as in the reference's
// dequant + BLAS path (src/backend/torch_source.cpp:1561-1566).
//
// Two kernels, by tile width:
//
// int4_tiled_kernel (256-column tiles, wide outputs). 256 rows of x by 256
// columns of W per workgroup of 8 waves, two per SIMD. A wave owns a 128 x 64
// block of MFMA 32x32x16 tiles; 64 inputs per step. Two waves per SIMD is what
// lets the matrix core run while a wave's loads and dequantization issue: on
// gfx950 an MFMA 32x32x16 holds its wave's issue for about 20 of its 32
// cycles, and a buffer load issued beside MFMA and VALU work stalls the wave
// for tens of cycles; the other wave of the SIMD covers both.
//
// Pipeline, per step ks (each wave):
//   * x moves HBM/L2 -> LDS without registers (buffer_load ... lds), two steps
//     ahead, into a ring of three 32 KB stages;
//   * the packed weights, scale and zero point of step ks + 3 are requested
//     into one of three register sets;
//   * the weights of the next step are dequantized into one of two W stages:
//     (q - z) * s = fma(q, s, -z * s) in f32 (exact), one rounding to the
//     16-bit type. The work of a step's weights is spread evenly over the 4 *
//     NMF MFMA slots from the last kk of step ks - 1 through kk = 2 of step ks
//     (about three VALU instructions per MFMA); each slot is its own
//     scheduling region (sched_barrier), which pins that interleave;
//   * one barrier, after kk = 2: every wave's x of step ks + 1 has landed and
//     its W stores are done; kk = 3 then runs while step ks + 1's kk = 0
//     operands are read and the dequantization of step ks + 2 begins in the W
//     stage step ks has finished with.
// The barrier is a bare s_barrier with explicit waits: __syncthreads()'s fence
// would wait for every outstanding load, including the ones two steps ahead.
// Stage indices are compile-time (the loop is unrolled by 6 = lcm(3, 2)).
//
// Rows of 64 elements are stored with their 16-byte columns XOR-swizzled by
// bits 1..3 of the row, so the MFMA operand reads hit distinct banks; the x
// loads pick their source column so that the contiguous LDS writes of one
// buffer_load ... lds land in that layout.
//
// Workgroups are numbered so that each XCD (workgroups b with one b % 8 run on one XCD)
// owns a contiguous run of tiles, ordered in groups of 4 row tiles: the
// tiles resident on one XCD share x and W tiles in its L2.
//
// int4_narrow_kernel (128-column tiles: one tile per CU at N = 4096, M =
// 2048). 4 waves, one per SIMD, each owning 32 columns of W for all 256 rows
// of x, so no column is dequantized twice and the dequantized weights never go
// through LDS: lane l of a wave loads the packed dwords of its column (l % 32)
// and dequantizes them straight into its MFMA operand registers. A 32x32x16
// operand lane holds 8 consecutive inputs of one column -- one packed dword --
// and lane half h = l / 32 takes input blocks 4 h .. 4 h + 3 of a 64-input
// step (16 bytes, one load), so MFMA kk (0..3) sums blocks kk and kk + 4; the
// x operand reads the same blocks from LDS. With W out of LDS, x gets a ring
// of four 32 KB stages, DMA'd three steps ahead. Measured against the
// 8-wave kernel with 128-column tiles on config 3's N = 4096 shapes (M =
// 2048): K = 4096 72 against 84-92 us, K = 14336 231 against 240-245 us.
#include "common.hpp"

namespace lnq {

namespace gemm {
constexpr int BM = 256;
constexpr int BK = 64;
constexpr int THREADS = 512;
constexpr int GROUP_M = 4;
constexpr int XCDS = 8;

template <int BN>
struct Cfg;
template <>
struct Cfg<256> {
  static constexpr int WAVES_N = 4;  // waves of 128 x 64, 2 x 4
  static constexpr int FA = 4;       // 32-row fragments of a wave
  static constexpr int FB = 2;       // 32-column fragments of a wave
};
}  // namespace gemm

template <int DT>
__device__ inline f32x16 mfma32x32x16(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (DT == LNQ_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
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
// row: an MFMA operand read takes 32 consecutive rows at one column, and rows
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
  // The last XCDs own one tile fewer when total % 8 != 0: the excess logical
  // ids fold back onto the tail workgroups' slots.
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

template <int DT, int BN>
__global__ __launch_bounds__(gemm::THREADS, 1) void int4_tiled_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scale,
    const uint8_t* __restrict__ zero, const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int M, int N, int K,
    int gshift) {
  using namespace gemm;
  using E = Elem<DT>;
  constexpr int FA = Cfg<BN>::FA, FB = Cfg<BN>::FB, WAVES_N = Cfg<BN>::WAVES_N;
  constexpr int NMF = FA * FB;   // MFMA slots of one kk
  constexpr int TPR = THREADS / BN;  // threads per W row
  constexpr int KPT = BK / TPR;  // inputs of a thread per step
  constexpr int DW = KPT / 8;    // packed dwords of a thread per step
  static_assert(DW * 8 == 4 * NMF, "one packed dword of dequantization per 8 MFMA slots");
  __shared__ __attribute__((aligned(16))) uint16_t X0[BM * BK];
  __shared__ __attribute__((aligned(16))) uint16_t X1[BM * BK];
  __shared__ __attribute__((aligned(16))) uint16_t W0[BN * BK];
  __shared__ __attribute__((aligned(16))) uint16_t W1[BN * BK];
  __shared__ __attribute__((aligned(16))) uint16_t X2[BM * BK];
  LNQ_MFMA_IN_AGPRS();

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WAVES_N;
  const int wn = wave % WAVES_N;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  if (tm >= tiles_m || tn >= tiles_n) return;
  const int m0 = tm * BM;
  const int n0 = tn * BN;
  const int groups = K >> gshift;
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

  // x: load i (0..3) of wave w writes LDS rows 64 i + 8 w .. + 7 (1 KB, lane l
  // at byte 16 l: row 64 i + 8 w + l / 8, stored column l % 8). The stored
  // column holds source column (l % 8) ^ key(row); key = (row >> 1) & 7 =
  // (4 w + l / 16) & 7 does not depend on i. Each load's row offset is in its
  // lane offset and only the step's k offset in the uniform one, so rows past M
  // are out of range whether or not the uniform offset is range-checked.
  const int xrow = 8 * wave + (lane >> 3);
  const int xcol = (lane & 7) ^ ((xrow >> 1) & 7);
  constexpr int X_LOADS = 4;  // x loads (one buffer_load ... lds each) of a wave a step
  int xoff[X_LOADS];
#pragma unroll
  for (int i = 0; i < X_LOADS; ++i) xoff[i] = (m0 + xrow + 64 * i) * K * 2 + xcol * 16;
  const int xlds = wave * 512;  // elements
  auto load_x = [&](uint16_t* dst, __amdgpu_buffer_rsrc_t r, int k0, int i) {
    const int v = xoff[i];  // through a local: an array element passed directly drops the host launch stub
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)(dst + xlds + i * 64 * BK), 16, v, 2 * k0, 0, 0);
  };

  // W: thread -> row n0 + tid / TPR, KPT weights (KPT / 2 packed bytes) at k
  // offset KPT * (tid % TPR), within one group (G is a power of two >= 32).
  const int brow = tid / TPR;
  const int bpart = tid % TPR;
  const int nsrc = n0 + brow;
  const int woff = nsrc * (K >> 1) + bpart * (KPT / 2);
  const int soff = nsrc * groups * 2;
  const int zoff = nsrc * groups;
  struct WRegs {
    uint32_t w[DW];
    uint32_t s, z;
  };
  // Vector-memory instructions of one load_w (scale, zero, the packed words as
  // one b128 or b64): the step's wait counts them with the X_LOADS x loads.
  constexpr int W_LOADS = 3;
  auto load_w = [&](WRegs& r, int ks) {
    const bool in = ks < steps;
    const int k0 = in ? ks * BK : 0;
    const int g = (k0 + KPT * bpart) >> gshift;
    const __amdgpu_buffer_rsrc_t qs = in ? rs : rnull, qz = in ? rz : rnull, qw = in ? rw : rnull;
    r.s = static_cast<uint16_t>(__builtin_amdgcn_raw_buffer_load_b16(qs, soff + 2 * g, 0, 0));
    r.z = __builtin_amdgcn_raw_buffer_load_b8(qz, zoff + g, 0, 0);
    if constexpr (DW == 4) {
      const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(qw, woff, k0 >> 1, 0));
      r.w[0] = v.x;
      r.w[1] = v.y;
      r.w[2] = v.z;
      r.w[3] = v.w;
    } else {
      const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(qw, woff, k0 >> 1, 0));
      r.w[0] = v.x;
      r.w[1] = v.y;
    }
  };

  // The dequantization of one step's weights as a stream of 4 * NMF positions,
  // 8 per packed dword (8 weights -> one 16-byte column of row brow): (q - z) s
  // in f32 (exact), one rounding. The codes become f16 halves without a
  // conversion -- (0x6400 | q) is 1024 + q, (0x6400 | 16 q) is 1024 + 16 q --
  // and v_fma_mix_f32 (an f16 half times an f32) gives (1024 + q) s -
  // (1024 + z) s and (1024 + 16 q) (s / 16) - (64 + z) s, each exactly
  // (q - z) s: codes 0 and 4 from w & 0x000f000f, 1 and 5 from w & 0x00f000f0,
  // 2, 6 and 3, 7 the same of w >> 8; 17 instructions a dword (4 and-or, 1
  // shift, 8 FMAs, 4 packs), spread over its 8 positions.
  struct Deq {
    uint32_t m0, m1, m2, m3, t;
    float v[8];
    u32x4 o;
  };
  Deq q;
  // scale, -(1024 + zero) * scale, scale / 16, -(64 + zero) * scale
  float sv = 0.f, cv = 0.f, sv16 = 0.f, cv16 = 0.f;
  uint32_t mlo = 0x000f000fu, mhi = 0x00f000f0u, magic = 0x64006400u;
  hide_in_vgpr(mlo);
  hide_in_vgpr(mhi);
  hide_in_vgpr(magic);
  auto half_of = [](uint32_t m, int h) -> float { return static_cast<float>(__builtin_bit_cast(f16x2, m)[h]); };
  auto set_scale = [&](const WRegs& r) {
    sv = E::to_f32(static_cast<uint16_t>(r.s));
    const float z = static_cast<float>(r.z & 0xffu);
    cv = -(1024.f + z) * sv;
    sv16 = sv * 0.0625f;
    cv16 = -(64.f + z) * sv;
  };
  auto deq_slot = [&](const WRegs& r, int pos, uint16_t* dst) {
    const int d = pos >> 3;
    switch (pos & 7) {
      case 0: q.m0 = and_or(r.w[d], mlo, magic); q.t = r.w[d] >> 8; break;
      case 1: q.m1 = and_or(r.w[d], mhi, magic); q.v[0] = fmaf(half_of(q.m0, 0), sv, cv); break;
      case 2: q.v[4] = fmaf(half_of(q.m0, 1), sv, cv); q.v[1] = fmaf(half_of(q.m1, 0), sv16, cv16); break;
      case 3: q.v[5] = fmaf(half_of(q.m1, 1), sv16, cv16); q.o.x = pack2<DT>(q.v[0], q.v[1]); break;
      case 4: q.m2 = and_or(q.t, mlo, magic); q.m3 = and_or(q.t, mhi, magic); break;
      case 5:
        q.v[2] = fmaf(half_of(q.m2, 0), sv, cv);
        q.v[3] = fmaf(half_of(q.m3, 0), sv16, cv16);
        q.o.y = pack2<DT>(q.v[2], q.v[3]);
        break;
      case 6:
        q.v[6] = fmaf(half_of(q.m2, 1), sv, cv);
        q.v[7] = fmaf(half_of(q.m3, 1), sv16, cv16);
        q.o.z = pack2<DT>(q.v[4], q.v[5]);
        break;
      default:
        q.o.w = pack2<DT>(q.v[6], q.v[7]);
        *reinterpret_cast<u32x4*>(&dst[swz(brow, DW * bpart + d)]) = q.o;
        break;
    }
  };

  f32x16 acc[FA][FB];
#pragma unroll
  for (int a = 0; a < FA; ++a)
#pragma unroll
    for (int b = 0; b < FB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

  const int lrow = lane & 31;
  const int lk = lane >> 5;  // which 8 of an MFMA's 16 inputs
  // Operand byte offsets within a stage, per kk. The fragments of one kk are
  // 32 rows (4096 bytes) apart and share the swizzle key (row >> 1) & 7, so
  // one offset register per kk serves them all through the immediate field.
  uint32_t aoff[4], boff[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const uint32_t col = static_cast<uint32_t>(((2 * kk + lk) ^ ((lrow >> 1) & 7)) << 4);
    aoff[kk] = static_cast<uint32_t>((wm * FA * 32 + lrow) * 128) + col;
    boff[kk] = static_cast<uint32_t>((wn * FB * 32 + lrow) * 128) + col;
  }
  auto rd = [&](const uint16_t* stage, uint32_t off, int frag) -> u32x4 {
    return *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(stage) + off + frag * 4096);
  };
  // Operand fragments: f0 holds even kk, f1 odd kk; kk + 1's are read while
  // kk's MFMAs run.
  u32x4 af0[FA], bf0[FB], af1[FA], bf1[FB];

  // One kk: NMF MFMA slots on (ca, cb). The first FA + FB slots read the next
  // kk's operands from (rxs, rws); slot s also carries dequantization position
  // pos0 + s of `deq` (into wd) and the loads vm(s).
  auto region = [&](const u32x4* ca, const u32x4* cb, u32x4* na, u32x4* nb, const uint16_t* rxs,
                    const uint16_t* rws, int nkk, const WRegs& deq, uint16_t* wd, int pos0, auto&& vm) {
#pragma unroll
    for (int s = 0; s < NMF; ++s) {
      acc[s / FB][s % FB] = mfma32x32x16<DT>(cb[s % FB], ca[s / FB], acc[s / FB][s % FB]);
      if (s < FA) na[s] = rd(rxs, aoff[nkk], s);
      else if (s < FA + FB) nb[s - FA] = rd(rws, boff[nkk], s - FA);
      deq_slot(deq, pos0 + s, wd);
      vm(s);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Step ks: MFMAs on (xc, wc) with kk = 0 already in f0. Regions kk = 0..2
  // also DMA x of step ks + 2 into xn2, dequantize positions NMF.. of step
  // ks + 1's weights (registers d1) into wn, and request step ks + 3's weights
  // into req. After the barrier, kk = 3 reads step ks + 1's kk = 0 operands
  // from (xn1, wn) and starts step ks + 2's weights (registers d2) in wc,
  // which no wave reads any more.
  auto step = [&](int ks, const uint16_t* xc, const uint16_t* xn1, uint16_t* xn2, uint16_t* wc, uint16_t* wn,
                  const WRegs& d1, const WRegs& d2, WRegs& req) {
    const bool xin = ks + 2 < steps;
    const __amdgpu_buffer_rsrc_t xr = xin ? rx : rnull;
    const int xk0 = xin ? (ks + 2) * BK : 0;
    constexpr int XGAP = NMF / X_LOADS + 1;  // slots between the x loads
    auto vm = [&](int r, int s) {
      const int p = r * NMF + s;
      if (p == 1) load_w(req, ks + 3);
      if (p >= 3 && (p - 3) % XGAP == 0 && (p - 3) / XGAP < X_LOADS) load_x(xn2, xr, xk0, (p - 3) / XGAP);
    };
    region(af0, bf0, af1, bf1, xc, wc, 1, d1, wn, NMF, [&](int s) { vm(0, s); });
    region(af1, bf1, af0, bf0, xc, wc, 2, d1, wn, 2 * NMF, [&](int s) { vm(1, s); });
    region(af0, bf0, af1, bf1, xc, wc, 3, d1, wn, 3 * NMF, [&](int s) { vm(2, s); });
    // This wave's x of step ks + 1 has arrived once at most the loads issued
    // after it -- this step's load_w (W_LOADS instructions) and load_x calls
    // (X_LOADS, one instruction each) -- remain; its W stores are done at
    // lgkmcnt(0). Past the barrier every wave's are, and no wave reads step ks's
    // stages again.
    wait_vm<W_LOADS + X_LOADS>();
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    set_scale(d2);
    region(af1, bf1, af0, bf0, xn1, wn, 0, d2, wc, 0, [&](int) {});
  };

  // Prologue: registers of steps 0..2 requested, x of steps 0 and 1 DMA'd;
  // step 0's weights dequantized into W0 and the first NMF positions of step
  // 1's into W1 (where the steady state's last region would have put them).
  WRegs ra, rb, rc;
  load_w(ra, 0);
#pragma unroll
  for (int i = 0; i < X_LOADS; ++i) load_x(X0, rx, 0, i);
  load_w(rb, 1);
#pragma unroll
  for (int i = 0; i < X_LOADS; ++i) load_x(X1, steps > 1 ? rx : rnull, steps > 1 ? BK : 0, i);
  load_w(rc, 2);
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  set_scale(ra);
#pragma unroll
  for (int p = 0; p < 4 * NMF; ++p) deq_slot(ra, p, W0);
  set_scale(rb);
#pragma unroll
  for (int p = 0; p < NMF; ++p) deq_slot(rb, p, W1);
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int a = 0; a < FA; ++a) af0[a] = rd(X0, aoff[0], a);
#pragma unroll
  for (int b = 0; b < FB; ++b) bf0[b] = rd(W0, boff[0], b);

  // x of step j in X[j % 3]; W of step j in W[j % 2]; registers of step j in
  // (ra, rb, rc)[j % 3].
  int ks = 0;
  for (; ks + 6 <= steps; ks += 6) {
    step(ks + 0, X0, X1, X2, W0, W1, rb, rc, ra);
    step(ks + 1, X1, X2, X0, W1, W0, rc, ra, rb);
    step(ks + 2, X2, X0, X1, W0, W1, ra, rb, rc);
    step(ks + 3, X0, X1, X2, W1, W0, rb, rc, ra);
    step(ks + 4, X1, X2, X0, W0, W1, rc, ra, rb);
    step(ks + 5, X2, X0, X1, W1, W0, ra, rb, rc);
  }
  // The last steps % 6 steps continue the same stage sequence.
  const int rest = steps - ks;
  if (rest > 0) step(ks + 0, X0, X1, X2, W0, W1, rb, rc, ra);
  if (rest > 1) step(ks + 1, X1, X2, X0, W1, W0, rc, ra, rb);
  if (rest > 2) step(ks + 2, X2, X0, X1, W0, W1, ra, rb, rc);
  if (rest > 3) step(ks + 3, X0, X1, X2, W1, W0, rb, rc, ra);
  if (rest > 4) step(ks + 4, X1, X2, X0, W0, W1, rc, ra, rb);
  // Loads of the steps past the end (zeros through rnull) may be in flight.
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Epilogue. The MFMAs compute the transposed tile (W as the A operand): lane
  // l, register r holds token m = l % 32 and output feature 8 (r / 4) + 4 (l /
  // 32) + r % 4 of its 32x32 tile, so registers 4q..4q+3 are four consecutive
  // features of one row of y: one 8-byte store (N % 4 == 0), else four.
  const bool vec_out = (N & 3) == 0;
#pragma unroll
  for (int a = 0; a < FA; ++a) {
    const int m = m0 + wm * FA * 32 + a * 32 + (lane & 31);
    if (m >= M) continue;
    uint16_t* yrow = y + static_cast<size_t>(m) * N;
#pragma unroll
    for (int b = 0; b < FB; ++b) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int n = n0 + wn * FB * 32 + b * 32 + 8 * q4 + 4 * (lane >> 5);
        uint16_t out[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          out[i] = E::from_f32(acc[a][b][4 * q4 + i]);
          if (bias != nullptr && n + i < N) out[i] = E::from_f32(E::to_f32(out[i]) + E::to_f32(bias[n + i]));
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

// ------------------------------------------------- 128-column tiles: int4_narrow_kernel
namespace narrow {
constexpr int WAVES = 4;
constexpr int THREADS = 64 * WAVES;
constexpr int WB = 32;            // columns of W a wave owns
constexpr int BN = WAVES * WB;    // 128
constexpr int NS = 4;             // x stages
}  // namespace narrow

// BM: rows of x a tile (256, or 128 where 256-row tiles would leave more than
// half the CUs without one: twice the tiles, each a wave's weights dequantized
// for half the rows).
template <int DT, int BM = gemm::BM>
__global__ __launch_bounds__(narrow::THREADS, 1) void int4_narrow_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scale,
    const uint8_t* __restrict__ zero, const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int M, int N, int K,
    int gshift) {
  using namespace narrow;
  using gemm::BK;
  using E = Elem<DT>;
  constexpr int FA = BM / 32;     // row fragments of 32 (8 or 4)
  constexpr int XL = FA;          // x DMAs a wave issues a step (1 KB each)
  constexpr int LPS = 3 + XL;     // loads a wave issues a step: weights, scale, zero, x DMAs
  constexpr int PPS = 8 / FA;     // dequantization positions a slot runs
  static_assert(FA == 8 || FA == 4, "256- or 128-row tiles");
  __shared__ __attribute__((aligned(16))) uint16_t XS[NS * BM * BK];
  LNQ_MFMA_IN_AGPRS();

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  if (tm >= tiles_m || tn >= tiles_n) return;
  const int m0 = tm * BM;
  const int n0 = tn * BN;
  const int groups = K >> gshift;
  const int steps = K / BK;

  // Rows past M (and columns past N) read zeros through the buffer range check;
  // a step past the end reads through a 0-byte descriptor.
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(x, static_cast<uint32_t>(static_cast<size_t>(M) * K * 2));
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(packed, static_cast<uint32_t>(static_cast<size_t>(N) * (K >> 1)));
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(scale, static_cast<uint32_t>(N * groups * 2));
  const __amdgpu_buffer_rsrc_t rz = buffer_rsrc(zero, static_cast<uint32_t>(N * groups));
  const __amdgpu_buffer_rsrc_t rnull = buffer_rsrc(packed, 0);

  // x: DMA i (0..FA-1) of wave w writes rows 32 i + 8 w .. + 7 of a stage, in the
  // swizzled layout of int4_tiled_kernel (the key (row >> 1) & 7 = (4 w + l /
  // 16) & 7 does not depend on i); the row offsets in the lane offsets.
  const int xrow = 8 * wave + (lane >> 3);
  const int xcol = (lane & 7) ^ ((xrow >> 1) & 7);
  int xoff[FA];
#pragma unroll
  for (int i = 0; i < FA; ++i) xoff[i] = (m0 + xrow + 32 * i) * K * 2 + xcol * 16;
  auto load_x = [&](int stage, __amdgpu_buffer_rsrc_t r, int k0, int i) {
    const int v = xoff[i];  // through a local: an array element passed directly drops the host launch stub
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)(XS + stage * BM * BK + wave * 512 + i * 32 * BK), 16, v,
                                              2 * k0, 0, 0);
  };

  // W: lane -> column n0 + 32 wave + lane % 32; half h = lane / 32 reads input
  // blocks 4 h .. 4 h + 3 of a step (16 bytes), all in one group (G >= 32).
  const int h = lane >> 5;
  const int ncol = n0 + wave * WB + (lane & 31);
  const int woff = ncol * (K >> 1) + 16 * h;
  const int soff = ncol * groups * 2;
  const int zoff = ncol * groups;
  struct WRegs {
    u32x4 w;
    uint32_t s, z;
  };
  auto load_w = [&](WRegs& r, int ks) {
    const bool in = ks < steps;
    const int k0 = in ? ks * BK : 0;
    const int g = (k0 + 32 * h) >> gshift;
    const __amdgpu_buffer_rsrc_t qs = in ? rs : rnull, qz = in ? rz : rnull, qw = in ? rw : rnull;
    r.w = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(qw, woff, k0 >> 1, 0));
    r.s = static_cast<uint16_t>(__builtin_amdgcn_raw_buffer_load_b16(qs, soff + 2 * g, 0, 0));
    r.z = __builtin_amdgcn_raw_buffer_load_b8(qz, zoff + g, 0, 0);
  };

  // A dword's 8 codes dequantized into one operand fragment, as 8 positions of
  // about two VALU instructions: (q - z) * s in f32 (exact), one rounding to the
  // 16-bit type, as int4_tiled_kernel does. The codes become f16 halves without
  // a conversion: (0x6400 | q) is 1024 + q and (0x6400 | 16 q) is 1024 + 16 q,
  // both exact, so v_fma_mix_f32 (an f16 half of a register times an f32)
  // gives (1024 + q) s - (1024 + z) s and (1024 + 16 q) (s / 16) - (64 + z) s,
  // each exactly (q - z) s: codes 0 and 4 come from w & 0x000f000f, 1 and 5
  // from w & 0x00f000f0, 2, 6 and 3, 7 the same of w >> 8.
  struct Deq {
    uint32_t m0, m1, m2, m3, t;
    float v[8];
  };
  Deq q;
  float sv = 0.f, cv = 0.f, sv16 = 0.f, cv16 = 0.f;
  uint32_t mlo = 0x000f000fu, mhi = 0x00f000f0u, magic = 0x64006400u;
  hide_in_vgpr(mlo);
  hide_in_vgpr(mhi);
  hide_in_vgpr(magic);
  auto half_of = [](uint32_t m, int h) -> float {
    return static_cast<float>(__builtin_bit_cast(f16x2, m)[h]);
  };
  auto set_scale = [&](const WRegs& r) {
    sv = E::to_f32(static_cast<uint16_t>(r.s));
    const float z = static_cast<float>(r.z & 0xffu);
    cv = -(1024.f + z) * sv;
    sv16 = sv * 0.0625f;
    cv16 = -(64.f + z) * sv;
  };
  auto deq_slot = [&](uint32_t w, int pos, u32x4& o) {
    switch (pos) {
      case 0: q.m0 = and_or(w, mlo, magic); q.t = w >> 8; break;
      case 1: q.m1 = and_or(w, mhi, magic); q.v[0] = fmaf(half_of(q.m0, 0), sv, cv); break;
      case 2: q.v[4] = fmaf(half_of(q.m0, 1), sv, cv); q.v[1] = fmaf(half_of(q.m1, 0), sv16, cv16); break;
      case 3: q.v[5] = fmaf(half_of(q.m1, 1), sv16, cv16); o.x = pack2<DT>(q.v[0], q.v[1]); break;
      case 4: q.m2 = and_or(q.t, mlo, magic); q.m3 = and_or(q.t, mhi, magic); break;
      case 5:
        q.v[2] = fmaf(half_of(q.m2, 0), sv, cv);
        q.v[3] = fmaf(half_of(q.m3, 0), sv16, cv16);
        o.y = pack2<DT>(q.v[2], q.v[3]);
        break;
      case 6:
        q.v[6] = fmaf(half_of(q.m2, 1), sv, cv);
        q.v[7] = fmaf(half_of(q.m3, 1), sv16, cv16);
        o.z = pack2<DT>(q.v[4], q.v[5]);
        break;
      default: o.w = pack2<DT>(q.v[6], q.v[7]); break;
    }
  };

  f32x16 acc[FA];
#pragma unroll
  for (int a = 0; a < FA; ++a)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[a][r] = 0.f;

  // x operand of MFMA kk, fragment a: rows 32 a + lane % 32, input block kk + 4 h.
  // The fragments of one kk share the swizzle key: one offset register per kk.
  const int lrow = lane & 31;
  uint32_t aoff[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
    aoff[kk] = static_cast<uint32_t>(lrow * 128 + (((kk + 4 * h) ^ ((lrow >> 1) & 7)) << 4));
  auto rd = [&](int stage, int kk, int a) -> u32x4 {
    return *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(XS) + stage * BM * BK * 2 + aoff[kk] +
                                           a * 4096);
  };

  u32x4 a0[FA], a1[FA];
  u32x4 b0[4], b1[4];

  // Region kk: FA MFMA slots on (ca, bc[kk]); slot s reads the next x fragment
  // s, runs dequantization positions PPS s .. PPS s + PPS - 1 of dword kk of the
  // next step's weights (registers dn, into bn[kk]) and the loads vm(s). Each
  // slot is its own scheduling region, which pins the interleave.
  auto region = [&](int kk, const u32x4* ca, u32x4* na, int nstage, int nkk, const u32x4* bc, u32x4* bn,
                    const WRegs& dn, auto&& vm) {
#pragma unroll
    for (int s = 0; s < FA; ++s) {
      acc[s] = mfma32x32x16<DT>(bc[kk], ca[s], acc[s]);
      na[s] = rd(nstage, nkk, s);
#pragma unroll
      for (int q2 = 0; q2 < PPS; ++q2) deq_slot(dn.w[kk], PPS * s + q2, bn[kk]);
      vm(s);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Step ks: MFMAs on x stage ks % NS and B fragments bc (dequantized during
  // step ks - 1); dequantizes step ks + 1's weights (dn) into bn, requests step
  // ks + 4's weights into req (step ks's registers, no longer read) and DMAs x
  // of step ks + 3 into stage (ks + 3) % NS (step ks - 1's, which every wave
  // finished reading before the previous barrier).
  auto step = [&](int ks, int st, const u32x4* bc, u32x4* bn, const WRegs& dn, WRegs& req) {
    const bool xin = ks + 3 < steps;
    const __amdgpu_buffer_rsrc_t xr = xin ? rx : rnull;
    const int xk0 = xin ? (ks + 3) * BK : 0;
    const int xst = (st + 3) % NS;
    auto vm = [&](int r, int s) {
      if (r == 0 && s == 0) load_w(req, ks + 4);
      if (r < 2 && (s & 1)) load_x(xst, xr, xk0, (XL / 2) * r + s / 2);  // XL / 2 a region
    };
    set_scale(dn);
    region(0, a0, a1, st, 1, bc, bn, dn, [&](int s) { vm(0, s); });
    region(1, a1, a0, st, 2, bc, bn, dn, [&](int s) { vm(1, s); });
    region(2, a0, a1, st, 3, bc, bn, dn, [&](int s) { vm(2, s); });
    // This wave's x DMA of step ks + 1 (issued in step ks - 2) has landed once
    // at most the loads of steps ks - 1 and ks remain; past the barrier every
    // wave's has, and region 3 reads step ks + 1's first x fragments.
    wait_vm<2 * LPS>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    region(3, a1, a0, (st + 1) % NS, 0, bc, bn, dn, [&](int s) { vm(3, s); });
  };

  // Prologue: weights of steps 0..3 requested, x of steps 0..2 DMA'd, step 0's
  // weights dequantized into b0, its first x fragments read.
  WRegs w0, w1, w2, w3;
  load_w(w0, 0);
#pragma unroll
  for (int i = 0; i < XL; ++i) load_x(0, rx, 0, i);
  load_w(w1, 1);
#pragma unroll
  for (int i = 0; i < XL; ++i) load_x(1, steps > 1 ? rx : rnull, steps > 1 ? BK : 0, i);
  load_w(w2, 2);
#pragma unroll
  for (int i = 0; i < XL; ++i) load_x(2, steps > 2 ? rx : rnull, steps > 2 ? 2 * BK : 0, i);
  load_w(w3, 3);
  wait_vm<0>();
  set_scale(w0);
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
#pragma unroll
    for (int p = 0; p < 8; ++p) deq_slot(w0.w[kk], p, b0[kk]);
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int a = 0; a < FA; ++a) a0[a] = rd(0, 0, a);

  // Step j: x stage j % 4, weight registers (w0..w3)[j % 4], B fragments b0 / b1 by parity.
  int ks = 0;
  for (; ks + 4 <= steps; ks += 4) {
    step(ks + 0, 0, b0, b1, w1, w0);
    step(ks + 1, 1, b1, b0, w2, w1);
    step(ks + 2, 2, b0, b1, w3, w2);
    step(ks + 3, 3, b1, b0, w0, w3);
  }
  const int rest = steps - ks;
  if (rest > 0) step(ks + 0, 0, b0, b1, w1, w0);
  if (rest > 1) step(ks + 1, 1, b1, b0, w2, w1);
  if (rest > 2) step(ks + 2, 2, b0, b1, w3, w2);
  // Loads of the steps past the end (zeros through rnull) may be in flight.
  wait_vm<0>();

  // Epilogue: lane l, register r of fragment a holds token 32 a + l % 32 and
  // feature 8 (r / 4) + 4 h + r % 4 of the wave's 32 columns: registers 4q..4q+3
  // are four consecutive features of one row of y.
  const bool vec_out = (N & 3) == 0;
#pragma unroll
  for (int a = 0; a < FA; ++a) {
    const int m = m0 + a * 32 + (lane & 31);
    if (m >= M) continue;
    uint16_t* yrow = y + static_cast<size_t>(m) * N;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int n = n0 + wave * WB + 8 * q4 + 4 * h;
      uint16_t out[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        out[i] = E::from_f32(acc[a][4 * q4 + i]);
        if (bias != nullptr && n + i < N) out[i] = E::from_f32(E::to_f32(out[i]) + E::to_f32(bias[n + i]));
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

// ------------------------------------------- persistent 256 x 256 form: int4_persistent_kernel
// One workgroup per CU walks its 256 x 256 tiles (tile b, b + G, .. of the
// XCD-grouped order of tile_of, G workgroups); the k-steps of all its tiles
// form one stream, so the loads of the next tile's first steps are in flight
// while a tile finishes.
//
// 4 waves, one per SIMD, each owning 128 x 128 outputs (4 x 4 MFMA 32x32x16
// tiles, 256 accumulator registers): per MFMA a wave reads half the LDS bytes
// of int4_tiled_kernel's 128 x 64 waves -- about 96 LDS bytes a clock per CU
// with the weights' stores, against 128. 64 inputs a step, two stages of x
// (256 rows) and of dequantized weights (256 rows of the 16-bit type), each a
// 32 KB array of 128-byte rows with 16-byte columns XOR-swizzled by bits 1..3
// of the row (x and weights in separate arrays: the compiler then waits for x's
// loads only before reading x):
//   * x moves HBM/L2 -> LDS by buffer_load ... lds, 8 rows x 128 bytes an
//     instruction (whole lines), issued in step g's last kk for step g + 2;
//   * thread t owns weight row t of the tile: its 32 packed bytes, scale and
//     zero point of step g + 3 are requested in step g's first kk (four
//     register sets, steps unrolled by four), and step g + 1's are dequantized
//     ((q - z) * s in f32, exact, one rounding: every product is x * bf16(W) as
//     in the reference's dequant + BLAS path) and stored over step g's first
//     three kk;
//   * one barrier a step, before the last kk: past it every wave's x and
//     weights of step g + 1 are in LDS and no wave reads step g's stage again,
//     so the last kk reads step g + 1's first operands and refills step g's x.
// A tile's first step starts its accumulators from C = 0; after its last the
// waves round their outputs (and add the bias) and store them.
namespace gemmp {
constexpr int BM = 256, BN = 256, BK = 64, NW = 4, THREADS = 64 * NW;
constexpr int FA = 4, FB = 4;          // 32-row / 32-column fragments of a wave
constexpr int PART = BM * BK * 2;      // bytes of a stage's x (or weight) array
constexpr int XL = PART / 1024 / NW;   // x loads (1 KB) of a wave a step
constexpr int WL = 4;                  // weight, scale and zero loads of a thread a step
constexpr int U = 4;                   // steps a loop iteration (K % 256 == 0)
static_assert(XL == 8 && BM == BN && BN == THREADS, "one weight row a thread");
}  // namespace gemmp

template <int DT>
__global__ __launch_bounds__(gemmp::THREADS, 1) void int4_persistent_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scale,
    const uint8_t* __restrict__ zero, const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int M, int N, int K,
    int gshift) {
  using namespace gemmp;
  using E = Elem<DT>;
  constexpr int KK = BK / 16;  // MFMA 32x32x16 sub-steps a step
  __shared__ __attribute__((aligned(16))) uint8_t X0[PART];
  __shared__ __attribute__((aligned(16))) uint8_t X1[PART];
  __shared__ __attribute__((aligned(16))) uint8_t W0[PART];
  __shared__ __attribute__((aligned(16))) uint8_t W1[PART];
  LNQ_MFMA_IN_AGPRS();

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = N / BN;
  const int total = tiles_m * tiles_n;
  const int G = gridDim.x;
  const int b0 = blockIdx.x;
  if (b0 >= total) return;
  const int mine = (total - 1 - b0) / G + 1;  // tiles b0, b0 + G, ..
  const int steps = K / BK;                   // a multiple of U
  const int nsteps = mine * steps;
  const int groups = K >> gshift;

  // Rows past M read zeros through the range check (the row offset is in the
  // lane offset, only the step's k offset in the uniform one); steps past the
  // stream read through 0-byte descriptors (no traffic, the same count of loads).
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(x, static_cast<uint32_t>(static_cast<size_t>(M) * K * 2));
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(packed, static_cast<uint32_t>(static_cast<size_t>(N) * (K >> 1)));
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(scale, static_cast<uint32_t>(N * groups * 2));
  const __amdgpu_buffer_rsrc_t rz = buffer_rsrc(zero, static_cast<uint32_t>(N * groups));
  const __amdgpu_buffer_rsrc_t rnull = buffer_rsrc(packed, 0);

  // A tile's x lane offsets and weight row: x load i (0..7) of wave w fills x
  // rows 32 i + 8 w + l / 8 (1 KB, lane l at byte 16 l, stored column l % 8
  // holding source column (l % 8) ^ key(row), key = (row >> 1) & 7, the same
  // for every i); thread t reads weight row n0 + t.
  const int xr = 8 * wave + (lane >> 3);
  const int x_lane = xr * K * 2 + 16 * ((lane & 7) ^ ((xr >> 1) & 7));
  struct TileOff {
    uint32_t x[XL];
    int n;  // weight row of this thread
  };
  auto tile_off = [&](int r, TileOff& o) __attribute__((always_inline)) {
    int tm, tn;
    tile_of(b0 + r * G, tiles_m, tiles_n, tm, tn);
#pragma unroll
    for (int i = 0; i < XL; ++i) o.x[i] = static_cast<uint32_t>((tm * BM + 32 * i) * K * 2 + x_lane);
    o.n = tn * BN + tid;
  };
  auto load_x = [&](uint8_t* st, bool in, const TileOff& o, int ks, int i) __attribute__((always_inline)) {
    // The lane offset through a local: a structure member passed to the builtin
    // directly makes the host pass drop the kernel's launch stub.
    const __amdgpu_buffer_rsrc_t q = in ? rx : rnull;
    const uint32_t v = o.x[i];
    __builtin_amdgcn_raw_ptr_buffer_load_lds(q, (lds_ptr)(st + (4 * i + wave) * 1024), 16, v, in ? ks * BK * 2 : 0, 0,
                                              0);
  };
  struct WRegs {
    u32x4 w0, w1;  // 64 codes
    uint32_t s, z;
  };
  auto load_w = [&](WRegs& r, bool in, const TileOff& o, int ks) __attribute__((always_inline)) {
    const int g = (ks * BK) >> gshift;
    const __amdgpu_buffer_rsrc_t qw = in ? rw : rnull, qs = in ? rs : rnull, qz = in ? rz : rnull;
    const uint32_t wo = static_cast<uint32_t>(o.n * (K >> 1) + ks * (BK / 2));
    r.w0 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(qw, wo, 0, 0));
    r.w1 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(qw, wo + 16, 0, 0));
    r.s = static_cast<uint16_t>(
        __builtin_amdgcn_raw_buffer_load_b16(qs, static_cast<uint32_t>((o.n * groups + g) * 2), 0, 0));
    r.z = __builtin_amdgcn_raw_buffer_load_b8(qz, static_cast<uint32_t>(o.n * groups + g), 0, 0);
  };

  // Dequantization of a step's 8 packed dwords into row tid of a weight stage,
  // as 64 positions (8 a dword, 17 VALU instructions a dword): the codes become
  // f16 halves without a conversion ((0x6400 | q) is 1024 + q, (0x6400 | 16 q)
  // is 1024 + 16 q) and v_fma_mix_f32 gives (1024 + q) s - (1024 + z) s and
  // (1024 + 16 q) (s / 16) - (64 + z) s, each exactly (q - z) s; one rounding a
  // pair. Dword d holds codes 8 d .. 8 d + 7 of the step: 16-byte column d.
  uint32_t mlo = 0x000f000fu, mhi = 0x00f000f0u, magic = 0x64006400u;
  hide_in_vgpr(mlo);
  hide_in_vgpr(mhi);
  hide_in_vgpr(magic);
  auto half_of = [](uint32_t m, int h) __attribute__((always_inline)) -> float { return static_cast<float>(__builtin_bit_cast(f16x2, m)[h]); };
  struct Deq {
    uint32_t m0, m1, m2, m3, t;
    float v[8];
    u32x4 o;
    float sv, cv, sv16, cv16;
  };
  Deq q;
  const int wkey = (tid >> 1) & 7;
  auto deq_pos = [&](const WRegs& r, int pos, uint8_t* wst) __attribute__((always_inline)) {
    const int d = pos >> 3;
    const uint32_t w = d < 4 ? r.w0[d] : r.w1[d - 4];
    switch (pos & 7) {
      case 0:
        if (d == 0) {
          q.sv = E::to_f32(static_cast<uint16_t>(r.s));
          const float z = static_cast<float>(r.z & 0xffu);
          q.cv = -(1024.f + z) * q.sv;
          q.sv16 = q.sv * 0.0625f;
          q.cv16 = -(64.f + z) * q.sv;
        }
        q.m0 = and_or(w, mlo, magic);
        q.t = w >> 8;
        break;
      case 1: q.m1 = and_or(w, mhi, magic); q.v[0] = fmaf(half_of(q.m0, 0), q.sv, q.cv); break;
      case 2: q.v[4] = fmaf(half_of(q.m0, 1), q.sv, q.cv); q.v[1] = fmaf(half_of(q.m1, 0), q.sv16, q.cv16); break;
      case 3: q.v[5] = fmaf(half_of(q.m1, 1), q.sv16, q.cv16); q.o.x = pack2<DT>(q.v[0], q.v[1]); break;
      case 4: q.m2 = and_or(q.t, mlo, magic); q.m3 = and_or(q.t, mhi, magic); break;
      case 5:
        q.v[2] = fmaf(half_of(q.m2, 0), q.sv, q.cv);
        q.v[3] = fmaf(half_of(q.m3, 0), q.sv16, q.cv16);
        q.o.y = pack2<DT>(q.v[2], q.v[3]);
        break;
      case 6:
        q.v[6] = fmaf(half_of(q.m2, 1), q.sv, q.cv);
        q.v[7] = fmaf(half_of(q.m3, 1), q.sv16, q.cv16);
        q.o.z = pack2<DT>(q.v[4], q.v[5]);
        break;
      default:
        q.o.w = pack2<DT>(q.v[6], q.v[7]);
        *reinterpret_cast<u32x4*>(wst + tid * 128 + ((d ^ wkey) << 4)) = q.o;
        break;
    }
  };

  f32x16 acc[FA][FB];
  const int lrow = lane & 31, lk = lane >> 5;
  // Operand offsets within a stage array per kk: fragments 32 rows (4096 bytes)
  // apart with the same key.
  uint32_t aoff[KK], boff[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
    aoff[kk] = static_cast<uint32_t>((wm * 128 + lrow) * 128 + (((2 * kk + lk) ^ ((lrow >> 1) & 7)) << 4));
    boff[kk] = static_cast<uint32_t>((wn * 128 + lrow) * 128 + (((2 * kk + lk) ^ ((lrow >> 1) & 7)) << 4));
  }
  u32x4 af[2][FA], bf[2][FB];
  constexpr int NMF = FA * FB;
  constexpr int READS = FA + FB;
  auto read_one = [&](int set, const uint8_t* xs, const uint8_t* ws, int kk, int r) __attribute__((always_inline)) {
    if (r < FA) af[set][r] = *reinterpret_cast<const u32x4*>(xs + aoff[kk] + r * 4096);
    else bf[set][r - FA] = *reinterpret_cast<const u32x4*>(ws + boff[kk] + (r - FA) * 4096);
  };

  // The epilogue of tile (m0, n0): lane l, register r of fragment (a, b) holds
  // row m0 + 128 wm + 32 a + l % 32 and column n0 + 128 wn + 32 b + 8 (r / 4) + 4
  // (l / 32) + r % 4 (the weights are the MFMA's A operand).
  auto epilogue = [&](int m0, int n0) __attribute__((always_inline)) {
#pragma unroll
    for (int b = 0; b < FB; ++b) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int n = n0 + wn * 128 + b * 32 + 8 * q4 + 4 * lk;
        float bv[4] = {0.f, 0.f, 0.f, 0.f};
        if (bias != nullptr) {
          const u32x2 bb = *reinterpret_cast<const u32x2*>(bias + n);
          bv[0] = E::to_f32(static_cast<uint16_t>(bb.x & 0xffffu));
          bv[1] = E::to_f32(static_cast<uint16_t>(bb.x >> 16));
          bv[2] = E::to_f32(static_cast<uint16_t>(bb.y & 0xffffu));
          bv[3] = E::to_f32(static_cast<uint16_t>(bb.y >> 16));
        }
#pragma unroll
        for (int a = 0; a < FA; ++a) {
          const int m = m0 + wm * 128 + a * 32 + lrow;
          uint32_t o[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            uint16_t v = E::from_f32(acc[a][b][4 * q4 + i]);
            if (bias != nullptr) v = E::from_f32(E::to_f32(v) + bv[i]);
            o[i] = v;
          }
          if (m < M)
            *reinterpret_cast<u32x2*>(y + static_cast<size_t>(m) * N + n) =
                u32x2{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
        }
      }
      // One column fragment at a time: the next tile's operands are live here.
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Step g on stages (xc, wc), step g + 1's on (xn, wn_): kk 0..2 run MFMAs on kk
  // while kk + 1's operands are read, dequantize step g + 1's weights (dq) into
  // wn_ (64 positions over their 48 slots) and, in kk 0, request step g + 3's
  // weights (into req); then this wave's x loads of step g + 1 have landed (only
  // this step's WL weight loads were issued after them) and its LDS stores and
  // reads are done, the barrier, and kk 3 reads step g + 1's first operands
  // and issues step g + 2's x loads into xc, one every other slot.
  auto step = [&](auto first_tag, uint8_t* xc, uint8_t* wc, uint8_t* xn, uint8_t* wn_, const WRegs& dq, WRegs& req,
                  bool w_in, const TileOff& wo, int w_ks, bool x_in, const TileOff& xo, int x_ks) __attribute__((always_inline)) {
    constexpr bool FIRST = decltype(first_tag)::value;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const int set = kk & 1;
      const bool last = kk == KK - 1;
      if (last) {
        wait_vm<WL>();
        __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int sl = 0; sl < NMF; ++sl) {
        const int a = sl / FB, b = sl % FB;
        if (FIRST && kk == 0) acc[a][b] = mfma32x32x16<DT>(bf[set][b], af[set][a], f32x16{});
        else acc[a][b] = mfma32x32x16<DT>(bf[set][b], af[set][a], acc[a][b]);
        static_assert(2 * READS == NMF, "one operand read every other slot");
        if ((sl & 1) == 0) {
          if (last) read_one(set ^ 1, xn, wn_, 0, sl >> 1);
          else read_one(set ^ 1, xc, wc, kk + 1, sl >> 1);
        }
        if (!last) {
          const int p0 = (kk * 64) / 3, p1 = ((kk + 1) * 64) / 3;
#pragma unroll
          for (int p = p0 + (sl * (p1 - p0)) / NMF; p < p0 + ((sl + 1) * (p1 - p0)) / NMF; ++p) deq_pos(dq, p, wn_);
        }
        if (kk == 0 && sl == 0) load_w(req, w_in, wo, w_ks);
        if (last && (sl & 1)) load_x(xc, x_in, xo, x_ks, sl >> 1);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  // Prologue (tile 0; a tile has at least U steps): x of steps 0 and 1 and the
  // weights of steps 0..2 requested; step 0's weights dequantized into W0;
  // barrier; step 0's first operands read.
  TileOff oc, on;
  tile_off(0, oc);
  WRegs wr[4];
#pragma unroll
  for (int i = 0; i < XL; ++i) load_x(X0, true, oc, 0, i);
#pragma unroll
  for (int i = 0; i < XL; ++i) load_x(X1, true, oc, 1, i);
  load_w(wr[0], true, oc, 0);
  load_w(wr[1], true, oc, 1);
  load_w(wr[2], true, oc, 2);
  wait_vm<2 * WL>();
#pragma unroll
  for (int pos = 0; pos < 64; ++pos) deq_pos(wr[0], pos, W0);
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int r = 0; r < READS; ++r) read_one(0, X0, W0, 0, r);

  // Groups of U = 4 steps (a tile is whole groups): step g + s of tile r at
  // k-step ks + s, on stage (g + s) % 2, weight registers (g + s) % 4. Step g + s
  // requests the weights of step g + s + 3 and the x of step g + s + 2: of tile r
  // while they lie in this group, else of the next group's tile (r, or r + 1
  // after a tile's last group). No branch inside a group: the compiler would
  // otherwise move the MFMAs across the blocks it split the group into. A tile's
  // first group is its own copy (accumulators started at zero).
  using T = std::integral_constant<bool, true>;
  using F = std::integral_constant<bool, false>;
  int r = 0;
  auto group = [&](int g, int ks, auto first_tag) __attribute__((always_inline)) {
    const bool ends = ks + U == steps;
    const int kn = ends ? 0 : ks + U;
    tile_off(r + (ends ? 1 : 0), on);
    step(first_tag, X0, W0, X1, W1, wr[1], wr[3], g + 3 < nsteps, oc, ks + 3, g + 2 < nsteps, oc, ks + 2);
    step(F{}, X1, W1, X0, W0, wr[2], wr[0], g + 4 < nsteps, on, kn, g + 3 < nsteps, oc, ks + 3);
    step(F{}, X0, W0, X1, W1, wr[3], wr[1], g + 5 < nsteps, on, kn + 1, g + 4 < nsteps, on, kn);
    step(F{}, X1, W1, X0, W0, wr[0], wr[2], g + 6 < nsteps, on, kn + 2, g + 5 < nsteps, on, kn + 1);
    oc = on;
  };
  int g = 0;
  for (; r < mine; ++r) {
    group(g, 0, T{});
    g += U;
    for (int ks = U; ks < steps; ks += U, g += U) group(g, ks, F{});
    int tm, tn;
    tile_of(b0 + r * G, tiles_m, tiles_n, tm, tn);
    epilogue(tm * BM, tn * BN);
  }
  // Loads of the steps past the stream (0-byte reads) may be in flight.
  wait_vm<0>();
}

bool int4_persistent_supports(int M, int N, int K, int G, int dtype) {
  // 256-column tiles (N % 256), groups of 4 steps of 64 inputs (K % 256), a step
  // within one group (G a multiple of 64), 32-bit buffer offsets.
  return (dtype == LNQ_BF16 || dtype == LNQ_F16) && M > 0 && N > 0 && N % gemmp::BN == 0 && K > 0 && K % 256 == 0 &&
         G >= 64 && G % 64 == 0 && (G & (G - 1)) == 0 && K % G == 0 && static_cast<size_t>(M) * K * 2 < (1ull << 31) &&
         static_cast<size_t>(N) * (K >> 1) < (1ull << 31);
}

bool int4_tiled_supports(int M, int N, int K, int G, int dtype) {
  // Buffer offsets are 32-bit: x and the packed weight stay under 2 GiB. A
  // thread's 16 or 32 weights of a step lie in one group: G is a power of two
  // of at least 32.
  return (dtype == LNQ_BF16 || dtype == LNQ_F16) && M > 0 && N > 0 && K % gemm::BK == 0 && K >= gemm::BK &&
         G >= 32 && (G & (G - 1)) == 0 && K % G == 0 && static_cast<size_t>(M) * K * 2 < (1ull << 31) &&
         static_cast<size_t>(N) * (K >> 1) < (1ull << 31);
}



template <int DT>
static void launch_tiled(const void* x, const uint8_t* packed, const void* scale, const uint8_t* zero,
                         const void* bias, void* y, int M, int N, int K, int gshift, bool wide, hipStream_t stream) {
  const int bn = wide ? 256 : narrow::BN;
  const int tiles = ((M + gemm::BM - 1) / gemm::BM) * ((N + bn - 1) / bn);
  const auto* xs = static_cast<const uint16_t*>(x);
  const auto* ss = static_cast<const uint16_t*>(scale);
  const auto* bs = static_cast<const uint16_t*>(bias);
  auto* ys = static_cast<uint16_t*>(y);
  if (wide)
    hipLaunchKernelGGL((int4_tiled_kernel<DT, 256>), dim3(tiles), dim3(gemm::THREADS), 0, stream, xs, packed, ss, zero,
                       bs, ys, M, N, K, gshift);
  else if (2 * tiles <= compute_units())
    // 256-row tiles would leave more than half the CUs idle: 128-row ones.
    hipLaunchKernelGGL((int4_narrow_kernel<DT, 128>), dim3(((M + 127) / 128) * ((N + bn - 1) / bn)),
                       dim3(narrow::THREADS), 0, stream, xs, packed, ss, zero, bs, ys, M, N, K, gshift);
  else
    hipLaunchKernelGGL((int4_narrow_kernel<DT>), dim3(tiles), dim3(narrow::THREADS), 0, stream, xs, packed, ss, zero,
                       bs, ys, M, N, K, gshift);
}

// Whether the persistent form takes the shape and has more 256 x 256 tiles than
// there are CUs (with one tile a workgroup it has no next tile to prefetch and
// the 8-wave tiled kernel is ahead).
bool int4_persistent_preferred(int M, int N, int K, int G, int dtype) {
  const long tiles = static_cast<long>((M + gemmp::BM - 1) / gemmp::BM) * ((N + gemmp::BN - 1) / gemmp::BN);
  return tiles > compute_units() && int4_persistent_supports(M, N, K, G, dtype);
}

// 256-column tiles read half the x bytes per FLOP of 128-column ones, but only
// pay while they still give nearly every compute unit a tile.
int int4_tiled_width(int M, int N) {
  // 256-column tiles once they fill at least 7/8 of the CUs: at M = 1024, N =
  // 14336 (224 tiles on 256 CUs) they take 114 us against 124 us for 448 tiles
  // of 256 x 128; at 128 tiles (N = 4096, M = 2048) the 128-column ones win (72
  // against 97 us).
  const long tiles256 = static_cast<long>((M + gemm::BM - 1) / gemm::BM) * ((N + 255) / 256);
  return 8 * tiles256 >= 7L * compute_units() ? 256 : 128;
}

LnqStatus launch_int4_persistent(const void* x, const uint8_t* packed, const void* scale, const uint8_t* zero,
                                 const void* bias, void* y, int M, int N, int K, int G, int dtype, hipStream_t stream) {
  const int gshift = __builtin_ctz(static_cast<unsigned>(G));
  const int tiles = ((M + gemmp::BM - 1) / gemmp::BM) * (N / gemmp::BN);
  const dim3 grid(tiles < compute_units() ? tiles : compute_units());
  const auto* xs = static_cast<const uint16_t*>(x);
  const auto* ss = static_cast<const uint16_t*>(scale);
  const auto* bs = static_cast<const uint16_t*>(bias);
  auto* ys = static_cast<uint16_t*>(y);
  if (dtype == LNQ_BF16)
    hipLaunchKernelGGL((int4_persistent_kernel<LNQ_BF16>), grid, dim3(gemmp::THREADS), 0, stream, xs, packed, ss, zero,
                       bs, ys, M, N, K, gshift);
  else
    hipLaunchKernelGGL((int4_persistent_kernel<LNQ_F16>), grid, dim3(gemmp::THREADS), 0, stream, xs, packed, ss, zero,
                       bs, ys, M, N, K, gshift);
  return launched("int4_persistent");
}

LnqStatus launch_int4_tiled(const void* x, const uint8_t* packed, const void* scale, const uint8_t* zero,
                            const void* bias, void* y, int M, int N, int K, int G, int dtype, int bn,
                            hipStream_t stream) {
  const int gshift = __builtin_ctz(static_cast<unsigned>(G));
  const bool wide = bn == 256;
  if (dtype == LNQ_BF16) launch_tiled<LNQ_BF16>(x, packed, scale, zero, bias, y, M, N, K, gshift, wide, stream);
  else launch_tiled<LNQ_F16>(x, packed, scale, zero, bias, y, M, N, K, gshift, wide, stream);
  return launched("int4_tiled");
}

}  // namespace lnq
