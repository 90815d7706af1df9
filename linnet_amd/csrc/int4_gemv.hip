// The one-token (M == 1) int4 group-wise dequant-GEMV on gfx950: y = x @ W^T,
// W[n, k] = (q[n, k] - z[n, k/G]) * s[n, k/G], the decode shape of
// std.quant::linear_int4_groups (stdlib/quant.linnet:132-140) as the reference
// launches it per token (linnet/torch/kernels.py:212-323; tinygemm below 8 rows).
//
// The path is bound by HBM: every packed byte is read once. The kernel is
// shaped around what one launch of ~30 MB can reach on MI355X:
//
// * Exact balance: one workgroup per CU. N rows are split into R = 8 * U8 rows
//   per workgroup with U8 = ceil(N / 2048) (14336 rows: 56 each, 256
//   workgroups), so every CU streams the same bytes.
// * Wide, contiguous weight reads: each wave owns R rows x 256 inputs; its
//   weights move HBM -> LDS with buffer_load ... lds, one instruction per
//   8 rows x 128 contiguous bytes (reads of 16 rows x 64 bytes, the footprint a
//   register load in MFMA operand order would have, stream ~20% slower). The
//   16-byte piece each lane fetches is chosen so that the reads in MFMA operand
//   order hit 16 distinct bank groups.
// * Few memory instructions per CU: a wave issues one x load, U8 weight loads
//   and one scale and one zero load, about 160 per CU for 14336 x 4096.
// * x first: each wave's slice of x is loaded first, staged in its own LDS
//   array (a separate array, so the compiler can see the weight loads do not
//   touch it and adds no wait for them) and turned into MFMA A operands; each
//   8-row pair of loads is multiplied as soon as it lands (explicit vmcnt
//   waits; loads retire in order).
// * Zero point and scale at the end: per tile and 128-input half the MFMA sums
//   C = sum x * (MAGIC + q) ((MAGIC | q) read as bf16 is 128 + q, f16 1024 + q)
//   and the wave folds acc = s * (C - (MAGIC + z) * sum x) after its scale and
//   zero loads (issued last) arrive; one barrier, then the 16 waves' partial
//   sums are added in a fixed order.
// * An odd U8 leaves a last tile of 8 rows: its two 128-input halves run as
//   one MFMA chain, half 0 in A row 0 / B columns 0-7 and half 1 in A row 1 /
//   B columns 8-15 (only row 0 of A carries x otherwise).
// * Inputs in another order (ORD: GPTQ's activation order, take_inputs of
//   stdlib/quant.linnet:142-149 ahead of the product, group 128): the packed
//   row's k-th weight is input order[k]'s. Each lane loads its 8 entries of
//   order with its x slice (before the weights, so nothing waits twice); once
//   they land, the workgroup's x slices sit in LDS in input order, each lane
//   reads x[order[k]] for its 8 k, and the taken slice continues as x does
//   above. The gather costs two LDS barriers and no extra HBM round trip.
// * The decode glue ahead of a projection, folded into the x staging (PRO,
//   bf16, group 128), so that it costs no launch of its own. RMSNorm: the
//   per-row factor r = rsqrt(mean(x^2) + eps) is a scalar of the one row, so
//   y = r * (W (x * w)): each wave loads its 256 norm weights with its x slice
//   and stages x * w (rounded to bf16) as x; the squares of its raw slice are
//   summed after its tiles, the waves' sums meet in LDS at the final barrier
//   (added in a fixed order) and r scales the output sums. Nothing of the norm
//   stands between x landing and the first MFMA; the staged values differ from
//   lnq_rmsnorm's x * r * w rounded to bf16 by that rounding. SiLU(g) * u: each
//   wave loads its u slice beside g; lanes l and l + 32 hold the same chunk, so
//   each half computes half of it and they exchange (the bits of lnq_silu_mul).
#include <type_traits>

#include "common.hpp"

namespace lnq {

namespace gemv {
// What x the one-token kernels multiply: x itself; RMSNorm(x) with weights
// pro.w and pro.eps (x * w staged, the row's factor applied to the sums);
// SiLU(x) * pro.u rounded to bf16.
enum { PRO_NONE = 0, PRO_NORM = 1, PRO_SILU = 2 };
constexpr int MAX_WAVES = 16;  // K <= 4096
constexpr int MAX_U8 = 8;      // R <= 64 rows per workgroup
constexpr int MAX_ROWS = 32;   // tokens of one few-token launch

// Weight tile T (loads 2T and 2T + 1, 1 KB each per wave) has an LDS array of
// its own. The compiler tracks buffer_load ... lds writes per LDS variable, so a
// tile's reads wait for that tile's two loads only; with one array for all
// loads it waits for every load before the first tile. Per-wave bytes of tile
// T, and the array's bytes (a 16-byte placeholder past the last tile):
constexpr int tile_wave_bytes(int u8, int t) { return 2 * t + 1 < u8 ? 2048 : 1024; }
constexpr int tile_bytes(int u8, int t) { return 2 * t < u8 ? tile_wave_bytes(u8, t) * MAX_WAVES : 16; }

// The 32-row kernel also takes 128 and 256 rows a workgroup (U8 = 16, 32; split
// K only), with at most wmax(U8) waves: 128 KB of weight tiles in all. Its
// tiles sit in four LDS arrays, tiles_per_array(U8) consecutive tiles each
// (one tile an array up to U8 = 8, the layout above).
constexpr int wmax(int u8) { return u8 <= 8 ? MAX_WAVES : 128 / u8; }
constexpr int tiles_per_array(int u8) { return ((u8 + 1) / 2 + 3) / 4; }
constexpr int array_wave_bytes(int u8, int a) {
  int bytes = 0;
  for (int t = a * tiles_per_array(u8); t < (a + 1) * tiles_per_array(u8) && 2 * t < u8; ++t)
    bytes += tile_wave_bytes(u8, t);
  return bytes;
}
constexpr int array_bytes(int u8, int a) { return array_wave_bytes(u8, a) > 0 ? array_wave_bytes(u8, a) * wmax(u8) : 16; }
}  // namespace gemv

// The prologue's operands (PRO_NORM: w, eps; PRO_SILU: u), by value.
struct GemvPrologue {
  const float* w;
  const uint16_t* u;
  float eps;
};

// The tile arrays of a kernel with U8 loads, and tile_lds(T, wave): wave's part
// of tile T (T a constant after unrolling).
#define LNQ_GEMV_TILE_ARRAYS(U8)                                                             \
  __shared__ __attribute__((aligned(16))) uint8_t L0[gemv::tile_bytes(U8, 0)];              \
  __shared__ __attribute__((aligned(16))) uint8_t L1[gemv::tile_bytes(U8, 1)];              \
  __shared__ __attribute__((aligned(16))) uint8_t L2[gemv::tile_bytes(U8, 2)];              \
  __shared__ __attribute__((aligned(16))) uint8_t L3[gemv::tile_bytes(U8, 3)];              \
  static_assert(U8 <= 8, "four tile arrays");                                                \
  auto tile_lds = [&](int T, int w) -> uint8_t* {                                            \
    uint8_t* base = T == 0 ? L0 : T == 1 ? L1 : T == 2 ? L2 : L3;                            \
    return base + w * gemv::tile_wave_bytes(U8, T);                                          \
  }

// The tile arrays of the 32-row kernel (four arrays of tiles_per_array(U8)
// tiles), and tile_lds(T, wave) as above.
#define LNQ_GEMV_TILE_GROUPS(U8)                                                                  \
  __shared__ __attribute__((aligned(16))) uint8_t L0[gemv::array_bytes(U8, 0)];                  \
  __shared__ __attribute__((aligned(16))) uint8_t L1[gemv::array_bytes(U8, 1)];                  \
  __shared__ __attribute__((aligned(16))) uint8_t L2[gemv::array_bytes(U8, 2)];                  \
  __shared__ __attribute__((aligned(16))) uint8_t L3[gemv::array_bytes(U8, 3)];                  \
  static_assert(U8 <= 8 || U8 % 8 == 0, "whole arrays past U8 = 8");                               \
  auto tile_lds = [&](int T, int w) -> uint8_t* {                                                 \
    constexpr int P = gemv::tiles_per_array(U8);                                                  \
    const int g = T / P;                                                                          \
    uint8_t* base = g == 0 ? L0 : g == 1 ? L1 : g == 2 ? L2 : L3;                                 \
    const int wb = g == 0 ? gemv::array_wave_bytes(U8, 0) : g == 1 ? gemv::array_wave_bytes(U8, 1) \
                 : g == 2 ? gemv::array_wave_bytes(U8, 2) : gemv::array_wave_bytes(U8, 3);        \
    return base + w * wb + (T % P) * 2048;                                                        \
  }

// The widened B operands of two packed dwords (16 codes): (MAGIC | q) pairs in
// pair order (dword s holds elements s and s + 4 of its 8). The three shifts of
// each dword are shared between the two as 64-bit funnel shifts; bits shifted
// in from the high dword land outside the 0x000f000f mask.
template <int DT>
__device__ inline void widen_pair(uint32_t lo, uint32_t hi, uint32_t mask, uint32_t magic, u32x4& b0, u32x4& b1) {
  const uint64_t v = (static_cast<uint64_t>(hi) << 32) | lo;
  const uint64_t v4 = v >> 4, v8 = v >> 8, v12 = v >> 12;
  b0 = u32x4{and_or(lo, mask, magic), and_or(static_cast<uint32_t>(v4), mask, magic),
             and_or(static_cast<uint32_t>(v8), mask, magic), and_or(static_cast<uint32_t>(v12), mask, magic)};
  b1 = u32x4{and_or(hi, mask, magic), and_or(static_cast<uint32_t>(v4 >> 32), mask, magic),
             and_or(static_cast<uint32_t>(v8 >> 32), mask, magic), and_or(static_cast<uint32_t>(v12 >> 32), mask, magic)};
}

// Workgroup: NW = K / 256 waves, R = 8 * U8 rows. G128: group 128 (a wave's two
// halves have consecutive groups, scales loaded as one dword); otherwise G is
// a multiple of 256 (both halves share one group).
template <int DT, int U8, bool G128, bool ORD = false, int PRO = gemv::PRO_NONE>
__global__ __launch_bounds__(64 * gemv::MAX_WAVES) void int4_gemv_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ packed,
    const uint16_t* __restrict__ scale, const uint8_t* __restrict__ zero,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int N, int K, int G,
    const int32_t* __restrict__ order, GemvPrologue pro) {
  using E = Elem<DT>;
  static_assert(!ORD || G128, "inputs in another order: group 128");
  static_assert(PRO == gemv::PRO_NONE || (DT == LNQ_BF16 && G128 && !ORD), "prologues: bf16, group 128, no order");
  constexpr int R = 8 * U8;
  constexpr int NF = U8 / 2;            // full 16-row tiles
  constexpr bool HALF = (U8 & 1) != 0;  // a last tile of 8 rows
  LNQ_GEMV_TILE_ARRAYS(U8);
  __shared__ __attribute__((aligned(16))) uint16_t Xsm[gemv::MAX_WAVES][256];
  __shared__ float Rsm[gemv::MAX_WAVES][R];  // wave-major: consecutive lanes, consecutive dwords
  __shared__ float Nsm[PRO == gemv::PRO_NORM ? gemv::MAX_WAVES : 1];  // each wave's sum of squares

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  const int col = lane & 15, j = lane >> 4;
  const int n0 = blockIdx.x * R;
  const int k0 = wave * 256;
  const int rowb = K >> 1;
  const int groups = K / G;
  uint16_t* Xw = Xsm[wave];
  // Buffer descriptors: rows past N read zeros through the range check.
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(packed, static_cast<uint32_t>(static_cast<size_t>(N) * rowb));
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(x, static_cast<uint32_t>(K * 2));
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(scale, static_cast<uint32_t>(N * groups * 2));
  const __amdgpu_buffer_rsrc_t rz = buffer_rsrc(zero, static_cast<uint32_t>(N * groups));

  // ---- loads: scales, zeros, x slice (lanes 0..31, 8 inputs each), weights.
  // The scale and zero loads go first: scattered (a row per lane) and needed only
  // at the end, they would otherwise return after all the weights.
  // Lane r < R: row n0 + r's scales and zero points of this wave's groups.
  const int srow = n0 + (lane < R ? lane : R - 1);
  const int g0 = k0 / G;
  uint32_t sv;
  uint16_t zv16;
  if constexpr (G128) {
    sv = __builtin_amdgcn_raw_buffer_load_b32(rs, (srow * groups + g0) * 2, 0, 0);  // s[g0] | s[g0 + 1] << 16
    zv16 = __builtin_amdgcn_raw_buffer_load_b16(rz, srow * groups + g0, 0, 0);      // z[g0] | z[g0 + 1] << 8
  } else {
    sv = __builtin_amdgcn_raw_buffer_load_b16(rs, (srow * groups + g0) * 2, 0, 0);
    zv16 = __builtin_amdgcn_raw_buffer_load_b8(rz, srow * groups + g0, 0, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
  u32x4 xv = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, (k0 + 8 * (lane & 31)) * 2, 0, 0));
  u32x4 ov0{}, ov1{};  // ORD: order[k0 + 8 (lane & 31) ...], 8 entries
  if constexpr (ORD) {
    const __amdgpu_buffer_rsrc_t ro = buffer_rsrc(order, static_cast<uint32_t>(K * 4));
    const int ob = (k0 + 8 * (lane & 31)) * 4;
    ov0 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ro, ob, 0, 0));
    ov1 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ro, ob + 16, 0, 0));
  }
  u32x4 pv0{}, pv1{};  // PRO: the norm's 8 f32 weights of the lane's x, or its 8 values of u
  if constexpr (PRO == gemv::PRO_NORM) {
    const __amdgpu_buffer_rsrc_t rp = buffer_rsrc(pro.w, static_cast<uint32_t>(K * 4));
    const int pb = (k0 + 8 * (lane & 31)) * 4;
    pv0 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, pb, 0, 0));
    pv1 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, pb + 16, 0, 0));
  } else if constexpr (PRO == gemv::PRO_SILU) {
    const __amdgpu_buffer_rsrc_t ru = buffer_rsrc(pro.u, static_cast<uint32_t>(K * 2));
    pv0 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ru, (k0 + 8 * (lane & 31)) * 2, 0, 0));
  }
  __builtin_amdgcn_sched_barrier(0);
  // Every wave's small loads enter the CU's memory pipeline before any weight
  // load: without this barrier the waves that reach their first load last find
  // it queued behind the other waves' weights (~100 KB), their x and scales land
  // late and their tiles are all multiplied after the stream has ended.
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  // Load u: rows n0 + 8u + (lane & 7) at 16-byte piece sigma of the wave's 128
  // bytes; sigma = 2 (lane / 16) + ((lane / 8) % 2 ^ u % 2) puts piece sigma of
  // row r at LDS slot 16 (sigma / 2) + 8 (sigma % 2 ^ u % 2) + r.
  auto load_weights = [&](int u) {
    const int a = lane >> 4, b = lane & 15;
    const int sigma = 2 * a + ((b >> 3) ^ (u & 1));
    const int row = n0 + 8 * u + (b & 7);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr)(tile_lds(u >> 1, wave) + 1024 * (u & 1)), 16,
                                             row * rowb + (k0 >> 1) + 16 * sigma, 0, 0, 2 /* non-temporal */);
  };
  // With an input order the gather needs every wave's x: only PRE loads go out
  // before it, so that no wave reaches its barrier late behind a queue of its
  // own weight loads; the rest follow the gather (loads still retire in issue
  // order, so the counts of the waits below are unchanged).
  constexpr int PRE = ORD && U8 > 4 ? 4 : U8;
#pragma unroll
  for (int u = 0; u < PRE; ++u) load_weights(u);
  __builtin_amdgcn_sched_barrier(0);

  // ---- x: wait for it (and the scales), stage it in pair order, sums of both halves.
  wait_vm<PRE>();
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (ORD) {
    // The workgroup's x in input order (Xsm holds exactly K values), then each
    // lane's 8 taken inputs; the second barrier keeps Xsm until all have read it.
    // Lanes 32..63 store the same values as lanes 0..31: a store under a lane
    // condition would let the compiler sink the x load into it, behind the weights.
    *reinterpret_cast<u32x4*>(Xw + 8 * (lane & 31)) = xv;
    lds_barrier();
    xv = gather_x8(&Xsm[0][0], ov0, ov1, static_cast<uint32_t>(K));
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = PRE; u < U8; ++u) load_weights(u);
    __builtin_amdgcn_sched_barrier(0);
  }
  const u32x4 xraw = xv;  // NORM: the raw slice, its squares summed after the tiles
  if constexpr (PRO == gemv::PRO_NORM) {
    xv = scale_bf16x8(xv, __builtin_bit_cast(f32x4, pv0), __builtin_bit_cast(f32x4, pv1));
  } else if constexpr (PRO == gemv::PRO_SILU) {
    xv = silu_mul_bf16x8_halves(xv, pv0, lane);
  }
  if (lane < 32) *reinterpret_cast<u32x4*>(Xw + 8 * lane) = permute_x8(xv);
  float sum = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t d = xv[e];
    sum += E::to_f32(static_cast<uint16_t>(d & 0xffffu)) + E::to_f32(static_cast<uint16_t>(d >> 16));
  }
  sum += __shfl_xor(sum, 1, 64);
  sum += __shfl_xor(sum, 2, 64);
  sum += __shfl_xor(sum, 4, 64);
  sum += __shfl_xor(sum, 8, 64);
  const float xs0 = __shfl(sum, 0, 64), xs1 = __shfl(sum, 16, 64);
  // A operands: half H, MFMA t of lane (., j) = x[k0 + 128 H + 32 j + 8 t ..] (pair
  // order); ac: the 8-row tile's, half 1 in A row 1 (lanes col == 1).
  u32x4 xa[2][4], ac[4];
#pragma unroll
  for (int H = 0; H < 2; ++H)
#pragma unroll
    for (int t = 0; t < 4; ++t) xa[H][t] = *reinterpret_cast<const u32x4*>(Xw + 128 * H + 32 * j + 8 * t);
#pragma unroll
  for (int t = 0; t < 4; ++t) ac[t] = *reinterpret_cast<const u32x4*>(Xw + (col == 1 ? 128 : 0) + 32 * j + 8 * t);
  __builtin_amdgcn_sched_barrier(0);

  uint32_t nib_mask = 0x000f000fu, nib_magic = E::MAGIC2;
  hide_in_vgpr(nib_mask);
  hide_in_vgpr(nib_magic);
  const int r7 = col & 7;
  // One MFMA chain over a lane's 16 bytes of weights; returns output register
  // `reg`.
  auto chain = [&](const u32x4 (&a)[4], const u32x4 w, int reg) -> float {
    u32x4 b0, b1, b2, b3;
    widen_pair<DT>(w.x, w.y, nib_mask, nib_magic, b0, b1);
    widen_pair<DT>(w.z, w.w, nib_mask, nib_magic, b2, b3);
    f32x4 C = f32x4{0.f, 0.f, 0.f, 0.f};
    C = mfma16x16x32<DT>(a[0], b0, C);
    C = mfma16x16x32<DT>(a[1], b1, C);
    C = mfma16x16x32<DT>(a[2], b2, C);
    C = mfma16x16x32<DT>(a[3], b3, C);
    return reg == 0 ? C[0] : C[1];
  };
  // ---- scales and zero points of each tile's rows (landed with x), so that a
  // tile's fold follows its MFMAs at once: acc = s0 (C0 - z0 xs0) + s1 (C1 - z1 xs1).
  uint32_t zv = zv16;
  if constexpr (!G128) {
    sv = (sv & 0xffffu) | (sv << 16);
    zv = (zv & 0xffu) | (zv << 8);
  }
  float fs0[NF + 1], fs1[NF + 1], fz0[NF + 1], fz1[NF + 1];
#pragma unroll
  for (int T = 0; T <= NF; ++T) {
    if (T == NF && !HALF) break;
    const int n = T < NF ? 8 * (2 * T + (col >> 3)) + r7 : 8 * (U8 - 1) + r7;  // the lane's output row
    const uint32_t sp = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(4 * n, static_cast<int>(sv)));
    const uint32_t zp = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(4 * n, static_cast<int>(zv)));
    fs0[T] = E::to_f32(static_cast<uint16_t>(sp & 0xffffu));
    fs1[T] = E::to_f32(static_cast<uint16_t>(sp >> 16));
    fz0[T] = -(E::MAGIC_VALUE + static_cast<float>(zp & 0xffu));
    fz1[T] = -(E::MAGIC_VALUE + static_cast<float>((zp >> 8) & 0xffu));
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- tiles as their loads land, each folded and stored for the cross-wave sum.
#pragma unroll
  for (int T = 0; T < NF; ++T) {
    // No LDS load below may be issued before the previous tile's MFMAs have read
    // their operands: the fences keep each tile's reads after the prior tile.
    __builtin_amdgcn_sched_barrier(0);
    wait_vm_rt(U8 - 1 - (2 * T + 1));
    __builtin_amdgcn_sched_barrier(0);
    const int h = col >> 3;
    const int p0 = 16 * (j >> 1) + 8 * ((j & 1) ^ h) + r7;        // piece j      (half 0)
    const int p1 = 16 * (2 + (j >> 1)) + 8 * ((j & 1) ^ h) + r7;  // piece 4 + j  (half 1)
    const uint8_t* Wt = tile_lds(T, wave) + 1024 * h;  // load 2 T + h
    const u32x4 w0 = *reinterpret_cast<const u32x4*>(Wt + 16 * p0);
    const u32x4 w1 = *reinterpret_cast<const u32x4*>(Wt + 16 * p1);
    const float c0 = chain(xa[0], w0, 0);
    const float c1 = chain(xa[1], w1, 0);
    const float acc = fmaf(fs0[T], fmaf(fz0[T], xs0, c0), fs1[T] * fmaf(fz1[T], xs1, c1));
    if (lane < 16) Rsm[wave][16 * T + lane] = acc;
  }
  if constexpr (HALF) {
    __builtin_amdgcn_sched_barrier(0);
    wait_vm<0>();
    __builtin_amdgcn_sched_barrier(0);
    constexpr int u = U8 - 1;
    const int H = col >> 3;
    const int sigma = 4 * H + j;
    const int pp = 16 * (sigma >> 1) + 8 * (sigma & 1) + r7;
    static_assert((u & 1) == 0, "the last load of an odd U8 is the first of its tile");
    const u32x4 w = *reinterpret_cast<const u32x4*>(tile_lds(NF, wave) + 16 * pp);
    const float c = chain(ac, w, H);
    const float part = H == 0 ? fs0[NF] * fmaf(fz0[NF], xs0, c) : fs1[NF] * fmaf(fz1[NF], xs1, c);
    const float acc = part + __shfl_xor(part, 8, 64);
    if (lane < 8) Rsm[wave][16 * NF + lane] = acc;
  }
  if constexpr (PRO == gemv::PRO_NORM) {
    // The wave's 256 inputs are 32-chunk group `wave` of the row (lanes 32..63
    // hold lanes 0..31's chunks).
    float v[8];
    unpack_bf16x8(xraw, v);
    const float g = sum_over_32_lanes(chunk_squares(v));
    if (lane == 0) Nsm[wave] = g;
  }
  __syncthreads();
  float rnorm = 1.f;  // NORM: the row's factor, the groups' sums added in order
  if constexpr (PRO == gemv::PRO_NORM) {
    float total = 0.f;
    for (int w = 0; w < nw; ++w) total += Nsm[w];
    rnorm = rsqrtf(total / static_cast<float>(K) + pro.eps);
  }
  // Four lanes per output row, each adding a quarter of the waves, then two
  // exchanges (a fixed order: the result does not depend on timing). A group of
  // four lanes is always active or inactive together.
  for (int t = threadIdx.x; t < 4 * R; t += blockDim.x) {
    const int r = t >> 2, part = t & 3;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < gemv::MAX_WAVES / 4; ++w) {
      const int wv = part * (gemv::MAX_WAVES / 4) + w;
      if (wv < nw) v += Rsm[wv][r];
    }
    v += __shfl_xor(v, 1, 64);
    v += __shfl_xor(v, 2, 64);
    if constexpr (PRO == gemv::PRO_NORM) v *= rnorm;
    const int n = n0 + r;
    if (part == 0 && n < N) {
      uint16_t out = E::from_f32(v);
      if (bias != nullptr) out = E::from_f32(E::to_f32(out) + E::to_f32(bias[n]));
      y[n] = out;
    }
  }
}

// One token, K > 4096 (the down projection's 14336): the one-token kernel with
// each wave owning S consecutive 256-input slices (K / (256 S) waves). Every
// slice keeps the one-token kernel's loads, LDS layout and MFMA chains; a
// tile's chains run per slice (A operands read back from LDS, a slice's fold
// coefficients fetched when it is used) and its folds are added in registers
// before the cross-wave sum. The LDS arrays are sized for SW(S) waves: tile
// arrays SW * S * U8 KB, x SW * S * 512 bytes.
namespace gemv {
constexpr int slice_waves(int s) { return s == 4 ? 14 : MAX_WAVES; }
constexpr int slice_max_u8(int s) { return s == 2 ? 4 : 2; }
constexpr int slice_tile_bytes(int u8, int t, int s) {
  return 2 * t < u8 ? tile_wave_bytes(u8, t) * s * slice_waves(s) : 16;
}
}  // namespace gemv

template <int DT, int U8, bool G128, int S, bool ORD = false, int PRO = gemv::PRO_NONE>
__global__ __launch_bounds__(64 * gemv::MAX_WAVES) void int4_gemv_slices_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ packed,
    const uint16_t* __restrict__ scale, const uint8_t* __restrict__ zero,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int N, int K, int G,
    const int32_t* __restrict__ order, GemvPrologue pro) {
  using E = Elem<DT>;
  static_assert(!ORD || G128, "inputs in another order: group 128");
  static_assert(PRO == gemv::PRO_NONE || (DT == LNQ_BF16 && G128 && !ORD), "prologues: bf16, group 128, no order");
  constexpr int R = 8 * U8;
  constexpr int NF = U8 / 2;
  constexpr bool HALF = (U8 & 1) != 0;
  constexpr int SW = gemv::slice_waves(S);
  static_assert(S >= 2 && S <= 4 && U8 <= gemv::slice_max_u8(S), "fits the LDS");
  __shared__ __attribute__((aligned(16))) uint8_t L0[gemv::slice_tile_bytes(U8, 0, S)];
  __shared__ __attribute__((aligned(16))) uint8_t L1[gemv::slice_tile_bytes(U8, 1, S)];
  __shared__ __attribute__((aligned(16))) uint16_t Xsm[SW][256 * S];
  __shared__ float Rsm[SW][R];
  __shared__ float Nsm[PRO == gemv::PRO_NORM ? SW * S : 1];  // each slice's sum of squares
  // Tile T's bytes of slice s of wave w (tiles 0 and 1 only: U8 <= 4).
  auto tile_lds = [&](int T, int w, int sl) -> uint8_t* {
    return (T == 0 ? L0 : L1) + (w * S + sl) * gemv::tile_wave_bytes(U8, T);
  };

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  const int col = lane & 15, j = lane >> 4;
  const int n0 = blockIdx.x * R;
  const int kw = wave * 256 * S;  // the wave's first input
  const int rowb = K >> 1;
  const int groups = K / G;
  uint16_t* Xw = Xsm[wave];
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(packed, static_cast<uint32_t>(static_cast<size_t>(N) * rowb));
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(x, static_cast<uint32_t>(K * 2));
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(scale, static_cast<uint32_t>(N * groups * 2));
  const __amdgpu_buffer_rsrc_t rz = buffer_rsrc(zero, static_cast<uint32_t>(N * groups));

  // ---- loads, small ones first (as in the one-token kernel): per slice the
  // scales and zero points of lane r's row, then x, then the weights.
  const int srow = n0 + (lane < R ? lane : R - 1);
  uint32_t sv[S], zv[S];
#pragma unroll
  for (int sl = 0; sl < S; ++sl) {
    const int g0 = (kw + 256 * sl) / G;
    if constexpr (G128) {
      sv[sl] = __builtin_amdgcn_raw_buffer_load_b32(rs, (srow * groups + g0) * 2, 0, 0);
      zv[sl] = __builtin_amdgcn_raw_buffer_load_b16(rz, srow * groups + g0, 0, 0);
    } else {
      sv[sl] = __builtin_amdgcn_raw_buffer_load_b16(rs, (srow * groups + g0) * 2, 0, 0);
      zv[sl] = __builtin_amdgcn_raw_buffer_load_b8(rz, srow * groups + g0, 0, 0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  u32x4 xv[S];
#pragma unroll
  for (int sl = 0; sl < S; ++sl)
    xv[sl] = __builtin_bit_cast(
        u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, (kw + 256 * sl + 8 * (lane & 31)) * 2, 0, 0));
  u32x4 ov[S][2];  // ORD: each slice's 8 entries of order
  if constexpr (ORD) {
    const __amdgpu_buffer_rsrc_t ro = buffer_rsrc(order, static_cast<uint32_t>(K * 4));
#pragma unroll
    for (int sl = 0; sl < S; ++sl) {
      const int ob = (kw + 256 * sl + 8 * (lane & 31)) * 4;
      ov[sl][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ro, ob, 0, 0));
      ov[sl][1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ro, ob + 16, 0, 0));
    }
  }
  u32x4 pv[S][2];  // PRO: each slice's 8 norm weights (f32), or its 8 values of u
  if constexpr (PRO == gemv::PRO_NORM) {
    const __amdgpu_buffer_rsrc_t rp = buffer_rsrc(pro.w, static_cast<uint32_t>(K * 4));
#pragma unroll
    for (int sl = 0; sl < S; ++sl) {
      const int pb = (kw + 256 * sl + 8 * (lane & 31)) * 4;
      pv[sl][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, pb, 0, 0));
      pv[sl][1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, pb + 16, 0, 0));
    }
  } else if constexpr (PRO == gemv::PRO_SILU) {
    const __amdgpu_buffer_rsrc_t ru = buffer_rsrc(pro.u, static_cast<uint32_t>(K * 2));
#pragma unroll
    for (int sl = 0; sl < S; ++sl)
      pv[sl][0] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(ru, (kw + 256 * sl + 8 * (lane & 31)) * 2, 0, 0));
  }
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  // Order: tile, then slice, then the tile's one or two loads, so that each
  // slice of a tile is multiplied as soon as its own loads land. Loads lo..hi-1
  // of that sequence:
  auto load_weights = [&](int lo, int hi) {
    const int a = lane >> 4, b = lane & 15;
    int i = 0;
#pragma unroll
    for (int T = 0; T < (U8 + 1) / 2; ++T) {
#pragma unroll
      for (int sl = 0; sl < S; ++sl) {
#pragma unroll
        for (int u = 2 * T; u < 2 * T + 2 && u < U8; ++u, ++i) {
          if (i < lo || i >= hi) continue;
          const int sigma = 2 * a + ((b >> 3) ^ (u & 1));
          const int row = n0 + 8 * u + (b & 7);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr)(tile_lds(T, wave, sl) + 1024 * (u & 1)), 16,
                                                   row * rowb + ((kw + 256 * sl) >> 1) + 16 * sigma, 0, 0,
                                                   2 /* non-temporal */);
        }
      }
    }
  };
  // As in the one-token kernel: with an input order, PRE loads before the gather.
  constexpr int PRE = ORD && S * U8 > 4 ? 4 : S * U8;
  load_weights(0, PRE);
  __builtin_amdgcn_sched_barrier(0);

  // ---- x of every slice to LDS in pair order; its sums over each half.
  wait_vm<PRE>();
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (ORD) {
    // As in the one-token kernel: x in input order (Xsm holds K values for the
    // nw * S slices), then each slice's taken inputs.
#pragma unroll
    for (int sl = 0; sl < S; ++sl) *reinterpret_cast<u32x4*>(Xw + 256 * sl + 8 * (lane & 31)) = xv[sl];
    lds_barrier();
#pragma unroll
    for (int sl = 0; sl < S; ++sl) xv[sl] = gather_x8(&Xsm[0][0], ov[sl][0], ov[sl][1], static_cast<uint32_t>(K));
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    load_weights(PRE, S * U8);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int sl = 0; sl < S; ++sl) {
    if constexpr (PRO == gemv::PRO_NORM) {
      // Slice sl of wave w is 32-chunk group S w + sl of the row. (Summed here, not
      // after the tiles as in the one-token kernel: kept across them, the partial
      // sums would push this kernel's registers past its budget.)
      float v[8];
      unpack_bf16x8(xv[sl], v);
      const float g = sum_over_32_lanes(chunk_squares(v));
      if (lane == 0) Nsm[wave * S + sl] = g;
      xv[sl] = scale_bf16x8(xv[sl], __builtin_bit_cast(f32x4, pv[sl][0]), __builtin_bit_cast(f32x4, pv[sl][1]));
    } else if constexpr (PRO == gemv::PRO_SILU) {
      xv[sl] = silu_mul_bf16x8_halves(xv[sl], pv[sl][0], lane);
    }
  }
  float xs0[S], xs1[S];
#pragma unroll
  for (int sl = 0; sl < S; ++sl) {
    if (lane < 32) *reinterpret_cast<u32x4*>(Xw + 256 * sl + 8 * lane) = permute_x8(xv[sl]);
    float sum = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t d = xv[sl][e];
      sum += E::to_f32(static_cast<uint16_t>(d & 0xffffu)) + E::to_f32(static_cast<uint16_t>(d >> 16));
    }
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    sum += __shfl_xor(sum, 4, 64);
    sum += __shfl_xor(sum, 8, 64);
    xs0[sl] = __shfl(sum, 0, 64);
    xs1[sl] = __shfl(sum, 16, 64);
    if constexpr (!G128) {
      sv[sl] = (sv[sl] & 0xffffu) | (sv[sl] << 16);
      zv[sl] = (zv[sl] & 0xffu) | (zv[sl] << 8);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  uint32_t nib_mask = 0x000f000fu, nib_magic = E::MAGIC2;
  hide_in_vgpr(nib_mask);
  hide_in_vgpr(nib_magic);
  const int r7 = col & 7;
  auto chain = [&](const u32x4 (&a)[4], const u32x4 w, int reg) -> float {
    u32x4 b0, b1, b2, b3;
    widen_pair<DT>(w.x, w.y, nib_mask, nib_magic, b0, b1);
    widen_pair<DT>(w.z, w.w, nib_mask, nib_magic, b2, b3);
    f32x4 C = f32x4{0.f, 0.f, 0.f, 0.f};
    C = mfma16x16x32<DT>(a[0], b0, C);
    C = mfma16x16x32<DT>(a[1], b1, C);
    C = mfma16x16x32<DT>(a[2], b2, C);
    C = mfma16x16x32<DT>(a[3], b3, C);
    return reg == 0 ? C[0] : C[1];
  };
  // Scale / zero point of output row n (workgroup-local) in slice sl: (s0, s1, -(M + z0), -(M + z1)).
  auto coeff = [&](int n, int sl, float& s0, float& s1, float& nz0, float& nz1) {
    const uint32_t sp = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(4 * n, static_cast<int>(sv[sl])));
    const uint32_t zp = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(4 * n, static_cast<int>(zv[sl])));
    s0 = E::to_f32(static_cast<uint16_t>(sp & 0xffffu));
    s1 = E::to_f32(static_cast<uint16_t>(sp >> 16));
    nz0 = -(E::MAGIC_VALUE + static_cast<float>(zp & 0xffu));
    nz1 = -(E::MAGIC_VALUE + static_cast<float>((zp >> 8) & 0xffu));
  };

  // ---- tiles as their loads land; each slice's chains, folded and added.
#pragma unroll
  for (int T = 0; T < NF; ++T) {
    const int h = col >> 3;
    const int p0 = 16 * (j >> 1) + 8 * ((j & 1) ^ h) + r7;
    const int p1 = 16 * (2 + (j >> 1)) + 8 * ((j & 1) ^ h) + r7;
    float acc = 0.f;
#pragma unroll
    for (int sl = 0; sl < S; ++sl) {
      float s0, s1, nz0, nz1;
      coeff(8 * (2 * T + h) + r7, sl, s0, s1, nz0, nz1);
      __builtin_amdgcn_sched_barrier(0);
      wait_vm_rt(S * U8 - (2 * S * T + 2 * (sl + 1)));  // this slice's two loads have landed
      __builtin_amdgcn_sched_barrier(0);
      u32x4 xa[2][4];
#pragma unroll
      for (int H = 0; H < 2; ++H)
#pragma unroll
        for (int t = 0; t < 4; ++t)
          xa[H][t] = *reinterpret_cast<const u32x4*>(Xw + 256 * sl + 128 * H + 32 * j + 8 * t);
      const uint8_t* Wt = tile_lds(T, wave, sl) + 1024 * h;
      const u32x4 w0 = *reinterpret_cast<const u32x4*>(Wt + 16 * p0);
      const u32x4 w1 = *reinterpret_cast<const u32x4*>(Wt + 16 * p1);
      const float c0 = chain(xa[0], w0, 0);
      const float c1 = chain(xa[1], w1, 0);
      acc += fmaf(s0, fmaf(nz0, xs0[sl], c0), s1 * fmaf(nz1, xs1[sl], c1));
    }
    if (lane < 16) Rsm[wave][16 * T + lane] = acc;
  }
  if constexpr (HALF) {
    const int H = col >> 3;
    const int sigma = 4 * H + j;
    const int pp = 16 * (sigma >> 1) + 8 * (sigma & 1) + r7;
    float part = 0.f;
#pragma unroll
    for (int sl = 0; sl < S; ++sl) {
      float s0, s1, nz0, nz1;
      coeff(8 * (U8 - 1) + r7, sl, s0, s1, nz0, nz1);
      __builtin_amdgcn_sched_barrier(0);
      wait_vm_rt(S - 1 - sl);  // the half tile's loads come last, one a slice
      __builtin_amdgcn_sched_barrier(0);
      u32x4 ac[4];
#pragma unroll
      for (int t = 0; t < 4; ++t)
        ac[t] = *reinterpret_cast<const u32x4*>(Xw + 256 * sl + (col == 1 ? 128 : 0) + 32 * j + 8 * t);
      const u32x4 w = *reinterpret_cast<const u32x4*>(tile_lds(NF, wave, sl) + 16 * pp);
      const float c = chain(ac, w, H);
      part += H == 0 ? s0 * fmaf(nz0, xs0[sl], c) : s1 * fmaf(nz1, xs1[sl], c);
    }
    const float acc = part + __shfl_xor(part, 8, 64);
    if (lane < 8) Rsm[wave][16 * NF + lane] = acc;
  }
  __syncthreads();
  float rnorm = 1.f;  // NORM: the row's factor, the groups' sums added in order
  if constexpr (PRO == gemv::PRO_NORM) {
    float total = 0.f;
    for (int g = 0; g < nw * S; ++g) total += Nsm[g];
    rnorm = rsqrtf(total / static_cast<float>(K) + pro.eps);
  }
  for (int t = threadIdx.x; t < 4 * R; t += blockDim.x) {
    const int r = t >> 2, part = t & 3;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < gemv::MAX_WAVES / 4; ++w) {
      const int wv = part * (gemv::MAX_WAVES / 4) + w;
      if (wv < nw) v += Rsm[wv][r];
    }
    v += __shfl_xor(v, 1, 64);
    v += __shfl_xor(v, 2, 64);
    if constexpr (PRO == gemv::PRO_NORM) v *= rnorm;
    const int n = n0 + r;
    if (part == 0 && n < N) {
      uint16_t out = E::from_f32(v);
      if (bias != nullptr) out = E::from_f32(E::to_f32(out) + E::to_f32(bias[n]));
      y[n] = out;
    }
  }
}

// A few tokens (2..MX rows, MX = 4 or 16): the one-token kernel's workgroup
// shape and weight streams, with A-operand row m of every MFMA holding x row m
// (lane col = m). The order of the inputs within a wave's 256 is free as long
// as A and B agree, so MFMA t of half H takes inputs 128 H + 32 t + 8 j .. + 7
// in lane (col, j): at 16 rows each lane loads its own A operands straight from
// x, an instruction reading 16 rows x 64 contiguous bytes (rows past M read
// zeros through the range check; up to 4 rows the loads are two rows x 512
// bytes, put in operand order through LDS). The B operands follow: lane (col,
// j) reads dword j of the 16-byte pieces 4 H + t of its weight row. The output
// registers of a tile hold rows 4 (lane / 16) + i; the fold takes each row's sum
// of x from the lanes that loaded it, and after a barrier the 16 waves' partial
// sums are added through LDS (the weight buffers, no longer read), four lanes an
// output.
template <int DT, int U8, bool G128, int MX>
__global__ __launch_bounds__(64 * gemv::MAX_WAVES) void int4_gemv_rows_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ packed,
    const uint16_t* __restrict__ scale, const uint8_t* __restrict__ zero,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int M, int N, int K, int G) {
  using E = Elem<DT>;
  constexpr int R = 8 * U8;
  constexpr int NT = (U8 + 1) / 2;  // 16-row tiles (an odd U8: the last one has 8 rows)
  LNQ_GEMV_TILE_ARRAYS(U8);
  // Once a wave has folded its tiles it writes its partial sums of tile T (16
  // output rows) over its own part of tile T's array, which only it reads:
  // element e = 64 i + lane (x row 4 (lane / 16) + i, output row 16 T +
  // lane % 16) at float 64 i + (lane ^ 4 w) of wave w's part. The XOR by 4 w
  // puts the four waves a read instruction touches (lanes 16 q + c read wave
  // 4 q + w, parts 2048 or 1024 bytes apart) in distinct banks.
  static_assert(gemv::tile_wave_bytes(U8, NT - 1) >= 256 * 4, "partial sums fit a wave's part of a tile");

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  const int col = lane & 15, j = lane >> 4;
  const int n0 = blockIdx.x * R;
  const int k0 = wave * 256;
  const int rowb = K >> 1;
  const int groups = K / G;
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(packed, static_cast<uint32_t>(static_cast<size_t>(N) * rowb));
  // Rows of x past M read zeros through the range check.
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(x, static_cast<uint32_t>(static_cast<size_t>(M) * K * 2));
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(scale, static_cast<uint32_t>(N * groups * 2));
  const __amdgpu_buffer_rsrc_t rz = buffer_rsrc(zero, static_cast<uint32_t>(N * groups));

  // ---- loads: scales and zeros (first: they are few, and the compiler may copy
  // them out of their registers early), x (row col, inputs k0 + 128 H + 32 t +
  // 8 j), weights.
  const int srow = n0 + (lane < R ? lane : R - 1);
  const int g0 = k0 / G;
  uint32_t sv;
  uint16_t zv16;
  if constexpr (G128) {
    sv = __builtin_amdgcn_raw_buffer_load_b32(rs, (srow * groups + g0) * 2, 0, 0);
    zv16 = __builtin_amdgcn_raw_buffer_load_b16(rz, srow * groups + g0, 0, 0);
  } else {
    sv = __builtin_amdgcn_raw_buffer_load_b16(rs, (srow * groups + g0) * 2, 0, 0);
    zv16 = __builtin_amdgcn_raw_buffer_load_b8(rz, srow * groups + g0, 0, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
  // 16 rows: each lane loads its A operands. Up to 4 rows, loads of two rows
  // x 256 inputs (lanes 0..31 row 2 i, 32..63 row 2 i + 1) move x to registers
  // with fewer instructions, and one pass through a wave-private LDS slot puts
  // it in operand order (A rows past 4 are zeros).
  u32x4 xa[2][4];
  u32x4 xc[2];
  if constexpr (MX == 16) {
#pragma unroll
    for (int H = 0; H < 2; ++H)
#pragma unroll
      for (int t = 0; t < 4; ++t)
        xa[H][t] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, (col * K + k0 + 128 * H + 32 * t + 8 * j) * 2, 0, 0));
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      xc[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            rx, ((2 * i + (lane >> 5)) * K + k0 + 8 * (lane & 31)) * 2, 0, 0));
  }
  __builtin_amdgcn_sched_barrier(0);
  {
    const int a = lane >> 4, b = lane & 15;
#pragma unroll
    for (int u = 0; u < U8; ++u) {
      const int sigma = 2 * a + ((b >> 3) ^ (u & 1));
      const int row = n0 + 8 * u + (b & 7);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr)(tile_lds(u >> 1, wave) + 1024 * (u & 1)), 16,
                                               row * rowb + (k0 >> 1) + 16 * sigma, 0, 0, 2 /* non-temporal */);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- x: wait for it (and the scales) alone; the sums of x row col over both
  // halves, then the A operands in pair order.
  wait_vm<U8>();
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (MX != 16) {
    static_assert(MX == 4, "4 or 16 rows");
    __shared__ __attribute__((aligned(16))) uint16_t Xst[gemv::MAX_WAVES][4 * 256];
    uint16_t* Xw = Xst[wave];
    *reinterpret_cast<u32x4*>(Xw + 256 * (lane >> 5) + 8 * (lane & 31)) = xc[0];
    *reinterpret_cast<u32x4*>(Xw + 256 * (2 + (lane >> 5)) + 8 * (lane & 31)) = xc[1];
#pragma unroll
    for (int H = 0; H < 2; ++H)
#pragma unroll
      for (int t = 0; t < 4; ++t) xa[H][t] = u32x4{0u, 0u, 0u, 0u};
    // Only the reads are under the lane condition.
    if (col < 4) {
#pragma unroll
      for (int H = 0; H < 2; ++H)
#pragma unroll
        for (int t = 0; t < 4; ++t)
          xa[H][t] = *reinterpret_cast<const u32x4*>(Xw + 256 * col + 128 * H + 32 * t + 8 * j);
    }
  }
  // The sums of x over each half on the matrix core (A = x, B = ones): lane
  // (col, j) register i is the sum of x row 4 j + i, the row its output
  // register i holds.
  u32x4 ones;
  ones.x = ones.y = ones.z = ones.w = E::ONE2;
  f32x4 xsum[2];
#pragma unroll
  for (int H = 0; H < 2; ++H) {
    xsum[H] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      xsum[H] = mfma16x16x32<DT>(xa[H][t], ones, xsum[H]);
      xa[H][t] = permute_x8(xa[H][t]);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  uint32_t nib_mask = 0x000f000fu, nib_magic = E::MAGIC2;
  hide_in_vgpr(nib_mask);
  hide_in_vgpr(nib_magic);
  const int r7 = col & 7;
  // One MFMA chain over four packed dwords (MFMA t takes dword t).
  auto chain = [&](const u32x4 (&a)[4], const u32x4 w) -> f32x4 {
    u32x4 b0, b1, b2, b3;
    widen_pair<DT>(w.x, w.y, nib_mask, nib_magic, b0, b1);
    widen_pair<DT>(w.z, w.w, nib_mask, nib_magic, b2, b3);
    f32x4 C = f32x4{0.f, 0.f, 0.f, 0.f};
    C = mfma16x16x32<DT>(a[0], b0, C);
    C = mfma16x16x32<DT>(a[1], b1, C);
    C = mfma16x16x32<DT>(a[2], b2, C);
    C = mfma16x16x32<DT>(a[3], b3, C);
    return C;
  };
  // ---- tiles as their loads land; tile T covers rows 16 T .. 16 T + 15 (the
  // last of an odd U8 only its first 8, the other 8 columns read again and
  // dropped). Piece sigma of row r7 of load u sits at 16-byte position
  // 16 (sigma / 2) + 8 ((sigma % 2) ^ (u % 2)) + r7; pieces t and t + 2 are 256
  // bytes apart, one ds_read2 a pair.
  f32x4 cf[NT][2];
#pragma unroll
  for (int T = 0; T < NT; ++T) {
    __builtin_amdgcn_sched_barrier(0);
    if (2 * T + 1 < U8) wait_vm_rt(U8 - 1 - (2 * T + 1));
    else wait_vm<0>();
    __builtin_amdgcn_sched_barrier(0);
    const int h = col >> 3;
    const int u = min(2 * T + h, U8 - 1);
    const int hh = u & 1;  // the piece order of load u (and its half of the tile array)
    const uint32_t* Wt = reinterpret_cast<const uint32_t*>(tile_lds(T, wave) + 1024 * hh);
    u32x4 w[2];
#pragma unroll
    for (int H = 0; H < 2; ++H)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        // pieces 4 H + t and 4 H + t + 2
        const int p = 16 * (2 * H) + 8 * ((t & 1) ^ hh) + r7;
        const uint32_t* at = Wt + 4 * p + j;
        w[H][t] = at[0];
        w[H][t + 2] = at[64];
      }
    cf[T][0] = chain(xa[0], w[0]);
    cf[T][1] = chain(xa[1], w[1]);
  }
  // ---- scales / zeros (landed before x), the fold.
  __builtin_amdgcn_sched_barrier(0);
  __asm__ volatile("" : "+v"(sv), "+v"(zv16));
  uint32_t zv = zv16;
  if constexpr (!G128) {
    sv = (sv & 0xffffu) | (sv << 16);
    zv = (zv & 0xffu) | (zv << 8);
  }
  // Sums of x rows 4 j + i (i = 0..3), the rows this lane's output registers hold.
  float xs[2][4];
#pragma unroll
  for (int H = 0; H < 2; ++H)
#pragma unroll
    for (int i = 0; i < 4; ++i) xs[H][i] = xsum[H][i];
  float acc[NT][4];
#pragma unroll
  for (int T = 0; T < NT; ++T) {
    const int n = 16 * T + col;  // output row within the workgroup (lane's column)
    const int src = n < R ? n : R - 1;
    const uint32_t sp = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(4 * src, static_cast<int>(sv)));
    const uint32_t zp = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(4 * src, static_cast<int>(zv)));
    const float s0 = E::to_f32(static_cast<uint16_t>(sp & 0xffffu)), s1 = E::to_f32(static_cast<uint16_t>(sp >> 16));
    const float z0 = E::MAGIC_VALUE + static_cast<float>(zp & 0xffu);
    const float z1 = E::MAGIC_VALUE + static_cast<float>((zp >> 8) & 0xffu);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      acc[T][i] = fmaf(s0, fmaf(-z0, xs[0][i], cf[T][0][i]), s1 * fmaf(-z1, xs[1][i], cf[T][1][i]));
  }
  // ---- the cross-wave sum through the wave's own (now unread) tile parts.
  // Element 64 i + l of a wave's part sits at 64 i + (l ^ 4 wave): the XOR spreads
  // the four waves a read instruction touches over distinct banks (as a rotation
  // by 4 wave would) and leaves 64 i a constant offset.
  const int lrot = lane ^ (4 * wave);
#pragma unroll
  for (int T = 0; T < NT; ++T) {
    float* red = reinterpret_cast<float*>(tile_lds(T, wave));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 4 * j + i;
      if (m < MX) red[64 * i + lrot] = acc[T][i];
    }
  }
  __syncthreads();
  // Output (T, m, c): lanes 16 q + c of a wave add waves 4 q .. 4 q + 3 (the
  // waves past nw masked), two exchanges finish the sum. Pass o (T = o / MX,
  // m = o % MX) covers 16 outputs; wave w takes passes w, w + nw, .., all its
  // reads issued before the first sum.
  constexpr int PASSES = NT * MX;
  constexpr int PW = (PASSES + gemv::MAX_WAVES - 1) / gemv::MAX_WAVES;  // passes a wave at 16 waves
  const int q = j;
  auto pass = [&](const int o, float (&r)[4]) {
    const int T = min(o / MX, NT - 1), m = o % MX;
    // (16 (m / 4) + col) ^ (4 wv) < 64: wave wv's element 64 (m % 4) + 16 (m / 4) + col.
    const int e = (16 * (m >> 2) + col) ^ (16 * q);
#pragma unroll
    for (int w = 0; w < gemv::MAX_WAVES / 4; ++w) {
      const int wv = 4 * q + w;
      r[w] = reinterpret_cast<const float*>(tile_lds(T, wv))[64 * (m & 3) + (e ^ (4 * w))];
    }
  };
  auto finish = [&](const int o, const float (&r)[4]) {
    const int T = o / MX, m = o % MX;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < gemv::MAX_WAVES / 4; ++w) v += 4 * q + w < nw ? r[w] : 0.f;
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    const int n = n0 + 16 * T + col;
    if (q == 0 && o < PASSES && m < M && 16 * T + col < R && n < N) {
      uint16_t out = E::from_f32(v);
      if (bias != nullptr) out = E::from_f32(E::to_f32(out) + E::to_f32(bias[n]));
      y[static_cast<size_t>(m) * N + n] = out;
    }
  };
  if (nw == gemv::MAX_WAVES) {
    float r[PW][4];
#pragma unroll
    for (int p = 0; p < PW; ++p) pass(wave + gemv::MAX_WAVES * p, r[p]);
#pragma unroll
    for (int p = 0; p < PW; ++p) finish(wave + gemv::MAX_WAVES * p, r[p]);
  } else {
    for (int o = wave; o < PASSES; o += nw) {
      float r[4];
      pass(o, r);
      finish(o, r);
    }
  }
}

// 17..32 tokens: the few-token kernel with two 16-row A blocks per weight
// tile, so that each packed byte is read and widened once for all 32 rows.
// Lane (col, j) holds the A operands of x rows col and 16 + col (inputs k0 +
// 128 H + 32 t + 8 j, rows past M read zeros), 64 registers; a wave may use 128
// in a 16-wave workgroup, so nothing else is held across tiles: the sums of
// each x row (MFMAs against ones) go to LDS once (XS), and each tile is folded
// with its scales and zero points as soon as its two MFMA chains end, its
// partial sums written over the
// wave's own part of the tile array (2 KB: 16 outputs x 32 rows, output-minor;
// the 8-row last tile of an odd U8 1 KB: its 8 outputs x 32 rows). The 16
// waves' sums are then added as in int4_gemv_rows_kernel.
//
// XT: x is given as x tiles (one 32-row chunk, x_tile_index): operand (b, H,
// t) of the wave's slice is one contiguous 1 KB load.
//
// SPLIT: the K range is cut into gridDim.y chunks of nw slices, workgroup
// (bx, c) taking chunk c of rows bx * R ..; its sums over the chunk go unrounded
// to part[c][m][n] (f32) and int4_split_reduce_kernel adds the chunks in order.
// Every workgroup reads x only over its own chunk, so a 64-row block with a
// quarter of K reads a quarter of x where the unsplit kernel's 16-row blocks
// read all of it (the down projection at 32 rows: 229 KB of x against 115 KB of
// weights a workgroup, in place of 917 KB against 115 KB).
template <int DT, int U8, bool G128, bool SPLIT = false, bool XT = false>
__global__ __launch_bounds__(64 * gemv::MAX_WAVES) void int4_gemv_rows32_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ packed,
    const uint16_t* __restrict__ scale, const uint8_t* __restrict__ zero,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int M, int N, int K, int G,
    float* __restrict__ part = nullptr) {
  using E = Elem<DT>;
  constexpr int R = 8 * U8;
  constexpr int NT = (U8 + 1) / 2;
  constexpr bool HALF = (U8 & 1) != 0;
  constexpr int SR = (R + 63) / 64;  // scale (and zero) registers: rows 64 i + lane
  static_assert(SPLIT || U8 <= 8, "more than 64 rows only with split K");
  LNQ_GEMV_TILE_GROUPS(U8);
  // Outputs of tile T a wave part holds (its floats: 32 times as many).
  auto outs = [](int T) { return HALF && T == NT - 1 ? 8 : 16; };
  static_assert(gemv::tile_wave_bytes(U8, NT - 1) == (HALF ? 1024 : 2048), "tile parts hold the partial sums");
  // Sums of x rows (block b, half H): XS[wave][b][H][row within the block].
  __shared__ __attribute__((aligned(16))) float XS[gemv::MAX_WAVES][2][2][16];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  const int col = lane & 15, j = lane >> 4;
  const int n0 = blockIdx.x * R;
  const int k0 = ((SPLIT ? blockIdx.y * nw : 0) + wave) * 256;
  const int rowb = K >> 1;
  const int groups = K / G;
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(packed, static_cast<uint32_t>(static_cast<size_t>(N) * rowb));
  const __amdgpu_buffer_rsrc_t rx =
      buffer_rsrc(x, static_cast<uint32_t>(static_cast<size_t>(XT ? 32 : M) * K * 2));
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(scale, static_cast<uint32_t>(N * groups * 2));
  const __amdgpu_buffer_rsrc_t rz = buffer_rsrc(zero, static_cast<uint32_t>(N * groups));

  // ---- loads: scales and zeros, x (16 per lane), weights.
  const int g0 = k0 / G;
  uint32_t sv[SR];
  uint16_t zv16[SR];
#pragma unroll
  for (int i = 0; i < SR; ++i) {
    const int srow = n0 + 64 * i + (lane < R - 64 * i ? lane : R - 64 * i - 1);
    if constexpr (G128) {
      sv[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, (srow * groups + g0) * 2, 0, 0);
      zv16[i] = __builtin_amdgcn_raw_buffer_load_b16(rz, srow * groups + g0, 0, 0);
    } else {
      sv[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, (srow * groups + g0) * 2, 0, 0);
      zv16[i] = __builtin_amdgcn_raw_buffer_load_b8(rz, srow * groups + g0, 0, 0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  u32x4 xa[2][2][4];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int H = 0; H < 2; ++H)
#pragma unroll
      for (int t = 0; t < 4; ++t)
        xa[b][H][t] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       rx, XT ? (((k0 >> 8) * 16 + 8 * b + 4 * H + t) * 64 + lane) * 16
                              : ((16 * b + col) * K + k0 + 128 * H + 32 * t + 8 * j) * 2, 0, 0));
  __builtin_amdgcn_sched_barrier(0);
  {
    const int a = lane >> 4, bb = lane & 15;
#pragma unroll
    for (int u = 0; u < U8; ++u) {
      const int sigma = 2 * a + ((bb >> 3) ^ (u & 1));
      const int row = n0 + 8 * u + (bb & 7);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr)(tile_lds(u >> 1, wave) + 1024 * (u & 1)), 16,
                                               row * rowb + (k0 >> 1) + 16 * sigma, 0, 0, 2 /* non-temporal */);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- x (and the scales) landed: the A operands in pair order (x tiles hold
  // them so already), then each row's sums over both halves on the matrix core
  // (A = x, B = ones: lane (col, j) register i is the sum of x row 16 b + 4 j +
  // i, the row its output register i holds), taken on the operands in pair order
  // in both cases so that tiles and row-major x give the same bits.
  wait_vm<U8>();
  __builtin_amdgcn_sched_barrier(0);
  u32x4 ones;
  ones.x = ones.y = ones.z = ones.w = E::ONE2;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int H = 0; H < 2; ++H) {
      f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if constexpr (!XT) xa[b][H][t] = permute_x8(xa[b][H][t]);
        sum = mfma16x16x32<DT>(xa[b][H][t], ones, sum);
      }
      if (col == 0) *reinterpret_cast<f32x4*>(&XS[wave][b][H][4 * j]) = sum;
    }
  __builtin_amdgcn_sched_barrier(0);

  uint32_t zv[SR];
#pragma unroll
  for (int r = 0; r < SR; ++r) {
    __asm__ volatile("" : "+v"(sv[r]), "+v"(zv16[r]));
    zv[r] = zv16[r];
    if constexpr (!G128) {
      sv[r] = (sv[r] & 0xffffu) | (sv[r] << 16);
      zv[r] = (zv[r] & 0xffu) | (zv[r] << 8);
    }
  }
  uint32_t nib_mask = 0x000f000fu, nib_magic = E::MAGIC2;
  hide_in_vgpr(nib_mask);
  hide_in_vgpr(nib_magic);
  const int r7 = col & 7;

  // ---- tiles as their loads land (the piece layout of int4_gemv_rows_kernel).
#pragma unroll
  for (int T = 0; T < NT; ++T) {
    __builtin_amdgcn_sched_barrier(0);
    if (2 * T + 1 < U8) wait_vm_rt(U8 - 1 - (2 * T + 1));
    else wait_vm<0>();
    __builtin_amdgcn_sched_barrier(0);
    const int h = col >> 3;
    const int u = min(2 * T + h, U8 - 1);
    const int hh = u & 1;
    const uint32_t* Wt = reinterpret_cast<const uint32_t*>(tile_lds(T, wave) + 1024 * hh);
    u32x4 w[2];
#pragma unroll
    for (int H = 0; H < 2; ++H)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int p = 16 * (2 * H) + 8 * ((t & 1) ^ hh) + r7;
        const uint32_t* at = Wt + 4 * p + j;
        w[H][t] = at[0];
        w[H][t + 2] = at[64];
      }
    f32x4 C[2][2];
#pragma unroll
    for (int H = 0; H < 2; ++H) {
      u32x4 b0, b1;
      C[0][H] = C[1][H] = f32x4{0.f, 0.f, 0.f, 0.f};
      widen_pair<DT>(w[H].x, w[H].y, nib_mask, nib_magic, b0, b1);
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        C[b][H] = mfma16x16x32<DT>(xa[b][H][0], b0, C[b][H]);
        C[b][H] = mfma16x16x32<DT>(xa[b][H][1], b1, C[b][H]);
      }
      widen_pair<DT>(w[H].z, w[H].w, nib_mask, nib_magic, b0, b1);
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        C[b][H] = mfma16x16x32<DT>(xa[b][H][2], b0, C[b][H]);
        C[b][H] = mfma16x16x32<DT>(xa[b][H][3], b1, C[b][H]);
      }
    }
    // Fold: output row 16 T + col, x rows 16 b + 4 j + i.
    const int n = 16 * T + col;
    const int src = (n < R ? n : R - 1) & 63;  // rows 16 T .. 16 T + 15 lie in register T / 4
    const uint32_t sp = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(4 * src, static_cast<int>(sv[T / 4])));
    const uint32_t zp = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(4 * src, static_cast<int>(zv[T / 4])));
    const float s0 = E::to_f32(static_cast<uint16_t>(sp & 0xffffu)), s1 = E::to_f32(static_cast<uint16_t>(sp >> 16));
    const float z0 = E::MAGIC_VALUE + static_cast<float>(zp & 0xffu);
    const float z1 = E::MAGIC_VALUE + static_cast<float>((zp >> 8) & 0xffu);
    const int CW = outs(T);
    float* red = reinterpret_cast<float*>(tile_lds(T, wave));
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const f32x4 x0 = *reinterpret_cast<const f32x4*>(&XS[wave][b][0][4 * j]);
      const f32x4 x1 = *reinterpret_cast<const f32x4*>(&XS[wave][b][1][4 * j]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = fmaf(s0, fmaf(-z0, x0[i], C[b][0][i]), s1 * fmaf(-z1, x1[i], C[b][1][i]));
        if (col < CW) red[((b * 4 + i) * 4 + j) * CW + col] = v;
      }
    }
  }
  __syncthreads();
  // The waves' partial sums added four outputs at a time: thread t takes quads
  // t, t + 64 nw, .. of the workgroup (tile T: 32 row slots x CW / 4 column
  // quads, slot s = 16 b + 4 i + j holding x row 16 b + 4 j + i), reads the quad
  // of every wave (16 contiguous bytes, at the same place in each wave's part:
  // one read instruction covers 1 KB of one part, so no bank is hit twice) and
  // adds them in wave order. No lane exchange: one LDS read a wave a quad. With
  // all 16 waves (K = 4096) the wave loop has no condition (no selects).
  constexpr int TQ = 32 * 16 / 4;  // quads of a full tile
  constexpr int QUADS = HALF ? (NT - 1) * TQ + TQ / 2 : NT * TQ;
  static_assert(TQ % 64 == 0 && QUADS % 64 == 0, "a wave's quads lie in one tile");
  for (int qd = threadIdx.x; qd < QUADS; qd += blockDim.x) {
    // The 64 quads of a wave are consecutive and a tile holds a multiple of 64:
    // the tile is the wave's (scalar), so its array is not selected lane by lane.
    const int T = __builtin_amdgcn_readfirstlane(qd / TQ), r = qd % TQ;
    const int cw = outs(T);
    const int cq = cw / 4;  // column quads of the tile
    const int slot = r / cq, c4 = 4 * (r % cq);
    const int e = slot * cw + c4;
    // Every wave's quad requested before the first add (one LDS round trip).
    auto gather = [&](auto all) -> f32x4 {
      f32x4 p[gemv::MAX_WAVES];
#pragma unroll
      for (int w = 0; w < gemv::MAX_WAVES; ++w)
        if (decltype(all)::value || w < nw)
          p[w] = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(tile_lds(T, w)) + e);
      f32x4 acc = p[0];
#pragma unroll
      for (int w = 1; w < gemv::MAX_WAVES; ++w)
        if (decltype(all)::value || w < nw)
          acc = f32x4{acc[0] + p[w][0], acc[1] + p[w][1], acc[2] + p[w][2], acc[3] + p[w][3]};
      return acc;
    };
    const f32x4 v = nw == gemv::MAX_WAVES ? gather(std::true_type{}) : gather(std::false_type{});
    const int m = (slot & 16) | ((slot & 3) << 2) | ((slot >> 2) & 3);
    const int n = n0 + 16 * T + c4;
    if (m >= M || 16 * T + c4 >= R) continue;
    if constexpr (SPLIT) {
      float* dst = part + (static_cast<size_t>(blockIdx.y) * M + m) * N + n;
      if (n + 3 < N && (N & 3) == 0) {
        *reinterpret_cast<f32x4*>(dst) = v;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (n + i < N) dst[i] = v[i];
      }
    } else {
      uint16_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[i] = E::from_f32(v[i]);
        if (bias != nullptr && n + i < N) o[i] = E::from_f32(E::to_f32(o[i]) + E::to_f32(bias[n + i]));
      }
      uint16_t* dst = y + static_cast<size_t>(m) * N + n;
      if (n + 3 < N && (N & 3) == 0 && (reinterpret_cast<uintptr_t>(y) & 7) == 0) {
        *reinterpret_cast<u32x2*>(dst) = u32x2{o[0] | (static_cast<uint32_t>(o[1]) << 16),
                                               o[2] | (static_cast<uint32_t>(o[3]) << 16)};
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (n + i < N) dst[i] = o[i];
      }
    }
  }
}

// The chunks of a split product added in chunk order (deterministic), rounded
// once to the output type, the bias added as the unsplit kernels add it
// (y = round(round(sum) + bias)). Thread t owns four consecutive outputs of one
// row (N % 4 == 0).
template <int DT>
__global__ __launch_bounds__(256) void int4_split_reduce_kernel(const float* __restrict__ part,
                                                                const uint16_t* __restrict__ bias,
                                                                uint16_t* __restrict__ y, int M, int N, int S) {
  using E = Elem<DT>;
  const size_t e = (static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  const size_t total = static_cast<size_t>(M) * N;
  if (e >= total) return;
  f32x4 v = *reinterpret_cast<const f32x4*>(part + e);
  for (int c = 1; c < S; ++c) {
    const f32x4 p = *reinterpret_cast<const f32x4*>(part + static_cast<size_t>(c) * total + e);
    v = f32x4{v[0] + p[0], v[1] + p[1], v[2] + p[2], v[3] + p[3]};
  }
  const int n = static_cast<int>(e % N);
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint16_t out = E::from_f32(v[i]);
    if (bias != nullptr) out = E::from_f32(E::to_f32(out) + E::to_f32(bias[n + i]));
    o[i] = out;
  }
  *reinterpret_cast<u32x2*>(y + e) = u32x2{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
}

// Whether the one-token kernel takes this shape (else the caller uses the
// general skinny kernel).
// Slices a wave takes in the K > 4096 one-token kernel (0: it does not take K):
// the fewest S in 2..4 with K / 256 = S * waves, waves <= slice_waves(S).
static int gemv_slices(int K) {
  if (K % 256 != 0 || K <= 256 * gemv::MAX_WAVES) return 0;
  const int k256 = K / 256;
  for (int sl = 2; sl <= 4; ++sl)
    if (k256 % sl == 0 && k256 / sl <= gemv::slice_waves(sl)) return sl;
  return 0;
}

static bool gemv_slices_supports(int N, int K, int G, const void* x, const void* packed, const void* scale,
                                 const void* zero) {
  const int sl = gemv_slices(K);
  if (sl == 0 || N <= 0 || (N + 2047) / 2048 > gemv::slice_max_u8(sl)) return false;
  if (!(G == 128 || G % 256 == 0) || K % G != 0) return false;
  if (static_cast<size_t>(N) * (K / 2) >= (1ull << 31)) return false;
  return aligned(x, 16) && aligned(packed, 16) && (G != 128 || aligned(scale, 4)) && (G != 128 || aligned(zero, 2));
}

bool int4_gemv_supports(int M, int N, int K, int G, const void* x, const void* packed, const void* scale,
                        const void* zero) {
  if (M < 1 || M > gemv::MAX_ROWS) return false;
  if (M == 1 && gemv_slices_supports(N, K, G, x, packed, scale, zero)) return true;
  if (K % 256 != 0 || K < 256 || K > 256 * gemv::MAX_WAVES) return false;
  if (!(G == 128 || G % 256 == 0) || K % G != 0) return false;
  // Past 16384 outputs the workgroups keep 64 rows each (U8 = 8) and the grid
  // grows past one workgroup a CU.
  if (N <= 0) return false;
  if (static_cast<size_t>(N) * (K / 2) >= (1ull << 31)) return false;
  // 16-byte x and weight loads; scale pairs as dwords (group 128).
  return aligned(x, 16) && aligned(packed, 16) && (G != 128 || aligned(scale, 4)) && (G != 128 || aligned(zero, 2));
}

// Whether the one-token kernels fuse an input order (take_inputs) for this shape:
// one row, group 128, order 16-byte aligned.
bool int4_gemv_takes_order(int M, int N, int K, int G, const void* x, const void* packed, const void* scale,
                           const void* zero, const void* order) {
  return M == 1 && G == 128 && aligned(order, 16) && int4_gemv_supports(M, N, K, G, x, packed, scale, zero);
}

template <int DT, int U8>
static void launch_gemv_u8(const void* x, const uint8_t* packed, const void* scale, const uint8_t* zero,
                           const void* bias, void* y, int N, int K, int G, const int32_t* order, int kind,
                           GemvPrologue pro, hipStream_t stream) {
  const dim3 grid((N + 8 * U8 - 1) / (8 * U8)), block(64 * (K / 256));
  const auto* xs = static_cast<const uint16_t*>(x);
  const auto* ss = static_cast<const uint16_t*>(scale);
  const auto* bs = static_cast<const uint16_t*>(bias);
  auto* ys = static_cast<uint16_t*>(y);
  if constexpr (DT == LNQ_BF16) {
    if (kind == gemv::PRO_NORM) {
      hipLaunchKernelGGL((int4_gemv_kernel<DT, U8, true, false, gemv::PRO_NORM>), grid, block, 0, stream, xs, packed, ss,
                         zero, bs, ys, N, K, G, nullptr, pro);
      return;
    }
    if (kind == gemv::PRO_SILU) {
      hipLaunchKernelGGL((int4_gemv_kernel<DT, U8, true, false, gemv::PRO_SILU>), grid, block, 0, stream, xs, packed, ss,
                         zero, bs, ys, N, K, G, nullptr, pro);
      return;
    }
  }
  if (order != nullptr)
    hipLaunchKernelGGL((int4_gemv_kernel<DT, U8, true, true>), grid, block, 0, stream, xs, packed, ss, zero, bs, ys, N,
                       K, G, order, pro);
  else if (G == 128)
    hipLaunchKernelGGL((int4_gemv_kernel<DT, U8, true>), grid, block, 0, stream, xs, packed, ss, zero, bs, ys, N, K, G,
                       nullptr, pro);
  else
    hipLaunchKernelGGL((int4_gemv_kernel<DT, U8, false>), grid, block, 0, stream, xs, packed, ss, zero, bs, ys, N, K,
                       G, nullptr, pro);
}

template <int DT>
static void launch_gemv_dt(const void* x, const uint8_t* packed, const void* scale, const uint8_t* zero,
                           const void* bias, void* y, int N, int K, int G, const int32_t* order, int kind,
                           GemvPrologue pro, hipStream_t stream) {
#define LNQ_GEMV_U8(U_) launch_gemv_u8<DT, U_>(x, packed, scale, zero, bias, y, N, K, G, order, kind, pro, stream)
  // Rows a workgroup, 8 * U8: the rounds of one workgroup a CU that 64-row
  // workgroups need, then the fewest rows that fill that many rounds (up to one
  // round: ceil(N / 2048) on 256 CUs; N = 28672: two full rounds of 56 rows,
  // not 1.75 of 64, the second leaving a quarter of the CUs idle).
  const int cus = compute_units();
  const int rounds = (N + 64 * cus - 1) / (64 * cus);
  switch ((N + 8 * cus * rounds - 1) / (8 * cus * rounds)) {
    case 1: LNQ_GEMV_U8(1); break;
    case 2: LNQ_GEMV_U8(2); break;
    case 3: LNQ_GEMV_U8(3); break;
    case 4: LNQ_GEMV_U8(4); break;
    case 5: LNQ_GEMV_U8(5); break;
    case 6: LNQ_GEMV_U8(6); break;
    case 7: LNQ_GEMV_U8(7); break;
    default: LNQ_GEMV_U8(8); break;
  }
#undef LNQ_GEMV_U8
}

template <int DT, int U8, int MX>
static void launch_rows_u8(const void* x, const uint8_t* packed, const void* scale, const uint8_t* zero,
                           const void* bias, void* y, int M, int N, int K, int G, hipStream_t stream) {
  const dim3 grid((N + 8 * U8 - 1) / (8 * U8)), block(64 * (K / 256));
  const auto* xs = static_cast<const uint16_t*>(x);
  const auto* ss = static_cast<const uint16_t*>(scale);
  const auto* bs = static_cast<const uint16_t*>(bias);
  auto* ys = static_cast<uint16_t*>(y);
  if (G == 128)
    hipLaunchKernelGGL((int4_gemv_rows_kernel<DT, U8, true, MX>), grid, block, 0, stream, xs, packed, ss, zero, bs, ys,
                       M, N, K, G);
  else
    hipLaunchKernelGGL((int4_gemv_rows_kernel<DT, U8, false, MX>), grid, block, 0, stream, xs, packed, ss, zero, bs,
                       ys, M, N, K, G);
}

template <int DT, int MX>
static void launch_rows_dt(const void* x, const uint8_t* packed, const void* scale, const uint8_t* zero,
                           const void* bias, void* y, int M, int N, int K, int G, hipStream_t stream) {
  // Rows a workgroup: ceil(N / 2048) up to 64 (one round on 256 CUs); past that
  // 64, unless 64-row workgroups would leave their last round less than half
  // full: then the fewest rows that fill whole rounds (each workgroup reads all
  // of x, so more of them cost more where the last round is nearly full anyway:
  // N = 28672 at 4 / 16 rows 15.5 / 21.4 us on 448 workgroups of 64 rows against
  // 16.3 / 22.0 on 512 of 56; N = 20000 14.96 / 20.96 on 313 of 64 against 12.58
  // / 18.47 on 500 of 40).
  const int cus = compute_units();
  const int rounds = (N + 64 * cus - 1) / (64 * cus);
  const int last = ((N + 63) / 64) % cus;
  const int u8 = rounds > 1 && (last == 0 || 2 * last >= cus) ? 8 : (N + 8 * cus * rounds - 1) / (8 * cus * rounds);
  switch (u8) {
    case 1: launch_rows_u8<DT, 1, MX>(x, packed, scale, zero, bias, y, M, N, K, G, stream); break;
    case 2: launch_rows_u8<DT, 2, MX>(x, packed, scale, zero, bias, y, M, N, K, G, stream); break;
    case 3: launch_rows_u8<DT, 3, MX>(x, packed, scale, zero, bias, y, M, N, K, G, stream); break;
    case 4: launch_rows_u8<DT, 4, MX>(x, packed, scale, zero, bias, y, M, N, K, G, stream); break;
    case 5: launch_rows_u8<DT, 5, MX>(x, packed, scale, zero, bias, y, M, N, K, G, stream); break;
    case 6: launch_rows_u8<DT, 6, MX>(x, packed, scale, zero, bias, y, M, N, K, G, stream); break;
    case 7: launch_rows_u8<DT, 7, MX>(x, packed, scale, zero, bias, y, M, N, K, G, stream); break;
    default: launch_rows_u8<DT, 8, MX>(x, packed, scale, zero, bias, y, M, N, K, G, stream); break;
  }
}

template <int DT, int U8, bool XT>
static void launch_rows32_u8(const void* x, const uint8_t* packed, const void* scale, const uint8_t* zero,
                             const void* bias, void* y, int M, int N, int K, int G, hipStream_t stream) {
  const dim3 grid((N + 8 * U8 - 1) / (8 * U8)), block(64 * (K / 256));
  const auto* xs = static_cast<const uint16_t*>(x);
  const auto* ss = static_cast<const uint16_t*>(scale);
  const auto* bs = static_cast<const uint16_t*>(bias);
  auto* ys = static_cast<uint16_t*>(y);
  if (G == 128)
    hipLaunchKernelGGL((int4_gemv_rows32_kernel<DT, U8, true, false, XT>), grid, block, 0, stream, xs, packed, ss, zero,
                       bs, ys, M, N, K, G, nullptr);
  else
    hipLaunchKernelGGL((int4_gemv_rows32_kernel<DT, U8, false, false, XT>), grid, block, 0, stream, xs, packed, ss,
                       zero, bs, ys, M, N, K, G, nullptr);
}

// Rows a workgroup of the 32-row GEMV, 8 * u8: u8 = ceil(N / 2048) as the
// one-token GEMV, except that 7 becomes 8 (N = 14336 at 32 rows: 224 workgroups
// of 64 rows in 13.3 us against 256 of 56 in 14.5, x tiles and row-major x alike).
template <int DT, bool XT>
static void launch_rows32_dt(const void* x, const uint8_t* packed, const void* scale, const uint8_t* zero,
                             const void* bias, void* y, int M, int N, int K, int G, hipStream_t stream) {
  switch ((N + 2047) / 2048) {
    case 1: launch_rows32_u8<DT, 1, XT>(x, packed, scale, zero, bias, y, M, N, K, G, stream); break;
    case 2: launch_rows32_u8<DT, 2, XT>(x, packed, scale, zero, bias, y, M, N, K, G, stream); break;
    case 3: launch_rows32_u8<DT, 3, XT>(x, packed, scale, zero, bias, y, M, N, K, G, stream); break;
    case 4: launch_rows32_u8<DT, 4, XT>(x, packed, scale, zero, bias, y, M, N, K, G, stream); break;
    case 5: launch_rows32_u8<DT, 5, XT>(x, packed, scale, zero, bias, y, M, N, K, G, stream); break;
    case 6: launch_rows32_u8<DT, 6, XT>(x, packed, scale, zero, bias, y, M, N, K, G, stream); break;
    default: launch_rows32_u8<DT, 8, XT>(x, packed, scale, zero, bias, y, M, N, K, G, stream); break;
  }
}

template <int DT, int U8, bool XT>
static void launch_split_u8(const void* x, const uint8_t* packed, const void* scale, const uint8_t* zero, int M,
                            int N, int K, int G, int S, float* part, hipStream_t stream) {
  const dim3 grid((N + 8 * U8 - 1) / (8 * U8), S), block(64 * (K / (256 * S)));
  const auto* xs = static_cast<const uint16_t*>(x);
  const auto* ss = static_cast<const uint16_t*>(scale);
  if (G == 128)
    hipLaunchKernelGGL((int4_gemv_rows32_kernel<DT, U8, true, true, XT>), grid, block, 0, stream, xs, packed, ss, zero,
                       nullptr, nullptr, M, N, K, G, part);
  else
    hipLaunchKernelGGL((int4_gemv_rows32_kernel<DT, U8, false, true, XT>), grid, block, 0, stream, xs, packed, ss,
                       zero, nullptr, nullptr, M, N, K, G, part);
}

template <int DT, bool XT>
static void launch_split_dt(const void* x, const uint8_t* packed, const void* scale, const uint8_t* zero,
                            const void* bias, void* y, int M, int N, int K, int G, int u8, int S, float* part,
                            hipStream_t stream, bool reduce) {
  if (u8 == 8) launch_split_u8<DT, 8, XT>(x, packed, scale, zero, M, N, K, G, S, part, stream);
  else launch_split_u8<DT, 16, XT>(x, packed, scale, zero, M, N, K, G, S, part, stream);
  if (!reduce) return;
  const size_t quads = static_cast<size_t>(M) * N / 4;
  hipLaunchKernelGGL((int4_split_reduce_kernel<DT>), dim3(static_cast<unsigned>((quads + 255) / 256)), dim3(256), 0,
                     stream, part, static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y), M, N, S);
}

// rows x K values, row-major, to x tiles (x_tile_index; chunks of 32 rows, rows
// past `rows` of the last chunk zero): thread t of workgroup (chunk, slice)
// moves the 16-byte pieces t, t + 256, t + 512, t + 768 of the slice's 16 KB,
// each put in pair order.
__global__ __launch_bounds__(256) void x_tiles_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ xt,
                                                      int rows, int K) {
  const int chunk = blockIdx.y, s = blockIdx.x;
  uint16_t* out = xt + static_cast<size_t>(chunk) * K * 32 + static_cast<size_t>(s) * 16 * 64 * 8;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int piece = threadIdx.x + 256 * r;  // operand piece / 64, lane piece % 64
    const int op = piece >> 6, lane = piece & 63;
    const int m = 32 * chunk + 16 * (op >> 3) + (lane & 15);
    const int k = 256 * s + 128 * ((op >> 2) & 1) + 32 * (op & 3) + 8 * (lane >> 4);
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (m < rows) v = permute_x8(*reinterpret_cast<const u32x4*>(x + static_cast<size_t>(m) * K + k));
    *reinterpret_cast<u32x4*>(out + static_cast<size_t>(piece) * 8) = v;
  }
}

LnqStatus launch_x_tiles(const void* x, void* xt, int rows, int K, hipStream_t stream) {
  if (rows <= 0) return LNQ_OK;
  const dim3 grid(K / 256, (rows + 31) / 32);
  hipLaunchKernelGGL(x_tiles_kernel, grid, dim3(256), 0, stream, static_cast<const uint16_t*>(x),
                     static_cast<uint16_t*>(xt), rows, K);
  return launched("x_tiles");
}

template <int DT, int U8, int S>
static void launch_slices_u8(const void* x, const uint8_t* packed, const void* scale, const uint8_t* zero,
                             const void* bias, void* y, int N, int K, int G, const int32_t* order, int kind,
                             GemvPrologue pro, hipStream_t stream) {
  const dim3 grid((N + 8 * U8 - 1) / (8 * U8)), block(64 * (K / (256 * S)));
  const auto* xs = static_cast<const uint16_t*>(x);
  const auto* ss = static_cast<const uint16_t*>(scale);
  const auto* bs = static_cast<const uint16_t*>(bias);
  auto* ys = static_cast<uint16_t*>(y);
  if constexpr (DT == LNQ_BF16) {
    if (kind == gemv::PRO_NORM) {
      hipLaunchKernelGGL((int4_gemv_slices_kernel<DT, U8, true, S, false, gemv::PRO_NORM>), grid, block, 0, stream, xs, packed, ss,
                         zero, bs, ys, N, K, G, nullptr, pro);
      return;
    }
    if (kind == gemv::PRO_SILU) {
      hipLaunchKernelGGL((int4_gemv_slices_kernel<DT, U8, true, S, false, gemv::PRO_SILU>), grid, block, 0, stream, xs, packed, ss,
                         zero, bs, ys, N, K, G, nullptr, pro);
      return;
    }
  }
  if (order != nullptr)
    hipLaunchKernelGGL((int4_gemv_slices_kernel<DT, U8, true, S, true>), grid, block, 0, stream, xs, packed, ss, zero,
                       bs, ys, N, K, G, order, pro);
  else if (G == 128)
    hipLaunchKernelGGL((int4_gemv_slices_kernel<DT, U8, true, S>), grid, block, 0, stream, xs, packed, ss, zero, bs, ys,
                       N, K, G, nullptr, pro);
  else
    hipLaunchKernelGGL((int4_gemv_slices_kernel<DT, U8, false, S>), grid, block, 0, stream, xs, packed, ss, zero, bs,
                       ys, N, K, G, nullptr, pro);
}

template <int DT>
static void launch_slices_dt(const void* x, const uint8_t* packed, const void* scale, const uint8_t* zero,
                             const void* bias, void* y, int N, int K, int G, const int32_t* order, int kind,
                             GemvPrologue pro, hipStream_t stream) {
  const int sl = gemv_slices(K), u8 = (N + 2047) / 2048;
#define LNQ_SLICES(S_, U_) \
  if (sl == S_ && u8 == U_)  \
    return launch_slices_u8<DT, U_, S_>(x, packed, scale, zero, bias, y, N, K, G, order, kind, pro, stream);
  LNQ_SLICES(2, 1) LNQ_SLICES(2, 2) LNQ_SLICES(2, 3) LNQ_SLICES(2, 4)
  LNQ_SLICES(3, 1) LNQ_SLICES(3, 2) LNQ_SLICES(4, 1) LNQ_SLICES(4, 2)
#undef LNQ_SLICES
}

// Whether the one-token kernels fold a prologue (1 RMSNorm, 2 SiLU(x) * u) into
// their x staging for this shape: one row, bf16, group 128, the prologue's
// operand 16-byte aligned, and at most 32768 outputs. Every workgroup repeats
// the prologue; past two rounds of 64-row workgroups on 256 CUs that costs more
// than the separate kernel (measured on the lm_head, N = 128256: 64.1 us folded
// against 60.0 for the norm kernel and the GEMV; N = 28672: 15.4 against 16.7).
bool int4_gemv_takes_prologue(int M, int N, int K, int G, int dtype, const void* x, const void* packed,
                              const void* scale, const void* zero, int prologue, const void* operand) {
  return M == 1 && dtype == LNQ_BF16 && G == 128 && (prologue == gemv::PRO_NORM || prologue == gemv::PRO_SILU) &&
         N <= 32768 && aligned(operand, 16) && int4_gemv_supports(M, N, K, G, x, packed, scale, zero);
}

// The split 32-row GEMV (1..32 rows): R = 8 * u8 rows a workgroup (u8 8 or 16),
// K in S chunks of at most wmax(u8) slices of 256 inputs (16 or 8),
// the chunks' f32 sums in part (S * M * N floats, 16-byte aligned), then added
// in order.
bool int4_gemv_split_supports(int M, int N, int K, int G, int u8, int S, const void* x, const void* packed,
                              const void* scale, const void* zero, const void* part) {
  if (M < 1 || M > gemv::MAX_ROWS || N <= 0 || N % 4 != 0 || S < 1) return false;
  if (!(u8 == 8 || u8 == 16)) return false;
  if (K <= 0 || K % (256 * S) != 0 || K / (256 * S) > gemv::wmax(u8)) return false;
  if (!(G == 128 || G % 256 == 0) || K % G != 0) return false;
  if (static_cast<size_t>(N) * (K / 2) >= (1ull << 31) || static_cast<size_t>(M) * K * 2 >= (1ull << 31)) return false;
  return aligned(x, 16) && aligned(packed, 16) && aligned(part, 16) && (G != 128 || aligned(scale, 4)) &&
         (G != 128 || aligned(zero, 2));
}

LnqStatus launch_int4_gemv_split(const void* x, const uint8_t* packed, const void* scale, const uint8_t* zero,
                                 const void* bias, void* y, int M, int N, int K, int G, int dtype, int u8, int S,
                                 float* part, hipStream_t stream, bool tiles, bool reduce) {
  if (!int4_gemv_split_supports(M, N, K, G, u8, S, x, packed, scale, zero, part)) {
    set_error("launch_int4_gemv_split: the split GEMV does not take rows=%d N=%d K=%d group=%d u8=%d splits=%d", M,
              N, K, G, u8, S);
    return LNQ_ERROR;
  }
  if (dtype == LNQ_BF16) {
    if (tiles) launch_split_dt<LNQ_BF16, true>(x, packed, scale, zero, bias, y, M, N, K, G, u8, S, part, stream, reduce);
    else launch_split_dt<LNQ_BF16, false>(x, packed, scale, zero, bias, y, M, N, K, G, u8, S, part, stream, reduce);
  } else {
    if (tiles) launch_split_dt<LNQ_F16, true>(x, packed, scale, zero, bias, y, M, N, K, G, u8, S, part, stream, reduce);
    else launch_split_dt<LNQ_F16, false>(x, packed, scale, zero, bias, y, M, N, K, G, u8, S, part, stream, reduce);
  }
  return launched("int4_gemv_split");
}

// The 32-row GEMV (1..32 rows, K <= 4096) on x tiles of one 32-row chunk; the
// shape limits of int4_gemv_supports at 17..32 rows.
LnqStatus launch_int4_gemv_tiles(const void* xt, const uint8_t* packed, const void* scale, const uint8_t* zero,
                                 const void* bias, void* y, int M, int N, int K, int G, int dtype, hipStream_t stream) {
  if (M < 1 || M > 32 || !int4_gemv_supports(32, N, K, G, xt, packed, scale, zero)) {
    set_error("launch_int4_gemv_tiles: the 32-row GEMV does not take rows=%d N=%d K=%d group=%d", M, N, K, G);
    return LNQ_ERROR;
  }
  if (dtype == LNQ_BF16) launch_rows32_dt<LNQ_BF16, true>(xt, packed, scale, zero, bias, y, M, N, K, G, stream);
  else launch_rows32_dt<LNQ_F16, true>(xt, packed, scale, zero, bias, y, M, N, K, G, stream);
  return launched("int4_gemv_tiles");
}

LnqStatus launch_int4_gemv(const void* x, const uint8_t* packed, const void* scale, const uint8_t* zero,
                           const void* bias, void* y, int M, int N, int K, int G, int dtype, hipStream_t stream,
                           const int32_t* order, int prologue, const float* norm_weight, const void* u, float eps) {
  if (order != nullptr && !int4_gemv_takes_order(M, N, K, G, x, packed, scale, zero, order)) {
    set_error("launch_int4_gemv: the one-token kernels take no input order for this shape");
    return LNQ_ERROR;
  }
  if (prologue != gemv::PRO_NONE &&
      (order != nullptr ||
       !int4_gemv_takes_prologue(M, N, K, G, dtype, x, packed, scale, zero, prologue,
                                 prologue == gemv::PRO_NORM ? static_cast<const void*>(norm_weight) : u))) {
    set_error("launch_int4_gemv: the one-token kernels fold no such prologue for this shape");
    return LNQ_ERROR;
  }
  const GemvPrologue pro{norm_weight, static_cast<const uint16_t*>(u), eps};
  if (M == 1 && gemv_slices_supports(N, K, G, x, packed, scale, zero)) {
    if (dtype == LNQ_BF16)
      launch_slices_dt<LNQ_BF16>(x, packed, scale, zero, bias, y, N, K, G, order, prologue, pro, stream);
    else launch_slices_dt<LNQ_F16>(x, packed, scale, zero, bias, y, N, K, G, order, prologue, pro, stream);
  } else if (M == 1) {
    if (dtype == LNQ_BF16)
      launch_gemv_dt<LNQ_BF16>(x, packed, scale, zero, bias, y, N, K, G, order, prologue, pro, stream);
    else launch_gemv_dt<LNQ_F16>(x, packed, scale, zero, bias, y, N, K, G, order, prologue, pro, stream);
  } else if (M <= 4) {
    if (dtype == LNQ_BF16) launch_rows_dt<LNQ_BF16, 4>(x, packed, scale, zero, bias, y, M, N, K, G, stream);
    else launch_rows_dt<LNQ_F16, 4>(x, packed, scale, zero, bias, y, M, N, K, G, stream);
  } else if (M <= 16) {
    if (dtype == LNQ_BF16) launch_rows_dt<LNQ_BF16, 16>(x, packed, scale, zero, bias, y, M, N, K, G, stream);
    else launch_rows_dt<LNQ_F16, 16>(x, packed, scale, zero, bias, y, M, N, K, G, stream);
  } else {
    if (dtype == LNQ_BF16) launch_rows32_dt<LNQ_BF16, false>(x, packed, scale, zero, bias, y, M, N, K, G, stream);
    else launch_rows32_dt<LNQ_F16, false>(x, packed, scale, zero, bias, y, M, N, K, G, stream);
  }
  return launched("int4_gemv");
}

}  // namespace lnq
