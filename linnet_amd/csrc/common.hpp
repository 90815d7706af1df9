// Shared helpers of the gfx950 weight-quantized linear kernels: vector types,
// bf16/f16 conversions, wave reductions, and the C ABI's error plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/linnet_quant.h"

namespace lnq {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Error plumbing (abi.cpp): a thread-local message behind lnq_last_error().
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// A failed HIP call becomes LNQ_ERROR with the call named.
#define LNQ_HIP_CHECK(expr)                                                             \
  do {                                                                                  \
    hipError_t lnq_err_ = (expr);                                                       \
    if (lnq_err_ != hipSuccess) {                                                       \
      ::lnq::set_error("%s failed: %s", #expr, hipGetErrorString(lnq_err_));            \
      return LNQ_ERROR;                                                                 \
    }                                                                                   \
  } while (0)

#define LNQ_REQUIRE(cond, ...)          \
  do {                                  \
    if (!(cond)) {                      \
      ::lnq::set_error(__VA_ARGS__);    \
      return LNQ_ERROR;                 \
    }                                   \
  } while (0)

// The launch's own error, checked right after it is enqueued.
inline LnqStatus launched(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(err));
    return LNQ_ERROR;
  }
  clear_error();
  return LNQ_OK;
}

// Compute units of the current device (256 if HIP cannot say), cached per device.
inline int compute_units() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

inline bool aligned(const void* p, size_t bytes) {
  return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

// ------------------------------------------------------------ conversions

__host__ __device__ inline float bf16_bits_to_f32(uint32_t bits) {
  return __builtin_bit_cast(float, bits << 16);
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// f32 -> bf16 bits, round to nearest even: gfx950's v_cvt_pk_bf16_f32.
// "x tiles": rows x K activations in the MFMA A-operand order of the 32-row
// GEMVs, so that each operand they load is 1 KB of contiguous memory (a wave
// instruction reading 16 rows x 64 bytes of row-major x runs at a third of the
// rate of one reading whole 128-byte lines). Rows come in chunks of 32 (K * 32
// values each); a chunk holds K / 256 slices of 16 operands 8 b + 4 H + t, and
// lane 16 j + c of an operand holds row 16 b + c, inputs 256 s + 128 H + 32 t +
// 8 j .. + 7 in pair order (0, 4, 1, 5, 2, 6, 3, 7: the order of the widened
// weights, see permute_x8), so the GEMVs multiply them as loaded. The index of
// value (m, k) (K % 256 == 0):
__host__ __device__ inline size_t x_tile_index(int m, int k, int K) {
  const int chunk = m >> 5, b = (m >> 4) & 1, c = m & 15;
  const int s = k >> 8, H = (k >> 7) & 1, t = (k >> 5) & 3, j = (k >> 3) & 3, e = k & 7;
  return static_cast<size_t>(chunk) * K * 32 +
         ((static_cast<size_t>(s) * 16 + 8 * b + 4 * H + t) * 64 + 16 * j + c) * 8 + 2 * (e & 3) + (e >> 2);
}

__device__ inline uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Two f32 values as a packed bf16 pair (low = a), one v_cvt_pk_bf16_f32.
__device__ inline uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

__device__ inline float f16_bits_to_f32(uint32_t bits) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}

// f32 -> f16 bits, round to nearest even, from the f32 value as it stands: the
// empty asm keeps the compiler from folding a preceding f32 multiply into a
// single-rounding mixed-precision FMA (v_fma_mixlo_f16), which would skip the
// f32 rounding every reference computes first.
__device__ inline uint16_t f32_to_f16_bits(float f) {
  __asm__ volatile("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Two f32 values exact in f16 (or whose double rounding does not matter) as a
// packed f16 pair (low = a), one v_cvt_pk_f16_f32.
__device__ inline uint32_t pack_f16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
}

// Element type of activations / scales / outputs, as a compile-time tag.
template <int DT>
struct Elem;

template <>
struct Elem<LNQ_BF16> {
  using storage = uint16_t;
  // (MAGIC | q) as this type is MAGIC_VALUE + q for a 4-bit q.
  static constexpr uint32_t MAGIC2 = 0x43004300u;  // bf16 128.0 in both halves
  static constexpr float MAGIC_VALUE = 128.0f;
  static constexpr uint32_t ONE2 = 0x3f803f80u;  // bf16 1.0 in both halves
  __device__ static float load(const storage* p) { return bf16_bits_to_f32(*p); }
  __device__ static float to_f32(storage v) { return bf16_bits_to_f32(v); }
  __device__ static storage from_f32(float f) { return f32_to_bf16_bits(f); }
};

template <>
struct Elem<LNQ_F16> {
  using storage = uint16_t;
  static constexpr uint32_t MAGIC2 = 0x64006400u;  // f16 1024.0 in both halves
  static constexpr float MAGIC_VALUE = 1024.0f;
  static constexpr uint32_t ONE2 = 0x3c003c00u;  // f16 1.0 in both halves
  __device__ static float load(const storage* p) { return f16_bits_to_f32(*p); }
  __device__ static float to_f32(storage v) { return f16_bits_to_f32(v); }
  __device__ static storage from_f32(float f) { return f32_to_f16_bits(f); }
};

template <>
struct Elem<LNQ_F32> {
  using storage = float;
  __device__ static float load(const storage* p) { return *p; }
  __device__ static float to_f32(storage v) { return v; }
  __device__ static storage from_f32(float f) { return f; }
};

// MFMA 16x16x32 on 8 bf16 / f16 values per lane (as four packed dwords).
template <int DT>
__device__ inline f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c);

template <>
__device__ inline f32x4 mfma16x16x32<LNQ_BF16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

template <>
__device__ inline f32x4 mfma16x16x32<LNQ_F16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// 8 packed 4-bit codes (nibble i = element i) as 8 half-precision values
// MAGIC + q in element order: dword s holds elements 2s (low) and 2s+1 (high).
template <int DT>
__device__ inline u32x4 nibbles_to_magic(uint32_t w) {
  const uint32_t lo = w & 0x0f0f0f0fu;         // bytes: q0 q2 q4 q6
  const uint32_t hi = (w >> 4) & 0x0f0f0f0fu;  // bytes: q1 q3 q5 q7
  u32x4 out;
  // v_perm_b32: selector bytes 0-3 pick from the second operand, 4-7 from the
  // first, 0x0c gives zero. Dword s = [lo.byte s, 0, hi.byte s, 0].
  out.x = __builtin_amdgcn_perm(hi, lo, 0x0c040c00u) | Elem<DT>::MAGIC2;
  out.y = __builtin_amdgcn_perm(hi, lo, 0x0c050c01u) | Elem<DT>::MAGIC2;
  out.z = __builtin_amdgcn_perm(hi, lo, 0x0c060c02u) | Elem<DT>::MAGIC2;
  out.w = __builtin_amdgcn_perm(hi, lo, 0x0c070c03u) | Elem<DT>::MAGIC2;
  return out;
}

// 8 packed 4-bit codes as MAGIC + q, pair order: dword s holds elements s (low)
// and s + 4 (high) -- one v_and_or per dword after a shift. The A operand must
// then hold x in the order 0,4,1,5,2,6,3,7 of each 8 (see permute_x8).
// (a & b) | c, selected as one v_and_or_b32 when the caller has hidden the
// constants b and c behind hide_in_vgpr (a gfx950 VOP3 instruction takes no
// literal constant, so the compiler would otherwise split it into v_and + v_or
// with literals). Plain code, not an asm statement: the hazard recognizer does
// not count an asm statement as a VALU write, so an MFMA that reads its result
// right after it gets no wait states and can read the register's old value.
__device__ inline uint32_t and_or(uint32_t a, uint32_t b, uint32_t c) { return (a & b) | c; }

// Makes v an opaque VGPR value (no instruction): the compiler then cannot fold
// it into a literal operand.
__device__ inline void hide_in_vgpr(uint32_t& v) { __asm__ volatile("" : "+v"(v)); }

// `mask` and `magic` are 0x000f000f and Elem<DT>::MAGIC2, held in VGPRs by the caller.
template <int DT>
__device__ inline u32x4 nibbles_to_magic_paired(uint32_t w, uint32_t mask, uint32_t magic) {
  u32x4 out;
  out.x = and_or(w, mask, magic);
  out.y = and_or(w >> 4, mask, magic);
  out.z = and_or(w >> 8, mask, magic);
  out.w = and_or(w >> 12, mask, magic);
  return out;
}

// 8 consecutive 16-bit values (4 dwords) reordered 0,4,1,5,2,6,3,7.
__device__ inline u32x4 permute_x8(u32x4 v) {
  u32x4 out;
  out.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);
  out.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);
  out.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);
  out.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);
  return out;
}

// `v` with every bit unknown to the compiler: keeps it from folding a preceding
// mask into each later byte extraction (v_bfe + v_cvt_f32_ubyte0 per byte
// instead of one v_cvt_f32_ubyteN).
__device__ inline uint32_t opaque(uint32_t v) {
  __asm__ volatile("" : "+v"(v));
  return v;
}

// A raw buffer descriptor (stride 0) over `bytes` bytes: lanes out of range read 0.
__device__ inline __amdgpu_buffer_rsrc_t buffer_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}


// LDS address space pointer, the destination type of buffer_load ... lds.
typedef __attribute__((address_space(3))) void* lds_ptr;

// s_waitcnt vmcnt(N): at most N vector-memory loads of this wave still in
// flight. Loads retire in issue order, so this waits for all but the N most
// recently issued.
template <int N>
__device__ inline void wait_vm() {
  __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier for LDS written with ds_write: waits for this wave's LDS
// operations only, not for its vector-memory loads still in flight (a fence
// would wait for every buffer_load ... lds too). The memory clobber keeps the
// compiler from moving LDS accesses across it.
__device__ inline void lds_barrier() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// x[o] for the 8 indices of o0, o1 (int32, as loaded), read from the n values at
// xall in LDS, packed two a dword in index order; an index outside [0, n) reads 0.
__device__ inline u32x4 gather_x8(const uint16_t* xall, u32x4 o0, u32x4 o1, uint32_t n) {
  auto at = [&](uint32_t i) -> uint32_t {
    const uint32_t v = xall[i < n ? i : 0u];
    return i < n ? v : 0u;
  };
  return u32x4{at(o0.x) | (at(o0.y) << 16), at(o0.z) | (at(o0.w) << 16), at(o1.x) | (at(o1.y) << 16),
               at(o1.z) | (at(o1.w) << 16)};
}

// wait_vm with a count known only after unrolling (folds to one s_waitcnt).
__device__ inline void wait_vm_rt(int n) {
  switch (n) {
#define LNQ_WAIT_CASE(i) \
  case i:                \
    wait_vm<i>();        \
    break;
    LNQ_WAIT_CASE(0) LNQ_WAIT_CASE(1) LNQ_WAIT_CASE(2) LNQ_WAIT_CASE(3) LNQ_WAIT_CASE(4)
    LNQ_WAIT_CASE(5) LNQ_WAIT_CASE(6) LNQ_WAIT_CASE(7) LNQ_WAIT_CASE(8) LNQ_WAIT_CASE(9)
    LNQ_WAIT_CASE(10) LNQ_WAIT_CASE(11) LNQ_WAIT_CASE(12) LNQ_WAIT_CASE(13) LNQ_WAIT_CASE(14)
    LNQ_WAIT_CASE(15) LNQ_WAIT_CASE(16) LNQ_WAIT_CASE(17) LNQ_WAIT_CASE(18) LNQ_WAIT_CASE(19)
#undef LNQ_WAIT_CASE
    default:
      wait_vm<0>();
      break;
  }
}

// MFMA accumulators in AGPRs: naming an AGPR in an asm clobber makes the
// compiler allocate MFMA destinations there (it uses VGPRs on its own when a
// kernel touches no AGPR). The register budget is then split evenly between
// VGPRs and AGPRs; the GEMM kernels keep their accumulator tiles in the AGPR
// half and their operands in the VGPR half.
#define LNQ_MFMA_IN_AGPRS() __asm__ volatile("" ::: "a0")

// Wave-wide reductions (64 lanes).
// Butterfly sum over the wave: every lane gets the same value, added in the
// same order on every lane.
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ inline float wave_min(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fminf(v, __shfl_xor(v, off, 64));
  return v;
}

// ------------------------------------------------ decode glue on 8 bf16 values
// The decode step's glue between linear layers, on one 16-byte chunk (8 bf16
// values, two a dword, low first), shared by its own kernels (lnq_rmsnorm,
// lnq_silu_mul) and the one-token GEMV's x staging.

__device__ inline void unpack_bf16x8(u32x4 d, float (&v)[8]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[2 * e] = bf16_bits_to_f32(d[e] & 0xffffu);
    v[2 * e + 1] = bf16_bits_to_f32(d[e] >> 16);
  }
}

// RMSNorm's sum of squares runs in one order wherever it is computed (the row
// kernel and the GEMV's norm prologue give the same factor): each chunk's 8
// squares in turn (chunk_squares), a butterfly over each 32 consecutive chunks
// held by lanes l..l+31 with lane & 31 = chunk % 32 (sum_over_32_lanes; every
// lane of the 32 gets the same bits), then the 32-chunk group sums one after
// another in chunk order.
__device__ inline float chunk_squares(const float (&v)[8]) {
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss = fmaf(v[e], v[e], ss);
  return ss;
}

__device__ inline float sum_over_32_lanes(float v) {
#pragma unroll
  for (int off = 1; off < 32; off <<= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// RMSNorm's output for a chunk: v * scale * w rounded to bf16 (w: the chunk's 8
// f32 weights), scale = rsqrt(sum of squares / hidden + eps).
__device__ inline u32x4 norm_bf16x8(const float (&v)[8], float scale, f32x4 w0, f32x4 w1) {
  u32x4 out;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const f32x4& w = e < 2 ? w0 : w1;
    const uint32_t lo = f32_to_bf16_bits(v[2 * e] * scale * w[(2 * e) & 3]);
    const uint32_t hi = f32_to_bf16_bits(v[2 * e + 1] * scale * w[(2 * e + 1) & 3]);
    out[e] = lo | (hi << 16);
  }
  return out;
}

// SiLU(g) * u in f32, as the MLP computes it, g / (1 + e^-g) * u, with the
// hardware's exp2 and reciprocal (v_exp_f32, v_rcp_f32; about 1 ulp each, far
// below the bf16 rounding of the result): g * rcp(1 + exp2(-g log2 e)) * u. The
// one-token GEMV evaluates it for every input in every workgroup, where the
// IEEE divide and the library exp cost ~20 instructions an element.
__device__ inline float silu_times(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(-g * 1.44269504088896341f);
  return g * __builtin_amdgcn_rcpf(1.f + e) * u;
}

// SiLU(g) * u of one dword of each (two bf16 values, low first), rounded to bf16.
__device__ inline uint32_t silu_mul_bf16x2(uint32_t g, uint32_t u) {
  const uint32_t lo = f32_to_bf16_bits(silu_times(bf16_bits_to_f32(g & 0xffffu), bf16_bits_to_f32(u & 0xffffu)));
  const uint32_t hi = f32_to_bf16_bits(silu_times(bf16_bits_to_f32(g >> 16), bf16_bits_to_f32(u >> 16)));
  return lo | (hi << 16);
}

// The same for a chunk that lanes l and l + 32 of a wave both hold: each half
// of the wave computes two of its four dwords (lanes 0..31 dwords 0 and 1,
// lanes 32..63 dwords 2 and 3) and the halves exchange them, so every lane ends
// with the whole chunk for half the arithmetic.
__device__ inline u32x4 silu_mul_bf16x8_halves(u32x4 g, u32x4 u, int lane) {
  const bool upper = lane >= 32;
  const uint32_t m0 = silu_mul_bf16x2(upper ? g[2] : g[0], upper ? u[2] : u[0]);
  const uint32_t m1 = silu_mul_bf16x2(upper ? g[3] : g[1], upper ? u[3] : u[1]);
  const uint32_t o0 = static_cast<uint32_t>(__shfl_xor(static_cast<int>(m0), 32, 64));
  const uint32_t o1 = static_cast<uint32_t>(__shfl_xor(static_cast<int>(m1), 32, 64));
  return upper ? u32x4{o0, o1, m0, m1} : u32x4{m0, m1, o0, o1};
}

// x * w rounded to bf16 for a chunk (w: its 8 f32 weights).
__device__ inline u32x4 scale_bf16x8(u32x4 x, f32x4 w0, f32x4 w1) {
  float v[8];
  unpack_bf16x8(x, v);
  u32x4 out;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const f32x4& w = e < 2 ? w0 : w1;
    out[e] = static_cast<uint32_t>(f32_to_bf16_bits(v[2 * e] * w[(2 * e) & 3])) |
             (static_cast<uint32_t>(f32_to_bf16_bits(v[2 * e + 1] * w[(2 * e + 1) & 3])) << 16);
  }
  return out;
}

}  // namespace lnq
