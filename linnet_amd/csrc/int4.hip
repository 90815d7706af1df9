// Group-wise 4-bit weights (std.quant::Int4GroupLinear) on gfx950:
//   - int4_skinny: the decode-shape dequant-GEMV / skinny GEMM on MFMA;
//   - int4_dequant: the whole weight dequantized, bit-exact with the reference;
//   - int4_quantize: round-to-nearest quantization, bit-exact with numpy;
//   - int4_pack / int4_unpack: the u4 / i4 byte layout.
//
// Layout (stdlib/quant.linnet:156-175, linnet/quant.py:1-12): packed [N, K/G, G/2]
// u8 with element 2k in the low nibble, scale [N, K/G], zero [N, K/G] u8;
// W[n, k] = (q[n, k] - zero[n, k/G]) * scale[n, k/G].
#include "common.hpp"

namespace lnq {

// ===================================================================== skinny
//
// One workgroup (4 waves) owns 16 output features (an MFMA column tile) and
// 16*MT rows of x; its 4 waves split K into contiguous quarters and add their
// partial sums through LDS at the end. The weight is streamed once from HBM in
// 128-element chunks (64 bytes of a row): lane (col = lane % 16, j = lane / 16)
// reads 16 bytes of row n0 + col, so the 64 lanes of a wave read 16 rows x 64
// contiguous bytes per chunk, fully used cache lines.
//
// The codes are widened without arithmetic: (MAGIC | q) read as bf16 is
// 128 + q (f16: 1024 + q). MFMA 16x16x32 then sums
//   C[m, n]  = sum_k x[m, k] * (MAGIC + q[n, k])     over one group
//   Cx[m, n] = sum_k x[m, k] * 1                      (B = ones)
// and one VALU epilogue per group folds zero point and scale in f32:
//   acc[m, n] += s[n, g] * (C - (MAGIC + z[n, g]) * Cx)
// which equals s * sum_k x * (q - z) -- the product with the exactly
// dequantized weight -- up to f32 rounding of the sums.
//
// Which 8 elements a lane contributes to each MFMA (the same for its A and
// B operands) depends on the group, so that one MFMA never spans two groups:
//   LOADW 16 (group % 128 == 0): one 16-byte load; dword t -> k = 32j + 8t
//   LOADW 8  (group 64):         two 8-byte loads; k = 64(t/2) + 16j + 8(t%2)
//   LOADW 4  (group 32):         four 4-byte loads; k = 32t + 8j

// Chunks each of nw waves takes: K split evenly, rounded up to whole batches of
// 4 chunks (so a wave's batches, and its scale / zero loads, stay aligned).
__host__ __device__ inline int skinny_per_wave(int chunks, int nw) {
  return (((chunks + nw - 1) / nw) + 3) & ~3;
}

template <int LOADW>
__device__ inline int chunk_koff(int t, int j) {
  if constexpr (LOADW == 16) return 32 * j + 8 * t;
  else if constexpr (LOADW == 8) return 64 * (t >> 1) + 16 * j + 8 * (t & 1);
  else return 32 * t + 8 * j;
}

template <int LOADW>
__device__ inline void load_chunk(const uint8_t* __restrict__ chunk, int j, uint32_t (&w)[4]) {
  if constexpr (LOADW == 16) {
    u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(chunk + 16 * j));
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else if constexpr (LOADW == 8) {
    u32x2 a = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(chunk + 8 * j));
    u32x2 b = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(chunk + 32 + 8 * j));
    w[0] = a.x; w[1] = a.y; w[2] = b.x; w[3] = b.y;
  } else {
#pragma unroll
    for (int t = 0; t < 4; ++t)
      w[t] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(chunk + 16 * t + 4 * j));
  }
}

// x (the A operand) comes either from LDS (XL) or from global memory.
//
// XL (the decode case, each wave's slice of x small): every wave copies its own
// K-slice of the workgroup's rows of x into a private LDS region, reordering
// each 8 elements 0,4,1,5,2,6,3,7 so that the codes widen in pair order (one
// v_and_or per dword), and issues those loads BEFORE its weight loads: loads
// retire in order, so a chunk's math then waits only for that chunk's weights.
// Otherwise x is read from global memory PD chunks ahead, in element order,
// and the codes widen in element order (v_perm + or).
//
// The weights stream in batches of U chunks, double-buffered: batch b + 1 is
// requested before batch b is multiplied. With one group a chunk (group % 128
// == 0) a chunk's epilogue runs after the next chunk's MFMAs are issued, so the
// MFMA latency is hidden. NW waves split K.
// SV: the scales and zero points of a batch's 4 chunks (4 groups of 128) come
// in one 8-byte and one 4-byte load per lane (aligned shapes, group 128).
template <int DT, int LOADW, int MT, bool XL, bool SV, int NW>
__global__ __launch_bounds__(64 * NW) void int4_skinny_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ packed,
    const uint16_t* __restrict__ scale, const uint8_t* __restrict__ zero,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int M, int N, int K, int G) {
  using E = Elem<DT>;
  // MFMAs t = 0..3 of a chunk; a group closes after every `tpg` of them.
  constexpr int tpg = LOADW == 16 ? 4 : (LOADW == 8 ? 2 : 1);
  constexpr int GPC = 4 / tpg;      // groups a chunk spans
  constexpr int U = 4;              // chunks of weight a batch
  constexpr int PD = XL ? 1 : 2;    // chunks of x in flight ahead of use
  __shared__ f32x4 red[NW][MT][64];
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;
  const int j = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int m0 = blockIdx.y * 16 * MT;
  const int mrows = min(M - m0, 16 * MT);  // rows of x this workgroup reads
  const int nrow = min(n0 + col, N - 1);   // rows past N read row N-1, never stored
  const int chunks = K >> 7;
  const int per_wave = skinny_per_wave(chunks, NW);
  const int cb = min(chunks, wave * per_wave);
  const int ce = min(chunks, cb + per_wave);
  const int groups = K / G;

  const uint8_t* wrow = packed + static_cast<size_t>(nrow) * (K >> 1);
  const uint16_t* srow = scale + static_cast<size_t>(nrow) * groups;
  const uint8_t* zrow = zero + static_cast<size_t>(nrow) * groups;
  // Buffer descriptors (SGPRs) with 32-bit lane offsets: a chunk's offset is an
  // SGPR / immediate, so the loads need no per-lane 64-bit address arithmetic.
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(packed, static_cast<uint32_t>(static_cast<size_t>(N) * (K >> 1)));
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(scale, static_cast<uint32_t>(N * groups * 2));
  const __amdgpu_buffer_rsrc_t rz = buffer_rsrc(zero, static_cast<uint32_t>(N * groups));
  const int vw = nrow * (K >> 1) + 16 * j;
  const int vs = nrow * groups * 2;
  const int vz = nrow * groups;

  // Row of x behind A-operand row `col` of m-tile mt; rows past M read a valid
  // row and only pollute output rows that are never stored.
  int xr[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xr[mt] = min(16 * mt + col, mrows - 1);

  // XL: this wave's LDS slice, rows of 128 * per_wave + 8 elements.
  const int wstride = 128 * per_wave + 8;
  uint16_t* xw = xs + wave * mrows * wstride;
  // A wave copies mrows x (ce - cb) chunks of x, 16 units (8 elements) a chunk
  // per row. With K % 512 == 0 every wave's chunk count is a multiple of 4, so
  // each lane copies P = (ce - cb) / 4 units of every row: unit q of a lane is
  // row q / P, unit lane + 64 * (q % P) -- scalar arithmetic only. The first XU
  // are requested before the weights (waiting for them then does not wait for
  // the weights) and stored after; the loads use clamped indices so the
  // compiler can count them.
  const int P = (ce - cb) >> 2;
  const int xq = XL ? mrows * P : 0;  // units this lane copies
  const int cbx = min(cb, chunks - 1);
  auto x_src = [&](int q) -> const u32x4* {
    const int qq = min(q, max(xq, 1) - 1);
    const int r = qq / P, u8 = lane + 64 * (qq - r * P);
    return reinterpret_cast<const u32x4*>(x + static_cast<size_t>(m0 + r) * K + 128 * cbx + 8 * u8);
  };
  auto x_store = [&](int q, u32x4 v) {
    const int qq = min(q, max(xq, 1) - 1);
    const int r = qq / P, u8 = lane + 64 * (qq - r * P);
    *reinterpret_cast<u32x4*>(xw + r * wstride + 8 * u8) = permute_x8(v);
  };
  constexpr int XU = 4;
  u32x4 xv[XU];
  if constexpr (XL) {
    if (xq > 0) {
#pragma unroll
      for (int q = 0; q < XU; ++q) xv[q] = *x_src(q);
    }
  }

  u32x4 ones;
  ones.x = ones.y = ones.z = ones.w = E::ONE2;
  // Constants of the pair-order widening, kept in VGPRs (see and_or).
  const uint32_t nib_mask = 0x000f000fu;
  const uint32_t nib_magic = E::MAGIC2;
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto load_x = [&](int c, u32x4 (&dst)[MT][4]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int k = 128 * c + chunk_koff<LOADW>(t, j);
        if constexpr (XL)
          dst[mt][t] = *reinterpret_cast<const u32x4*>(xw + xr[mt] * wstride + (k - 128 * cb));
        else
          dst[mt][t] = *reinterpret_cast<const u32x4*>(x + static_cast<size_t>(m0 + xr[mt]) * K + k);
      }
  };

  struct Batch {
    uint32_t w[U][4];
    float s[U][GPC], zz[U][GPC];
  };
  auto load_batch = [&](int c0, Batch& bt) {
    if constexpr (SV) {
      // c0 % 4 == 0 and one group a chunk: groups c0..c0+3 of this row (an
      // idle wave's c0 == chunks reads the row's last 4, unused).
      const int g0 = min(c0, chunks - 4);
      const u32x2 sv = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, vs, 2 * g0, 0));
      const uint32_t zv = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(rz, vz, g0, 0));
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t half = (u < 2 ? sv.x : sv.y) >> (16 * (u & 1));
        bt.s[u][0] = E::to_f32(static_cast<uint16_t>(half & 0xffffu));
        bt.zz[u][0] = E::MAGIC_VALUE + static_cast<float>((zv >> (8 * u)) & 0xffu);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = max(min(c0 + u, ce - 1), 0);  // past the end: re-read the last chunk, unused
      if constexpr (LOADW == 16) {
        const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, vw, 64 * c, 0));
        bt.w[u][0] = v.x; bt.w[u][1] = v.y; bt.w[u][2] = v.z; bt.w[u][3] = v.w;
      } else {
        load_chunk<LOADW>(wrow + 64 * c, j, bt.w[u]);
      }
      if constexpr (!SV) {
#pragma unroll
        for (int q = 0; q < GPC; ++q) {
          const int g = (128 * c + chunk_koff<LOADW>(q * tpg, 0)) / G;
          bt.s[u][q] = E::to_f32(srow[g]);
          bt.zz[u][q] = E::MAGIC_VALUE + static_cast<float>(zrow[g]);
        }
      }
    }
  };

  auto widen = [&](uint32_t w) -> u32x4 {
    if constexpr (XL) return nibbles_to_magic_paired<DT>(w, nib_mask, nib_magic);
    else return nibbles_to_magic<DT>(w);
  };
  auto fold = [&](const f32x4& C, const f32x4& Cx, float s, float zz, f32x4& a) {
#pragma unroll
    for (int r = 0; r < 4; ++r) a[r] = fmaf(s, fmaf(-zz, Cx[r], C[r]), a[r]);
  };

  auto run_batch = [&](int c0, const Batch& bt) {
    u32x4 xa[PD + 1][MT][4];
#pragma unroll
    for (int d = 0; d < PD; ++d)
      if (c0 + d < ce) load_x(c0 + d, xa[d]);
    if constexpr (tpg == 4) {
      // One group a chunk: chunk u's MFMAs, then chunk u-1's epilogue.
      f32x4 C[2][MT], Cx[2][MT];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u;
        if (c < ce) {
          if (u + PD < U && c + PD < ce) load_x(c + PD, xa[(u + PD) % (PD + 1)]);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            C[u & 1][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
            Cx[u & 1][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const u32x4 b = widen(bt.w[u][t]);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              const u32x4 a = xa[u % (PD + 1)][mt][t];
              C[u & 1][mt] = mfma16x16x32<DT>(a, b, C[u & 1][mt]);
              Cx[u & 1][mt] = mfma16x16x32<DT>(a, ones, Cx[u & 1][mt]);
            }
          }
        }
        if (u > 0 && c - 1 < ce) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            fold(C[(u - 1) & 1][mt], Cx[(u - 1) & 1][mt], bt.s[u - 1][0], bt.zz[u - 1][0], acc[mt]);
        }
      }
      if (c0 + U - 1 < ce) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          fold(C[(U - 1) & 1][mt], Cx[(U - 1) & 1][mt], bt.s[U - 1][0], bt.zz[U - 1][0], acc[mt]);
      }
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u;
        if (c >= ce) break;
        if (u + PD < U && c + PD < ce) load_x(c + PD, xa[(u + PD) % (PD + 1)]);
        f32x4 C[MT], Cx[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          C[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
          Cx[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const u32x4 b = widen(bt.w[u][t]);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const u32x4 a = xa[u % (PD + 1)][mt][t];
            C[mt] = mfma16x16x32<DT>(a, b, C[mt]);
            Cx[mt] = mfma16x16x32<DT>(a, ones, Cx[mt]);
          }
          if ((t + 1) % tpg == 0) {
            const int q = t / tpg;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              fold(C[mt], Cx[mt], bt.s[u][q], bt.zz[u][q], acc[mt]);
              C[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
              Cx[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
          }
        }
      }
    }
  };

  Batch even, odd;
  // Unconditional (addresses clamped for an idle wave) so the compiler can count
  // the loads in flight when it waits for x below.
  load_batch(cb, even);
  if constexpr (XL) {
    if (xq > 0) {
#pragma unroll
      for (int q = 0; q < XU; ++q) x_store(q, xv[q]);  // past xq: a repeat of the last unit
      for (int q = XU; q < xq; ++q) x_store(q, *x_src(q));
    }
    // The slice is read only by this wave; a wave's LDS requests are served in
    // order, and the fence keeps the compiler from moving reads above writes.
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  }
  for (int c0 = cb; c0 < ce; c0 += 2 * U) {
    if (c0 + U < ce) load_batch(c0 + U, odd);
    run_batch(c0, even);
    if (c0 + U >= ce) break;
    if (c0 + 2 * U < ce) load_batch(c0 + 2 * U, even);
    run_batch(c0 + U, odd);
  }

#pragma unroll
  for (int mt = 0; mt < MT; ++mt) red[wave][mt][lane] = acc[mt];
  __syncthreads();

  // One output per thread per m-tile: (lane, r) of the 16x16 tile, r < 4.
  if (threadIdx.x < 256) {
    const int olane = threadIdx.x & 63;
    const int r = threadIdx.x >> 6;
    const int n = n0 + (olane & 15);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = m0 + 16 * mt + 4 * (olane >> 4) + r;
      if (m < M && n < N) {
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) v += red[w][mt][olane][r];
        uint16_t out = E::from_f32(v);
        if (bias != nullptr) out = E::from_f32(E::to_f32(out) + E::to_f32(bias[n]));
        y[static_cast<size_t>(m) * N + n] = out;
      }
    }
  }
}

// =================================================================== dequant
// out[n, k] = (q - z) * s in f32, rounded once to the scale's dtype: the value
// the reference's `_int4_unpack` (Triton, f32 then cast) and the CPU
// `(q.to(T) - z.to(T)) * s` both give, (q - z) * s being exact in f32 for
// bf16 / f16 scales.

// 4 packed bytes (8 elements of one group) per thread, consecutive threads on
// consecutive bytes: each wave reads 256 contiguous bytes and writes 1 KB (2 KB
// for f32) contiguous. K % 8 == 0, G % 8 == 0. Grid: x over a row's 8-element
// units, y over rows (no division).
template <int DT>
__global__ __launch_bounds__(256) void int4_dequant_fast(
    const uint8_t* __restrict__ packed, const typename Elem<DT>::storage* __restrict__ scale,
    const uint8_t* __restrict__ zero, typename Elem<DT>::storage* __restrict__ out, int K, int gshift,
    int G) {
  using E = Elem<DT>;
  using S = typename E::storage;
  const int per_row = K >> 3;
  const int unit = blockIdx.x * blockDim.x + threadIdx.x;
  if (unit >= per_row) return;
  const int64_t n = blockIdx.y;
  const int k0 = unit << 3;
  const int groups = K / G;
  const int g = gshift >= 0 ? k0 >> gshift : k0 / G;
  const float s = E::load(scale + n * groups + g);
  const float zf = static_cast<float>(zero[n * groups + g]);
  const uint32_t w = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(packed + n * (K >> 1)) + unit);
  // (q - z) * s as the reference writes it: q - z is exact, and so is the product
  // for a 16-bit scale (5 bits times at most 11), then one rounding to the output
  // type; an f32 scale rounds once in f32. (fma(q, s, -z s) would equal it but
  // give +0 where q == z and s < 0; the product gives -0, as the reference does.)
  const uint32_t lo = opaque(w & 0x0f0f0f0fu);
  const uint32_t hi = opaque((w >> 4) & 0x0f0f0f0fu);
  float v[8];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const float q0 = static_cast<float>((lo >> (8 * b)) & 0xffu);
    const float q1 = static_cast<float>((hi >> (8 * b)) & 0xffu);
    v[2 * b] = (q0 - zf) * s;
    v[2 * b + 1] = (q1 - zf) * s;
  }
  S* dst = out + n * K + k0;
  if constexpr (DT == LNQ_BF16) {
    *reinterpret_cast<u32x4*>(dst) = u32x4{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                           pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
  } else if constexpr (DT == LNQ_F16) {
    *reinterpret_cast<u32x4*>(dst) = u32x4{pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3]),
                                           pack_f16x2(v[4], v[5]), pack_f16x2(v[6], v[7])};
  } else {
    reinterpret_cast<f32x4*>(dst)[0] = f32x4{v[0], v[1], v[2], v[3]};
    reinterpret_cast<f32x4*>(dst)[1] = f32x4{v[4], v[5], v[6], v[7]};
  }
}

// Any even group: one byte (two elements) per thread.
template <int DT>
__global__ __launch_bounds__(256) void int4_dequant_any(
    const uint8_t* __restrict__ packed, const typename Elem<DT>::storage* __restrict__ scale,
    const uint8_t* __restrict__ zero, typename Elem<DT>::storage* __restrict__ out,
    int64_t bytes, int K, int G) {
  using E = Elem<DT>;
  const int64_t b = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= bytes) return;
  const int64_t half = K >> 1;
  const int64_t n = b / half;
  const int k = static_cast<int>(b - n * half) << 1;
  const int groups = K / G;
  const int g = k / G;
  const float s = E::load(scale + n * groups + g);
  const float z = static_cast<float>(zero[n * groups + g]);
  const uint32_t byte = packed[b];
  out[n * K + k] = E::from_f32((static_cast<float>(byte & 15u) - z) * s);
  out[n * K + k + 1] = E::from_f32((static_cast<float>(byte >> 4) - z) * s);
}

// ================================================================== quantize
// One wave per group of G inputs of a row: min / max over the group, then the
// codes, in exactly numpy's f32 order of operations (linnet/quant.py:92-98):
// scale = (max - min) / 15 (not > 0 -> 1), zero = clip(rint(-min / scale), 0, 15),
// q = clip(rint(w / scale) + zero, 0, 15); rint rounds half to even, divisions
// are IEEE (hip-clang's default correctly rounded f32 divide).
__global__ __launch_bounds__(256) void int4_quantize_kernel(const float* __restrict__ w,
                                                            uint8_t* __restrict__ packed,
                                                            float* __restrict__ scale,
                                                            uint8_t* __restrict__ zero,
                                                            int64_t total_groups, int G) {
  const int lane = threadIdx.x & 63;
  const int64_t grp = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (grp >= total_groups) return;
  const float* p = w + grp * G;
  float lo = __builtin_huge_valf();
  float hi = -__builtin_huge_valf();
  for (int i = lane; i < G; i += 64) {
    const float v = p[i];
    lo = fminf(lo, v);
    hi = fmaxf(hi, v);
  }
  lo = wave_min(lo);
  hi = wave_max(hi);
  float s = (hi - lo) / 15.0f;
  if (!(s > 0.0f)) s = 1.0f;
  const float z = fminf(fmaxf(rintf(-lo / s), 0.0f), 15.0f);
  uint8_t* dst = packed + grp * (G >> 1);
  for (int i = 2 * lane; i < G; i += 128) {
    const float q0 = fminf(fmaxf(rintf(p[i] / s) + z, 0.0f), 15.0f);
    const float q1 = fminf(fmaxf(rintf(p[i + 1] / s) + z, 0.0f), 15.0f);
    dst[i >> 1] = static_cast<uint8_t>(static_cast<uint32_t>(q0) | (static_cast<uint32_t>(q1) << 4));
  }
  if (lane == 0) {
    scale[grp] = s;
    zero[grp] = static_cast<uint8_t>(z);
  }
}

// ============================================================ pack / unpack

__global__ __launch_bounds__(256) void int4_pack_kernel(const uint8_t* __restrict__ codes,
                                                        uint8_t* __restrict__ packed,
                                                        int64_t pairs) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= pairs) return;
  packed[i] = static_cast<uint8_t>((codes[2 * i] & 15u) | ((codes[2 * i + 1] & 15u) << 4));
}

__global__ __launch_bounds__(256) void int4_unpack_kernel(const uint8_t* __restrict__ packed,
                                                          uint8_t* __restrict__ codes,
                                                          int64_t pairs, int is_signed) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= pairs) return;
  const uint32_t b = packed[i];
  uint32_t lo = b & 15u, hi = b >> 4;
  if (is_signed) {
    lo = static_cast<uint32_t>(static_cast<int32_t>(lo ^ 8u) - 8) & 0xffu;
    hi = static_cast<uint32_t>(static_cast<int32_t>(hi ^ 8u) - 8) & 0xffu;
  }
  codes[2 * i] = static_cast<uint8_t>(lo);
  codes[2 * i + 1] = static_cast<uint8_t>(hi);
}

// std.quant::Int4Linear's weight (signed 4-bit i4, one scale a row) in the
// group layout the fused kernels read: the code c = nibble ^ 8 is v + 8 for the
// signed value v, so with zero point 8 every group gives (c - 8) * s = v * s,
// the product the reference forms before its one rounding (stdlib/quant.linnet:
// 24-29, 101-111). Thread t: bytes 16 t .. 16 t + 15 of the weight (a whole
// number of 16-byte pieces: rows of in/2 bytes, in % 32 == 0), and entry t of the
// per-group scales and zero points.
template <int DT>
__global__ __launch_bounds__(256) void int4_row_prepare_kernel(const uint8_t* __restrict__ weight,
                                                               const typename Elem<DT>::storage* __restrict__ scale,
                                                               uint8_t* __restrict__ packed,
                                                               typename Elem<DT>::storage* __restrict__ group_scale,
                                                               uint8_t* __restrict__ zero, int64_t pieces,
                                                               int64_t entries, int groups) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t < pieces) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(weight + 16 * t);
    *reinterpret_cast<u32x4*>(packed + 16 * t) = w ^ 0x88888888u;
  }
  if (t < entries) {
    group_scale[t] = scale[t / groups];
    zero[t] = 8;
  }
}

// std.quant::take_inputs (stdlib/quant.linnet:142-149): taken[r, k] = x[r, order[k]]
// over `rows` rows of n elements of type T; an index outside [0, n) reads 0.
// One thread an output element; a row's gathered reads stay within its n
// elements, which the caches hold after the first touch.
template <typename T>
__global__ __launch_bounds__(256) void take_inputs_kernel(const T* __restrict__ x, const int32_t* __restrict__ order,
                                                          T* __restrict__ taken, int64_t total, int64_t n) {
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = t / n, k = t - r * n;
    const int64_t i = order[k];
    taken[t] = (i >= 0 && i < n) ? x[r * n + i] : T(0);
  }
}

// ============================================================ launch helpers

template <int DT, int LOADW, int MT, bool XL, bool SV>
static void launch_skinny_v(const uint16_t* xs, const uint8_t* packed, const uint16_t* ss,
                            const uint8_t* zero, const uint16_t* bs, uint16_t* ys, int M, int N,
                            int K, int G, hipStream_t stream) {
  // Eight waves split K when each still gets at least one batch of chunks, up
  // to 16 rows. At 64 rows (MT = 4) two waves a SIMD leave 256 registers a wave,
  // which spills, while one wave a SIMD holds all of its tile; at 17-32 rows
  // four waves are as fast or a little faster (K = 14336: 31.0 against 31.4 us
  // at 32 rows).
  const int chunks = K >> 7;
  const bool eight = chunks >= 64 && MT < 2;
  const int nw = eight ? 8 : 4;
  const dim3 grid((N + 15) / 16, (M + 16 * MT - 1) / (16 * MT)), block(64 * nw);
  const int rows = min(M, 16 * MT);
  const int per_wave = skinny_per_wave(chunks, nw);
  const size_t lds = XL ? static_cast<size_t>(nw) * rows * (128 * per_wave + 8) * 2 : 0;
  // Every row count runs the four-row epilogue (one row leaves rows 1..3 of the
  // accumulators zero).
#define LNQ_SKINNY(NW)                                                                        \
  hipLaunchKernelGGL((int4_skinny_kernel<DT, LOADW, MT, XL, SV, NW>), grid, block, lds, stream, \
                     xs, packed, ss, zero, bs, ys, M, N, K, G)
  if constexpr (MT < 2) {
    if (eight) {
      LNQ_SKINNY(8);
      return;
    }
  }
  LNQ_SKINNY(4);
#undef LNQ_SKINNY
}

// LDS bytes a workgroup may spend on its rows of x (decode shapes fit).
constexpr int kXLdsBudget = 48 * 1024;

template <int DT, int LOADW, int MT>
static void launch_skinny_mt(const uint16_t* xs, const uint8_t* packed, const uint16_t* ss,
                             const uint8_t* zero, const uint16_t* bs, uint16_t* ys, int M, int N,
                             int K, int G, hipStream_t stream) {
  const int rows = min(M, 16 * MT);
  // Upper bound of what launch_skinny_v asks for (any NW): 8 padded slices.
  const size_t lds = static_cast<size_t>(rows) * (128 * 8 * skinny_per_wave(K >> 7, 8) + 8 * 8) * 2;
  // Vector scale loads: group 128 and rows of a multiple of 4 groups (every
  // wave's first chunk is a multiple of 4), aligned scale / zero rows.
  const bool sv = LOADW == 16 && G == 128 && (K / G) % 4 == 0 && aligned(ss, 8) && aligned(zero, 4) &&
                  static_cast<size_t>(N) * (K >> 1) < (1ull << 31);
  if (lds <= kXLdsBudget && K % 512 == 0 && static_cast<size_t>(N) * (K >> 1) < (1ull << 31)) {
    if (sv) launch_skinny_v<DT, LOADW, MT, true, true>(xs, packed, ss, zero, bs, ys, M, N, K, G, stream);
    else launch_skinny_v<DT, LOADW, MT, true, false>(xs, packed, ss, zero, bs, ys, M, N, K, G, stream);
  } else {
    if (sv) launch_skinny_v<DT, LOADW, MT, false, true>(xs, packed, ss, zero, bs, ys, M, N, K, G, stream);
    else launch_skinny_v<DT, LOADW, MT, false, false>(xs, packed, ss, zero, bs, ys, M, N, K, G, stream);
  }
}

template <int DT, int LOADW>
static LnqStatus launch_skinny_lw(const void* x, const uint8_t* packed, const void* scale,
                                  const uint8_t* zero, const void* bias, void* y, int M, int N,
                                  int K, int G, hipStream_t stream) {
  const auto* xs = static_cast<const uint16_t*>(x);
  const auto* ss = static_cast<const uint16_t*>(scale);
  const auto* bs = static_cast<const uint16_t*>(bias);
  auto* ys = static_cast<uint16_t*>(y);
  if (M <= 16)
    launch_skinny_mt<DT, LOADW, 1>(xs, packed, ss, zero, bs, ys, M, N, K, G, stream);
  else if (M <= 32)
    launch_skinny_mt<DT, LOADW, 2>(xs, packed, ss, zero, bs, ys, M, N, K, G, stream);
  else
    launch_skinny_mt<DT, LOADW, 4>(xs, packed, ss, zero, bs, ys, M, N, K, G, stream);
  return launched("int4_skinny");
}

template <int DT>
static LnqStatus launch_skinny(const void* x, const uint8_t* packed, const void* scale,
                               const uint8_t* zero, const void* bias, void* y, int M, int N,
                               int K, int G, hipStream_t stream) {
  if (G % 128 == 0)
    return launch_skinny_lw<DT, 16>(x, packed, scale, zero, bias, y, M, N, K, G, stream);
  if (G == 64) return launch_skinny_lw<DT, 8>(x, packed, scale, zero, bias, y, M, N, K, G, stream);
  return launch_skinny_lw<DT, 4>(x, packed, scale, zero, bias, y, M, N, K, G, stream);
}

// Defined in int4_gemm.hip: the prefill dequant-GEMM. `bn` is the tile width
// (128 or 256 output columns); int4_tiled_width gives the automatic one.
LnqStatus launch_int4_tiled(const void* x, const uint8_t* packed, const void* scale,
                            const uint8_t* zero, const void* bias, void* y, int M, int N, int K,
                            int G, int dtype, int bn, hipStream_t stream);
bool int4_tiled_supports(int M, int N, int K, int G, int dtype);
int int4_tiled_width(int M, int N);
LnqStatus launch_int4_persistent(const void* x, const uint8_t* packed, const void* scale, const uint8_t* zero,
                                 const void* bias, void* y, int M, int N, int K, int G, int dtype, hipStream_t stream);
bool int4_persistent_supports(int M, int N, int K, int G, int dtype);
bool int4_persistent_preferred(int M, int N, int K, int G, int dtype);

// Defined in int4_gemv.hip: the one-token dequant-GEMV.
bool int4_gemv_supports(int M, int N, int K, int G, const void* x, const void* packed, const void* scale,
                        const void* zero);
LnqStatus launch_int4_gemv(const void* x, const uint8_t* packed, const void* scale, const uint8_t* zero,
                           const void* bias, void* y, int M, int N, int K, int G, int dtype, hipStream_t stream,
                           const int32_t* order = nullptr, int prologue = 0, const float* norm_weight = nullptr,
                           const void* u = nullptr, float eps = 0.f);
bool int4_gemv_takes_order(int M, int N, int K, int G, const void* x, const void* packed, const void* scale,
                           const void* zero, const void* order);
bool int4_gemv_takes_prologue(int M, int N, int K, int G, int dtype, const void* x, const void* packed,
                              const void* scale, const void* zero, int prologue, const void* operand);

// Defined in int4_gemv.hip: the 32-row GEMV with K split over workgroups.
bool int4_gemv_split_supports(int M, int N, int K, int G, int u8, int S, const void* x, const void* packed,
                              const void* scale, const void* zero, const void* part);
LnqStatus launch_int4_gemv_split(const void* x, const uint8_t* packed, const void* scale, const uint8_t* zero,
                                 const void* bias, void* y, int M, int N, int K, int G, int dtype, int u8, int S,
                                 float* part, hipStream_t stream, bool tiles = false, bool reduce = true);
LnqStatus launch_int4_gemv_tiles(const void* xt, const uint8_t* packed, const void* scale, const uint8_t* zero,
                                 const void* bias, void* y, int M, int N, int K, int G, int dtype, hipStream_t stream);
LnqStatus launch_x_tiles(const void* x, void* xt, int rows, int K, hipStream_t stream);

// The split GEMV's workgroup shape for K: past K = 4096 (where the few-row
// GEMV stops), 64-row blocks and the fewest K chunks of at most 16 slices of
// 256 inputs, if that leaves a chunk 8 or more (K = 14336: 4 chunks of 14;
// 8192: 2 of 16); at K = 4096, 128-row blocks in 2 chunks of 8 slices.
static bool split_shape(int K, int& u8, int& S) {
  if (K % 256 != 0) return false;
  const int slices = K / 256;
  if (K == 4096) {
    u8 = 16;
    S = 2;
    return true;
  }
  if (K <= 4096) return false;
  for (int s = 2; s <= slices; ++s)
    if (slices % s == 0 && slices / s <= 16) {
      u8 = 8;
      S = s;
      return slices / s >= 8;
    }
  return false;
}

// Whether the automatic choice with a workspace takes the split GEMV (rows run
// in 32-row chunks). Measured (bf16, group 128, graphs over rotating weight
// copies): K = 14336, N = 4096 at 32 rows 18.7-19.2 us against 32.3 for the
// skinny kernel, 16 rows 16.7 against 19.7, 8 rows 17.3 against 15.9; K = 4096
// only over the widest outputs (N = 128256 at 32 rows 109.9 against 117.5 for
// the unsplit 32-row GEMV; N = 28672: 31.5 against 30.6, N = 4096: 11.7 against
// 11.5, so the rest keep their kernels).
static bool split_preferred(int M, int N, int K) {
  if (M < 16 || M > 64 || N % 4 != 0) return false;
  if (K > 4096) return true;
  return K == 4096 && M > 16 && N >= 65536;
}

static int64_t split_workspace_bytes(int M, int N, int S) {
  return static_cast<int64_t>(S) * (M < 32 ? M : 32) * N * 4;
}

// The argument checks of lnq_int4_linear that do not look at the operands;
// false (with the message set) when one fails.
static bool check_int4_linear(int64_t rows, int64_t in_features, int64_t out_features, int64_t group,
                              int32_t dtype, int32_t kernel, const char* who) {
  if (!(dtype == LNQ_BF16 || dtype == LNQ_F16)) {
    set_error("%s: activations are bf16 or f16, not dtype %d", who, dtype);
    return false;
  }
  if (!(rows >= 0 && out_features > 0 && in_features > 0)) {
    set_error("%s: bad shape rows=%lld in=%lld out=%lld", who, (long long)rows, (long long)in_features,
              (long long)out_features);
    return false;
  }
  if (in_features % 128 != 0) {
    set_error("%s: in_features %lld is not a multiple of 128", who, (long long)in_features);
    return false;
  }
  if (!(group > 0 && in_features % group == 0 && (group == 32 || group == 64 || group % 128 == 0))) {
    set_error("%s: a group of %lld is not 32, 64 or a multiple of 128 dividing %lld", who, (long long)group,
              (long long)in_features);
    return false;
  }
  if (!(rows <= INT32_MAX && in_features <= INT32_MAX && out_features <= INT32_MAX)) {
    set_error("%s: sizes exceed 2^31", who);
    return false;
  }
  if (!(kernel >= LNQ_KERNEL_AUTO && kernel <= LNQ_KERNEL_PERSISTENT)) {
    set_error("%s: unknown kernel %d", who, kernel);
    return false;
  }
  return true;
}

// The prefill kernel for a shape the tiled kernel takes: where 256-column tiles
// give (nearly) every CU a tile, the 256-column tiled kernel, or the persistent
// 256 x 256 form where it takes the shape and there are more tiles than CUs
// (config 3, (K, N) = (4096, 14336) at 2048 rows, 448 tiles: 1104-1114 against
// 1043-1067 TFLOP/s for int4_tiled_kernel<256> in the same runs; at 1024 rows,
// 224 tiles, one a workgroup: 1036 against 1064); otherwise 128-column tiles.
static int prefill_kernel(int M, int N, int K, int G, int dtype) {
  if (int4_tiled_width(M, N) != 256) return LNQ_KERNEL_TILED_128;
  return int4_persistent_preferred(M, N, K, G, dtype) ? LNQ_KERNEL_PERSISTENT : LNQ_KERNEL_TILED_256;
}

// The kernel lnq_int4_linear runs (LNQ_KERNEL_GEMV, _SKINNY, _TILED_128,
// _TILED_256 or _PERSISTENT), or -1 with the message set when the one asked for
// does not take the shape. GEMV at 33..64 rows means the few-token GEMV per
// 32-row chunk.
static int choose_int4_kernel(int M, int N, int K, int G, int dtype, int kernel, const void* x,
                              const void* packed, const void* scale, const void* zero) {
  // The one-workgroup-per-CU GEMV takes 1..32 rows (1: one x row broadcast; 2..32:
  // x row m in MFMA A row m of one or two A blocks).
  const bool gemv_ok = int4_gemv_supports(M, N, K, G, x, packed, scale, zero);
  if (kernel == LNQ_KERNEL_GEMV) {
    if (!gemv_ok) {
      set_error("lnq_int4_linear: the one-token kernel does not take rows=%d N=%d K=%d group=%d", M, N, K, G);
      return -1;
    }
    return LNQ_KERNEL_GEMV;
  }
  if (kernel == LNQ_KERNEL_AUTO) {
    // Measured (bf16, group 128, K = 4096, graphs over rotating weight copies):
    // one row always takes the GEMV (N = 128256: 56 against 69 us; 16384: 7.8
    // against 9.4). Up to 6 rows the GEMV is ahead at every width (4 rows: N =
    // 4096 4.7 against 6.3 us; 14336 9.5 against 11.7; 28672 16.2 against 19.7;
    // 128256 60.7 against 73.1). Over a wide output (N >= 6144) it stays ahead
    // at 5..32 rows in one launch -- up to 16 rows one A block, 17..32 two
    // blocks over each weight tile (N = 14336: 12.0 against 21.7 us at 16 rows,
    // 18.0 against 35.7 at 32; 128256: 128 against 264 at 32) -- and at 33..64
    // rows once per 32-row chunk (N = 14336: 35.6 against 68.9 at 64). Over N
    // <= 4096 the two are level from 16 to 32 rows (N = 4096: 7.2 / 7.5 us at
    // 16, 11.3 / 11.2 at 32) and the skinny kernel is ahead at 64 (18.6 against
    // 22.5 for two 32-row launches).
    const bool wide = N >= 6144;
    const bool few = M <= 6;
    if (gemv_ok && (M == 1 || few || (M > 4 && wide))) return LNQ_KERNEL_GEMV;
    if (wide && M > 32 && M <= 64 && int4_gemv_supports(32, N, K, G, x, packed, scale, zero)) return LNQ_KERNEL_GEMV;
    if (M > 64 && int4_tiled_supports(M, N, K, G, dtype)) return prefill_kernel(M, N, K, G, dtype);
    return LNQ_KERNEL_SKINNY;
  }
  if (kernel == LNQ_KERNEL_SKINNY) return LNQ_KERNEL_SKINNY;
  if (kernel == LNQ_KERNEL_PERSISTENT) {
    if (!int4_persistent_supports(M, N, K, G, dtype)) {
      set_error("lnq_int4_linear: the persistent kernel does not take M=%d N=%d K=%d group=%d", M, N, K, G);
      return -1;
    }
    return LNQ_KERNEL_PERSISTENT;
  }
  if (!int4_tiled_supports(M, N, K, G, dtype)) {
    set_error("lnq_int4_linear: the tiled kernel does not take M=%d N=%d K=%d group=%d", M, N, K, G);
    return -1;
  }
  if (kernel == LNQ_KERNEL_TILED) return prefill_kernel(M, N, K, G, dtype);
  return kernel;
}

}  // namespace lnq

using namespace lnq;

extern "C" {

LNQ_API LnqStatus lnq_int4_linear(const void* x, const uint8_t* packed, const void* scale,
                                  const uint8_t* zero, const void* bias, void* y, int64_t rows,
                                  int64_t in_features, int64_t out_features, int64_t group,
                                  int32_t dtype, int32_t kernel, void* stream) {
  if (!check_int4_linear(rows, in_features, out_features, group, dtype, kernel, "lnq_int4_linear"))
    return LNQ_ERROR;
  LNQ_REQUIRE(x && packed && scale && zero && y, "lnq_int4_linear: null pointer");
  LNQ_REQUIRE(aligned(x, 16) && aligned(packed, 16),
              "lnq_int4_linear: x and packed must be 16-byte aligned");
  if (rows == 0) {
    clear_error();
    return LNQ_OK;
  }
  const int M = static_cast<int>(rows), N = static_cast<int>(out_features);
  const int K = static_cast<int>(in_features), G = static_cast<int>(group);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int code = choose_int4_kernel(M, N, K, G, dtype, kernel, x, packed, scale, zero);
  if (code < 0) return LNQ_ERROR;
  if (code == LNQ_KERNEL_GEMV) {
    if (M <= 32) return launch_int4_gemv(x, packed, scale, zero, bias, y, M, N, K, G, dtype, s);
    // 33..64 rows over a wide output: the few-token GEMV once per 32-row chunk.
    const size_t xrow = static_cast<size_t>(K) * 2, yrow = static_cast<size_t>(N) * 2;
    for (int c = 0; c < M; c += 32) {
      const int rc = M - c < 32 ? M - c : 32;
      const LnqStatus st = launch_int4_gemv(static_cast<const uint8_t*>(x) + c * xrow, packed, scale, zero, bias,
                                            static_cast<uint8_t*>(y) + c * yrow, rc, N, K, G, dtype, s);
      if (st != LNQ_OK) return st;
    }
    return LNQ_OK;
  }
  if (code == LNQ_KERNEL_PERSISTENT)
    return launch_int4_persistent(x, packed, scale, zero, bias, y, M, N, K, G, dtype, s);
  if (code == LNQ_KERNEL_TILED_128 || code == LNQ_KERNEL_TILED_256)
    return launch_int4_tiled(x, packed, scale, zero, bias, y, M, N, K, G, dtype,
                             code == LNQ_KERNEL_TILED_256 ? 256 : 128, s);
  if (dtype == LNQ_BF16)
    return launch_skinny<LNQ_BF16>(x, packed, scale, zero, bias, y, M, N, K, G, s);
  return launch_skinny<LNQ_F16>(x, packed, scale, zero, bias, y, M, N, K, G, s);
}

LNQ_API LnqStatus lnq_int4_linear_plan(int64_t rows, int64_t in_features, int64_t out_features,
                                       int64_t group, int32_t dtype, int32_t kernel,
                                       int32_t* chosen) {
  LNQ_REQUIRE(chosen != nullptr, "lnq_int4_linear_plan: null pointer");
  if (!check_int4_linear(rows, in_features, out_features, group, dtype, kernel, "lnq_int4_linear_plan"))
    return LNQ_ERROR;
  if (rows == 0) {
    *chosen = LNQ_KERNEL_SKINNY;
    clear_error();
    return LNQ_OK;
  }
  // Any 16-byte aligned address stands for the operands.
  static const uint8_t* const kAligned = reinterpret_cast<const uint8_t*>(static_cast<uintptr_t>(256));
  const int code = choose_int4_kernel(static_cast<int>(rows), static_cast<int>(out_features),
                                      static_cast<int>(in_features), static_cast<int>(group), dtype, kernel,
                                      kAligned, kAligned, kAligned, kAligned);
  if (code < 0) return LNQ_ERROR;
  *chosen = code;
  clear_error();
  return LNQ_OK;
}

LNQ_API LnqStatus lnq_int4_linear_workspace(int64_t rows, int64_t in_features, int64_t out_features, int64_t group,
                                            int32_t dtype, int32_t kernel, int32_t* chosen,
                                            int64_t* workspace_bytes) {
  LNQ_REQUIRE(chosen != nullptr && workspace_bytes != nullptr, "lnq_int4_linear_workspace: null pointer");
  const int32_t base = kernel == LNQ_KERNEL_SPLIT ? LNQ_KERNEL_AUTO : kernel;
  if (!check_int4_linear(rows, in_features, out_features, group, dtype, base, "lnq_int4_linear_workspace"))
    return LNQ_ERROR;
  *workspace_bytes = 0;
  const int M = static_cast<int>(rows), N = static_cast<int>(out_features), K = static_cast<int>(in_features);
  int u8 = 0, S = 0;
  const bool shaped = rows > 0 && split_shape(K, u8, S);
  if (kernel == LNQ_KERNEL_SPLIT || (kernel == LNQ_KERNEL_AUTO && shaped && split_preferred(M, N, K))) {
    static const uint8_t* const kAligned = reinterpret_cast<const uint8_t*>(static_cast<uintptr_t>(256));
    LNQ_REQUIRE(rows == 0 || (shaped && rows <= 64 &&
                              int4_gemv_split_supports(M < 32 ? M : 32, N, K, static_cast<int>(group), u8, S,
                                                       kAligned, kAligned, kAligned, kAligned, kAligned) &&
                              (M <= 32 || int4_gemv_split_supports(M - 32, N, K, static_cast<int>(group), u8, S,
                                                                   kAligned, kAligned, kAligned, kAligned,
                                                                   kAligned))),
                "lnq_int4_linear_workspace: the split GEMV does not take rows=%lld in=%lld out=%lld group=%lld",
                (long long)rows, (long long)in_features, (long long)out_features, (long long)group);
    *chosen = LNQ_KERNEL_SPLIT;
    *workspace_bytes = rows == 0 ? 0 : split_workspace_bytes(M, N, S);
    clear_error();
    return LNQ_OK;
  }
  return lnq_int4_linear_plan(rows, in_features, out_features, group, dtype, kernel, chosen);
}

LNQ_API LnqStatus lnq_int4_linear_ws(const void* x, const uint8_t* packed, const void* scale, const uint8_t* zero,
                                     const void* bias, void* y, int64_t rows, int64_t in_features,
                                     int64_t out_features, int64_t group, int32_t dtype, int32_t kernel,
                                     void* workspace, int64_t workspace_bytes, void* stream) {
  int32_t chosen = -1;
  int64_t need = 0;
  if (lnq_int4_linear_workspace(rows, in_features, out_features, group, dtype, kernel, &chosen, &need) != LNQ_OK)
    return LNQ_ERROR;
  const bool fits = workspace != nullptr && aligned(workspace, 16) && workspace_bytes >= need;
  if (chosen != LNQ_KERNEL_SPLIT || rows == 0 || (kernel == LNQ_KERNEL_AUTO && !fits))
    return lnq_int4_linear(x, packed, scale, zero, bias, y, rows, in_features, out_features, group, dtype,
                           kernel == LNQ_KERNEL_SPLIT ? LNQ_KERNEL_AUTO : kernel, stream);
  LNQ_REQUIRE(fits, "lnq_int4_linear_ws: the split GEMV needs %lld workspace bytes, 16-byte aligned (got %lld)",
              (long long)need, (long long)workspace_bytes);
  LNQ_REQUIRE(x && packed && scale && zero && y, "lnq_int4_linear_ws: null pointer");
  const int M = static_cast<int>(rows), N = static_cast<int>(out_features);
  const int K = static_cast<int>(in_features), G = static_cast<int>(group);
  int u8 = 0, S = 0;
  split_shape(K, u8, S);
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* part = static_cast<float*>(workspace);
  const size_t xrow = static_cast<size_t>(K) * 2, yrow = static_cast<size_t>(N) * 2;
  // 33..64 rows: one 32-row chunk after another on the stream, sharing the workspace.
  for (int c = 0; c < M; c += 32) {
    const int rc = M - c < 32 ? M - c : 32;
    const void* xc = static_cast<const uint8_t*>(x) + c * xrow;
    LNQ_REQUIRE(int4_gemv_split_supports(rc, N, K, G, u8, S, xc, packed, scale, zero, part),
                "lnq_int4_linear_ws: the split GEMV does not take these operands (rows=%d in=%d out=%d group=%d; x, "
                "packed and the workspace 16-byte aligned, group 128 scales 4- and zeros 2-byte aligned)",
                rc, K, N, G);
    const LnqStatus st = launch_int4_gemv_split(xc, packed, scale, zero, bias, static_cast<uint8_t*>(y) + c * yrow,
                                                rc, N, K, G, dtype, u8, S, part, s);
    if (st != LNQ_OK) return st;
  }
  return LNQ_OK;
}

LNQ_API LnqStatus lnq_x_tiles(const void* x, void* xt, int64_t rows, int64_t in_features, void* stream) {
  LNQ_REQUIRE(rows >= 0 && rows <= INT32_MAX && in_features > 0 && in_features % 256 == 0 &&
                  in_features * 64 <= INT32_MAX,
              "lnq_x_tiles: bad shape rows=%lld in=%lld (in %% 256 == 0)", (long long)rows, (long long)in_features);
  if (rows == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(x && xt, "lnq_x_tiles: null pointer");
  LNQ_REQUIRE(aligned(x, 16) && aligned(xt, 16), "lnq_x_tiles: x and xt must be 16-byte aligned");
  return launch_x_tiles(x, xt, static_cast<int>(rows), static_cast<int>(in_features), static_cast<hipStream_t>(stream));
}

LNQ_API LnqStatus lnq_int4_linear_tiles(const void* xt, const uint8_t* packed, const void* scale, const uint8_t* zero,
                                        const void* bias, void* y, int64_t rows, int64_t in_features,
                                        int64_t out_features, int64_t group, int32_t dtype, int32_t kernel,
                                        void* workspace, int64_t workspace_bytes, void* stream) {
  if (!check_int4_linear(rows, in_features, out_features, group, dtype, LNQ_KERNEL_AUTO, "lnq_int4_linear_tiles"))
    return LNQ_ERROR;
  LNQ_REQUIRE(kernel == LNQ_KERNEL_AUTO || kernel == LNQ_KERNEL_GEMV || kernel == LNQ_KERNEL_SPLIT,
              "lnq_int4_linear_tiles: kernel is AUTO, GEMV or SPLIT, not %d", kernel);
  LNQ_REQUIRE(rows <= 64 && in_features % 256 == 0,
              "lnq_int4_linear_tiles: x tiles of up to 64 rows with in %% 256 == 0, got rows=%lld in=%lld",
              (long long)rows, (long long)in_features);
  if (rows == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(xt && packed && scale && zero && y, "lnq_int4_linear_tiles: null pointer");
  LNQ_REQUIRE(kernel != LNQ_KERNEL_GEMV || in_features <= 4096,
              "lnq_int4_linear_tiles: the 32-row GEMV takes in <= 4096, got %lld", (long long)in_features);
  const int M = static_cast<int>(rows), N = static_cast<int>(out_features);
  const int K = static_cast<int>(in_features), G = static_cast<int>(group);
  int u8 = 0, S = 0;
  const bool shaped = split_shape(K, u8, S);
  const int64_t need = shaped ? split_workspace_bytes(M, N, S) : 0;
  const bool fits = workspace != nullptr && aligned(workspace, 16) && workspace_bytes >= need;
  // The split GEMV past K = 4096, where the 32-row GEMV stops; up to it the
  // 32-row GEMV (on tiles it is ahead of the split form at every width measured,
  // 32 rows: N = 128256 92.9 against 100.1 us, 28672: 24.6 against 27.1, 6144:
  // 9.9 against 10.9, 4096: 8.2 against 10.2).
  const bool split = kernel == LNQ_KERNEL_SPLIT || K > 4096;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t tile_chunk = static_cast<size_t>(K) * 64, yrow = static_cast<size_t>(N) * 2;
  for (int c = 0; c < M; c += 32) {
    const int rc = M - c < 32 ? M - c : 32;
    const void* xc = static_cast<const uint8_t*>(xt) + (c / 32) * tile_chunk;
    void* yc = static_cast<uint8_t*>(y) + c * yrow;
    if (split) {
      LNQ_REQUIRE(shaped, "lnq_int4_linear_tiles: the split GEMV does not take in=%d", K);
      LNQ_REQUIRE(fits, "lnq_int4_linear_tiles: the split GEMV needs %lld workspace bytes, 16-byte aligned (got %lld)",
                  (long long)need, (long long)workspace_bytes);
      LNQ_REQUIRE(int4_gemv_split_supports(rc, N, K, G, u8, S, xc, packed, scale, zero, workspace),
                  "lnq_int4_linear_tiles: the split GEMV does not take rows=%d in=%d out=%d group=%d", rc, K, N, G);
      const LnqStatus st = launch_int4_gemv_split(xc, packed, scale, zero, bias, yc, rc, N, K, G, dtype, u8, S,
                                                  static_cast<float*>(workspace), s, true);
      if (st != LNQ_OK) return st;
    } else {
      const LnqStatus st = launch_int4_gemv_tiles(xc, packed, scale, zero, bias, yc, rc, N, K, G, dtype, s);
      if (st != LNQ_OK) return st;
    }
  }
  return LNQ_OK;
}

LNQ_API LnqStatus lnq_int4_linear_tiles_parts(const void* xt, const uint8_t* packed, const void* scale,
                                              const uint8_t* zero, float* parts, int64_t parts_bytes, int64_t rows,
                                              int64_t in_features, int64_t out_features, int64_t group,
                                              int32_t dtype, int32_t* splits, void* stream) {
  if (!check_int4_linear(rows, in_features, out_features, group, dtype, LNQ_KERNEL_AUTO,
                         "lnq_int4_linear_tiles_parts"))
    return LNQ_ERROR;
  LNQ_REQUIRE(splits != nullptr, "lnq_int4_linear_tiles_parts: null pointer");
  const int M = static_cast<int>(rows), N = static_cast<int>(out_features);
  const int K = static_cast<int>(in_features), G = static_cast<int>(group);
  int u8 = 0, S = 0;
  LNQ_REQUIRE(K > 4096 && split_shape(K, u8, S) && rows >= 1 && rows <= 32,
              "lnq_int4_linear_tiles_parts: the split GEMV's parts take 1..32 rows and in > 4096 split into chunks "
              "of 8..16 slices, got rows=%lld in=%lld", (long long)rows, (long long)in_features);
  const int64_t need = split_workspace_bytes(M, N, S);
  LNQ_REQUIRE(xt && packed && scale && zero && parts, "lnq_int4_linear_tiles_parts: null pointer");
  LNQ_REQUIRE(aligned(parts, 16) && parts_bytes >= need,
              "lnq_int4_linear_tiles_parts: the parts take %lld bytes, 16-byte aligned (got %lld)", (long long)need,
              (long long)parts_bytes);
  LNQ_REQUIRE(int4_gemv_split_supports(M, N, K, G, u8, S, xt, packed, scale, zero, parts),
              "lnq_int4_linear_tiles_parts: the split GEMV does not take rows=%d in=%d out=%d group=%d", M, K, N, G);
  *splits = S;
  return launch_int4_gemv_split(xt, packed, scale, zero, nullptr, nullptr, M, N, K, G, dtype, u8, S, parts,
                                static_cast<hipStream_t>(stream), true, false);
}

LNQ_API LnqStatus lnq_int4_dequantize(const uint8_t* packed, const void* scale,
                                      const uint8_t* zero, void* out, int64_t out_features,
                                      int64_t in_features, int64_t group, int32_t dtype,
                                      void* stream) {
  LNQ_REQUIRE(dtype == LNQ_BF16 || dtype == LNQ_F16 || dtype == LNQ_F32,
              "lnq_int4_dequantize: scales are bf16, f16 or f32, not dtype %d", dtype);
  LNQ_REQUIRE(out_features >= 0 && in_features >= 0 && in_features % 2 == 0,
              "lnq_int4_dequantize: bad shape out=%lld in=%lld", (long long)out_features,
              (long long)in_features);
  LNQ_REQUIRE(group > 0 && group % 2 == 0 && (in_features == 0 || in_features % group == 0),
              "lnq_int4_dequantize: groups of %lld must be even and divide %lld", (long long)group,
              (long long)in_features);
  LNQ_REQUIRE(in_features <= INT32_MAX, "lnq_int4_dequantize: in_features exceeds 2^31");
  if (out_features == 0 || in_features == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(packed && scale && zero && out, "lnq_int4_dequantize: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int K = static_cast<int>(in_features), G = static_cast<int>(group);
  const bool fast = K % 8 == 0 && G % 8 == 0 && aligned(packed, 4) && aligned(out, 16);
  if (fast && out_features <= 65535) {
    const int per_row = K / 8;
    const int gshift = (G & (G - 1)) == 0 ? __builtin_ctz(static_cast<unsigned>(G)) : -1;
    const dim3 grid(static_cast<unsigned>((per_row + 255) / 256), static_cast<unsigned>(out_features));
    if (dtype == LNQ_BF16)
      hipLaunchKernelGGL((int4_dequant_fast<LNQ_BF16>), grid, dim3(256), 0, s, packed,
                         static_cast<const uint16_t*>(scale), zero, static_cast<uint16_t*>(out), K,
                         gshift, G);
    else if (dtype == LNQ_F16)
      hipLaunchKernelGGL((int4_dequant_fast<LNQ_F16>), grid, dim3(256), 0, s, packed,
                         static_cast<const uint16_t*>(scale), zero, static_cast<uint16_t*>(out), K,
                         gshift, G);
    else
      hipLaunchKernelGGL((int4_dequant_fast<LNQ_F32>), grid, dim3(256), 0, s, packed,
                         static_cast<const float*>(scale), zero, static_cast<float*>(out), K, gshift,
                         G);
  } else {
    const int64_t bytes = out_features * (K / 2);
    const dim3 grid(static_cast<unsigned>((bytes + 255) / 256));
    if (dtype == LNQ_BF16)
      hipLaunchKernelGGL((int4_dequant_any<LNQ_BF16>), grid, dim3(256), 0, s, packed,
                         static_cast<const uint16_t*>(scale), zero, static_cast<uint16_t*>(out),
                         bytes, K, G);
    else if (dtype == LNQ_F16)
      hipLaunchKernelGGL((int4_dequant_any<LNQ_F16>), grid, dim3(256), 0, s, packed,
                         static_cast<const uint16_t*>(scale), zero, static_cast<uint16_t*>(out),
                         bytes, K, G);
    else
      hipLaunchKernelGGL((int4_dequant_any<LNQ_F32>), grid, dim3(256), 0, s, packed,
                         static_cast<const float*>(scale), zero, static_cast<float*>(out), bytes,
                         K, G);
  }
  return launched("int4_dequant");
}

LNQ_API LnqStatus lnq_int4_quantize(const float* weight, uint8_t* packed, float* scale,
                                    uint8_t* zero, int64_t out_features, int64_t in_features,
                                    int64_t group, void* stream) {
  LNQ_REQUIRE(out_features >= 0 && in_features >= 0, "lnq_int4_quantize: bad shape");
  LNQ_REQUIRE(group > 0 && group % 2 == 0 && (in_features == 0 || in_features % group == 0),
              "lnq_int4_quantize: groups of %lld must be even and divide the %lld inputs",
              (long long)group, (long long)in_features);
  LNQ_REQUIRE(group <= INT32_MAX, "lnq_int4_quantize: group exceeds 2^31");
  const int64_t total = out_features * (in_features / group);
  if (total == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(weight && packed && scale && zero, "lnq_int4_quantize: null pointer");
  const dim3 grid(static_cast<unsigned>((total + 3) / 4));
  hipLaunchKernelGGL(int4_quantize_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                     weight, packed, scale, zero, total, static_cast<int>(group));
  return launched("int4_quantize");
}

LNQ_API LnqStatus lnq_int4_pack(const uint8_t* codes, uint8_t* packed, int64_t pairs,
                                void* stream) {
  LNQ_REQUIRE(pairs >= 0, "lnq_int4_pack: negative size");
  if (pairs == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(codes && packed, "lnq_int4_pack: null pointer");
  hipLaunchKernelGGL(int4_pack_kernel, dim3(static_cast<unsigned>((pairs + 255) / 256)), dim3(256),
                     0, static_cast<hipStream_t>(stream), codes, packed, pairs);
  return launched("int4_pack");
}

LNQ_API LnqStatus lnq_int4_row_prepare(const uint8_t* weight, const void* scale, uint8_t* packed,
                                       void* group_scale, uint8_t* zero, int64_t out_features,
                                       int64_t in_features, int64_t group, int32_t dtype, void* stream) {
  LNQ_REQUIRE(dtype == LNQ_BF16 || dtype == LNQ_F16 || dtype == LNQ_F32,
              "lnq_int4_row_prepare: scales are bf16, f16 or f32, not dtype %d", dtype);
  LNQ_REQUIRE(out_features >= 0 && in_features >= 0 && in_features % 32 == 0,
              "lnq_int4_row_prepare: bad shape out=%lld in=%lld (in %% 32 == 0)", (long long)out_features,
              (long long)in_features);
  LNQ_REQUIRE(group > 0 && group % 2 == 0 && (in_features == 0 || in_features % group == 0),
              "lnq_int4_row_prepare: groups of %lld must be even and divide %lld", (long long)group,
              (long long)in_features);
  const int64_t pieces = out_features * (in_features / 32);
  const int64_t entries = out_features * (in_features / group);
  if (pieces == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(weight && scale && packed && group_scale && zero, "lnq_int4_row_prepare: null pointer");
  LNQ_REQUIRE(aligned(weight, 16) && aligned(packed, 16), "lnq_int4_row_prepare: weights must be 16-byte aligned");
  LNQ_REQUIRE(in_features / group <= INT32_MAX, "lnq_int4_row_prepare: too many groups");
  const int64_t n = pieces > entries ? pieces : entries;
  const dim3 grid(static_cast<unsigned>((n + 255) / 256));
  const int groups = static_cast<int>(in_features / group);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define LNQ_ROWS(DT)                                                                                           \
  hipLaunchKernelGGL((int4_row_prepare_kernel<DT>), grid, dim3(256), 0, s, weight,                             \
                     static_cast<const typename Elem<DT>::storage*>(scale), packed,                             \
                     static_cast<typename Elem<DT>::storage*>(group_scale), zero, pieces, entries, groups)
  if (dtype == LNQ_BF16) LNQ_ROWS(LNQ_BF16);
  else if (dtype == LNQ_F16) LNQ_ROWS(LNQ_F16);
  else LNQ_ROWS(LNQ_F32);
#undef LNQ_ROWS
  return launched("int4_row_prepare");
}

LNQ_API LnqStatus lnq_take_inputs(const void* x, const int32_t* order, void* taken, int64_t rows, int64_t n,
                                  int32_t dtype, void* stream) {
  LNQ_REQUIRE(dtype == LNQ_BF16 || dtype == LNQ_F16 || dtype == LNQ_F32,
              "lnq_take_inputs: x is bf16, f16 or f32, not dtype %d", dtype);
  LNQ_REQUIRE(rows >= 0 && n >= 0, "lnq_take_inputs: bad shape rows=%lld n=%lld", (long long)rows, (long long)n);
  if (rows == 0 || n == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(x && order && taken, "lnq_take_inputs: null pointer");
  LNQ_REQUIRE(x != taken, "lnq_take_inputs: taken must not be x");
  const int64_t total = rows * n;
  const int64_t blocks = (total + 255) / 256;
  const dim3 grid(static_cast<unsigned>(blocks < 65536 ? blocks : 65536));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == LNQ_F32)
    hipLaunchKernelGGL((take_inputs_kernel<uint32_t>), grid, dim3(256), 0, s, static_cast<const uint32_t*>(x), order,
                       static_cast<uint32_t*>(taken), total, n);
  else
    hipLaunchKernelGGL((take_inputs_kernel<uint16_t>), grid, dim3(256), 0, s, static_cast<const uint16_t*>(x), order,
                       static_cast<uint16_t*>(taken), total, n);
  return launched("take_inputs");
}

LNQ_API LnqStatus lnq_int4_linear_ordered(const void* x, const int32_t* order, const uint8_t* packed,
                                          const void* scale, const uint8_t* zero, const void* bias, void* y,
                                          void* taken, int64_t rows, int64_t in_features, int64_t out_features,
                                          int64_t group, int32_t dtype, int32_t kernel, void* stream) {
  if (order == nullptr)
    return lnq_int4_linear(x, packed, scale, zero, bias, y, rows, in_features, out_features, group, dtype, kernel,
                           stream);
  if (!check_int4_linear(rows, in_features, out_features, group, dtype, kernel, "lnq_int4_linear_ordered"))
    return LNQ_ERROR;
  LNQ_REQUIRE(x && packed && scale && zero && y, "lnq_int4_linear_ordered: null pointer");
  LNQ_REQUIRE(aligned(x, 16) && aligned(packed, 16), "lnq_int4_linear_ordered: x and packed must be 16-byte aligned");
  if (rows == 0) {
    clear_error();
    return LNQ_OK;
  }
  const int M = static_cast<int>(rows), N = static_cast<int>(out_features);
  const int K = static_cast<int>(in_features), G = static_cast<int>(group);
  if ((kernel == LNQ_KERNEL_AUTO || kernel == LNQ_KERNEL_GEMV) &&
      int4_gemv_takes_order(M, N, K, G, x, packed, scale, zero, order))
    return launch_int4_gemv(x, packed, scale, zero, bias, y, M, N, K, G, dtype, static_cast<hipStream_t>(stream),
                            order);
  LNQ_REQUIRE(taken != nullptr && aligned(taken, 16),
              "lnq_int4_linear_ordered: %d rows x %d inputs need a 16-byte aligned `taken` buffer of as many elements "
              "(the gather is fused only for one row, group 128)", M, K);
  if (lnq_take_inputs(x, order, taken, rows, in_features, dtype, stream) != LNQ_OK) return LNQ_ERROR;
  return lnq_int4_linear(taken, packed, scale, zero, bias, y, rows, in_features, out_features, group, dtype, kernel,
                         stream);
}

LNQ_API LnqStatus lnq_int4_linear_prologue(const void* x, const void* u, const float* norm_weight, float eps,
                                           int32_t prologue, const uint8_t* packed, const void* scale,
                                           const uint8_t* zero, const void* bias, void* y, void* staged, int64_t rows,
                                           int64_t in_features, int64_t out_features, int64_t group, int32_t dtype,
                                           int32_t kernel, void* stream) {
  LNQ_REQUIRE(prologue == LNQ_PROLOGUE_RMSNORM || prologue == LNQ_PROLOGUE_SILU_MUL,
              "lnq_int4_linear_prologue: prologue is LNQ_PROLOGUE_RMSNORM or LNQ_PROLOGUE_SILU_MUL");
  LNQ_REQUIRE(dtype == LNQ_BF16, "lnq_int4_linear_prologue: the prologues compute in bf16");
  if (!check_int4_linear(rows, in_features, out_features, group, dtype, kernel, "lnq_int4_linear_prologue"))
    return LNQ_ERROR;
  LNQ_REQUIRE(x && packed && scale && zero && y, "lnq_int4_linear_prologue: null pointer");
  LNQ_REQUIRE(prologue == LNQ_PROLOGUE_RMSNORM ? norm_weight != nullptr : u != nullptr,
              "lnq_int4_linear_prologue: RMSNorm needs norm_weight, SiLU(x) * u needs u");
  if (rows == 0) {
    clear_error();
    return LNQ_OK;
  }
  const int M = static_cast<int>(rows), N = static_cast<int>(out_features);
  const int K = static_cast<int>(in_features), G = static_cast<int>(group);
  const void* operand = prologue == LNQ_PROLOGUE_RMSNORM ? static_cast<const void*>(norm_weight) : u;
  if ((kernel == LNQ_KERNEL_AUTO || kernel == LNQ_KERNEL_GEMV) &&
      int4_gemv_takes_prologue(M, N, K, G, dtype, x, packed, scale, zero, prologue, operand))
    return launch_int4_gemv(x, packed, scale, zero, bias, y, M, N, K, G, dtype, static_cast<hipStream_t>(stream),
                            nullptr, prologue, norm_weight, u, eps);
  LNQ_REQUIRE(staged != nullptr && aligned(staged, 16),
              "lnq_int4_linear_prologue: %d rows x %d inputs need a 16-byte aligned `staged` buffer of as many "
              "elements (the prologue is fused only for one row, group 128, on the one-token kernels)", M, K);
  const LnqStatus st =
      prologue == LNQ_PROLOGUE_RMSNORM
          ? lnq_rmsnorm(const_cast<void*>(x), nullptr, norm_weight, staged, rows, in_features, eps, stream)
          : lnq_silu_mul(x, u, staged, rows * in_features, stream);
  if (st != LNQ_OK) return st;
  return lnq_int4_linear(staged, packed, scale, zero, bias, y, rows, in_features, out_features, group, dtype, kernel,
                         stream);
}

LNQ_API LnqStatus lnq_int4_unpack(const uint8_t* packed, void* codes, int64_t pairs,
                                  int32_t is_signed, void* stream) {
  LNQ_REQUIRE(pairs >= 0, "lnq_int4_unpack: negative size");
  if (pairs == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(codes && packed, "lnq_int4_unpack: null pointer");
  hipLaunchKernelGGL(int4_unpack_kernel, dim3(static_cast<unsigned>((pairs + 255) / 256)),
                     dim3(256), 0, static_cast<hipStream_t>(stream), packed,
                     static_cast<uint8_t*>(codes), pairs, is_signed ? 1 : 0);
  return launched("int4_unpack");
}

}  // extern "C"
