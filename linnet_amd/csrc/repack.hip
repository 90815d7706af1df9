// Calibrated 4-bit checkpoints (GPTQ, AWQ) repacked into Int4GroupLinear's bytes
// on the GPU: the work of the reference's `import_quantized`
// (`python/linnet/src/linnet/quant.py:222-240, 300-340`, numpy there).
//
// Both formats hold eight 4-bit codes in an int32, lowest bits first:
//   GPTQ  qweight [in/8, out]: word [c, o] holds input 8c + k of output o at bits 4k
//         (codes packed along the inputs); with activation order the result takes
//         input order[i] of the checkpoint as its input i.
//   AWQ   qweight [in, out/8]: word [i, c] holds output 8c + AWQ_ORDER[k] at bits 4k
//         (codes packed along the outputs, interleaved).
//   qzeros [groups, out/8]: zero points packed along the outputs as each format's
//         qweight packs its codes (GPTQ in order, AWQ interleaved), GPTQ's first
//         format storing each less one (zero_offset 1).
// Int4GroupLinear's weight is [out, in/2] bytes, input 2b in the low nibble of
// byte b, so a dword of it holds inputs 8c .. 8c + 7 of one output at bits 4k --
// the bit order of a GPTQ word. The repack is therefore a transpose of 8-code
// words, with a gather of codes for activation order and an 8 x 8 code transpose
// for AWQ.
//
// Byte work (HBM-bound): each workgroup owns 64 outputs x 256 inputs (a 64 x 32
// tile of output dwords), builds it in LDS from reads coalesced along the
// outputs, and writes it as 64 rows of 128 contiguous bytes.
#include "common.hpp"

namespace lnq {

namespace repack {
constexpr int OUTS = 64;    // outputs per workgroup
constexpr int WORDS = 32;   // output dwords (8 inputs each) per output row
constexpr int THREADS = 256;
}  // namespace repack

// Bit position (in units of 4 bits) of output 8c + j within an AWQ word: the k
// with AWQ_ORDER[k] = j for AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7).
__device__ inline int awq_slot(int j) { return (j >> 1) + 4 * (j & 1); }

__global__ __launch_bounds__(repack::THREADS) void int4_repack_kernel(
    const int32_t* __restrict__ qweight, const int32_t* __restrict__ order, int packing,
    int64_t in_features, int64_t out_features, uint32_t* __restrict__ packed) {
  __shared__ uint32_t tile[repack::OUTS][repack::WORDS + 1];
  const int t = threadIdx.x;
  const int64_t o0 = static_cast<int64_t>(blockIdx.x) * repack::OUTS;
  const int64_t c0 = static_cast<int64_t>(blockIdx.y) * repack::WORDS;  // first output dword of the row
  const int64_t words = in_features / 8;                                 // output dwords per row
  const int ol = t % repack::OUTS;
  const int64_t o = o0 + ol;
  const bool live = o < out_features;
  // Thread (ol, quarter) builds output dwords c0 + 8 quarter + r, r = 0..7, of output o.
  for (int r = 0; r < 8; ++r) {
    const int cl = 8 * (t / repack::OUTS) + r;
    const int64_t c = c0 + cl;
    uint32_t word = 0;
    if (live && c < words) {
      if (packing == LNQ_PACKING_AWQ) {
        const int shift = 4 * awq_slot(static_cast<int>(o & 7));
        const int64_t stride = out_features / 8;
        for (int k = 0; k < 8; ++k) {
          const uint32_t w = static_cast<uint32_t>(qweight[(8 * c + k) * stride + (o >> 3)]);
          word |= ((w >> shift) & 15u) << (4 * k);
        }
      } else if (order != nullptr) {
        // The eight source inputs first, then their eight words (independent
        // loads, all in flight), then the codes.
        int src[8];
        uint32_t w[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) src[k] = order[8 * c + k];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int sk = min(max(src[k], 0), static_cast<int>(in_features) - 1);
          w[k] = static_cast<uint32_t>(qweight[static_cast<int64_t>(sk >> 3) * out_features + o]);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const bool ok = src[k] >= 0 && src[k] < in_features;  // not a permutation entry: code 0
          word |= (ok ? (w[k] >> (4 * (src[k] & 7))) & 15u : 0u) << (4 * k);
        }
      } else {
        word = static_cast<uint32_t>(qweight[c * out_features + o]);
      }
    }
    tile[ol][cl] = word;
  }
  __syncthreads();
  for (int idx = t; idx < repack::OUTS * repack::WORDS; idx += repack::THREADS) {
    const int rl = idx / repack::WORDS, cl = idx % repack::WORDS;
    const int64_t ro = o0 + rl, c = c0 + cl;
    if (ro < out_features && c < words) packed[ro * words + c] = tile[rl][cl];
  }
}

__global__ void int4_repack_zero_kernel(const int32_t* __restrict__ qzeros, int packing, int zero_offset,
                                        int64_t out_features, int64_t groups, uint8_t* __restrict__ zero) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= out_features * groups) return;
  const int64_t o = idx / groups, g = idx % groups;
  const uint32_t w = static_cast<uint32_t>(qzeros[g * (out_features / 8) + (o >> 3)]);
  const int j = static_cast<int>(o & 7);
  const int slot = packing == LNQ_PACKING_AWQ ? awq_slot(j) : j;
  zero[idx] = static_cast<uint8_t>(((w >> (4 * slot)) & 15u) + static_cast<uint32_t>(zero_offset));
}

}  // namespace lnq

using namespace lnq;

extern "C" {

LNQ_API LnqStatus lnq_int4_repack(const int32_t* qweight, const int32_t* qzeros, const int32_t* order,
                                  int32_t packing, int32_t zero_offset, int64_t in_features,
                                  int64_t out_features, int64_t groups, uint8_t* packed, uint8_t* zero,
                                  void* stream) {
  LNQ_REQUIRE(packing == LNQ_PACKING_GPTQ || packing == LNQ_PACKING_AWQ,
              "lnq_int4_repack: packing %d is neither GPTQ (0) nor AWQ (1)", packing);
  LNQ_REQUIRE(in_features >= 0 && out_features >= 0 && groups >= 0, "lnq_int4_repack: negative size");
  LNQ_REQUIRE(in_features % 8 == 0 && out_features % 8 == 0,
              "lnq_int4_repack: %lld inputs and %lld outputs must be multiples of 8 (eight codes a word)",
              static_cast<long long>(in_features), static_cast<long long>(out_features));
  LNQ_REQUIRE(groups >= 1 || in_features == 0, "lnq_int4_repack: no groups");
  LNQ_REQUIRE(groups == 0 || in_features % groups == 0,
              "lnq_int4_repack: %lld inputs do not make %lld equal groups", static_cast<long long>(in_features),
              static_cast<long long>(groups));
  LNQ_REQUIRE(zero_offset == 0 || zero_offset == 1, "lnq_int4_repack: zero_offset is 0 or 1, got %d", zero_offset);
  LNQ_REQUIRE(order == nullptr || packing == LNQ_PACKING_GPTQ, "lnq_int4_repack: only GPTQ has an activation order");
  LNQ_REQUIRE(in_features / 8 <= (int64_t{1} << 31) && out_features <= (int64_t{1} << 31),
              "lnq_int4_repack: too large");
  if (in_features == 0 || out_features == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(qweight && qzeros && packed && zero, "lnq_int4_repack: null pointer");
  LNQ_REQUIRE(aligned(packed, 4), "lnq_int4_repack: packed is not 4-byte aligned");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>((out_features + repack::OUTS - 1) / repack::OUTS),
                  static_cast<unsigned>((in_features / 8 + repack::WORDS - 1) / repack::WORDS));
  LNQ_REQUIRE(grid.y <= 65535, "lnq_int4_repack: %lld inputs are too many", static_cast<long long>(in_features));
  hipLaunchKernelGGL(int4_repack_kernel, grid, dim3(repack::THREADS), 0, s, qweight, order, packing, in_features,
                     out_features, reinterpret_cast<uint32_t*>(packed));
  LnqStatus st = launched("int4_repack");
  if (st != LNQ_OK) return st;
  const int64_t n = out_features * groups;
  LNQ_REQUIRE((n + 255) / 256 < (int64_t{1} << 31), "lnq_int4_repack: too many zero points");
  hipLaunchKernelGGL(int4_repack_zero_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, qzeros,
                     packing, zero_offset, out_features, groups, zero);
  return launched("int4_repack_zero");
}

}  // extern "C"
