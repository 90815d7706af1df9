// Decode-step glue for the int4 Llama-shaped workload (the "Full int4
// Llama-3.1-8B decode step" that BASELINE config 5 measures): everything a
// decoder layer does between its quantized linear layers, as three kernels
// instead of ~40 small framework ops a layer (each a ~3 us graph node here).
//
//   rmsnorm:           x += delta (rounded to bf16), h = x * rsqrt(mean(x^2) + eps) * w
//   decode_attention:  rotary embedding of q and k, k and v written into the KV
//                      cache at `pos`, softmax(q K^T / sqrt(hd)) V over 0..pos
//   silu_mul:          a = silu(g) * u
//
// All arithmetic is f32 (activations and KV caches stored bf16) in a fixed order,
// so results do not depend on timing. The reference gets these ops from its
// generated module (framework ops on the GPU); they are not part of its
// quantized-linear path.
#include <mutex>

#include "common.hpp"

namespace lnq {

namespace decode {
constexpr int THREADS = 256;
constexpr int MAX_GROUP = 8;  // query heads per KV head
constexpr int CHUNK = 64;  // cache positions a workgroup takes
constexpr int MAX_CHUNKS = 4096;  // chunks the merge holds: positions up to 262144
constexpr int MAX_DEVICES = 64;
}  // namespace decode

static_assert(LNQ_DECODE_ATTENTION_SCRATCH_FLOATS % 64 == 0, "scratch size");

// The split-K partial results of lnq_decode_attention_noalloc: one array on each
// GPU the library runs on, held until the process ends. Host code never passes
// this name to a kernel (on the host it stands for no device address); it
// passes the address hipGetSymbolAddress gives for the current device.
static __device__ __align__(256) float scratch[LNQ_DECODE_ATTENTION_SCRATCH_FLOATS];

namespace {
std::mutex scratch_mutex;
float* scratch_address[decode::MAX_DEVICES] = {};
}  // namespace

// The device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept; nullptr with the error set if
// the lookup fails.
static float* scratch_on_current_device() {
  int device = -1;
  const hipError_t got = hipGetDevice(&device);
  if (got != hipSuccess || device < 0 || device >= decode::MAX_DEVICES) {
    set_error("lnq_decode_attention_noalloc: no current device (%s)", hipGetErrorString(got));
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (scratch_address[device] == nullptr) {
    void* address = nullptr;
    const hipError_t found = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (found != hipSuccess || address == nullptr) {
      set_error("lnq_decode_attention_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", device,
                hipGetErrorString(found));
      return nullptr;
    }
    scratch_address[device] = static_cast<float*>(address);
  }
  return scratch_address[device];
}

// Sum over the block (256 threads), the same value returned to every thread.
__device__ inline float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ inline float block_max(float v, float* red) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// One workgroup per row.
__global__ __launch_bounds__(decode::THREADS) void rmsnorm_kernel(uint16_t* __restrict__ x,
                                                                  const uint16_t* __restrict__ delta,
                                                                  const float* __restrict__ w,
                                                                  uint16_t* __restrict__ h, int hidden, float eps) {
  __shared__ float red[4];
  uint16_t* xr = x + static_cast<size_t>(blockIdx.x) * hidden;
  uint16_t* hr = h + static_cast<size_t>(blockIdx.x) * hidden;
  const uint16_t* dr = delta ? delta + static_cast<size_t>(blockIdx.x) * hidden : nullptr;
  float ss = 0.f;
  for (int i = threadIdx.x; i < hidden; i += decode::THREADS) {
    float v = bf16_bits_to_f32(xr[i]);
    if (dr) {
      const uint16_t r = f32_to_bf16_bits(v + bf16_bits_to_f32(dr[i]));
      xr[i] = r;
      v = bf16_bits_to_f32(r);
    }
    ss = fmaf(v, v, ss);
  }
  const float scale = rsqrtf(block_sum(ss, red) / static_cast<float>(hidden) + eps);
  for (int i = threadIdx.x; i < hidden; i += decode::THREADS)
    hr[i] = f32_to_bf16_bits(bf16_bits_to_f32(xr[i]) * scale * w[i]);
}

// The same with the row held in registers: thread t owns 16-byte chunks t,
// t + 256, ... (CH of them, up to 8: hidden <= 2048 CH, hidden % 8 == 0), every load of x,
// delta and the weight issued before any is used (the scalar loop above waits on
// each of its 16 loads a thread in turn: 14 us for one 4096-wide row).
// TILES: h is written as x tiles (x_tile_index) for the 32-row GEMVs.
// parts (else nullptr): the delta is the sum of `splits` f32 partial sums
// parts[s][row][k] added in order and rounded once to bf16 -- what the split
// GEMV's reduction writes as its output with no bias -- read in place of delta.
template <int CH, bool TILES = false>
__global__ __launch_bounds__(decode::THREADS) void rmsnorm_vec_kernel(uint16_t* __restrict__ x,
                                                                      const uint16_t* __restrict__ delta,
                                                                      const float* __restrict__ w,
                                                                      uint16_t* __restrict__ h, int hidden, float eps,
                                                                      const float* __restrict__ parts = nullptr,
                                                                      int splits = 0) {
  __shared__ float group_ss[CH * decode::THREADS / 32];
  uint16_t* xr = x + static_cast<size_t>(blockIdx.x) * hidden;
  uint16_t* hr = h + static_cast<size_t>(blockIdx.x) * hidden;
  const uint16_t* dr = delta ? delta + static_cast<size_t>(blockIdx.x) * hidden : nullptr;
  const bool has_delta = dr != nullptr || parts != nullptr;
  const size_t part_stride = static_cast<size_t>(gridDim.x) * hidden;  // one chunk's [rows, hidden]
  const float* pr = parts ? parts + static_cast<size_t>(blockIdx.x) * hidden : nullptr;
  const int chunks = hidden >> 3;
  u32x4 xv[CH], dv[CH];
  f32x4 wv[CH][2];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int i = threadIdx.x + c * decode::THREADS;
    if (i < chunks) {
      xv[c] = *reinterpret_cast<const u32x4*>(xr + 8 * i);
      dv[c] = dr ? *reinterpret_cast<const u32x4*>(dr + 8 * i) : u32x4{0u, 0u, 0u, 0u};
      wv[c][0] = *reinterpret_cast<const f32x4*>(w + 8 * i);
      wv[c][1] = *reinterpret_cast<const f32x4*>(w + 8 * i + 4);
    }
  }
  if (pr != nullptr) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int i = threadIdx.x + c * decode::THREADS;
      if (i >= chunks) continue;
      f32x4 a = *reinterpret_cast<const f32x4*>(pr + 8 * i), b = *reinterpret_cast<const f32x4*>(pr + 8 * i + 4);
      for (int sp = 1; sp < splits; ++sp) {
        const float* q = pr + sp * part_stride + 8 * i;
        const f32x4 qa = *reinterpret_cast<const f32x4*>(q), qb = *reinterpret_cast<const f32x4*>(q + 4);
        a = f32x4{a[0] + qa[0], a[1] + qa[1], a[2] + qa[2], a[3] + qa[3]};
        b = f32x4{b[0] + qb[0], b[1] + qb[1], b[2] + qb[2], b[3] + qb[3]};
      }
      dv[c] = u32x4{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3]), pack_bf16x2(b[0], b[1]), pack_bf16x2(b[2], b[3])};
    }
  }
  float v[CH][8];
  float ss[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int i = threadIdx.x + c * decode::THREADS;
    ss[c] = 0.f;
    if (i >= chunks) continue;
    u32x4 out;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float lo = bf16_bits_to_f32(static_cast<uint16_t>(xv[c][e] & 0xffffu));
      float hi = bf16_bits_to_f32(static_cast<uint16_t>(xv[c][e] >> 16));
      if (has_delta) {
        lo = bf16_bits_to_f32(f32_to_bf16_bits(lo + bf16_bits_to_f32(static_cast<uint16_t>(dv[c][e] & 0xffffu))));
        hi = bf16_bits_to_f32(f32_to_bf16_bits(hi + bf16_bits_to_f32(static_cast<uint16_t>(dv[c][e] >> 16))));
      }
      v[c][2 * e] = lo;
      v[c][2 * e + 1] = hi;
      out[e] = static_cast<uint32_t>(f32_to_bf16_bits(lo)) | (static_cast<uint32_t>(f32_to_bf16_bits(hi)) << 16);
    }
    if (has_delta) *reinterpret_cast<u32x4*>(xr + 8 * i) = out;
    ss[c] = chunk_squares(v[c]);
  }
  // The sum of squares in the order the one-token GEMV's norm prologue uses (so
  // both give the same bits): chunk i = t + 256 c sits in 32-chunk group i / 32 =
  // t / 32 + 8 c at lane t % 32 of its half wave; chunks past the row add 0.
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const float g = sum_over_32_lanes(ss[c]);
    if ((threadIdx.x & 31) == 0) group_ss[(threadIdx.x >> 5) + c * (decode::THREADS / 32)] = g;
  }
  __syncthreads();
  float total = 0.f;
  for (int g = 0; g < (chunks + 31) / 32; ++g) total += group_ss[g];
  const float scale = rsqrtf(total / static_cast<float>(hidden) + eps);
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int i = threadIdx.x + c * decode::THREADS;
    if (i >= chunks) continue;
    uint16_t* dst = TILES ? h + x_tile_index(blockIdx.x, 8 * i, hidden) : hr + 8 * i;
    const u32x4 out = norm_bf16x8(v[c], scale, wv[c][0], wv[c][1]);
    *reinterpret_cast<u32x4*>(dst) = TILES ? permute_x8(out) : out;  // tiles: 8 values in pair order
  }
}

// Split-K decode attention. Workgroup (row, KV head, chunk c) takes positions
// [64 c, 64 c + 64) of that head's cache for its G query heads: scores, their
// max m and sum s of exp(score - m), and acc = sum exp(score - m) V, written to
// the workspace; decode_combine_kernel merges the chunks. Keys and values move
// four values (8 bytes) at a time: a thread's key loads cover 4 positions x
// HD/16 dimensions (the partial scores of the 16 dimension groups are added
// through LDS), its value loads 4 dimensions x 64/(256/(HD/4)) positions. Every
// workgroup applies the rotary embedding itself (q, and k for position pos, which
// it reads from LDS rather than the cache, rounded to bf16 as the cache holds
// it); the one whose chunk holds pos writes k and v into the caches. bf16 caches:
// K transposed, [rows, kv_heads, HD, cap]; V [rows, kv_heads, cap, HD]; cap a
// multiple of 4.
template <int HD, int GT>
__global__ __launch_bounds__(decode::THREADS) void decode_attention_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const float* __restrict__ cosv, const float* __restrict__ sinv, uint16_t* __restrict__ kt,
    uint16_t* __restrict__ vc, float* __restrict__ work, int heads, int kv_heads, int cap, int pos, int chunks,
    int64_t q_stride, int64_t kv_stride, const int32_t* __restrict__ pos_dev) {
  constexpr int C = decode::CHUNK;       // 64 positions
  constexpr int DG = 16;                 // dimension groups of the scores
  constexpr int DPG = HD / DG;           // dimensions a score thread takes
  constexpr int DV = HD / 4;             // value threads across the dimensions
  constexpr int PG = decode::THREADS / DV;  // value threads across the positions
  // GT: query heads per KV head the LDS arrays hold (G <= GT); smaller arrays
  // let more workgroups share a CU (G = 4: ~35 KB against ~70 KB at 8).
  constexpr int G8 = GT;
  __shared__ float qs[G8][HD];
  __shared__ float kn[HD], vn[HD];
  __shared__ float sp[DG][G8][C];   // partial scores
  __shared__ float p[G8][C];        // exp(score - m)
  __shared__ float stat[G8][2];     // m, s
  __shared__ __attribute__((aligned(16))) float pacc[PG][G8][HD];
  const int G = heads / kv_heads;
  const int c = blockIdx.x % chunks;
  const int rk = blockIdx.x / chunks;  // row * kv_heads + kvh
  const int row = rk / kv_heads, kvh = rk % kv_heads;
  const int l0 = c * C;
  if (pos_dev != nullptr) {
    // The position in device memory (a captured step advances it on the device):
    // the grid covers the whole cache, the chunks past pos have nothing to do, and
    // cos / sin are tables [cap, HD / 2] read at row pos.
    pos = *pos_dev;
    if (pos < 0 || pos >= cap || l0 > pos) return;
    cosv += static_cast<size_t>(pos) * (HD / 2);
    sinv += static_cast<size_t>(pos) * (HD / 2);
  }
  const int n = min(C, pos + 1 - l0);  // live positions of this chunk
  const int tid = threadIdx.x;
  constexpr int HALF = HD / 2;
  const float scale = rsqrtf(static_cast<float>(HD));
  const uint16_t* qr = q + row * q_stride + kvh * G * HD;
  const uint16_t* kr = k + row * kv_stride + kvh * HD;
  const uint16_t* vr = v + row * kv_stride + kvh * HD;
  uint16_t* ktb = kt + static_cast<size_t>(rk) * HD * cap;
  uint16_t* vcb = vc + static_cast<size_t>(rk) * cap * HD;
  const bool owner = pos >= l0 && pos < l0 + C;

  // The new token's inputs first -- q of the G heads and k (pairs i, i + HD/2),
  // cos / sin at pos, v -- so that the rotary embedding runs while the chunk's
  // keys and values, loaded next, are in flight (loads retire in issue order).
  constexpr int RT = ((decode::MAX_GROUP + 1) * HALF + decode::THREADS - 1) / decode::THREADS;
  // (Every load is unconditional -- an item past the last reads the last one's
  // inputs again -- so that they all issue together instead of each behind its
  // own branch and wait.)
  float ra_in[RT], rb_in[RT], rcos[RT], rsin[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const int t = min(tid + r * decode::THREADS, (G + 1) * HALF - 1);
    const int g = t / HALF, i = t % HALF;
    const uint16_t* src = g < G ? qr + g * HD : kr;
    ra_in[r] = bf16_bits_to_f32(src[i]);
    rb_in[r] = bf16_bits_to_f32(src[i + HALF]);
    rcos[r] = cosv[i];
    rsin[r] = sinv[i];
  }
  const uint16_t vnew = vr[min(tid, HD - 1)];
  // (A compiler barrier: the chunk's loads below may not move above these.)
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);

  // The chunk's keys and values: every load issued before any is used
  // (registers), the scores after. Key thread (dimension group dg, positions
  // 4 p4 .. 4 p4 + 3); value thread (dimensions 4 d4 .. 4 d4 + 3, positions pg,
  // pg + PG, ...). Position pos is the new key / value (from LDS).
  const int p4 = tid & 15, dg = tid >> 4;
  const int lp = l0 + 4 * p4;
  const int d4 = tid % DV, pg = tid / DV;
  constexpr int VJ = C / PG;  // value positions a thread takes
  // (bf16 caches: four values are 8 bytes.)
  // Buffer loads, unconditional: keys past the cache's end read zeros through the
  // range check of this (row, KV head)'s block (keys past pos are read and their
  // scores masked); values from pos on read zeros (the range ends at pos: past it
  // the cache may hold anything, and 0 * NaN would not vanish).
  u32x2 kreg[DPG], vreg[VJ];
  const __amdgpu_buffer_rsrc_t rkt = buffer_rsrc(ktb, static_cast<uint32_t>(HD * cap * 2));
  const __amdgpu_buffer_rsrc_t rvc = buffer_rsrc(vcb, static_cast<uint32_t>(pos * HD * 2));
#pragma unroll
  for (int dd = 0; dd < DPG; ++dd) {
    const int d = dg * DPG + dd;
    kreg[dd] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rkt, (d * cap + lp) * 2, 0, 0));
  }
#pragma unroll
  for (int jj = 0; jj < VJ; ++jj) {
    const int j = pg + jj * PG;
    vreg[jj] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rvc, ((l0 + j) * HD + 4 * d4) * 2, 0, 0));
  }
  auto widen = [](u32x2 w) {
    return make_float4(bf16_bits_to_f32(static_cast<uint16_t>(w.x & 0xffffu)), bf16_bits_to_f32(static_cast<uint16_t>(w.x >> 16)),
                       bf16_bits_to_f32(static_cast<uint16_t>(w.y & 0xffffu)), bf16_bits_to_f32(static_cast<uint16_t>(w.y >> 16)));
  };

  // Rotary embedding (pairs i, i + HD/2); the new key and value into LDS, and into
  // the caches by the chunk that holds pos.
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    // (Items past the last repeat it: the same values to the same places.)
    const int t = min(tid + r * decode::THREADS, (G + 1) * HALF - 1);
    const int g = t / HALF, i = t % HALF;
    const float a = ra_in[r], b = rb_in[r];
    const float ra = a * rcos[r] - b * rsin[r], rb = b * rcos[r] + a * rsin[r];
    if (g < G) {
      qs[g][i] = ra * scale;
      qs[g][i + HALF] = rb * scale;
    } else {
      // The new key as the cache holds it (rounded to bf16).
      const uint16_t ba = f32_to_bf16_bits(ra), bb = f32_to_bf16_bits(rb);
      kn[i] = bf16_bits_to_f32(ba);
      kn[i + HALF] = bf16_bits_to_f32(bb);
      if (owner) {
        ktb[static_cast<size_t>(i) * cap + pos] = ba;
        ktb[static_cast<size_t>(i + HALF) * cap + pos] = bb;
      }
    }
  }
  // Heads past G (G < G8) hold zeros: the score and value loops below then run
  // over all G8 heads without a branch (their LDS reads issue together).
  for (int t = G * HD + tid; t < G8 * HD; t += decode::THREADS) qs[t / HD][t % HD] = 0.f;
  static_assert(HD <= decode::THREADS, "a thread stores one value of the new token");
  if (tid < HD) {
    vn[tid] = bf16_bits_to_f32(vnew);
    if (owner) vcb[static_cast<size_t>(pos) * HD + tid] = vnew;
  }
  __syncthreads();

  // Partial scores of this thread's dimension group.
  {
    float acc[G8][4];
#pragma unroll
    for (int g = 0; g < G8; ++g)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[g][e] = 0.f;
#pragma unroll
    for (int dd = 0; dd < DPG; ++dd) {
      const int d = dg * DPG + dd;
      const float4 kw = widen(kreg[dd]);
      float kk[4] = {kw.x, kw.y, kw.z, kw.w};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (lp + e == pos) kk[e] = kn[d];
#pragma unroll
      for (int g = 0; g < G8; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[g][e] = fmaf(qs[g][d], kk[e], acc[g][e]);
    }
#pragma unroll
    for (int g = 0; g < G8; ++g)
#pragma unroll
      for (int e = 0; e < 4; ++e) sp[dg][g][4 * p4 + e] = acc[g][e];
  }
  __syncthreads();
  // Scores (16 groups added in order); a wave holds one head's 64 positions
  // (C = 64), so its max and its sum of exp(score - max) are wave reductions.
  static_assert(C == 64, "one head's chunk a wave");
  for (int t = tid; t < G8 * C; t += decode::THREADS) {
    const int g = t / C, j = t % C;
    if (g >= G) {  // (wave-uniform: a wave holds one head)
      p[g][j] = 0.f;
      continue;
    }
    float sc = 0.f;
#pragma unroll
    for (int q = 0; q < DG; ++q) sc += sp[q][g][j];
    sc = j < n ? sc : -INFINITY;
    const float m = wave_max(sc);
    const float e = j < n ? expf(sc - m) : 0.f;
    const float sum = wave_sum(e);
    p[g][j] = e;
    if (j == 0) {
      stat[g][0] = m;
      stat[g][1] = sum;
    }
  }
  __syncthreads();
  // acc[g][d] = sum_j p[g][j] V[j][d] over this thread's positions.
  {
    float acc[G8][4];
#pragma unroll
    for (int g = 0; g < G8; ++g)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[g][e] = 0.f;
#pragma unroll
    for (int jj = 0; jj < VJ; ++jj) {
      const int j = pg + jj * PG;  // past pos: p is 0 and the value read 0
      const float4 vv =
          l0 + j == pos ? make_float4(vn[4 * d4], vn[4 * d4 + 1], vn[4 * d4 + 2], vn[4 * d4 + 3]) : widen(vreg[jj]);
#pragma unroll
      for (int g = 0; g < G8; ++g) {
        const float pj = p[g][j];
        acc[g][0] = fmaf(pj, vv.x, acc[g][0]);
        acc[g][1] = fmaf(pj, vv.y, acc[g][1]);
        acc[g][2] = fmaf(pj, vv.z, acc[g][2]);
        acc[g][3] = fmaf(pj, vv.w, acc[g][3]);
      }
    }
#pragma unroll
    for (int g = 0; g < G8; ++g)
      *reinterpret_cast<float4*>(&pacc[pg][g][4 * d4]) = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
  }
  __syncthreads();
  float* wrow = work + static_cast<size_t>(blockIdx.x) * decode::MAX_GROUP * (HD + 2);
  for (int t = tid; t < G * HD; t += decode::THREADS) {
    const int g = t / HD, d = t % HD;
    float o = 0.f;
#pragma unroll
    for (int pp = 0; pp < PG; ++pp) o += pacc[pp][g][d];
    wrow[g * (HD + 2) + 2 + d] = o;
  }
  if (tid < G) {
    wrow[tid * (HD + 2)] = stat[tid][0];
    wrow[tid * (HD + 2) + 1] = stat[tid][1];
  }
}

// out[row, head] = sum_c acc_c exp(m_c - M) / sum_c s_c exp(m_c - M), chunks in order;
// with `tiles`, out is written as x tiles of the [rows, heads * HD] output.
template <int HD>
__global__ __launch_bounds__(HD) void decode_combine_kernel(const float* __restrict__ work, uint16_t* __restrict__ out,
                                                            int heads, int kv_heads, int chunks,
                                                            const int32_t* __restrict__ pos_dev, int cap, bool tiles) {
  // One round trip to memory: every load is issued as the kernel starts -- the
  // chunks' (m, s) (thread t: chunks t, t + HD, ...) and thread d's dimension
  // of the first PRE chunks' sums -- then the max and the sum of the weights
  // (block reductions, the weights exp(m - M) kept in LDS), then thread d adds
  // its dimension over the chunks in order.
  constexpr int WAVES = HD / 64;
  constexpr int PRE = 32;  // chunks whose sums a thread holds in registers (context 2048)
  __shared__ float wts[decode::MAX_CHUNKS];
  __shared__ float red[WAVES];
  const int G = heads / kv_heads;
  const int row = blockIdx.x / heads, head = blockIdx.x % heads;
  const int kvh = head / G, g = head % G;
  const int d = threadIdx.x;
  const size_t o_at = tiles ? x_tile_index(row, head * HD + d, heads * HD)
                            : (static_cast<size_t>(row) * heads + head) * HD + d;
  const float* base = work + (static_cast<size_t>(row) * kv_heads + kvh) * chunks * decode::MAX_GROUP * (HD + 2) +
                      g * (HD + 2);
  const size_t stride = static_cast<size_t>(decode::MAX_GROUP) * (HD + 2);
  // With the position in device memory, the chunks up to pos's (the workspace
  // keeps the whole cache's chunk stride); a position outside the cache gives zeros.
  int live = chunks;
  if (pos_dev != nullptr) {
    const int p = *pos_dev;
    live = p >= 0 && p < cap ? p / decode::CHUNK + 1 : 0;
    if (live == 0) {
      out[o_at] = 0;
      return;
    }
  }
  // (Loads past the live chunks read the last live chunk again and are unused:
  // unconditional, so that they issue together.)
  float a_pre[PRE];
#pragma unroll
  for (int i = 0; i < PRE; ++i) a_pre[i] = base[static_cast<size_t>(min(i, live - 1)) * stride + 2 + d];
  float m_own = -INFINITY, s_own = 0.f;  // thread d's first chunk (d < live)
  if (d < live) {
    m_own = base[static_cast<size_t>(d) * stride];
    s_own = base[static_cast<size_t>(d) * stride + 1];
  }
  auto block_reduce = [&](float v, bool is_max) {
    v = is_max ? wave_max(v) : wave_sum(v);
    __syncthreads();
    if ((d & 63) == 0) red[d >> 6] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < WAVES; ++i) r = is_max ? fmaxf(r, red[i]) : r + red[i];
    return r;
  };
  float m = m_own;
  for (int c = d + HD; c < live; c += HD) m = fmaxf(m, base[c * stride]);
  const float M = block_reduce(m, true);
  float sp = 0.f;
  if (d < live) {
    const float w = expf(m_own - M);
    wts[d] = w;
    sp = s_own * w;
  }
  for (int c = d + HD; c < live; c += HD) {
    const float w = expf(base[c * stride] - M);
    wts[c] = w;
    sp = fmaf(base[c * stride + 1], w, sp);
  }
  const float S = block_reduce(sp, false);  // its barriers also publish wts
  float o = 0.f;
#pragma unroll
  for (int i = 0; i < PRE; ++i)
    if (i < live) o = fmaf(a_pre[i], wts[i], o);
  for (int c = PRE; c < live; ++c) o = fmaf(base[c * stride + 2 + d], wts[c], o);
  out[o_at] = f32_to_bf16_bits(o / S);
}

// A prompt's rotary embedding and cache writes, one kernel for what the torch
// glue does in ~15: workgroup (head slot hs, 64-position tile). Slots 0..heads-1
// are q heads, then the kv_heads k heads, then the v heads. A tile of 64
// positions x HD values moves through LDS (coalesced loads along each
// position's HD values); q and k are rotated in f32 (pairs i, i + HD/2, cos / sin
// tables [cap, HD/2] at each position) and rounded to bf16, as the decode kernel
// and the torch reference round them; q, k and v go out head-major [head, P, HD]
// (the fused attention's layout), k also transposed into Kt [kv_heads, HD, cap]
// and v into V [kv_heads, cap, HD] at positions 0..P-1.
template <int HD>
__global__ __launch_bounds__(decode::THREADS) void prefill_rope_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int64_t in_stride,
    const float* __restrict__ cosv, const float* __restrict__ sinv, uint16_t* __restrict__ q_out,
    uint16_t* __restrict__ k_out, uint16_t* __restrict__ v_out, uint16_t* __restrict__ kt, uint16_t* __restrict__ vc,
    int P, int heads, int kv_heads, int cap) {
  constexpr int C = 64;                  // positions a tile
  constexpr int HALF = HD / 2;
  constexpr int CH = HD / 8;             // 16-byte chunks a position
  __shared__ uint16_t tile[C][HD + 2];   // (+2: the transposed reads of Kt hit distinct banks)
  const int hs = blockIdx.y;
  const int p0 = blockIdx.x * C;
  const int tid = threadIdx.x;
  const bool is_q = hs < heads, is_k = !is_q && hs < heads + kv_heads;
  const int h = is_q ? hs : is_k ? hs - heads : hs - heads - kv_heads;
  const uint16_t* src = (is_q ? q : is_k ? k : v) + static_cast<size_t>(h) * HD;
  for (int c = tid; c < C * CH; c += decode::THREADS) {
    const int pl = c / CH, dc = c % CH;
    u32x4 val{0u, 0u, 0u, 0u};
    if (p0 + pl < P) val = *reinterpret_cast<const u32x4*>(src + static_cast<size_t>(p0 + pl) * in_stride + 8 * dc);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      tile[pl][8 * dc + 2 * e] = static_cast<uint16_t>(val[e] & 0xffffu);
      tile[pl][8 * dc + 2 * e + 1] = static_cast<uint16_t>(val[e] >> 16);
    }
  }
  __syncthreads();
  if (is_q || is_k) {
    for (int t = tid; t < C * HALF; t += decode::THREADS) {
      const int pl = t / HALF, i = t % HALF;
      if (p0 + pl >= P) continue;
      const float a = bf16_bits_to_f32(tile[pl][i]), b = bf16_bits_to_f32(tile[pl][i + HALF]);
      const float c = cosv[static_cast<size_t>(p0 + pl) * HALF + i], sn = sinv[static_cast<size_t>(p0 + pl) * HALF + i];
      tile[pl][i] = f32_to_bf16_bits(a * c - b * sn);
      tile[pl][i + HALF] = f32_to_bf16_bits(b * c + a * sn);
    }
    __syncthreads();
  }
  uint16_t* out = (is_q ? q_out : is_k ? k_out : v_out) + static_cast<size_t>(h) * P * HD;
  for (int c = tid; c < C * HD; c += decode::THREADS) {
    const int pl = c / HD, d = c % HD;
    if (p0 + pl < P) out[static_cast<size_t>(p0 + pl) * HD + d] = tile[pl][d];
  }
  if (is_k) {
    uint16_t* ktb = kt + static_cast<size_t>(h) * HD * cap;
    for (int c = tid; c < HD * C; c += decode::THREADS) {
      const int d = c / C, pl = c % C;  // consecutive threads: consecutive positions of one dimension
      if (p0 + pl < P) ktb[static_cast<size_t>(d) * cap + p0 + pl] = tile[pl][d];
    }
  } else if (!is_q) {
    uint16_t* vcb = vc + static_cast<size_t>(h) * cap * HD;
    for (int c = tid; c < C * HD; c += decode::THREADS) {
      const int pl = c / HD, d = c % HD;
      if (p0 + pl < P) vcb[static_cast<size_t>(p0 + pl) * HD + d] = tile[pl][d];
    }
  }
}

__global__ __launch_bounds__(decode::THREADS) void silu_mul_kernel(const uint16_t* __restrict__ g,
                                                                   const uint16_t* __restrict__ u,
                                                                   uint16_t* __restrict__ a, int64_t n, int64_t width,
                                                                   int64_t g_stride, int64_t u_stride, bool tiles) {
  // Element i of a [rows, width]: row i / width of g and u, whose rows are
  // g_stride and u_stride elements apart (the two halves of a joined gate|up
  // projection's output, say); with `tiles`, a is written as x tiles.
  for (int64_t i = blockIdx.x * static_cast<int64_t>(decode::THREADS) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * decode::THREADS) {
    const int64_t r = i / width, c = i - r * width;
    const size_t o = tiles ? x_tile_index(static_cast<int>(r), static_cast<int>(c), static_cast<int>(width))
                           : static_cast<size_t>(i);
    a[o] = f32_to_bf16_bits(silu_times(bf16_bits_to_f32(g[r * g_stride + c]), bf16_bits_to_f32(u[r * u_stride + c])));
  }
}

}  // namespace lnq

using namespace lnq;

extern "C" {

LNQ_API int64_t lnq_decode_attention_workspace(int64_t rows, int64_t kv_heads, int64_t head_dim, int64_t pos);

LNQ_API LnqStatus lnq_rmsnorm(void* x, const void* delta, const float* weight, void* h, int64_t rows,
                              int64_t hidden, float eps, void* stream) {
  LNQ_REQUIRE(rows >= 0 && hidden > 0 && hidden <= INT32_MAX && rows <= INT32_MAX, "lnq_rmsnorm: bad shape");
  if (rows == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(x && weight && h, "lnq_rmsnorm: null pointer");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  auto* xs = static_cast<uint16_t*>(x);
  const auto* ds = static_cast<const uint16_t*>(delta);
  auto* hs = static_cast<uint16_t*>(h);
  const int H = static_cast<int>(hidden);
  const int ch = (H + 8 * decode::THREADS - 1) / (8 * decode::THREADS);
  const bool vec = H % 8 == 0 && ch <= 8 && aligned(x, 16) && aligned(h, 16) && aligned(weight, 16) &&
                   (delta == nullptr || aligned(delta, 16));
  const dim3 grid(static_cast<unsigned>(rows)), block(decode::THREADS);
  if (vec && ch == 1) hipLaunchKernelGGL(rmsnorm_vec_kernel<1>, grid, block, 0, s, xs, ds, weight, hs, H, eps);
  else if (vec && ch == 2) hipLaunchKernelGGL(rmsnorm_vec_kernel<2>, grid, block, 0, s, xs, ds, weight, hs, H, eps);
  else if (vec && ch <= 4) hipLaunchKernelGGL(rmsnorm_vec_kernel<4>, grid, block, 0, s, xs, ds, weight, hs, H, eps);
  else if (vec) hipLaunchKernelGGL(rmsnorm_vec_kernel<8>, grid, block, 0, s, xs, ds, weight, hs, H, eps);
  else hipLaunchKernelGGL(rmsnorm_kernel, grid, block, 0, s, xs, ds, weight, hs, H, eps);
  return launched("rmsnorm");
}

LNQ_API LnqStatus lnq_rmsnorm_tiles(void* x, const void* delta, const float* weight, void* xt, int64_t rows,
                                    int64_t hidden, float eps, void* stream) {
  LNQ_REQUIRE(rows >= 0 && rows <= INT32_MAX && hidden > 0 && hidden % 256 == 0 && hidden <= 64 * decode::THREADS,
              "lnq_rmsnorm_tiles: bad shape rows=%lld hidden=%lld (hidden %% 256 == 0, <= %d)", (long long)rows,
              (long long)hidden, 64 * decode::THREADS);
  if (rows == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(x && weight && xt, "lnq_rmsnorm_tiles: null pointer");
  LNQ_REQUIRE(aligned(x, 16) && aligned(xt, 16) && aligned(weight, 16) && (delta == nullptr || aligned(delta, 16)),
              "lnq_rmsnorm_tiles: operands must be 16-byte aligned");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  auto* xs = static_cast<uint16_t*>(x);
  const auto* ds = static_cast<const uint16_t*>(delta);
  auto* hs = static_cast<uint16_t*>(xt);
  const int H = static_cast<int>(hidden);
  const int ch = (H + 8 * decode::THREADS - 1) / (8 * decode::THREADS);
  const dim3 grid(static_cast<unsigned>(rows)), block(decode::THREADS);
  if (ch == 1) hipLaunchKernelGGL((rmsnorm_vec_kernel<1, true>), grid, block, 0, s, xs, ds, weight, hs, H, eps);
  else if (ch == 2) hipLaunchKernelGGL((rmsnorm_vec_kernel<2, true>), grid, block, 0, s, xs, ds, weight, hs, H, eps);
  else if (ch <= 4) hipLaunchKernelGGL((rmsnorm_vec_kernel<4, true>), grid, block, 0, s, xs, ds, weight, hs, H, eps);
  else hipLaunchKernelGGL((rmsnorm_vec_kernel<8, true>), grid, block, 0, s, xs, ds, weight, hs, H, eps);
  return launched("rmsnorm_tiles");
}

LNQ_API LnqStatus lnq_rmsnorm_parts(void* x, const float* parts, int32_t splits, const float* weight, void* h,
                                    int32_t h_tiles, int64_t rows, int64_t hidden, float eps, void* stream) {
  LNQ_REQUIRE(rows >= 0 && rows <= INT32_MAX && hidden > 0 && hidden % 256 == 0 && hidden <= 64 * decode::THREADS &&
                  splits >= 1,
              "lnq_rmsnorm_parts: bad shape rows=%lld hidden=%lld splits=%d (hidden %% 256 == 0, <= %d)",
              (long long)rows, (long long)hidden, splits, 64 * decode::THREADS);
  if (rows == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(x && parts && weight && h, "lnq_rmsnorm_parts: null pointer");
  LNQ_REQUIRE(aligned(x, 16) && aligned(h, 16) && aligned(weight, 16) && aligned(parts, 16),
              "lnq_rmsnorm_parts: operands must be 16-byte aligned");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  auto* xs = static_cast<uint16_t*>(x);
  auto* hs = static_cast<uint16_t*>(h);
  const int H = static_cast<int>(hidden);
  const int ch = (H + 8 * decode::THREADS - 1) / (8 * decode::THREADS);
  const dim3 grid(static_cast<unsigned>(rows)), block(decode::THREADS);
#define LNQ_RMS_PARTS(C_)                                                                                             \
  if (h_tiles) hipLaunchKernelGGL((rmsnorm_vec_kernel<C_, true>), grid, block, 0, s, xs, nullptr, weight, hs, H, eps,  \
                                  parts, splits);                                                                      \
  else hipLaunchKernelGGL((rmsnorm_vec_kernel<C_, false>), grid, block, 0, s, xs, nullptr, weight, hs, H, eps, parts,  \
                          splits)
  if (ch == 1) { LNQ_RMS_PARTS(1); }
  else if (ch == 2) { LNQ_RMS_PARTS(2); }
  else if (ch <= 4) { LNQ_RMS_PARTS(4); }
  else { LNQ_RMS_PARTS(8); }
#undef LNQ_RMS_PARTS
  return launched("rmsnorm_parts");
}

// pos_dev: nullptr (the position is `pos`) or the device address of the int32
// position, the grid then sized for position `pos` = cap - 1 (the whole cache).
static LnqStatus decode_attention(const void* q, const void* k, const void* v, const float* cos, const float* sin,
                                  void* kt_cache, void* v_cache, void* out, float* workspace,
                                  int64_t workspace_floats, int64_t rows, int64_t heads, int64_t kv_heads,
                                  int64_t head_dim, int64_t cap, int64_t pos, int64_t q_stride, int64_t kv_stride,
                                  const int32_t* pos_dev, void* stream, bool tiles = false) {
  LNQ_REQUIRE(head_dim == 64 || head_dim == 128, "lnq_decode_attention: head_dim is 64 or 128, not %lld",
              static_cast<long long>(head_dim));
  LNQ_REQUIRE(rows >= 0 && kv_heads > 0 && heads % kv_heads == 0 && heads / kv_heads <= decode::MAX_GROUP,
              "lnq_decode_attention: heads must be a multiple (at most %d) of kv_heads", decode::MAX_GROUP);
  LNQ_REQUIRE(pos >= 0 && pos < cap && cap <= INT32_MAX, "lnq_decode_attention: position %lld outside the cache",
              static_cast<long long>(pos));
  LNQ_REQUIRE(cap % 4 == 0, "lnq_decode_attention: the cache capacity %lld is not a multiple of 4",
              static_cast<long long>(cap));
  const int64_t chunks = (pos + decode::CHUNK) / decode::CHUNK;
  LNQ_REQUIRE(chunks <= decode::MAX_CHUNKS, "lnq_decode_attention: position %lld past the %d the merge takes",
              static_cast<long long>(pos), decode::MAX_CHUNKS * decode::CHUNK - 1);
  const int64_t need = lnq_decode_attention_workspace(rows, kv_heads, head_dim, pos);
  LNQ_REQUIRE(workspace_floats >= need, "lnq_decode_attention: the workspace holds %lld floats, %lld needed",
              static_cast<long long>(workspace_floats), static_cast<long long>(need));
  LNQ_REQUIRE(rows * kv_heads * chunks <= INT32_MAX && rows * heads <= INT32_MAX, "lnq_decode_attention: too many rows");
  if (rows == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(q && k && v && cos && sin && kt_cache && v_cache && out && workspace, "lnq_decode_attention: null pointer");
  LNQ_REQUIRE(aligned(kt_cache, 16) && aligned(v_cache, 16), "lnq_decode_attention: caches must be 16-byte aligned");
  const dim3 grid(static_cast<unsigned>(rows * kv_heads * chunks)), grid2(static_cast<unsigned>(rows * heads));
  hipStream_t s = static_cast<hipStream_t>(stream);
#define LNQ_ATT_G(HD_, GT_)                                                                                       \
  hipLaunchKernelGGL((decode_attention_kernel<HD_, GT_>), grid, dim3(decode::THREADS), 0, s,                      \
                     static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),                              \
                     static_cast<const uint16_t*>(v), cos, sin, static_cast<uint16_t*>(kt_cache),                    \
                     static_cast<uint16_t*>(v_cache), workspace,                                                    \
                     static_cast<int>(heads), static_cast<int>(kv_heads), static_cast<int>(cap), static_cast<int>(pos), \
                     static_cast<int>(chunks), qs_, kvs_, pos_dev);                                                 \
  hipLaunchKernelGGL(decode_combine_kernel<HD_>, grid2, dim3(HD_), 0, s, workspace, static_cast<uint16_t*>(out),   \
                     static_cast<int>(heads), static_cast<int>(kv_heads), static_cast<int>(chunks), pos_dev,         \
                     static_cast<int>(cap), tiles)
#define LNQ_ATT(HD_)                                      \
  switch (group <= 1 ? 1 : group <= 2 ? 2 : group <= 4 ? 4 : 8) { \
    case 1: LNQ_ATT_G(HD_, 1); break;                     \
    case 2: LNQ_ATT_G(HD_, 2); break;                     \
    case 4: LNQ_ATT_G(HD_, 4); break;                     \
    default: LNQ_ATT_G(HD_, 8); break;                    \
  }
  const int64_t group = heads / kv_heads;
  // Row strides of q and of k / v in elements, so q, k and v may be column
  // slices of one joined projection's output. Past one row each stride spans at
  // least a row: a stride of 0 (a row broadcast over rows) is refused rather
  // than read as rows that are not there. One row reads no stride.
  LNQ_REQUIRE(rows == 1 || (q_stride >= heads * head_dim && kv_stride >= kv_heads * head_dim),
              "lnq_decode_attention: row strides %lld / %lld shorter than a row", static_cast<long long>(q_stride),
              static_cast<long long>(kv_stride));
  LNQ_REQUIRE(!tiles || ((heads * head_dim) % 256 == 0 && aligned(out, 16)),
              "lnq_decode_attention_tiles: x tiles take heads * head_dim %% 256 == 0 and a 16-byte aligned output");
  const int64_t qs_ = rows == 1 ? heads * head_dim : q_stride;
  const int64_t kvs_ = rows == 1 ? kv_heads * head_dim : kv_stride;
  if (head_dim == 64) {
    LNQ_ATT(64);
  } else {
    LNQ_ATT(128);
  }
#undef LNQ_ATT
#undef LNQ_ATT_G
  return launched("decode_attention");
}

LNQ_API LnqStatus lnq_decode_attention(const void* q, const void* k, const void* v, const float* cos,
                                       const float* sin, void* kt_cache, void* v_cache, void* out, float* workspace,
                                       int64_t workspace_floats, int64_t rows, int64_t heads, int64_t kv_heads,
                                       int64_t head_dim, int64_t cap, int64_t pos, int64_t q_stride,
                                       int64_t kv_stride, void* stream) {
  return decode_attention(q, k, v, cos, sin, kt_cache, v_cache, out, workspace, workspace_floats, rows, heads,
                          kv_heads, head_dim, cap, pos, q_stride, kv_stride, nullptr, stream);
}

LNQ_API LnqStatus lnq_decode_attention_at(const void* q, const void* k, const void* v, const float* cos_table,
                                          const float* sin_table, void* kt_cache, void* v_cache, void* out,
                                          float* workspace, int64_t workspace_floats, int64_t rows, int64_t heads,
                                          int64_t kv_heads, int64_t head_dim, int64_t cap, const int32_t* pos,
                                          int64_t q_stride, int64_t kv_stride, void* stream) {
  LNQ_REQUIRE(pos != nullptr || rows == 0, "lnq_decode_attention_at: null position");
  LNQ_REQUIRE(cap > 0, "lnq_decode_attention_at: empty cache");
  return decode_attention(q, k, v, cos_table, sin_table, kt_cache, v_cache, out, workspace, workspace_floats, rows,
                          heads, kv_heads, head_dim, cap, cap - 1, q_stride, kv_stride, pos, stream);
}

LNQ_API LnqStatus lnq_decode_attention_tiles(const void* q, const void* k, const void* v, const float* cos,
                                             const float* sin, void* kt_cache, void* v_cache, void* out_tiles,
                                             float* workspace, int64_t workspace_floats, int64_t rows, int64_t heads,
                                             int64_t kv_heads, int64_t head_dim, int64_t cap, int64_t pos,
                                             const int32_t* pos_dev, int64_t q_stride, int64_t kv_stride,
                                             void* stream) {
  if (pos_dev != nullptr) {
    LNQ_REQUIRE(cap > 0, "lnq_decode_attention_tiles: empty cache");
    pos = cap - 1;
  }
  return decode_attention(q, k, v, cos, sin, kt_cache, v_cache, out_tiles, workspace, workspace_floats, rows, heads,
                          kv_heads, head_dim, cap, pos, q_stride, kv_stride, pos_dev, stream, true);
}

LNQ_API int64_t lnq_decode_attention_workspace(int64_t rows, int64_t kv_heads, int64_t head_dim, int64_t pos) {
  const int64_t chunks = (pos + decode::CHUNK) / decode::CHUNK;
  return rows * kv_heads * chunks * decode::MAX_GROUP * (head_dim + 2);
}

LNQ_API LnqStatus lnq_decode_attention_noalloc(const void* q, const void* k, const void* v, const float* cos,
                                               const float* sin, void* kt_cache, void* v_cache, void* out,
                                               int64_t rows, int64_t heads, int64_t kv_heads, int64_t head_dim,
                                               int64_t cap, int64_t pos, int64_t q_stride, int64_t kv_stride,
                                               void* stream) {
  // The sizes the workspace depends on, checked before any device call.
  LNQ_REQUIRE(head_dim == 64 || head_dim == 128, "lnq_decode_attention_noalloc: head_dim is 64 or 128, not %lld",
              static_cast<long long>(head_dim));
  LNQ_REQUIRE(rows >= 0 && rows <= INT32_MAX && kv_heads > 0 && kv_heads <= INT32_MAX && pos >= 0 &&
                  pos < decode::MAX_CHUNKS * decode::CHUNK,
              "lnq_decode_attention_noalloc: bad shape rows=%lld kv_heads=%lld pos=%lld",
              static_cast<long long>(rows), static_cast<long long>(kv_heads), static_cast<long long>(pos));
  const int64_t need = lnq_decode_attention_workspace(rows, kv_heads, head_dim, pos);
  LNQ_REQUIRE(need <= LNQ_DECODE_ATTENTION_SCRATCH_FLOATS,
              "lnq_decode_attention_noalloc: the step needs %lld workspace floats, more than the %lld the library "
              "holds (use lnq_decode_attention with a workspace of that size)",
              static_cast<long long>(need), static_cast<long long>(LNQ_DECODE_ATTENTION_SCRATCH_FLOATS));
  float* work = nullptr;
  if (rows > 0) {
    work = scratch_on_current_device();
    if (work == nullptr) return LNQ_ERROR;
  }
  // The kernels write every workspace entry the merge reads in the same call, so
  // nothing in `scratch` has to start at zero.
  return lnq_decode_attention(q, k, v, cos, sin, kt_cache, v_cache, out, work, LNQ_DECODE_ATTENTION_SCRATCH_FLOATS,
                              rows, heads, kv_heads, head_dim, cap, pos, q_stride, kv_stride, stream);
}

LNQ_API LnqStatus lnq_prefill_rope(const void* q, const void* k, const void* v, int64_t in_stride,
                                   const float* cos_table, const float* sin_table, void* q_out, void* k_out,
                                   void* v_out, void* kt_cache, void* v_cache, int64_t positions, int64_t heads,
                                   int64_t kv_heads, int64_t head_dim, int64_t cap, void* stream) {
  LNQ_REQUIRE(head_dim == 64 || head_dim == 128, "lnq_prefill_rope: head_dim is 64 or 128, not %lld",
              static_cast<long long>(head_dim));
  LNQ_REQUIRE(positions >= 0 && positions <= cap && cap <= INT32_MAX && heads > 0 && kv_heads > 0 &&
                  heads % kv_heads == 0 && heads + 2 * kv_heads <= 65535,
              "lnq_prefill_rope: bad shape (positions <= cap, heads a multiple of kv_heads)");
  LNQ_REQUIRE(in_stride >= head_dim && in_stride % 8 == 0, "lnq_prefill_rope: in_stride is a multiple of 8 elements");
  // A position's q row spans heads * head_dim elements (k and v rows kv_heads *
  // head_dim <= that): a shorter stride would read rows that overlap.
  LNQ_REQUIRE(positions <= 1 || in_stride >= heads * head_dim,
              "lnq_prefill_rope: row stride %lld is shorter than a q row of %lld elements",
              static_cast<long long>(in_stride), static_cast<long long>(heads * head_dim));
  if (positions == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(q && k && v && cos_table && sin_table && q_out && k_out && v_out && kt_cache && v_cache,
              "lnq_prefill_rope: null pointer");
  LNQ_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(v, 16), "lnq_prefill_rope: q, k and v 16-byte aligned");
  const dim3 grid(static_cast<unsigned>((positions + 63) / 64), static_cast<unsigned>(heads + 2 * kv_heads));
  const auto s = static_cast<hipStream_t>(stream);
  const auto* qs = static_cast<const uint16_t*>(q);
  const auto* ks = static_cast<const uint16_t*>(k);
  const auto* vs = static_cast<const uint16_t*>(v);
  auto* qo = static_cast<uint16_t*>(q_out);
  auto* ko = static_cast<uint16_t*>(k_out);
  auto* vo = static_cast<uint16_t*>(v_out);
  auto* kt = static_cast<uint16_t*>(kt_cache);
  auto* vc = static_cast<uint16_t*>(v_cache);
  const int P = static_cast<int>(positions), H = static_cast<int>(heads), KVH = static_cast<int>(kv_heads);
  if (head_dim == 128)
    hipLaunchKernelGGL(prefill_rope_kernel<128>, grid, dim3(decode::THREADS), 0, s, qs, ks, vs, in_stride, cos_table,
                       sin_table, qo, ko, vo, kt, vc, P, H, KVH, static_cast<int>(cap));
  else
    hipLaunchKernelGGL(prefill_rope_kernel<64>, grid, dim3(decode::THREADS), 0, s, qs, ks, vs, in_stride, cos_table,
                       sin_table, qo, ko, vo, kt, vc, P, H, KVH, static_cast<int>(cap));
  return launched("prefill_rope");
}

LNQ_API LnqStatus lnq_silu_mul(const void* g, const void* u, void* a, int64_t n, void* stream) {
  LNQ_REQUIRE(n >= 0, "lnq_silu_mul: bad size");
  if (n == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(g && u && a, "lnq_silu_mul: null pointer");
  const int64_t blocks = (n + decode::THREADS - 1) / decode::THREADS;
  hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<unsigned>(blocks < 4096 ? blocks : 4096)),
                     dim3(decode::THREADS), 0, static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(g),
                     static_cast<const uint16_t*>(u), static_cast<uint16_t*>(a), n, n, int64_t{0}, int64_t{0}, false);
  return launched("silu_mul");
}

LNQ_API LnqStatus lnq_silu_mul_rows(const void* g, const void* u, void* a, int64_t rows, int64_t width,
                                    int64_t g_stride, int64_t u_stride, void* stream) {
  LNQ_REQUIRE(rows >= 0 && width >= 0 && g_stride >= width && u_stride >= width, "lnq_silu_mul_rows: bad shape");
  if (rows == 0 || width == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(g && u && a, "lnq_silu_mul_rows: null pointer");
  const int64_t n = rows * width;
  const int64_t blocks = (n + decode::THREADS - 1) / decode::THREADS;
  hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<unsigned>(blocks < 4096 ? blocks : 4096)),
                     dim3(decode::THREADS), 0, static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(g),
                     static_cast<const uint16_t*>(u), static_cast<uint16_t*>(a), n, width, g_stride, u_stride, false);
  return launched("silu_mul_rows");
}

LNQ_API LnqStatus lnq_silu_mul_tiles(const void* g, const void* u, void* xt, int64_t rows, int64_t width,
                                     int64_t g_stride, int64_t u_stride, void* stream) {
  LNQ_REQUIRE(rows >= 0 && rows <= INT32_MAX && width > 0 && width % 256 == 0 && width <= INT32_MAX &&
                  g_stride >= width && u_stride >= width,
              "lnq_silu_mul_tiles: bad shape (width %% 256 == 0)");
  if (rows == 0) {
    clear_error();
    return LNQ_OK;
  }
  LNQ_REQUIRE(g && u && xt, "lnq_silu_mul_tiles: null pointer");
  const int64_t n = rows * width;
  const int64_t blocks = (n + decode::THREADS - 1) / decode::THREADS;
  hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<unsigned>(blocks < 4096 ? blocks : 4096)),
                     dim3(decode::THREADS), 0, static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(g),
                     static_cast<const uint16_t*>(u), static_cast<uint16_t*>(xt), n, width, g_stride, u_stride, true);
  return launched("silu_mul_tiles");
}

}  // extern "C"
