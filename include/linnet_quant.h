/* linnet_quant.h -- C ABI of the MI355X (gfx950) weight-quantized linear kernels.
 *
 * The boundary of `liblinnet_quant_hip.so`: plain pointers to device memory,
 * element counts and a HIP stream. No PyTorch types cross it. Conventions follow
 * the reference's native runtime ABI (include/linnet/runtime/runtime.h):
 *
 *   - every entry point returns a status: LNQ_OK 0, LNQ_ERROR 1, LNQ_UNAVAILABLE 2
 *     (runtime.h:37-40), and on failure leaves a message for lnq_last_error(),
 *     a thread-local string (runtime.h:99, runtime.cpp:28);
 *   - work is enqueued on `stream` (a hipStream_t; NULL is the null stream) and the
 *     call returns without waiting for it, as LnExecutable.execute does
 *     (runtime.h:79-94); no entry point allocates device memory or synchronizes,
 *     so every call may be recorded into a HIP graph;
 *   - tensors are borrowed: caller-owned, contiguous, row-major.
 *
 * Each entry point below names the reference interface it replaces (paths are
 * relative to the reference checkout; the Python package is python/linnet/src/linnet).
 */
#ifndef LINNET_QUANT_H
#define LINNET_QUANT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LNQ_API __attribute__((visibility("default")))

#define LNQ_ABI_VERSION 1

typedef int32_t LnqStatus;
#define LNQ_OK 0
#define LNQ_ERROR 1
#define LNQ_UNAVAILABLE 2 /* not on this device */

/* Element types of activations, scales and outputs. */
#define LNQ_BF16 0
#define LNQ_F16 1
#define LNQ_F32 2

/* Kernel families lnq_int4_linear may be told to use (LNQ_KERNEL_AUTO picks by rows). */
#define LNQ_KERNEL_AUTO 0
#define LNQ_KERNEL_SKINNY 1 /* dequant-GEMV/skinny GEMM on MFMA, rows <= 64 */
#define LNQ_KERNEL_TILED 2  /* prefill dequant-GEMM, LDS-staged bf16 tiles on MFMA */
#define LNQ_KERNEL_GEMV 3   /* few-token dequant-GEMV, one workgroup per CU (rows 1..32;
                               in % 256 == 0 and <= 4096, group 128 or a multiple of 256;
                               past 16384 outputs, more workgroups of 64 rows than CUs;
                               one row also in = 256 * S * waves for S = 2..4
                               slices a wave (e.g. 6144, 8192, 12288, 14336) with out <=
                               8192 (S = 2) or 4096 (S = 3, 4)) */
#define LNQ_KERNEL_TILED_128 4 /* the tiled kernel with tiles of 128 output columns */
#define LNQ_KERNEL_TILED_256 5 /* the tiled kernel with tiles of 256 output columns */
#define LNQ_KERNEL_PERSISTENT 6 /* the persistent prefill dequant-GEMM: 256 x 256 tiles,
                                   one workgroup a CU walking its tiles (out % 256 == 0,
                                   in % 256 == 0, group a power of two >= 64) */
#define LNQ_KERNEL_SPLIT 7 /* the 32-row GEMV with `in` split over workgroups, the chunks'
                              f32 sums in a caller workspace (lnq_int4_linear_ws only):
                              rows 1..64 (33..64 as two chunks), out % 4 == 0, in = 4096
                              or a multiple of 256 above it whose slices of 256 split into
                              chunks of 8..16 (e.g. 6144, 8192, 12288, 14336) */

/* The ABI version this library implements (LNQ_ABI_VERSION). */
LNQ_API uint32_t lnq_abi_version(void);

/* The message of the last failed call on this thread ("" if none). */
LNQ_API const char* lnq_last_error(void);

/* Number of GPUs HIP sees, and whether device `device` is a gfx950 (1) or not (0). */
LNQ_API LnqStatus lnq_device_probe(int32_t device, int32_t* is_gfx950, int32_t* compute_units);

/* ---------------------------------------------------------------- int4 groups
 * Layout of std.quant::Int4GroupLinear (stdlib/quant.linnet:156-175):
 *   packed [out, in/group, group/2] u8, element 2k in the low nibble;
 *   scale  [out, in/group] in `dtype`;  zero [out, in/group] u8 in 0..15;
 *   weight[o, i] = (q[o, i] - zero[o, i/group]) * scale[o, i/group].
 */

/* y[rows, out] = x[rows, in] @ W^T (+ bias[out]), x/scale/bias/y of `dtype` (bf16 or
 * f16), summed in f32, rounded once to `dtype`; with a bias, the rounded product plus
 * the bias rounded again (the reference adds the bias after the product).
 * in % 128 == 0; group 32, 64 or a multiple of 128 dividing `in`.
 * Replaces: kernels.py:277-323 `int4_linear` and the generated `_int4_linear`
 * (src/backend/torch_source.cpp:1553-1570; tinygemm below 8 rows, Triton to 128,
 * dequant + cuBLAS above). */
LNQ_API LnqStatus lnq_int4_linear(const void* x, const uint8_t* packed, const void* scale,
                                  const uint8_t* zero, const void* bias, void* y, int64_t rows,
                                  int64_t in_features, int64_t out_features, int64_t group,
                                  int32_t dtype, int32_t kernel, void* stream);

/* std.quant::take_inputs (stdlib/quant.linnet:142-149): taken[r, k] = x[r, order[k]]
 * for `rows` rows of n elements of `dtype` (bf16, f16 or f32); order [n] int32. An
 * index outside [0, n) reads 0 (the reference's index_select raises; checkpoint
 * import checks that an order is a permutation). taken must not be x.
 * Replaces: the `torch.index_select` candidate (src/opt/candidates.cpp:18) as the
 * generated module emits it (src/backend/torch_source.cpp:397-398) and the
 * interpreter's entry (python/linnet/src/linnet/torch/native.py:269-271). */
LNQ_API LnqStatus lnq_take_inputs(const void* x, const int32_t* order, void* taken, int64_t rows, int64_t n,
                                  int32_t dtype, void* stream);

/* Int4GroupLinear.forward with an input order (GPTQ's activation order,
 * stdlib/quant.linnet:163-174): lnq_int4_linear of take_inputs(x, order). One row at
 * group 128 (the decode step) runs one kernel, the gather fused into the one-token
 * GEMV's staging of x (order 16-byte aligned, kernel AUTO or GEMV); any other call
 * gathers into `taken` (rows * in elements of `dtype`, 16-byte aligned; may be NULL
 * when the gather is fused) and multiplies that. order NULL: lnq_int4_linear.
 * Replaces: the two steps the generated module runs for the layer
 * (torch_source.cpp:397-398, then `_int4_linear`, :1553-1570). */
LNQ_API LnqStatus lnq_int4_linear_ordered(const void* x, const int32_t* order, const uint8_t* packed,
                                          const void* scale, const uint8_t* zero, const void* bias, void* y,
                                          void* taken, int64_t rows, int64_t in_features, int64_t out_features,
                                          int64_t group, int32_t dtype, int32_t kernel, void* stream);

/* What lnq_int4_linear_prologue multiplies in place of x. */
#define LNQ_PROLOGUE_RMSNORM 1  /* x * rsqrt(mean(x^2) + eps) * norm_weight, rounded to bf16 */
#define LNQ_PROLOGUE_SILU_MUL 2 /* silu(x) * u = x / (1 + exp(-x)) * u, rounded to bf16 */

/* lnq_int4_linear of the decode glue ahead of a projection (bf16): RMSNorm of x
 * (weight norm_weight f32 [in], eps; what lnq_rmsnorm with no delta computes) or
 * silu(x) * u (u [rows, in], as lnq_silu_mul), then the int4 product, + bias. One row
 * at group 128 runs one kernel, the prologue folded into the one-token GEMV's staging
 * of x (operand 16-byte aligned, kernel AUTO or GEMV): SiLU with the bits of the two
 * kernels; RMSNorm as r * (W (x * w)) with r = rsqrt(mean(x^2) + eps) the row's
 * factor, x * w rounded to bf16 where lnq_rmsnorm rounds x * r * w (so the two
 * differ by that rounding). Any other call writes the prologue's output to `staged`
 * (rows * in bf16, 16-byte aligned) and multiplies that. With one row and bias = the
 * residual stream's row, y = residual + product rounded as a residual add.
 * Replaces: the ops the generated module runs around a quantized linear in the
 * decode step -- `torch.rms_norm` (src/backend/torch_source.cpp:686-689) or SiLU
 * (:670) times up (stdlib/nn/mlp.linnet:22) -- then `_int4_linear` (:1553-1570). */
LNQ_API LnqStatus lnq_int4_linear_prologue(const void* x, const void* u, const float* norm_weight, float eps,
                                           int32_t prologue, const uint8_t* packed, const void* scale,
                                           const uint8_t* zero, const void* bias, void* y, void* staged, int64_t rows,
                                           int64_t in_features, int64_t out_features, int64_t group, int32_t dtype,
                                           int32_t kernel, void* stream);

/* The kernel lnq_int4_linear runs for these arguments on the current device, its
 * operands 16-byte aligned: *chosen = LNQ_KERNEL_GEMV, LNQ_KERNEL_SKINNY,
 * LNQ_KERNEL_TILED_128, LNQ_KERNEL_TILED_256 or LNQ_KERNEL_PERSISTENT (GEMV also
 * for 33..64 rows run as 32-row chunks). Fails as lnq_int4_linear would on arguments it refuses.
 * No counterpart in the reference (its dispatch is Python, torch_source.cpp:1553-1570):
 * lets a caller or a test see which kernel a shape takes. */
LNQ_API LnqStatus lnq_int4_linear_plan(int64_t rows, int64_t in_features, int64_t out_features,
                                       int64_t group, int32_t dtype, int32_t kernel,
                                       int32_t* chosen);

/* lnq_int4_linear with scratch memory of the caller's: `workspace` (16-byte aligned,
 * workspace_bytes long; NULL with 0 is allowed) lets the automatic choice take
 * LNQ_KERNEL_SPLIT where it is faster (16..64 rows with in > 4096 -- the down
 * projection of a decode batch -- and 17..64 rows over out >= 65536 at in = 4096),
 * the K chunks' partial sums written there and added in chunk order (deterministic).
 * Without enough workspace it chooses as lnq_int4_linear does; kernel
 * LNQ_KERNEL_SPLIT runs the split GEMV or fails. Calls that overlap on one
 * workspace race. Other kernels as lnq_int4_linear.
 * Replaces: the same reference calls as lnq_int4_linear (torch_source.cpp:1553-1570,
 * Triton's `int4_linear` at 16..64 rows); the workspace is the caller allocator's
 * memory a generated module hands over, as it does for the reference's BLAS calls. */
LNQ_API LnqStatus lnq_int4_linear_ws(const void* x, const uint8_t* packed, const void* scale,
                                     const uint8_t* zero, const void* bias, void* y, int64_t rows,
                                     int64_t in_features, int64_t out_features, int64_t group,
                                     int32_t dtype, int32_t kernel, void* workspace,
                                     int64_t workspace_bytes, void* stream);

/* The kernel lnq_int4_linear_ws runs for these arguments given enough workspace
 * (*chosen as lnq_int4_linear_plan's, or LNQ_KERNEL_SPLIT) and the workspace bytes
 * it needs (*workspace_bytes: 0 unless LNQ_KERNEL_SPLIT, then K chunks * min(rows, 32)
 * * out * 4). No counterpart in the reference (its dispatch is Python,
 * torch_source.cpp:1553-1570): lets a caller size the workspace. */
LNQ_API LnqStatus lnq_int4_linear_workspace(int64_t rows, int64_t in_features, int64_t out_features,
                                            int64_t group, int32_t dtype, int32_t kernel,
                                            int32_t* chosen, int64_t* workspace_bytes);

/* x tiles: activations laid out for the few-row GEMVs' matrix-core operands, so
 * that each 1 KB operand they load is contiguous (row-major x makes every load
 * instruction read 16 rows x 64 bytes, a third of the rate of whole lines). For rows
 * x in values (in % 256 == 0), chunks of 32 rows of in * 32 values; within a chunk,
 * value (m, k) sits at ((k / 256 * 16 + 8 (m / 16 % 2) + 4 (k / 128 % 2) + k / 32 % 4)
 * * 64 + 16 (k / 8 % 4) + m % 16) * 8 + 2 (k % 4) + k % 8 / 4 (each 8 consecutive
 * inputs in the order 0, 4, 1, 5, 2, 6, 3, 7). lnq_x_tiles writes them from row-major
 * x (2-byte values; rows of the last chunk past `rows` zero; x, xt 16-byte aligned).
 * No counterpart in the reference (a layout of this library's decode kernels). */
LNQ_API LnqStatus lnq_x_tiles(const void* x, void* xt, int64_t rows, int64_t in_features, void* stream);

/* lnq_int4_linear_ws on x given as x tiles (rows 1..64, in % 256 == 0): the 32-row
 * GEMV (in <= 4096; kernel AUTO or GEMV) or the split GEMV (kernel SPLIT, where the
 * automatic choice of lnq_int4_linear_ws takes it with this workspace, and always
 * past in = 4096, which then needs the workspace lnq_int4_linear_workspace names).
 * The products are those of the same kernels on row-major x, bit for bit.
 * Replaces: the same reference calls as lnq_int4_linear (torch_source.cpp:1553-1570),
 * for a caller whose previous kernel wrote x tiles (lnq_rmsnorm_tiles,
 * lnq_silu_mul_tiles). */
LNQ_API LnqStatus lnq_int4_linear_tiles(const void* xt, const uint8_t* packed, const void* scale,
                                        const uint8_t* zero, const void* bias, void* y, int64_t rows,
                                        int64_t in_features, int64_t out_features, int64_t group,
                                        int32_t dtype, int32_t kernel, void* workspace,
                                        int64_t workspace_bytes, void* stream);

/* The split GEMV of lnq_int4_linear_tiles (1..32 rows, in > 4096) without its
 * last step: the K chunks' f32 partial sums are left in parts [*splits, rows, out]
 * (16-byte aligned, lnq_int4_linear_workspace's bytes) for a consumer that adds
 * them in chunk order and rounds once, giving the bits of lnq_int4_linear_tiles
 * with no bias (lnq_rmsnorm_parts takes them as its residual delta). */
LNQ_API LnqStatus lnq_int4_linear_tiles_parts(const void* xt, const uint8_t* packed, const void* scale,
                                              const uint8_t* zero, float* parts, int64_t parts_bytes, int64_t rows,
                                              int64_t in_features, int64_t out_features, int64_t group,
                                              int32_t dtype, int32_t* splits, void* stream);

/* out[out, in] = (q - zero) * scale computed in f32 and rounded once to `dtype`
 * (the scale's dtype: bf16, f16 or f32). Any even group dividing `in`.
 * Replaces: `_int4_unpack`/`_int4_weight` (torch_source.cpp:1518-1550) and the
 * dequantized branch of `_int4_pack` (torch_source.cpp:1501-1504). */
LNQ_API LnqStatus lnq_int4_dequantize(const uint8_t* packed, const void* scale,
                                      const uint8_t* zero, void* out, int64_t out_features,
                                      int64_t in_features, int64_t group, int32_t dtype,
                                      void* stream);

/* Round-to-nearest asymmetric 4-bit quantization of an f32 weight [out, in], bit for
 * bit as numpy does it: scale = (max - min) / 15 (0 -> 1), zero = clip(rint(-min /
 * scale), 0, 15), q = clip(rint(w / scale) + zero, 0, 15); writes packed [out, in/2]
 * u8, scale [out, in/group] f32, zero [out, in/group] u8.
 * Replaces: linnet/quant.py:83-99 `quantize_int4_groups` + :242-248 `pack_int4_groups`. */
LNQ_API LnqStatus lnq_int4_quantize(const float* weight, uint8_t* packed, float* scale,
                                    uint8_t* zero, int64_t out_features, int64_t in_features,
                                    int64_t group, void* stream);

/* Codes (any integer bytes, wrapped to 4 bits) two a byte, low first: packed[i] =
 * (codes[2i] & 15) | (codes[2i+1] & 15) << 4, for `pairs` bytes.
 * Replaces: torch/packed.py:61-75 `pack4` (i4/u4) and quant.py:242-248. */
LNQ_API LnqStatus lnq_int4_pack(const uint8_t* codes, uint8_t* packed, int64_t pairs,
                                void* stream);

/* The inverse: 2*pairs codes, u4 as uint8 (is_signed 0) or i4 sign-extended to int8
 * (is_signed 1). Replaces: torch/packed.py:27-35 `unpack4` (i4/u4). */
LNQ_API LnqStatus lnq_int4_unpack(const uint8_t* packed, void* codes, int64_t pairs,
                                  int32_t is_signed, void* stream);

/* std.quant::Int4Linear (stdlib/quant.linnet:24-29, 101-111): a signed 4-bit weight
 * [out, in] (i4 bytes [out, in/2], element 2k low, two's complement) with one scale a
 * row, weight[o, i] = q[o, i] * scale[o], in the group layout lnq_int4_linear takes:
 * packed [out, in/group, group/2] = weight ^ 0x88 (the code q + 8 of each value),
 * group_scale [out, in/group] = scale[o] (in `dtype`: bf16, f16 or f32), zero [out,
 * in/group] = 8, so that (code - zero) * scale is q * scale exactly, the product the
 * reference forms before its one rounding. in % 32 == 0, even groups dividing in.
 * No fused candidate exists in the reference (the layer runs its body, dequantize and
 * `linear`): the layout change is prepare-time, holding in * out / 2 bytes more, as the
 * reference's tinygemm repack of Int4GroupLinear does (torch_source.cpp:1482-1500). */
LNQ_API LnqStatus lnq_int4_row_prepare(const uint8_t* weight, const void* scale, uint8_t* packed,
                                       void* group_scale, uint8_t* zero, int64_t out_features,
                                       int64_t in_features, int64_t group, int32_t dtype, void* stream);

/* Packings of calibrated 4-bit checkpoints lnq_int4_repack reads. */
#define LNQ_PACKING_GPTQ 0
#define LNQ_PACKING_AWQ 1

/* A 4-bit GPTQ or AWQ layer's int32 words as Int4GroupLinear's weight and zero
 * points, eight codes a word, lowest bits first:
 *   GPTQ: qweight [in/8, out], word [c, o] holds input 8c+k of output o at bits 4k;
 *   AWQ:  qweight [in, out/8], word [i, c] holds output 8c+ORDER[k] at bits 4k,
 *         ORDER = (0, 2, 4, 6, 1, 3, 5, 7);
 *   qzeros [groups, out/8] packs the zero points along the outputs the same way
 *   (GPTQ in order, AWQ interleaved); zero_offset (0 or 1) is added to each (1 for
 *   GPTQ's first checkpoint format, which stores each less one).
 * order: GPTQ in activation order, [in] int32 (a permutation; else NULL): input i
 * of the result is checkpoint input order[i]. The entries are device memory and are
 * not checked here (an entry outside 0..in-1 reads as code 0, not a zero weight):
 * the caller passes a permutation (the Python wrapper checks it).
 * Writes packed [out, in/2] (= [out, groups, in/groups/2], low nibble first) and
 * zero [out, groups] u8. in and out are multiples of 8, groups divides in.
 * Replaces: quant.py:222-240, 300-340 (`import_quantized`'s numpy repack: `_nibbles`,
 * the AWQ column reversal, the `order` gather and `pack_int4_groups`). */
LNQ_API LnqStatus lnq_int4_repack(const int32_t* qweight, const int32_t* qzeros,
                                  const int32_t* order, int32_t packing, int32_t zero_offset,
                                  int64_t in_features, int64_t out_features, int64_t groups,
                                  uint8_t* packed, uint8_t* zero, void* stream);

/* ------------------------------------------------------- executables
 * The reference runtime's executable shape (include/linnet/runtime/runtime.h:44-94):
 * DLPack-laid-out tensors, a per-call context, and an executable of four callbacks that
 * a plan calls (ln_plan_add / ln_plan_run, runtime.h:112-131). The layouts are the
 * reference's, so its runtime can hold an executable made here; when its header is
 * included first, its declarations are used. The stream is a hipStream_t. */
#ifndef LINNET_RUNTIME_H
#define LN_CPU 1
#define LN_CUDA 2
typedef struct LnDevice {
  int32_t type; /* DLPack device type: LN_CPU, LN_CUDA; 10 is DLPack's ROCm */
  int32_t id;
} LnDevice;
typedef struct LnDataType {
  uint8_t code; /* DLPack: 0 int, 1 uint, 2 float, 4 bfloat */
  uint8_t bits;
  uint16_t lanes;
} LnDataType;
typedef struct LnTensor {
  void* data;
  LnDevice device;
  int32_t ndim;
  LnDataType dtype;
  int64_t* shape;
  int64_t* strides; /* in elements; NULL for a contiguous tensor */
  uint64_t byte_offset;
} LnTensor;
typedef struct LnContext {
  uint32_t abi_version;
  LnDevice device;
  void* stream; /* here a hipStream_t (NULL: the null stream) */
  void* workspace;
  size_t workspace_bytes;
  int32_t capturing; /* nonzero while a graph records the stream */
} LnContext;
typedef struct LnExecutable {
  uint32_t abi_version;
  void* state;
  int (*prepare)(void* state, LnContext* context);
  int (*execute)(void* state, const LnTensor* inputs, size_t input_count, LnTensor* outputs,
                 size_t output_count, LnContext* context);
  const char* (*error)(void* state);
  void (*destroy)(void* state);
} LnExecutable;
#endif

#define LNQ_DL_ROCM 10 /* DLPack's device type of a ROCm GPU */

/* An executable for std.quant::linear_int4_groups of one layer shape (in_features,
 * out_features, group; checked as lnq_int4_linear checks them; kernel an LNQ_KERNEL_*):
 * inputs x [*S, in] (bf16 or f16, contiguous), packed [out, in/group, group/2] u8,
 * scale [out, in/group] of x's dtype, zero [out, in/group] u8, and an optional fifth,
 * bias [out]; output y [*S, out] of x's dtype. Tensors are borrowed (contiguous, on a
 * ROCm or CUDA-typed device); the context's abi_version is LNQ_ABI_VERSION.
 * prepare checks the device is a gfx950 (LNQ_UNAVAILABLE otherwise) and holds nothing;
 * execute enqueues on context->stream and never waits or allocates, so it may run under
 * graph capture; error gives the state's last message; destroy frees the state.
 * *out is filled in; the caller owns it and calls destroy once.
 * Replaces: the linnet.backends executable a plugin returns for linear_int4_groups
 * (backends/contract.py:228-323, runtime.h:82-94), with the generated `_int4_linear`'s
 * semantics (torch_source.cpp:1553-1570). */
LNQ_API LnqStatus lnq_int4_linear_executable(int64_t in_features, int64_t out_features,
                                             int64_t group, int32_t kernel, LnExecutable* out);

/* ----------------------------------------------------------------- 8-bit
 * Weights [out, in] of int8 (fp8 0) or FP8 E4M3 bytes (fp8 1). Scales (f32): one per
 * row ([out], group 0), or [out/row_block, in/group] (int8 groups: row_block 1;
 * FP8 blocks: group = row_block = block).
 */

/* Symmetric int8 quantization of an f32 weight [out, in] in groups of `group` inputs:
 * scale = max|w| / 127 (0 -> 1) rounded to `scale_dtype` first, q = clip(rint(w /
 * scale), -127, 127); scale written as f32 [out, in/group].
 * Replaces: linnet/quant.py:102-121 `quantize_int8_groups`. */
LNQ_API LnqStatus lnq_int8_quantize(const float* weight, int8_t* q, float* scale,
                                    int64_t out_features, int64_t in_features, int64_t group,
                                    int32_t scale_dtype, void* stream);

/* y[rows, out] = x[rows, in] @ (w * scale)^T with the weight widened in registers and
 * x unrounded, f32 sums, rounded once to `dtype`; per-row scales multiply the sum,
 * group scales each group. in % 128 == 0 (and % group).
 * Replaces: kernels.py:375-434 `gemv8` (rows 1) and :437-592 `w8a16` (rows <= 64). */
LNQ_API LnqStatus lnq_w8a16(const void* x, const uint8_t* weight, const float* scale, void* y,
                            int64_t rows, int64_t out_features, int64_t in_features,
                            int32_t fp8, int64_t group, int64_t row_block, int32_t dtype,
                            void* stream);

/* The 8-bit weight dequantized: out[o, i] = widen(w[o, i]) * scale, f32 product
 * rounded once to `dtype`. Replaces: kernels.py:595-666 `dequantize8`. */
LNQ_API LnqStatus lnq_dequantize8(const uint8_t* weight, const float* scale, void* out,
                                  int64_t out_features, int64_t in_features, int32_t fp8,
                                  int64_t group, int64_t row_block, int32_t dtype, void* stream);

/* Each row of x [rows, in] (`dtype`) rounded to 8 bits with its own scale:
 * scale[r] = max(max|x[r]|, 1e-12) / (448 | 127), q = e4m3(clamp(x / scale, +-448))
 * rounded to nearest even, or int8 clamp(trunc(x / scale +- 0.5), +-127).
 * Replaces: kernels.py:669-753 `fp8_rows` / `int8_rows`. */
LNQ_API LnqStatus lnq_rows8(const void* x, uint8_t* q, float* x_scale, int64_t rows,
                            int64_t in_features, int32_t fp8, int32_t dtype, void* stream);

/* y[rows, out] = (q[rows, in] @ w[out, in]^T) * x_scale[rows] * scale[out] in `dtype`:
 * int8 x int8 summed exactly in int32 (fp8 0), or e4m3 x e4m3 summed in f32 (fp8 1),
 * on MFMA. in % 128 == 0.
 * Replaces: kernels.py:805-915 `int8_mm`, and `torch._scaled_mm` as
 * torch/quantized.py:129 calls it (row scales, bf16/f16 out). */
LNQ_API LnqStatus lnq_mm8(const uint8_t* q, const uint8_t* weight, const float* x_scale,
                          const float* scale, void* y, int64_t rows, int64_t out_features,
                          int64_t in_features, int32_t fp8, int32_t dtype, void* stream);

/* lnq_mm8 with the kernel named: tile_n 128 or 256 output columns a workgroup,
 * LNQ_MM8_PERSISTENT (1) the persistent form (256 x 256 tiles, one workgroup a
 * compute unit walking its tiles; out % 256 == 0, in % 256 == 0),
 * LNQ_MM8_STREAM (2) the weight-streaming form (256 x 128 tiles with x and
 * weights in stages of their own, loaded by waves of their own), 0 for
 * lnq_mm8's own choice. Every form sums the same MFMAs in the same k order:
 * the same bits.
 * No counterpart in the reference (`torch._scaled_mm` / `int8_mm` choose
 * internally): lets a test run each instance. */
#define LNQ_MM8_PERSISTENT 1
#define LNQ_MM8_STREAM 2
LNQ_API LnqStatus lnq_mm8_tiles(const uint8_t* q, const uint8_t* weight, const float* x_scale,
                                const float* scale, void* y, int64_t rows, int64_t out_features,
                                int64_t in_features, int32_t fp8, int32_t dtype, int32_t tile_n,
                                void* stream);

/* The kernel lnq_mm8 takes for rows x out_features x in_features (fp8 1: e4m3
 * operands, 0: int8) on the current device, as lnq_mm8_tiles names it (1, 2,
 * 128 or 256). */
LNQ_API LnqStatus lnq_mm8_plan(int64_t rows, int64_t out_features, int64_t in_features,
                               int32_t fp8, int32_t* tile_n);

/* Each 128 inputs (group = 128) of each row of x [rows, in] (`dtype`: bf16, f16 or f32)
 * rounded to FP8 E4M3 with a scale of their own: scale = max(max|x|, 1e-12) / 448
 * (f32, IEEE divide), q = E4M3 round-to-nearest-even of clamp(x / scale, +-448); rows
 * rows .. padded-1 are zeros with scale 1. Writes q [padded, in] and x_scale [in/128,
 * padded] f32 (x_scale[g * padded + row], the column-major scales of the reference).
 * Replaces: torch/kernels.py:757-802 `fp8_groups`. */
LNQ_API LnqStatus lnq_fp8_groups(const void* x, uint8_t* q, float* x_scale, int64_t rows,
                                 int64_t padded, int64_t in_features, int64_t group,
                                 int32_t dtype, void* stream);

/* Block-scaled FP8 x FP8: y[rows, out] = sum over 128-input blocks b of
 * (q[:, b] @ w[:, b]^T) * x_scale[b * xs_stride + row] * scale[out / 128, b], E4M3
 * operands on the FP8 MFMA, f32 sums, rounded once to `dtype` (bf16 or f16). q [rows,
 * in], w [out, in] E4M3 bytes (16-byte aligned), x_scale as lnq_fp8_groups writes it
 * (xs_stride = its padded rows), scale [out/128, in/128] f32. in, out % 128 == 0.
 * Replaces: `torch._scaled_mm` with block-wise scales as torch/quantized.py:159-166
 * (`fp8_block_linear`, rounded) calls it. */
LNQ_API LnqStatus lnq_mm8_block(const uint8_t* qx, const uint8_t* weight, const float* x_scale,
                                int64_t xs_stride, const float* scale, void* y, int64_t rows,
                                int64_t out_features, int64_t in_features, int32_t dtype,
                                void* stream);

/* ------------------------------------------------------------------- MXFP4
 * gpt-oss's expert weights: blocks [E, out, in/32, 16] bytes (32 FP4 E2M1 values a
 * block, element 2j in the low nibble of byte j), scales [E, out, in/32] E8M0 bytes
 * (a block's weights are its E2M1 values times 2^(scale - 127)).
 */

/* y[r, k, o] = sum_i x[r, k, i] * W[experts[r, k], o, i] for rows x chosen (r, k)
 * pairs, x [rows, chosen, in] of `dtype` (bf16 or f16) with element strides
 * x_row_stride and x_slot_stride (0 for an input the chosen experts of a row
 * share; both multiples of 8, x 16-byte aligned, its last axis contiguous),
 * experts [rows, chosen] int64, y [rows, chosen, out] of `dtype`. Each block's
 * products are summed in f32 and scaled, the blocks added in f32, the sum rounded
 * once. An expert index outside 0 .. num_experts-1 gives zeros. in % 32 == 0,
 * in <= 8192. Replaces: torch/kernels.py:94-209 `mxfp4_experts` (the generated
 * `_mxfp4_experts`, src/backend/torch_source.cpp:1579-1600). */
LNQ_API LnqStatus lnq_mxfp4_experts(const void* x, int64_t x_row_stride, int64_t x_slot_stride,
                                    const uint8_t* blocks, const uint8_t* scales,
                                    const int64_t* experts, void* y, int64_t rows, int64_t chosen,
                                    int64_t num_experts, int64_t out_features,
                                    int64_t in_features, int32_t dtype, void* stream);

/* ------------------------------------------------------------------------- NF4
 * std.quant::Nf4Linear (stdlib/quant.linnet:177-215): codes [out, in/2] bytes of
 * QLoRA's 4-bit NormalFloat, the first input of a pair in the low nibble, and
 * absmax [out, in/block] f32, one scale for each `block` consecutive inputs of a
 * row: weight[o, i] = nf4(q[o, i]) * absmax[o, i / block]. All three enqueue on
 * `stream` and return at once.
 */

/* The weight in `dtype` (bf16, f16 or f32), [out, in]: the code's f32 value times
 * its scale in f32, rounded once to nearest even -- bit for bit the reference's
 * `dequantize_nf4` (stdlib/quant.linnet:180-187). block even, in % block == 0.
 * Replaces: the generated torch module's lowering of `dequantize_nf4` (the
 * codebook cast, src/emit/source.cpp:120-143, then the multiply). */
LNQ_API LnqStatus lnq_nf4_dequant(const uint8_t* codes, const float* absmax, void* out,
                                  int64_t out_features, int64_t in_features, int64_t block,
                                  int32_t dtype, void* stream);

/* y[r, o] = sum_i x[r, i] * weight[o, i] (+ bias[o]) for `rows` rows of x
 * (row strides in elements), x / bias / y of `dtype` (bf16 or f16). The weight
 * is read as stored: each code's value, rounded once to `dtype`, meets x in an
 * f32 dot product; a block's sum is scaled by its absmax and the blocks added in
 * f32, the row rounded once. Up to 8 rows of x a pass over the weight (4 past
 * in = 8192). block %
 * 16 == 0, in % block == 0, in <= 32768, the codes under 2 GiB; x 16-byte aligned
 * with x_stride % 8 == 0. Replaces: `linear_nf4`'s body, the widened weight and
 * its product (stdlib/quant.linnet:189-199), for the few-row calls. */
LNQ_API LnqStatus lnq_nf4_linear(const void* x, int64_t x_stride, int64_t rows, const uint8_t* codes,
                                 const float* absmax, const void* bias, void* y, int64_t y_stride,
                                 int64_t out_features, int64_t in_features, int64_t block,
                                 int32_t dtype, void* stream);

/* A bitsandbytes 4-bit NF4 layer as Nf4Linear holds it: `codes` = `packed`
 * ([out * in / 2] bytes, the first code of a pair in the high nibble) with each
 * byte's nibbles swapped; `absmax` [out * in / block] f32 = `absmax_in` (f32)
 * as it is, or, with double quantization (nested_map and nested_absmax given),
 * absmax_in's uint8 codes decoded as nested_map[code] * nested_absmax[i /
 * nested_block] + offset, in f32 (two roundings). Replaces: quant.py:414-466
 * `_bnb_nf4` (numpy). */
LNQ_API LnqStatus lnq_nf4_repack(const uint8_t* packed, const void* absmax_in, const float* nested_absmax,
                                 const float* nested_map, int64_t nested_block, float offset,
                                 uint8_t* codes, float* absmax, int64_t out_features,
                                 int64_t in_features, int64_t block, void* stream);

/* ------------------------------------------------------- decode-step glue (bf16)
 * What a decoder layer runs between its quantized linear layers, for the int4
 * Llama-shaped decode step of BASELINE config 5. No counterpart in the reference's
 * quantized-linear path: its generated module runs these as framework ops
 * (the model card's norms, rotary embedding, attention and MLP,
 * examples/01-llama/src/lib.linnet, stdlib/nn/mlp.linnet:16-24).
 */

/* Per row of x [rows, hidden]: with delta (else NULL), x += delta rounded to bf16 in
 * place; then h = x * rsqrt(mean(x^2) + eps) * weight (weight f32 [hidden]). */
LNQ_API LnqStatus lnq_rmsnorm(void* x, const void* delta, const float* weight, void* h, int64_t rows,
                              int64_t hidden, float eps, void* stream);

/* lnq_rmsnorm with h written as x tiles (lnq_x_tiles; hidden % 256 == 0 and <=
 * 16384, operands 16-byte aligned): the same bits, for lnq_int4_linear_tiles. */
LNQ_API LnqStatus lnq_rmsnorm_tiles(void* x, const void* delta, const float* weight, void* xt, int64_t rows,
                                    int64_t hidden, float eps, void* stream);

/* lnq_rmsnorm (h_tiles 0) or lnq_rmsnorm_tiles (1) whose delta is the sum of `splits`
 * f32 partial sums parts [splits, rows, hidden] added in order and rounded once to
 * bf16 -- the output lnq_int4_linear_tiles_parts leaves in parts -- read in place
 * of a bf16 delta (hidden % 256 == 0 and <= 16384; operands 16-byte aligned). */
LNQ_API LnqStatus lnq_rmsnorm_parts(void* x, const float* parts, int32_t splits, const float* weight, void* h,
                                    int32_t h_tiles, int64_t rows, int64_t hidden, float eps, void* stream);

/* One decode step of grouped-query attention: q [rows, heads*head_dim], k and v
 * [rows, kv_heads*head_dim] (bf16); rotary embedding of q and k with cos/sin f32
 * [head_dim/2] (pairs i, i + head_dim/2); k and v stored (rounded to bf16) at `pos`
 * of the bf16 caches kt_cache [rows, kv_heads, head_dim, cap] (transposed) and
 * v_cache [rows, kv_heads, cap, head_dim]; out [rows, heads*head_dim] = softmax(q K^T / sqrt(head_dim)) V over
 * positions 0..pos, in chunks of 64 positions merged in order (split-K). head_dim 64
 * or 128; heads / kv_heads <= 8; pos < 262144; cap a multiple of 4 and the caches
 * 16-byte aligned.
 * `workspace` (f32, caller-owned) holds lnq_decode_attention_workspace(rows, kv_heads,
 * head_dim, pos) floats. q_stride and kv_stride are the row strides (elements) of q
 * and of k / v, at least a row each when rows > 1 (unread at one row): q, k and v may
 * be column slices of one joined q|k|v projection's output. */
LNQ_API LnqStatus lnq_decode_attention(const void* q, const void* k, const void* v, const float* cos,
                                       const float* sin, void* kt_cache, void* v_cache, void* out,
                                       float* workspace, int64_t workspace_floats, int64_t rows,
                                       int64_t heads, int64_t kv_heads, int64_t head_dim, int64_t cap,
                                       int64_t pos, int64_t q_stride,
                                       int64_t kv_stride, void* stream);

/* lnq_decode_attention with the position in device memory (`pos`: one int32), so
 * that a step recorded into a graph moves along the cache on each replay when the
 * graph also advances the position. cos_table / sin_table are f32 [cap, head_dim/2]
 * (row p: cos / sin of p times the rotary frequencies), read at row pos; the
 * workspace is sized for position cap - 1 and the grid covers the whole cache
 * (chunks past pos return at once). A position outside [0, cap) writes nothing to
 * the caches and zeros to `out`.
 * Replaces: the rotary-position bookkeeping of the generated decode step
 * (python/linnet/src/linnet/torch/compiled.py:430-503), which passes the position
 * from the host on every call. */
LNQ_API LnqStatus lnq_decode_attention_at(const void* q, const void* k, const void* v, const float* cos_table,
                                          const float* sin_table, void* kt_cache, void* v_cache, void* out,
                                          float* workspace, int64_t workspace_floats, int64_t rows, int64_t heads,
                                          int64_t kv_heads, int64_t head_dim, int64_t cap, const int32_t* pos,
                                          int64_t q_stride, int64_t kv_stride, void* stream);

/* lnq_decode_attention (pos_dev NULL: position pos, cos / sin at it) or
 * lnq_decode_attention_at (pos_dev the device position, cos / sin the tables over
 * the cache, pos ignored), the output written as x tiles (lnq_x_tiles; heads *
 * head_dim % 256 == 0, out_tiles 16-byte aligned): the same bits, for the o
 * projection's lnq_int4_linear_tiles. */
LNQ_API LnqStatus lnq_decode_attention_tiles(const void* q, const void* k, const void* v, const float* cos,
                                             const float* sin, void* kt_cache, void* v_cache, void* out_tiles,
                                             float* workspace, int64_t workspace_floats, int64_t rows, int64_t heads,
                                             int64_t kv_heads, int64_t head_dim, int64_t cap, int64_t pos,
                                             const int32_t* pos_dev, int64_t q_stride, int64_t kv_stride,
                                             void* stream);

/* Floats of lnq_decode_attention's workspace: rows * kv_heads * ceil((pos + 1) / 64)
 * * 8 * (head_dim + 2). */
LNQ_API int64_t lnq_decode_attention_workspace(int64_t rows, int64_t kv_heads, int64_t head_dim,
                                               int64_t pos);

/* Floats of the workspace lnq_decode_attention_noalloc holds on each GPU (32 MiB). */
#define LNQ_DECODE_ATTENTION_SCRATCH_FLOATS 8388608

/* lnq_decode_attention without a workspace argument and without allocating: the
 * split-K partial results go to a static device array of the library,
 * LNQ_DECODE_ATTENTION_SCRATCH_FLOATS floats on each GPU it runs on, held until the
 * process ends (its address looked up once per device on the first call there).
 * Refuses a step whose workspace (lnq_decode_attention_workspace) exceeds it, e.g.
 * past 32 rows x 8 KV heads x 1984 positions at head_dim 128. Every call on a GPU
 * shares that GPU's array, which keeps the last call's contents (no entry needs to
 * start at zero): calls that overlap on one GPU (two streams, two threads) race.
 * No counterpart in the reference: for callers that cannot allocate device memory --
 * code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc. */
LNQ_API LnqStatus lnq_decode_attention_noalloc(const void* q, const void* k, const void* v,
                                               const float* cos, const float* sin, void* kt_cache,
                                               void* v_cache, void* out, int64_t rows, int64_t heads,
                                               int64_t kv_heads, int64_t head_dim, int64_t cap,
                                               int64_t pos, int64_t q_stride, int64_t kv_stride,
                                               void* stream);

/* A prompt's rotary embedding and cache writes (bf16): for positions 0..positions-1,
 * q [positions, heads*head_dim], k and v [positions, kv_heads*head_dim] (rows
 * in_stride elements apart: column slices of a joined q|k|v output); q and k
 * rotated in f32 (pairs i, i + head_dim/2, cos / sin tables f32 [cap, head_dim/2]
 * read at each position) and rounded to bf16; q_out [heads, positions, head_dim],
 * k_out and v_out [kv_heads, positions, head_dim]; k also into kt_cache [kv_heads,
 * head_dim, cap] (transposed) and v into v_cache [kv_heads, cap, head_dim] at
 * positions 0..positions-1. One sequence (one row of the caches).
 * Replaces: the rotary embedding (examples/01-llama/src/rope.linnet:11), the
 * head split and the cache writes of the decoder card's prompt attention
 * (examples/01-llama/src/attention.linnet:35-56, 114-119), which the generated
 * module runs as framework ops. */
LNQ_API LnqStatus lnq_prefill_rope(const void* q, const void* k, const void* v, int64_t in_stride,
                                   const float* cos_table, const float* sin_table, void* q_out, void* k_out,
                                   void* v_out, void* kt_cache, void* v_cache, int64_t positions, int64_t heads,
                                   int64_t kv_heads, int64_t head_dim, int64_t cap, void* stream);

/* a = silu(g) * u = g / (1 + exp(-g)) * u for n bf16 elements, f32 math. */
LNQ_API LnqStatus lnq_silu_mul(const void* g, const void* u, void* a, int64_t n, void* stream);

/* The same over rows: a [rows, width] (contiguous) = silu(g) * u with the rows of
 * g and u g_stride and u_stride elements apart (e.g. the halves of a joined
 * gate|up projection's output [rows, 2*width]: u = g + width, both strides 2*width). */
LNQ_API LnqStatus lnq_silu_mul_rows(const void* g, const void* u, void* a, int64_t rows, int64_t width,
                                    int64_t g_stride, int64_t u_stride, void* stream);

/* lnq_silu_mul_rows with a written as x tiles (lnq_x_tiles; width % 256 == 0): the
 * same bits, for lnq_int4_linear_tiles. */
LNQ_API LnqStatus lnq_silu_mul_tiles(const void* g, const void* u, void* xt, int64_t rows, int64_t width,
                                     int64_t g_stride, int64_t u_stride, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LINNET_QUANT_H */
