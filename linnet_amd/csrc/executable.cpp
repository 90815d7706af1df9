// The int4 linear as an executable of the reference runtime's shape
// (include/linnet/runtime/runtime.h:44-94): a state behind four callbacks, tensors
// described DLPack's way, work enqueued on the context's stream.
//
// The executable holds the layer's shape only: its weights arrive as inputs on
// every call (borrowed, as a plan passes them), nothing is prepared into device
// memory, and execute allocates nothing and never waits, so a plan may capture
// it into a graph.
#include <cstdlib>
#include <cstring>
#include <new>

#include "common.hpp"

namespace lnq {
namespace {

struct Int4Executable {
  int64_t in_features;
  int64_t out_features;
  int64_t group;
  int32_t kernel;
  int32_t device = -1;  // the device prepare checked
  char message[512] = {0};
};

int fail(Int4Executable* e, int code, const char* fmt, ...) __attribute__((format(printf, 3, 4)));
int fail(Int4Executable* e, int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(e->message, sizeof(e->message), fmt, args);
  va_end(args);
  return code;
}

bool on_gpu(const LnDevice& d) { return d.type == LNQ_DL_ROCM || d.type == LN_CUDA; }

// Element count of a contiguous tensor's dimensions, or -1 when the strides are
// not row-major.
int64_t contiguous_numel(const LnTensor& t) {
  int64_t n = 1;
  for (int i = t.ndim - 1; i >= 0; --i) {
    if (t.shape[i] < 0) return -1;
    if (t.strides != nullptr && t.shape[i] > 1 && t.strides[i] != n) return -1;
    n *= t.shape[i];
  }
  return n;
}

bool same_dtype(const LnDataType& a, const LnDataType& b) {
  return a.code == b.code && a.bits == b.bits && a.lanes == b.lanes;
}

const char* dtype_name(const LnDataType& t) {
  if (t.code == 4 && t.bits == 16) return "bf16";
  if (t.code == 2 && t.bits == 16) return "f16";
  if (t.code == 1 && t.bits == 8) return "u8";
  return "another type";
}

void* address(const LnTensor& t) { return static_cast<char*>(t.data) + t.byte_offset; }

int prepare(void* state, LnContext* context) {
  auto* e = static_cast<Int4Executable*>(state);
  if (context == nullptr || context->abi_version != LNQ_ABI_VERSION)
    return fail(e, LNQ_ERROR, "int4_linear: context ABI %u, this library implements %u",
                context == nullptr ? 0u : context->abi_version, static_cast<unsigned>(LNQ_ABI_VERSION));
  if (!on_gpu(context->device))
    return fail(e, LNQ_UNAVAILABLE, "int4_linear: the HIP kernels run on a GPU, not device type %d",
                context->device.type);
  int32_t gfx950 = 0, cus = 0;
  if (lnq_device_probe(context->device.id, &gfx950, &cus) != LNQ_OK || !gfx950)
    return fail(e, LNQ_UNAVAILABLE, "int4_linear: device %d is not a gfx950 (MI355X)", context->device.id);
  e->device = context->device.id;
  e->message[0] = '\0';
  return LNQ_OK;
}

int execute(void* state, const LnTensor* inputs, size_t input_count, LnTensor* outputs, size_t output_count,
            LnContext* context) {
  auto* e = static_cast<Int4Executable*>(state);
  if (context == nullptr || context->abi_version != LNQ_ABI_VERSION)
    return fail(e, LNQ_ERROR, "int4_linear: context ABI %u, this library implements %u",
                context == nullptr ? 0u : context->abi_version, static_cast<unsigned>(LNQ_ABI_VERSION));
  if (e->device < 0) return fail(e, LNQ_ERROR, "int4_linear: execute before prepare");
  if (!(input_count == 4 || input_count == 5) || output_count != 1 || inputs == nullptr || outputs == nullptr)
    return fail(e, LNQ_ERROR, "int4_linear: takes (x, packed, scale, zero[, bias]) -> (y), got %zu -> %zu",
                input_count, output_count);
  const LnTensor& x = inputs[0];
  const LnTensor& packed = inputs[1];
  const LnTensor& scale = inputs[2];
  const LnTensor& zero = inputs[3];
  const LnTensor* bias = input_count == 5 ? &inputs[4] : nullptr;
  const LnTensor& y = outputs[0];
  const LnTensor* all[] = {&x, &packed, &scale, &zero, &y, bias};
  for (const LnTensor* t : all) {
    if (t == nullptr) continue;
    if (!on_gpu(t->device) || t->device.id != e->device)
      return fail(e, LNQ_ERROR, "int4_linear: a tensor on device (%d, %d), the executable runs on GPU %d",
                  t->device.type, t->device.id, e->device);
    if (t->ndim < 1 || t->shape == nullptr || contiguous_numel(*t) < 0)
      return fail(e, LNQ_ERROR, "int4_linear: tensors are contiguous and at least 1-D");
    if (t->data == nullptr) return fail(e, LNQ_ERROR, "int4_linear: null tensor data");
  }
  const LnDataType bf16{4, 16, 1}, f16{2, 16, 1}, u8{1, 8, 1};
  int32_t dtype;
  if (same_dtype(x.dtype, bf16)) dtype = LNQ_BF16;
  else if (same_dtype(x.dtype, f16)) dtype = LNQ_F16;
  else return fail(e, LNQ_ERROR, "int4_linear: x is bf16 or f16, not %s", dtype_name(x.dtype));
  const int64_t in = e->in_features, out = e->out_features, g = e->group;
  if (x.shape[x.ndim - 1] != in)
    return fail(e, LNQ_ERROR, "int4_linear: x's last axis is %lld, the layer takes %lld",
                static_cast<long long>(x.shape[x.ndim - 1]), static_cast<long long>(in));
  const int64_t rows = contiguous_numel(x) / in;
  if (!(packed.ndim == 3 && packed.shape[0] == out && packed.shape[1] == in / g && packed.shape[2] == g / 2 &&
        same_dtype(packed.dtype, u8)))
    return fail(e, LNQ_ERROR, "int4_linear: packed is [%lld, %lld, %lld] u8", static_cast<long long>(out),
                static_cast<long long>(in / g), static_cast<long long>(g / 2));
  if (!(scale.ndim == 2 && scale.shape[0] == out && scale.shape[1] == in / g && same_dtype(scale.dtype, x.dtype)))
    return fail(e, LNQ_ERROR, "int4_linear: scale is [%lld, %lld] of x's type (%s)", static_cast<long long>(out),
                static_cast<long long>(in / g), dtype_name(x.dtype));
  if (!(zero.ndim == 2 && zero.shape[0] == out && zero.shape[1] == in / g && same_dtype(zero.dtype, u8)))
    return fail(e, LNQ_ERROR, "int4_linear: zero is [%lld, %lld] u8", static_cast<long long>(out),
                static_cast<long long>(in / g));
  if (bias != nullptr && !(bias->ndim == 1 && bias->shape[0] == out && same_dtype(bias->dtype, x.dtype)))
    return fail(e, LNQ_ERROR, "int4_linear: bias is [%lld] of x's type", static_cast<long long>(out));
  bool y_ok = y.ndim == x.ndim && y.shape[y.ndim - 1] == out && same_dtype(y.dtype, x.dtype);
  for (int i = 0; y_ok && i + 1 < x.ndim; ++i) y_ok = y.shape[i] == x.shape[i];
  if (!y_ok) return fail(e, LNQ_ERROR, "int4_linear: y is x's shape with the last axis %lld, of x's type",
                         static_cast<long long>(out));
  // The kernel choice reads the current device's properties: the executable's
  // device for the call, the caller's again after it.
  int current = -1;
  if (hipGetDevice(&current) != hipSuccess) current = -1;
  if (current != e->device && hipSetDevice(e->device) != hipSuccess)
    return fail(e, LNQ_ERROR, "int4_linear: cannot select device %d", e->device);
  const LnqStatus status =
      lnq_int4_linear(address(x), static_cast<const uint8_t*>(address(packed)), address(scale),
                      static_cast<const uint8_t*>(address(zero)), bias == nullptr ? nullptr : address(*bias), address(y),
                      rows, in, out, g, dtype, e->kernel, context->stream);
  if (current >= 0 && current != e->device) (void)hipSetDevice(current);
  if (status != LNQ_OK) return fail(e, status, "%s", lnq_last_error());
  e->message[0] = '\0';
  return LNQ_OK;
}

const char* error(void* state) { return static_cast<Int4Executable*>(state)->message; }

void destroy(void* state) { delete static_cast<Int4Executable*>(state); }

}  // namespace
}  // namespace lnq

using namespace lnq;

extern "C" {

LNQ_API LnqStatus lnq_int4_linear_executable(int64_t in_features, int64_t out_features, int64_t group, int32_t kernel,
                                             LnExecutable* out) {
  LNQ_REQUIRE(out != nullptr, "lnq_int4_linear_executable: null executable");
  int32_t chosen = 0;
  // The shape checks of lnq_int4_linear (one row stands for any).
  if (lnq_int4_linear_plan(1, in_features, out_features, group, LNQ_BF16,
                           kernel == LNQ_KERNEL_GEMV ? LNQ_KERNEL_AUTO : kernel, &chosen) != LNQ_OK)
    return LNQ_ERROR;
  auto* state = new (std::nothrow) Int4Executable{in_features, out_features, group, kernel};
  LNQ_REQUIRE(state != nullptr, "lnq_int4_linear_executable: out of host memory");
  out->abi_version = LNQ_ABI_VERSION;
  out->state = state;
  out->prepare = prepare;
  out->execute = execute;
  out->error = error;
  out->destroy = destroy;
  clear_error();
  return LNQ_OK;
}

}  // extern "C"
