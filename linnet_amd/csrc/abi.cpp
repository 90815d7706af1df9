// The C ABI's bookkeeping: version, thread-local last error, device probe.
// Mirrors the reference runtime's status / ln_last_error convention
// (include/linnet/runtime/runtime.h:37-40, :99; src/runtime/runtime.cpp:28).
#include <cstring>
#include <string>

#include "common.hpp"

namespace lnq {

static thread_local std::string last_error;

void set_error(const char* fmt, ...) {
  char buffer[1024];
  va_list args;
  va_start(args, fmt);
  std::vsnprintf(buffer, sizeof buffer, fmt, args);
  va_end(args);
  last_error = buffer;
}

void clear_error() { last_error.clear(); }

}  // namespace lnq

extern "C" {

LNQ_API uint32_t lnq_abi_version(void) { return LNQ_ABI_VERSION; }

LNQ_API const char* lnq_last_error(void) { return lnq::last_error.c_str(); }

LNQ_API LnqStatus lnq_device_probe(int32_t device, int32_t* is_gfx950, int32_t* compute_units) {
  int count = 0;
  hipError_t err = hipGetDeviceCount(&count);
  if (err != hipSuccess || count == 0) {
    lnq::set_error("no HIP device: %s", err == hipSuccess ? "count 0" : hipGetErrorString(err));
    return LNQ_UNAVAILABLE;
  }
  LNQ_REQUIRE(device >= 0 && device < count, "device %d out of range (%d devices)", device, count);
  hipDeviceProp_t props;
  LNQ_HIP_CHECK(hipGetDeviceProperties(&props, device));
  if (is_gfx950) *is_gfx950 = std::strncmp(props.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
  if (compute_units) *compute_units = props.multiProcessorCount;
  lnq::clear_error();
  return LNQ_OK;
}

}  // extern "C"
