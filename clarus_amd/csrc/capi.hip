// Library-wide C entry points: ABI version, struct sizes, per-thread error text.
#include <atomic>
#include <string.h>

#include "capi.hpp"

namespace clarus {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = 0; }

static std::atomic<int> g_cus[64];

int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int n = g_cus[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    g_cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

static thread_local char g_kernel[160];

void note_kernel(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_kernel, sizeof(g_kernel), fmt, ap);
  va_end(ap);
}

}  // namespace clarus

extern "C" {

int clarus_hip_abi_version(void) { return CLARUS_HIP_ABI_VERSION; }

size_t clarus_hip_sizeof_gemm_args(void) { return sizeof(ClarusGemmArgs); }

size_t clarus_hip_sizeof_conv_args(void) { return sizeof(ClarusConvArgs); }

const char* clarus_hip_last_error(void) { return clarus::g_err; }

const char* clarus_hip_last_kernel(void) { return clarus::g_kernel; }

}  // extern "C"
