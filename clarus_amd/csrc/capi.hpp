// Host-side helpers shared by the C entry points: error reporting and launch checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/clarus_hip.h"

namespace clarus {

// record the calling thread's last failure (read by clarus_hip_last_error)
void set_error(const char* fmt, ...);
void clear_error();
// compute units of the calling thread's current device (hipDeviceAttributeMultiprocessorCount,
// looked up once per device; 256 on a whole MI355X, fewer on a partition); sizes persistent grids
int device_cus();

// record the kernel a launching entry point chose for the calling thread's current call (read by
// clarus_hip_last_kernel); a diagnostic only, never read by the dispatch
void note_kernel(const char* fmt, ...);

inline bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// returns CLARUS_ELAUNCH (with the HIP error text) if the last launch failed, else CLARUS_OK
inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return CLARUS_ELAUNCH;
  }
  return CLARUS_OK;
}

#define CLARUS_REQUIRE(cond, ...)   \
  do {                              \
    if (!(cond)) {                  \
      ::clarus::set_error(__VA_ARGS__); \
      return CLARUS_EINVAL;         \
    }                               \
  } while (0)

}  // namespace clarus
