// Host-side helpers shared by the libhsmoe translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hsmoe.h"

namespace hsmoe {

// Records a printf-style message as this thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Returns HSMOE_OK, or HSMOE_ERR_LAUNCH with the HIP error recorded.
int check_launch(const char* what);

inline bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// Expert weights are read through buffer resources with 32-bit offsets: an
// expert matrix (d x i, up to 2 bytes per element) must stay below 4 GiB.
inline bool expert_fits(int64_t d, int64_t i) { return (uint64_t)d * (uint64_t)i * 2 < (1ull << 32); }

// Compute units of the current device (256, the MI355X's count, when the query fails).
inline int device_cus() {
  int cus = 256, dev = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
    cus = 256;
  return cus;
}

}  // namespace hsmoe
