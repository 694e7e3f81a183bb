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

}  // namespace hsmoe
