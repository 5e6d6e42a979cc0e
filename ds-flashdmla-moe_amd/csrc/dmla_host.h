// Host-side helpers shared by the C-ABI entry points: error reporting and argument checks.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "flashdmla.h"

namespace dmla {

// Records a printf-style message for dmla_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Clears the thread's error message; every entry point calls it first.
void clear_error();

// Converts a pending launch error into DMLA_ERR_HIP.
int check_launch(const char* what);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool mult8(int64_t s) { return (s % 8) == 0; }

// Number of compute units of the current device (cached per device).
int device_cu_count();

}  // namespace dmla
