// Error reporting shared by the C-ABI entry points (include/solort_hip.h).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../../include/solort_hip.h"

namespace solort {

// Records a printf-style message for solort_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Returns 0 if the last launch on this thread succeeded, else records and
// returns the hipError_t.
int check_launch(const char* what);

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace solort
