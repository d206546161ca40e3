// q4mi_internal.h -- host-side helpers shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/q4mi.h"

namespace q4mi {

// Status of the launch just enqueued (does not synchronize).
inline int launch_status() {
    return hipGetLastError() == hipSuccess ? Q4MI_OK : Q4MI_E_LAUNCH;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace q4mi
