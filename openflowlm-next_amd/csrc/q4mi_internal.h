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

// The kernels move packed weights, activations, outputs and workspaces in 16-byte vectors.
inline bool misaligned16(const void* p) { return ((uintptr_t)p & 15u) != 0; }

}  // namespace q4mi
