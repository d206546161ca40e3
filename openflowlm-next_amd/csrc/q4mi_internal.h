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

// Whether the byte ranges [a, a + na) and [b, b + nb) intersect (a NULL pointer or an
// empty range intersects nothing).
inline bool overlaps(const void* a, int64_t na, const void* b, int64_t nb) {
    const char *ca = (const char*)a, *cb = (const char*)b;
    return a && b && na > 0 && nb > 0 && ca < cb + nb && cb < ca + na;
}

// x_out = res + the S partial planes (split order) and xn = bf16 of its RMSNorm (q4_rmsnorm_add's
// arithmetic) in one launch, M rows of N <= 4096 (norm.hip).
int rmsnorm_planes(const float* res, const float* part, int S, const void* w, int w_dtype, float* x_out, void* xn,
                   int M, int64_t N, float eps, void* stream);

}  // namespace q4mi
