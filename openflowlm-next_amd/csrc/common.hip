// common.hip -- version and status text of the C ABI.
#include "q4mi_internal.h"

extern "C" int q4mi_version(void) { return 100; }

extern "C" const char* q4mi_strerror(int status) {
    switch (status) {
        case Q4MI_OK: return "ok";
        case Q4MI_E_SHAPE: return "shape not supported by the layout (N % 64, K % 32, or a kernel's own multiple)";
        case Q4MI_E_ARG: return "invalid argument (NULL pointer, dtype, block width or mode)";
        case Q4MI_E_WORKSPACE: return "workspace missing or smaller than the *_workspace_bytes query";
        case Q4MI_E_LAUNCH: return "HIP kernel launch failed";
        case Q4MI_E_RANGE: return "count out of the supported range";
        default: return "unknown status";
    }
}
