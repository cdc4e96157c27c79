// Host-side helpers shared by the C-ABI launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "flaggems_vllm_amd.h"

namespace fgv {

// Records msg as this thread's last error and returns code.
int fail(int code, const char* msg);

inline bool aligned(const void* p, uintptr_t bytes) {
    return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0;
}

// Status of the launch just issued: 0, or the positive hipError_t.
inline int launch_status() {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? FGV_OK : static_cast<int>(e);
}

}  // namespace fgv
