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

// CUs of the current device (256 on MI355X).
inline int cu_count() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    return cus;
}

}  // namespace fgv
