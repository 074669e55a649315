// Host-side argument checks shared by the C-ABI entry points.  Each check maps
// to one status code of include/grout_attn_hip.h and runs before any HIP call,
// so a rejected call never touches the device.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "grout_attn_hip.h"

namespace grout {

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline hipStream_t to_hip(grout_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Launch status: 0 or the positive hipError_t of the last launch.
inline int32_t launch_status() {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? GROUT_OK : static_cast<int32_t>(e);
}

}  // namespace grout

#define GROUT_REQUIRE(cond, code) \
    do {                          \
        if (!(cond)) return (code); \
    } while (0)

#define GROUT_REQUIRE_PTR(p)                                  \
    do {                                                      \
        if ((p) == nullptr) return GROUT_ERR_NULL_POINTER;    \
        if (!::grout::aligned16(p)) return GROUT_ERR_ALIGNMENT; \
    } while (0)
