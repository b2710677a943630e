// vt_internal.h -- host-side helpers of the C ABI: error state, argument
// checks, launch checks.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/vt_abi.h"

namespace vt {

void set_error(const char *fmt, ...);
void clear_error();

inline hipStream_t as_stream(vt_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Return VT_ERR_HIP if a HIP call or the last launch failed.
#define VT_HIP_CHECK(expr)                                                                                        \
    do {                                                                                                          \
        hipError_t e_ = (expr);                                                                                   \
        if (e_ != hipSuccess) {                                                                                   \
            ::vt::set_error("%s: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, __LINE__);                \
            return VT_ERR_HIP;                                                                                    \
        }                                                                                                         \
    } while (0)

#define VT_LAUNCH_CHECK(what)                                                                                     \
    do {                                                                                                          \
        hipError_t e_ = hipGetLastError();                                                                        \
        if (e_ != hipSuccess) {                                                                                   \
            ::vt::set_error("launch of %s failed: %s", what, hipGetErrorString(e_));                              \
            return VT_ERR_HIP;                                                                                    \
        }                                                                                                         \
    } while (0)

#define VT_REQUIRE(cond, ...)                                                                                     \
    do {                                                                                                          \
        if (!(cond)) {                                                                                            \
            ::vt::set_error(__VA_ARGS__);                                                                         \
            return VT_ERR_INVALID;                                                                                \
        }                                                                                                         \
    } while (0)

} // namespace vt
