// Host-side helpers shared by the C-ABI entry points: argument checks that
// return a status instead of aborting, per-thread error text, launch checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/soinfer_amd.h"

namespace soi {

void set_last_error(const char* fmt, ...);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int64_t ceil_div64(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Check the last launch on this thread; map failure to SOI_ERR_HIP.
inline int launch_status(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_last_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
        return SOI_ERR_HIP;
    }
    return SOI_OK;
}

}  // namespace soi

#define SOI_REQUIRE(cond, ...)                   \
    do {                                         \
        if (!(cond)) {                           \
            ::soi::set_last_error(__VA_ARGS__);  \
            return SOI_ERR_INVALID_ARGUMENT;     \
        }                                        \
    } while (0)

#define SOI_HIP_TRY(expr, what)                                                               \
    do {                                                                                      \
        hipError_t _soi_e = (expr);                                                           \
        if (_soi_e != hipSuccess) {                                                           \
            ::soi::set_last_error("%s: %s failed: %s", what, #expr, hipGetErrorString(_soi_e)); \
            return SOI_ERR_HIP;                                                               \
        }                                                                                     \
    } while (0)
