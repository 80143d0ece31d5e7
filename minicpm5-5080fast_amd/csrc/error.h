// error.h - thread-local diagnostics behind mc_last_error (the reference's
// convention, native/runtime/error.{h,cpp}: status code + English message).
#pragma once

#include <hip/hip_runtime.h>

#include "minicpm_runtime.h"

namespace mckv {

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

// Maps a HIP launch/API error to MC_E_CUDA with a message; MC_OK otherwise.
mc_status_t check_hip(hipError_t e, const char* what);

// Last launch error of this thread (hipGetLastError) as an mc_status_t.
inline mc_status_t check_launch(const char* what) {
    return check_hip(hipGetLastError(), what);
}

}  // namespace mckv

// Runs a body that may throw and converts any exception to MC_E_INTERNAL, so
// no C++ exception crosses the C ABI.
#define MC_GUARD_BEGIN try {
#define MC_GUARD_END                                              \
    }                                                             \
    catch (const std::exception& ex) {                            \
        mckv::set_error("internal error: %s", ex.what());         \
        return MC_E_INTERNAL;                                     \
    }                                                             \
    catch (...) {                                                 \
        mckv::set_error("internal error: unknown exception");     \
        return MC_E_INTERNAL;                                     \
    }
