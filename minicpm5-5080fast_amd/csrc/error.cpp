// error.cpp - thread-local error buffer and mc_last_error.
#include "error.h"

#include <cstdarg>
#include <cstdio>
#include <cstdlib>

#include "trace.h"

namespace mckv {

namespace {
thread_local char g_err[512] = "";
}

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

mc_status_t check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return MC_OK;
    (void)hipGetLastError();
    set_error("%s: %s", what, hipGetErrorString(e));
    return MC_E_CUDA;
}

bool trace_enabled() {
    static const bool on = std::getenv("MC_ROCTX") != nullptr;
    return on;
}

}  // namespace mckv

extern "C" const char* mc_last_error(void) { return mckv::g_err; }
